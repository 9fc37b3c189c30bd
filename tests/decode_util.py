"""Builders shared by the decode-step tests: a synthetic model as the
reference's int4_hip argument lists (device tensors) plus the matching
oracle layers (host arrays)."""
import numpy as np
import torch

import int4_hip
import r4q_oracle as O
import r4q_synth as S


class Model:
    pass


def build(dev, *, D, I, H, Hk, L, vocab, max_seq, seed, bits=None, lm_bits=16, batch=1,
          fill=0, kv_scale=False, rope_len=None):
    """bits: {(layer, group): 4|8}.  The first `fill` cache positions hold FP8
    codes of N(0,1) values (encoded with the oracle)."""
    hd = 128
    g = S.gen(seed)
    m = Model()
    m.D, m.I, m.H, m.Hk, m.L, m.hd, m.vocab, m.max_seq, m.eps = D, I, H, Hk, L, hd, vocab, max_seq, 1e-6
    m.batch = batch
    m.cpu_layers, m.oracle_layers = [], []
    names = ("qkv", "o", "gu", "down")
    lists = {k: [] for k in ("qkv_w", "qkv_s", "qkv_N", "o_w", "o_s", "o_N", "gu_w", "gu_s",
                             "gu_N", "down_w", "down_s", "down_N", "in_norm_w", "post_norm_w",
                             "q_norm_w", "k_norm_w")}
    for li in range(L):
        lb = {n: (bits or {}).get((li, n), 4) for n in names}
        ly = S.make_layer(D, I, H, Hk, hd, g, bits=lb)
        m.cpu_layers.append(ly)
        kw = {}
        for n in names:
            kw[n + "_w"] = ly[n + "_w"].numpy()
            kw[n + "_s"] = None if ly[n + "_s"] is None else ly[n + "_s"].numpy().reshape(ly[n + "_N"], -1, 2)
            kw[n + "_bits"] = ly[n + "_bits"]
            lists[n + "_w"].append(ly[n + "_w"].to(dev))
            lists[n + "_s"].append(None if ly[n + "_s"] is None else ly[n + "_s"].to(dev))
            lists[n + "_N"].append(ly[n + "_N"])
        for src, dst in (("in_norm", "in_norm_w"), ("post_norm", "post_norm_w"),
                         ("q_norm", "q_norm_w"), ("k_norm", "k_norm_w")):
            kw[src] = ly[src].numpy()
            lists[dst].append(ly[src].to(dev))
        m.oracle_layers.append(O.Layer(**kw))
    m.lists = lists
    m.final_norm = S.norm_weight(D, g)
    lw, ls = S.weight(vocab, D, lm_bits, g)
    m.lm_w, m.lm_s, m.lm_bits = lw, ls, lm_bits
    m.embed = (torch.randn(vocab, D, generator=g) * 0.5).half()
    m.cos, m.sin = S.rope_tables(hd, rope_len or max_seq)
    # caches
    m.kc_np = np.zeros((L, batch, Hk, max_seq, hd), np.uint8)
    m.vc_np = np.zeros_like(m.kc_np)
    if fill:
        for li in range(L):
            m.kc_np[li, :, :, :fill] = O.fp8_encode(
                torch.randn(batch, Hk, fill, hd, generator=g).float().numpy())
            m.vc_np[li, :, :, :fill] = O.fp8_encode(
                torch.randn(batch, Hk, fill, hd, generator=g).float().numpy())
    m.k_scales = m.v_scales = None
    if kv_scale:
        m.k_scales = [(0.5 + torch.rand(Hk, generator=g)).float() for _ in range(L)]
        m.v_scales = [(0.5 + torch.rand(Hk, generator=g)).float() for _ in range(L)]
    m.dev = dev
    m.reset_caches()
    m.final_norm_d = m.final_norm.to(dev)
    m.lm_w_d = m.lm_w.to(dev)
    m.lm_s_d = None if m.lm_s is None else m.lm_s.to(dev)
    m.embed_d = m.embed.to(dev)
    m.cos_d, m.sin_d = m.cos.to(dev), m.sin.to(dev)
    m.kv_scales = None if not kv_scale else ([t.to(dev) for t in m.k_scales],
                                             [t.to(dev) for t in m.v_scales])
    return m


def _reset(self):
    self.k_caches = [torch.from_numpy(self.kc_np[li].copy()).to(self.dev) for li in range(self.L)]
    self.v_caches = [torch.from_numpy(self.vc_np[li].copy()).to(self.dev) for li in range(self.L)]


Model.reset_caches = _reset


def layer_args(m, pos):
    l = m.lists
    return (l["qkv_w"], l["qkv_s"], l["qkv_N"], l["o_w"], l["o_s"], l["o_N"], l["gu_w"], l["gu_s"],
            l["gu_N"], l["down_w"], l["down_s"], l["down_N"], l["in_norm_w"], l["post_norm_w"],
            l["q_norm_w"], l["k_norm_w"], m.cos_d, m.sin_d, pos, m.H, m.Hk, m.hd, m.D, m.I, m.eps)


def step_logits(m, hidden, pos):
    had = torch.zeros(32, 32, dtype=torch.float16, device=m.dev)
    return int4_hip.decode_step_logits(hidden, *layer_args(m, pos), m.k_caches, m.v_caches,
                                       m.final_norm_d, m.lm_w_d, m.lm_s_d, m.vocab, m.D, had,
                                       kv_scales=m.kv_scales)


def bench_args(m, start_pos):
    had = torch.zeros(32, 32, dtype=torch.float16, device=m.dev)
    return layer_args(m, start_pos) + (m.k_caches, m.v_caches, m.final_norm_d, m.lm_w_d, m.lm_s_d,
                                       m.vocab, m.D, had)


def gpu_kv_at(m, pos, b=0):
    """Per layer (k_bytes, v_bytes) [Hk, hd] the GPU wrote at `pos`."""
    return [(m.k_caches[li][b, :, pos].cpu().numpy(), m.v_caches[li][b, :, pos].cpu().numpy())
            for li in range(m.L)]


def check_forced_kv(forced, kv_trace, rel=2.0 ** -8):
    """Every GPU KV code that differs from the oracle's own must be the code
    of a value within `rel` (relative to max(|x|, row rms)) of the oracle's
    pre-quantisation value x: the difference comes from last-bit rounding
    upstream of the encoder, never from the encoder or the indexing.
    Returns the number of differing codes."""
    n_diff = 0
    for (gk, gv), (ok, ov, kpre, vpre) in zip(forced, kv_trace):
        for g, o, x in ((gk, ok, kpre), (gv, ov, vpre)):
            x = x.astype(np.float64)
            rms = np.sqrt((x ** 2).mean(axis=-1, keepdims=True))
            slack = rel * np.maximum(np.abs(x), rms)
            vlo = O.fp8_decode_ref(O.fp8_encode((x - slack).astype(np.float32)))
            vhi = O.fp8_decode_ref(O.fp8_encode((x + slack).astype(np.float32)))
            vg = O.fp8_decode_ref(g)
            ok_ = (vg >= np.minimum(vlo, vhi)) & (vg <= np.maximum(vlo, vhi))
            n_diff += int((g != o).sum())
            assert ok_.all(), f"{int((~ok_).sum())} KV codes not explained by rounding"
    return n_diff


def oracle_step(m, hidden16, pos, kc, vc, b=0, forced_kv=None, kv_trace=None):
    """Oracle decode step for batch row b; kc/vc: per-layer [Hk, max_seq, hd]
    arrays mutated in place.  Returns (hidden, logits)."""
    ks = None if m.k_scales is None else [t.numpy() for t in m.k_scales]
    vs = None if m.v_scales is None else [t.numpy() for t in m.v_scales]
    return O.decode_step(m.oracle_layers, hidden16, pos, kc, vc, H=m.H, Hk=m.Hk, D=m.hd,
                         hidden=m.D, inter=m.I, eps=m.eps, rope_cos=m.cos.numpy(),
                         rope_sin=m.sin.numpy(), final_norm=m.final_norm.numpy(),
                         lm_w=m.lm_w.numpy(),
                         lm_s=None if m.lm_s is None else m.lm_s.numpy().reshape(m.vocab, -1, 2),
                         lm_bits=m.lm_bits, k_scales=ks, v_scales=vs, forced_kv=forced_kv,
                         kv_trace=kv_trace)


def plan(m, B, n=2):
    """r4q_decode_plan of the model: (attention split count, layers whose
    gate/up applies the SiLU gate in the same launch[, layers whose qkv split
    partials the attention prologue sums (n = 3)])."""
    import ctypes as C

    import r4q_lib as R
    had = torch.zeros(32, 32, dtype=torch.float16, device=m.dev)
    args = layer_args(m, 0)
    md = int4_hip.build_model(*args[:18], *args[19:], m.k_caches, m.v_caches, m.final_norm_d,
                              m.lm_w_d, m.lm_s_d, m.vocab, m.D)
    del had
    out = (C.c_int32 * n)()
    R.call("r4q_decode_plan", C.byref(md.struct), B, out, n)
    return tuple(int(v) for v in out)


def oracle_batch_forced(m, h, pos):
    """Batched oracle step for every row with the GPU's KV codes at `pos`
    (each differing code checked to be explainable by last-bit rounding);
    returns (hidden [B, D], logits [B, V], number of differing codes, total)."""
    B = m.batch
    kc = [m.kc_np[li].copy() for li in range(m.L)]
    vc = [m.vc_np[li].copy() for li in range(m.L)]
    forced = [(m.k_caches[li][:, :, pos].cpu().numpy(), m.v_caches[li][:, :, pos].cpu().numpy())
              for li in range(m.L)]
    trace = []
    ks = None if m.k_scales is None else [t.numpy() for t in m.k_scales]
    vs = None if m.v_scales is None else [t.numpy() for t in m.v_scales]
    hid, logits = O.decode_step_batch(
        m.oracle_layers, h.reshape(B, -1), pos, kc, vc, H=m.H, Hk=m.Hk, D=m.hd, hidden=m.D,
        inter=m.I, eps=m.eps, rope_cos=m.cos.numpy(), rope_sin=m.sin.numpy(),
        final_norm=m.final_norm.numpy(), lm_w=m.lm_w.numpy(),
        lm_s=None if m.lm_s is None else m.lm_s.numpy().reshape(m.vocab, -1, 2),
        lm_bits=m.lm_bits, k_scales=ks, v_scales=vs, forced_kv=forced, kv_trace=trace)
    n = check_forced_kv(forced, trace)
    total = sum(k.size + v.size for k, v in forced)
    return hid, logits, n, total
