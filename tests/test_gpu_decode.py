"""Decode-step parity: the int4_hip drop-in (decode_step_logits, decode_step,
decode_bench[_graph], decode_loop, decode_profile) against the oracle, plus
size-independent properties (graph == eager, batch rows == single rows)."""
import numpy as np
import pytest
import torch

import int4_hip
import r4q_synth as S
from conftest import rel_l2
from decode_util import (bench_args, build, check_forced_kv, gpu_kv_at, layer_args,
                         oracle_batch_forced, oracle_step, plan, step_logits)

pytestmark = pytest.mark.gpu
TOL = 5e-3


def _oracle_forced(m, h, pos, want_hidden=False):
    """Oracle step fed with the GPU's FP8 codes at `pos` (each checked to be
    explainable by last-bit rounding of the oracle's own value)."""
    kc = [m.kc_np[li, 0].copy() for li in range(m.L)]
    vc = [m.vc_np[li, 0].copy() for li in range(m.L)]
    forced, trace = gpu_kv_at(m, pos), []
    hid, logits = oracle_step(m, h.numpy().reshape(-1), pos, kc, vc, forced_kv=forced,
                              kv_trace=trace)
    n = check_forced_kv(forced, trace)
    total = sum(k.size + v.size for k, v in forced)
    assert n <= 0.05 * total, f"{n} of {total} KV codes differ"
    return hid if want_hidden else logits


def _hidden(m, seed, rows=1):
    return (torch.randn(rows, 1, m.D, generator=S.gen(seed)) * 0.5).half()


@pytest.mark.parametrize("kv_scale", [False, True])
def test_small_model_step_vs_oracle(dev, kv_scale):
    bits = {(0, "o"): 8, (1, "down"): 8, (1, "qkv"): 8}
    m = build(dev, D=256, I=512, H=4, Hk=2, L=2, vocab=1000, max_seq=64, seed=3, bits=bits,
              fill=5, kv_scale=kv_scale)
    h = _hidden(m, 1)
    pos = 5
    logits = step_logits(m, h.to(dev), pos).cpu().float().numpy().reshape(-1)
    want = _oracle_forced(m, h, pos)
    assert rel_l2(logits, want) <= TOL
    for li in range(m.L):  # positions before pos untouched
        assert np.array_equal(m.k_caches[li][0, :, :pos].cpu().numpy(), m.kc_np[li, 0, :, :pos])


def test_qwen3_width_two_layers_vs_oracle(dev):
    bits = {(0, "gu"): 8, (1, "down"): 8}
    m = build(dev, D=5120, I=17408, H=40, Hk=8, L=2, vocab=4096, max_seq=160, seed=11, bits=bits,
              fill=100, kv_scale=True)
    h = _hidden(m, 2)
    pos = 100
    logits = step_logits(m, h.to(dev), pos).cpu().float().numpy().reshape(-1)
    assert np.all(np.isfinite(logits))
    assert rel_l2(logits, _oracle_forced(m, h, pos)) <= TOL


def test_qwen3_width_batch8_step_vs_oracle(dev):
    """Batch 8 at full Qwen3-14B width: skinny MFMA GEMMs with the step's own
    split-K workspace, the gate/up GEMM applying SiLU + FWHT-32 in its
    epilogue, its 32 units past two whole rounds of 256 cut along K into
    pieces whose last arrival sums them (both layers, INT8 and INT4), batched
    row norms; every row against the oracle under KV teacher forcing."""
    bits = {(0, "gu"): 8, (1, "down"): 8, (1, "qkv"): 8}
    m = build(dev, D=5120, I=17408, H=40, Hk=8, L=2, vocab=4096, max_seq=96, seed=13, bits=bits,
              batch=8, fill=60, kv_scale=True)
    nsplit, fused = plan(m, 8)
    assert fused == 2, "batched gate/up did not take the fused SiLU reduce"
    h = _hidden(m, 12, rows=8)
    pos = 60
    logits = step_logits(m, h.to(dev), pos).cpu().float().numpy().reshape(8, -1)
    assert np.all(np.isfinite(logits))
    _, want, n, total = oracle_batch_forced(m, h.numpy().reshape(8, -1), pos)
    assert n <= 0.05 * total, f"{n} of {total} KV codes differ"
    for b in range(8):
        assert rel_l2(logits[b], want[b]) <= TOL, (b, rel_l2(logits[b], want[b]))


def test_batch8_gate_up_tail_pieces_vs_oracle(dev):
    """I = 9600: 300 SiLU units, one whole round of 256 and 44 tail units
    that the batched gate/up GEMM cuts along K into two pieces each (INT8
    layer 0, INT4 layer 1); every row against the oracle, and a second step
    on the same inputs bit-identical to the first (each launch leaves the
    tail's arrival counters at zero for the next)."""
    bits = {(0, "gu"): 8}
    m = build(dev, D=1024, I=9600, H=16, Hk=8, L=2, vocab=512, max_seq=48, seed=31, bits=bits,
              batch=8, fill=20)
    nsplit, fused = plan(m, 8)
    assert fused == 2, fused
    h = _hidden(m, 32, rows=8)
    pos = 20
    first = step_logits(m, h.to(dev), pos).cpu()
    second = step_logits(m, h.to(dev), pos).cpu()
    assert torch.equal(first.view(torch.int16), second.view(torch.int16))
    logits = first.float().numpy().reshape(8, -1)
    assert np.all(np.isfinite(logits))
    _, want, n, total = oracle_batch_forced(m, h.numpy().reshape(8, -1), pos)
    assert n <= 0.05 * total, f"{n} of {total} KV codes differ"
    for b in range(8):
        assert rel_l2(logits[b], want[b]) <= TOL, (b, rel_l2(logits[b], want[b]))


def test_qwen3_width_batch8_ctx2048_step_vs_oracle(dev):
    """Batch 8 at ctx 2048 (position 2048, cache capacity 2088): 4 attention
    splits per (sequence, KV head) whose prologue sums the qkv split partials,
    INT4 and INT8 layers; every row against the oracle under KV teacher
    forcing."""
    bits = {(0, "qkv"): 8, (1, "o"): 8}
    m = build(dev, D=5120, I=17408, H=40, Hk=8, L=2, vocab=1024, max_seq=2088, seed=25,
              bits=bits, batch=8, fill=2048, kv_scale=True)
    nsplit, fused = plan(m, 8)
    assert nsplit == 4 and fused == 2, (nsplit, fused)
    h = _hidden(m, 26, rows=8)
    pos = 2048
    logits = step_logits(m, h.to(dev), pos).cpu().float().numpy().reshape(8, -1)
    assert np.all(np.isfinite(logits))
    _, want, n, total = oracle_batch_forced(m, h.numpy().reshape(8, -1), pos)
    assert n <= 0.05 * total, f"{n} of {total} KV codes differ"
    for b in range(8):
        assert rel_l2(logits[b], want[b]) <= TOL, (b, rel_l2(logits[b], want[b]))


def test_qwen3_width_batch3_step_vs_oracle(dev):
    """Batch 3 at full width: gate_up runs unsplit with the SiLU gate in the
    skinny GEMM's epilogue on 3 of its 8 activation rows (the rest repeat the
    last row and are not stored), INT4 and INT8; every row against the
    oracle under KV teacher forcing."""
    bits = {(1, "gu"): 8, (0, "down"): 8}
    m = build(dev, D=5120, I=17408, H=40, Hk=8, L=2, vocab=2048, max_seq=96, seed=21, bits=bits,
              batch=3, fill=40, kv_scale=True)
    nsplit, fused = plan(m, 3)
    assert fused == 2, "batched gate/up did not apply the SiLU gate in the same launch"
    h = _hidden(m, 22, rows=3)
    pos = 40
    logits = step_logits(m, h.to(dev), pos).cpu().float().numpy().reshape(3, -1)
    assert np.all(np.isfinite(logits))
    _, want, n, total = oracle_batch_forced(m, h.numpy().reshape(3, -1), pos)
    assert n <= 0.05 * total, f"{n} of {total} KV codes differ"
    for b in range(3):
        assert rel_l2(logits[b], want[b]) <= TOL, (b, rel_l2(logits[b], want[b]))


def test_qwen3_width_batch8_split_partials_summed_in_consumers_bit_exact(dev):
    """Batch 8 at full width: the split-K partials of the qkv, o and down
    projections summed by the kernels that consume them (attention prologue,
    residual + row norm; split order, rounded to fp16) give the same logits
    and FP8 K/V bytes, bit for bit, as separate reduce launches (split_reduce
    override); INT4 and INT8 layers."""
    import r4q_lib as R
    bits = {(1, "qkv"): 8, (0, "o"): 8, (1, "down"): 8}
    m = build(dev, D=5120, I=17408, H=40, Hk=8, L=2, vocab=4096, max_seq=96, seed=14, bits=bits,
              batch=8, fill=60, kv_scale=True)
    assert plan(m, 8, 3)[2] == 6, "split partials not summed by their consumers"
    h = _hidden(m, 15, rows=8).to(dev)
    pos = 60
    runs = []
    for knob in (0, 1):
        R.tune("split_reduce", knob)
        try:
            assert plan(m, 8, 3)[2] == (6 if knob == 0 else 0)
            lg = step_logits(m, h, pos).clone()
            kv = [gpu_kv_at(m, pos, b) for b in range(8)]
        finally:
            R.tune("split_reduce", 0)
        runs.append((lg, kv))
    (la, kva), (lb, kvb) = runs
    assert torch.isfinite(la.float()).all()
    assert torch.equal(la.view(torch.int16), lb.view(torch.int16))
    for b in range(8):
        for (ka, va), (kb, vb) in zip(kva[b], kvb[b]):
            assert np.array_equal(ka, kb) and np.array_equal(va, vb), b


def test_qwen3_width_ctx2048_step_vs_oracle(dev):
    """Batch 1 at ctx 2048 (position 2048, cache capacity 2088): the 17-split
    attention with the head norm + RoPE + FP8 KV prologue in its owner
    workgroup, against the oracle under KV teacher forcing."""
    m = build(dev, D=5120, I=17408, H=40, Hk=8, L=2, vocab=2048, max_seq=2088, seed=17,
              bits={(1, "o"): 8}, fill=2048, kv_scale=True)
    nsplit, fused = plan(m, 1)
    assert nsplit == 17 and fused == 2, (nsplit, fused)
    h = _hidden(m, 14)
    pos = 2048
    logits = step_logits(m, h.to(dev), pos).cpu().float().numpy().reshape(-1)
    assert np.all(np.isfinite(logits))
    assert rel_l2(logits, _oracle_forced(m, h, pos)) <= TOL


@pytest.mark.parametrize("D,I,H,Hk,B", [(256, 512, 4, 2, 3), (5120, 17408, 40, 8, 1)])
def test_graph_step_equals_eager_step(dev, D, I, H, Hk, B):
    """decode_step_logits replays a captured step (the position set on the
    device) by default: logits and KV bytes bit-identical to the eager
    launches, at several positions through one cached graph."""
    m = build(dev, D=D, I=I, H=H, Hk=Hk, L=2, vocab=1024, max_seq=80, seed=23, batch=B, fill=30,
              bits={(0, "down"): 8})
    h = _hidden(m, 9, rows=B).to(dev)
    had = torch.zeros(32, 32, dtype=torch.float16, device=dev)
    res = {}
    for use_graph in (False, True):
        m.reset_caches()
        outs = []
        for pos in (30, 31, 45):
            lg = int4_hip.decode_step_logits(h, *layer_args(m, pos), m.k_caches, m.v_caches,
                                             m.final_norm_d, m.lm_w_d, m.lm_s_d, m.vocab, m.D,
                                             had, use_graph=use_graph)
            hid = int4_hip.decode_step(h, *layer_args(m, pos + 1), m.k_caches, m.v_caches, had,
                                       use_graph=use_graph)
            outs.append((lg.cpu(), hid.cpu()))
        res[use_graph] = (outs, [t.cpu() for t in m.k_caches + m.v_caches])
    for (a, b), (c, d) in zip(res[False][0], res[True][0]):
        assert torch.equal(a, c) and torch.equal(b, d)
    for a, b in zip(res[False][1], res[True][1]):
        assert torch.equal(a, b)


def test_graph_loop_recaptures_after_sampling_workspace_moves(dev):
    """A captured sampling loop bakes in the sampling workspace; a larger
    r4q_sample call on the same context reallocates that workspace, so the
    next replay must capture again rather than use the freed buffer.  The
    tokens then equal the eager loop's."""
    m = build(dev, D=256, I=512, H=4, Hk=2, L=2, vocab=700, max_seq=64, seed=29, fill=12)
    h = _hidden(m, 10).to(dev)
    had = torch.zeros(32, 32, dtype=torch.float16, device=dev)
    kw = dict(temperature=0.8, top_p=0.9, seed=5)

    def run(use_graph):
        m.reset_caches()
        return int4_hip.decode_loop(m.embed_d, m.final_norm_d, m.lm_w_d, m.lm_s_d, m.vocab, m.D,
                                    h, 6, *layer_args(m, 12), m.k_caches, m.v_caches, had,
                                    use_graph=use_graph, **kw)

    first = run(True)
    big = torch.randn(300, m.vocab, generator=S.gen(3)).half().to(dev)
    int4_hip.sample(big, temperature=1.0, top_p=0.95, seed=1)  # grows the workspace
    torch.cuda.synchronize()
    again = run(True)
    eager = run(False)
    assert torch.equal(first, eager) and torch.equal(again, eager)


def test_decode_step_hidden_matches_oracle(dev):
    m = build(dev, D=256, I=512, H=8, Hk=2, L=3, vocab=64, max_seq=32, seed=5, fill=0)
    h = _hidden(m, 3)
    had = torch.zeros(32, 32, dtype=torch.float16, device=dev)
    out = int4_hip.decode_step(h.to(dev), *layer_args(m, 0), m.k_caches, m.v_caches, had)
    assert out.shape == (1, 1, m.D)
    want = _oracle_forced(m, h, 0, want_hidden=True)
    assert rel_l2(out.cpu().float().numpy().reshape(-1), want) <= TOL


def test_batch_rows_equal_single_rows(dev):
    m = build(dev, D=256, I=512, H=4, Hk=2, L=2, vocab=500, max_seq=40, seed=9, batch=3, fill=7)
    h = _hidden(m, 4, rows=3)
    batched = step_logits(m, h.to(dev), 7).cpu()
    for b in range(3):
        m.k_caches = [torch.from_numpy(m.kc_np[li, b:b + 1].copy()).to(dev) for li in range(m.L)]
        m.v_caches = [torch.from_numpy(m.vc_np[li, b:b + 1].copy()).to(dev) for li in range(m.L)]
        single = step_logits(m, h[b:b + 1].to(dev), 7).cpu()
        # batched rows take the skinny MFMA GEMM and separate norms, single
        # rows the fused-norm GEMV: same math, different accumulation order
        assert rel_l2(batched[b], single[0]) <= TOL


def test_batch_rows_vs_oracle(dev):
    m = build(dev, D=256, I=512, H=8, Hk=2, L=2, vocab=400, max_seq=48, seed=19, batch=4, fill=9,
              bits={(1, "gu"): 8})
    h = _hidden(m, 5, rows=4)
    pos = 9
    batched = step_logits(m, h.to(dev), pos).cpu().float().numpy().reshape(4, -1)
    for b in range(4):
        kc = [m.kc_np[li, b].copy() for li in range(m.L)]
        vc = [m.vc_np[li, b].copy() for li in range(m.L)]
        forced, trace = gpu_kv_at(m, pos, b), []
        _, want = oracle_step(m, h[b].numpy().reshape(-1), pos, kc, vc, b=b, forced_kv=forced,
                              kv_trace=trace)
        check_forced_kv(forced, trace)
        assert rel_l2(batched[b], want) <= TOL, b


@pytest.mark.parametrize("D,I,H,Hk,vocab", [(256, 512, 4, 2, 300), (5120, 17408, 40, 8, 2048)])
def test_graph_replay_equals_eager(dev, D, I, H, Hk, vocab):
    m = build(dev, D=D, I=I, H=H, Hk=Hk, L=2, vocab=vocab, max_seq=96, seed=21, fill=40,
              bits={(1, "o"): 8})
    h = _hidden(m, 6).to(dev)
    n = 12
    toks_e = int4_hip.decode_loop(m.embed_d, m.final_norm_d, m.lm_w_d, m.lm_s_d, m.vocab, m.D, h, n,
                                  *layer_args(m, 40), m.k_caches, m.v_caches,
                                  torch.zeros(32, 32, dtype=torch.float16, device=dev))
    kc_e = [t.cpu().clone() for t in m.k_caches]
    m.reset_caches()
    toks_g = torch.empty(n, 1, dtype=torch.int64, device=dev)
    int4_hip._bench(h, m.embed_d, n, bench_args(m, 40), True, tokens_out=toks_g)
    torch.cuda.synchronize()
    assert torch.equal(toks_e, toks_g.cpu()[:, 0])
    for a, b in zip(kc_e, m.k_caches):
        assert torch.equal(a, b.cpu())
    # a second replay from the same state reuses the captured graph
    m.reset_caches()
    toks_g2 = torch.empty(n, 1, dtype=torch.int64, device=dev)
    int4_hip._bench(h, m.embed_d, n, bench_args(m, 40), True, tokens_out=toks_g2)
    torch.cuda.synchronize()
    assert torch.equal(toks_g2, toks_g)


def test_decode_loop_matches_host_greedy(dev):
    m = build(dev, D=256, I=512, H=4, Hk=2, L=2, vocab=300, max_seq=64, seed=31, fill=10)
    h = _hidden(m, 7).to(dev)
    n = 8
    had = torch.zeros(32, 32, dtype=torch.float16, device=dev)
    toks = int4_hip.decode_loop(m.embed_d, m.final_norm_d, m.lm_w_d, m.lm_s_d, m.vocab, m.D, h, n,
                                *layer_args(m, 10), m.k_caches, m.v_caches, had)
    m.reset_caches()
    hid = h
    want = []
    for t in range(n):
        lg = step_logits(m, hid, 10 + t)
        tok = int(lg.float().reshape(-1).argmax())
        want.append(tok)
        hid = m.embed_d[tok].view(1, 1, m.D).contiguous()
    assert toks.tolist() == want


def test_decode_bench_and_profile_run(dev):
    m = build(dev, D=256, I=512, H=4, Hk=2, L=2, vocab=300, max_seq=64, seed=41, fill=10)
    h = _hidden(m, 8).to(dev)
    int4_hip.decode_bench(h, m.embed_d, 5, *bench_args(m, 10))
    int4_hip.decode_bench_graph(h, m.embed_d, 5, *bench_args(m, 10))
    prof = int4_hip.decode_profile(h, m.embed_d, *bench_args(m, 20))
    assert len(prof) == 5 and prof[0] > 0
    assert prof[1] + prof[2] + prof[3] <= prof[0] * 1.01


def test_decode_rejects_position_beyond_cache(dev):
    m = build(dev, D=256, I=512, H=4, Hk=2, L=1, vocab=100, max_seq=16, seed=1)
    with pytest.raises(RuntimeError):
        step_logits(m, _hidden(m, 1).to(dev), 16)
