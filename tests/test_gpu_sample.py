"""On-device temperature / top-p sampling (r4q_sample, r4q_decode_generate)
against the oracle's restatement of the engine's Python sampler
(int4_engine_v5.py:330-335, 387-399).

A sampled token must be the oracle's token or, where the outcome hinges on
float rounding (fp32 sums over 151,936 tokens on the GPU, float64 in the
oracle), a token whose oracle CDF interval lies within 1e-5 of the draw u, or
whose cumulative mass before it is within 1e-5 of top_p; most draws must
match exactly.  Frequencies over many draws are
checked against the kept distribution with a chi-square bound, and the
sampled decode loop is checked eager == graph and step by step against
host-side sampling of the same logits."""
import numpy as np
import pytest
import torch

import int4_hip
import r4q_oracle as O
import r4q_synth as S
from decode_util import bench_args, build, layer_args, step_logits

pytestmark = pytest.mark.gpu
MARGIN = 1e-5


def _logits(V, seed, scale=2.5, ties=True):
    g = S.gen(seed)
    x = (torch.randn(V, generator=g) * scale).half()
    if ties:
        x[: V // 3] = (x[: V // 3] * 2).round() / 2  # many exact ties
        x[V // 3] = -0.0
        x[V // 3 + 1] = 0.0
    return x


@pytest.mark.parametrize("temperature", [0.0, 0.6, 1.0, 1.5])
@pytest.mark.parametrize("top_p", [0.5, 0.9, 1.0])
def test_sample_matches_oracle_full_vocab(dev, temperature, top_p):
    V, seed = 151936, 12345
    x = _logits(V, int(temperature * 10 + top_p * 100))
    xd = x.to(dev)
    exact = 0
    for counter in range(8):
        got = int(int4_hip.sample(xd, temperature, top_p, seed, counter).item())
        u = O.sample_uniform(seed, counter, 0)
        want, info = O.sample_top_p(x.numpy(), temperature, top_p, u, return_info=True)
        exact += got == want
        assert O.sample_distance(got, info) <= MARGIN, (counter, got, want)
    assert exact >= 4


def test_sample_greedy_is_torch_argmax(dev):
    for seed in range(6):
        x = _logits(5000 + seed, seed)
        x[100 + seed] = x.max()  # tie for the maximum
        if seed == 0:
            x[:] = -1.0
            x[7] = -0.0
            x[3] = 0.0  # +0 and -0 tie at the maximum: the lower index wins
        got = int(int4_hip.sample(x.to(dev), 0.0).item())
        assert got == int(torch.argmax(x.float()))


def test_sample_rows_stride_and_counter(dev):
    """Rows of a strided view; a one-row call before and between leaves the
    context's tables valid for more rows (the workspace layout does not
    depend on the row count)."""
    V, B = 3000, 3
    base = torch.stack([_logits(V, 70 + b) for b in range(B)])
    big = torch.zeros(B, V + 64, dtype=torch.float16)
    big[:, :V] = base
    bd = big.to(dev)
    view = bd[:, :V]  # row stride V + 64
    int4_hip.sample(bd[0, :V], 0.8, 0.95, 99, 3)
    for counter in (0, 5, 1 << 40):
        int4_hip.sample(bd[1, :V], 1.0, 1.0, 1, counter)
        got = int4_hip.sample(view, 0.8, 0.95, 99, counter).cpu().tolist()
        for b in range(B):
            u = O.sample_uniform(99, counter, b)
            want, info = O.sample_top_p(base[b].numpy(), 0.8, 0.95, u, return_info=True)
            assert O.sample_distance(got[b], info) <= MARGIN, (counter, b, got[b], want)


def test_sample_frequencies_chi_square(dev):
    """4096 draws (512 identical rows x 8 counters) from a 16-token row."""
    x = torch.tensor([2.0, 1.5, 1.5, 0.5, 0.0, -0.5, 3.0, 1.0, 2.5, -1.0, 0.25, 1.5, 2.0, -2.0,
                      0.75, 1.25], dtype=torch.float16)
    T, top_p, rows = 0.9, 0.9, 512
    xd = x.to(dev).repeat(rows, 1)
    draws = torch.cat([int4_hip.sample(xd, T, top_p, 2024, c) for c in range(8)]).cpu().numpy()
    # kept set and its renormalised probabilities (literal sort / cumsum restatement)
    z = x.double() / T
    sl, si = torch.sort(z, descending=True, stable=True)
    p = torch.softmax(sl, 0)
    keep = ~((torch.cumsum(p, 0) - p) >= top_p)
    kept = si[keep].numpy()
    pk = torch.softmax(z[kept], 0).numpy()
    assert set(np.unique(draws)) <= set(kept.tolist())
    counts = np.array([(draws == k).sum() for k in kept])
    n = draws.size
    chi2 = float(((counts - n * pk) ** 2 / (n * pk)).sum())
    # dof = len(kept) - 1 <= 15: P(chi2 > 50) < 1e-5 under the null
    assert chi2 < 50.0, (chi2, counts, n * pk)


def test_sample_rejects_bad_arguments(dev):
    x = torch.zeros(10, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="top_p"):
        int4_hip.sample(x, 1.0, 0.0)
    with pytest.raises(ValueError):
        int4_hip.sample(x.float(), 1.0, 0.9)


def _loop(m, h, n, pos, **kw):
    had = torch.zeros(32, 32, dtype=torch.float16, device=h.device)
    return int4_hip.decode_loop(m.embed_d, m.final_norm_d, m.lm_w_d, m.lm_s_d, m.vocab, m.D, h, n,
                                *layer_args(m, pos), m.k_caches, m.v_caches, had, **kw)


def test_sampled_decode_loop_eager_graph_and_host(dev):
    m = build(dev, D=256, I=512, H=4, Hk=2, L=2, vocab=300, max_seq=64, seed=51, fill=10)
    h = (torch.randn(1, 1, m.D, generator=S.gen(9)) * 0.5).half().to(dev)
    n, T, top_p, seed = 10, 1.2, 0.95, 777
    toks_e = _loop(m, h, n, 10, temperature=T, top_p=top_p, seed=seed)
    m.reset_caches()
    toks_g = _loop(m, h, n, 10, temperature=T, top_p=top_p, seed=seed, use_graph=True)
    assert torch.equal(toks_e, toks_g)
    m.reset_caches()
    greedy = _loop(m, h, n, 10)
    assert not torch.equal(toks_e, greedy)  # 10 draws at T = 1.2 over 300 tokens
    # host replay: the step's logits sampled with the same (seed, position)
    m.reset_caches()
    hid = h
    for t in range(n):
        lg = step_logits(m, hid, 10 + t)
        tok = int(int4_hip.sample(lg.reshape(-1), T, top_p, seed, 10 + t).item())
        assert tok == int(toks_e[t]), t
        hid = m.embed_d[tok].view(1, 1, m.D).contiguous()
