"""Pins the oracle's temperature / top-p sampler (f3) on the CPU.

* splitmix64 against the published sequence of its reference implementation
  (seed 1234567);
* temperature 0 is torch.argmax (first index of the maximum);
* the kept set equals a literal torch restatement of the reference's top-p
  code (int4_engine_v5.py:387-399: sort descending, cumsum of softmax, mask
  cumulative-before >= top_p) in float64, with a stable sort for ties;
* the inverse-CDF draw over a fine uniform grid of u reproduces the kept
  tokens' renormalised probabilities.
"""
import numpy as np
import pytest
import torch

import r4q_oracle as O


def test_splitmix64_published_sequence():
    g, m = 0x9E3779B97F4A7C15, (1 << 64) - 1
    got = [O.splitmix64((1234567 + k * g) & m) for k in range(3)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423]


def test_uniform_is_in_unit_interval_and_spread():
    u = np.array([O.sample_uniform(7, c, r) for c in range(2000) for r in range(2)])
    assert u.min() >= 0.0 and u.max() < 1.0
    hist = np.histogram(u, bins=10, range=(0, 1))[0]
    assert hist.min() > 300 and hist.max() < 500  # 4000 draws, 400 expected per bin


def _logits(V, seed, ties=True):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(V, generator=g) * 3.0).half()
    if ties:  # coarse values force many exact ties, ±0 included
        x[: V // 4] = (x[: V // 4] * 2).round() / 2
        x[V // 4] = -0.0
        x[V // 4 + 1] = 0.0
    return x


@pytest.mark.parametrize("seed", range(5))
def test_temperature_zero_is_argmax(seed):
    x = _logits(3000, seed)
    x[17] = x.max()  # a tie for the maximum at a low index
    assert O.sample_top_p(x.numpy(), 0.0, 0.9, 0.5) == int(torch.argmax(x.float()))


def _reference_kept(x16, temperature, top_p):
    """The reference's code path, literally (float64, stable sort)."""
    z = x16.double() / temperature
    sorted_logits, sorted_idx = torch.sort(z, descending=True, stable=True)
    probs = torch.softmax(sorted_logits, dim=-1)
    cum = torch.cumsum(probs, dim=-1)
    mask = cum - probs >= top_p
    return set(sorted_idx[~mask].tolist())


@pytest.mark.parametrize("temperature", [0.6, 1.0, 1.7])
@pytest.mark.parametrize("top_p", [0.3, 0.9, 0.97])
def test_kept_set_matches_reference_code(temperature, top_p):
    checked = 0
    for seed in range(6):
        x = _logits(4096, seed * 11 + int(top_p * 100))
        tok, info = O.sample_top_p(x.numpy(), temperature, top_p, 0.5, return_info=True)
        if info["cut_margin"] < 1e-12:
            continue
        want = _reference_kept(x, temperature, top_p)
        assert info["kept"] == len(want)
        assert tok in want
        checked += 1
    assert checked >= 5


def test_draw_frequencies_follow_kept_distribution():
    x = torch.tensor([2.0, 1.5, 1.5, 0.0, -1.0, 3.0, -0.0, 1.5], dtype=torch.float16)
    T, top_p = 0.8, 0.9
    kept = sorted(_reference_kept(x, T, top_p))
    z = x.double() / T
    p = torch.softmax(z[kept], dim=0).numpy()
    n = 20000
    counts = {k: 0 for k in kept}
    for i in range(n):
        counts[O.sample_top_p(x.numpy(), T, top_p, (i + 0.5) / n)] += 1
    freq = np.array([counts[k] / n for k in kept])
    assert np.max(np.abs(freq - p)) < 2.0 / n + 1e-12


def test_top_p_one_keeps_everything_and_ties_draw_by_index():
    x = torch.tensor([1.0, 1.0, 1.0, 1.0], dtype=torch.float16)
    # four equal tokens: u in [k/4, (k+1)/4) draws token k (index order)
    for k in range(4):
        assert O.sample_top_p(x.numpy(), 1.0, 1.0, (k + 0.5) / 4) == k
    # top_p 0.5 keeps the first two tied tokens (mass before: 0, 0.25 < 0.5; 0.5 is not)
    _, info = O.sample_top_p(x.numpy(), 1.0, 0.5, 0.1, return_info=True)
    assert info["kept"] == 2
