"""GPU parity of the MFMA prefill GEMM with on-the-fly dequantisation
(config 3 shapes and ragged edges) against the oracle.  rel-L2 <= 5e-3."""
import numpy as np
import pytest
import torch

import int4_hip
import r4q_oracle as O
import r4q_synth as S
from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 5e-3


def _run(dev, bits, M, N, K, seed):
    g = S.gen(seed)
    w, sz = S.weight(N, K, bits, g)
    x = (torch.randn(M, K, generator=g)).half()
    y = int4_hip.dbg_gemm(x.to(dev), w.to(dev), None if sz is None else sz.to(dev), M, N, K)
    want = O.gemm(x.numpy(), w.numpy(), None if sz is None else sz.numpy(), bits)
    return y.cpu().numpy(), want


@pytest.mark.parametrize("M,N,K", [(512, 17408, 5120), (512, 5120, 17408)])
def test_prefill_gemm_config3(dev, M, N, K):
    got, want = _run(dev, 4, M, N, K, seed=3)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) <= TOL


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("M,N,K", [(17, 100, 32), (130, 129, 96), (256, 384, 1024), (64, 64, 64)])
def test_prefill_gemm_ragged(dev, bits, M, N, K):
    got, want = _run(dev, bits, M, N, K, seed=M + N + K + bits)
    assert rel_l2(got, want) <= TOL


def test_small_m_path_matches_gemv(dev):
    """M <= 16 streams the weights per row; every row equals the GEMV."""
    g = S.gen(5)
    N, K = 1000, 5120
    w, sz = S.int4_weight(N, K, g)
    x = torch.randn(8, K, generator=g).half()
    W, SZ, X = w.to(dev), sz.to(dev), x.to(dev)
    y = int4_hip.dbg_gemm(X, W, SZ, 8, N, K)
    for r in range(8):
        assert torch.equal(y[r], int4_hip.dbg_gemv(X[r].contiguous(), W, SZ, N, K))
