"""GPU parity of the MFMA prefill GEMM with on-the-fly dequantisation
(config 3 shapes and ragged edges) against the oracle.  rel-L2 <= 5e-3."""
import ctypes as C

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


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("M,N,K", [(2, 7168, 5120), (8, 17408, 5120), (8, 5120, 17408),
                                   (16, 1000, 5120), (9, 300, 1024), (3, 77, 256),
                                   (5, 33, 128), (12, 65, 512)])
def test_skinny_gemm_vs_oracle(dev, bits, M, N, K):
    """2 <= M <= 16 rows (batched decode): weights streamed once through the
    LDS ring, MFMA; the workspace the library asks for lets narrow shapes
    split along K.  Shapes whose K is not a whole number of ring steps take
    the per-row GEMV path (checked the same way)."""
    got, want = _run(dev, bits, M, N, K, seed=7 * M + N + K + bits)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) <= TOL
    for r in range(M):
        assert rel_l2(got[r], want[r]) <= TOL


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("M,N,K", [(8, 5120, 17408), (16, 200, 2048), (4, 130, 1024)])
def test_skinny_gemm_without_workspace(dev, bits, M, N, K):
    """r4q_gemm (no workspace): one pass over K per 64-row tile, no split."""
    import r4q_lib as R
    g = S.gen(3 * M + N + K + bits)
    w, sz = S.weight(N, K, bits, g)
    x = (torch.randn(M, K, generator=g) * 0.5).half()
    want = O.gemm(x.numpy(), w.numpy(), None if sz is None else sz.numpy(), bits)
    xd, wd = x.to(dev), w.to(dev)
    sd = None if sz is None else sz.to(dev)
    y = torch.empty(M, N, dtype=torch.float16, device=dev)
    R.call("r4q_gemm", xd.data_ptr(), wd.data_ptr(), None if sd is None else sd.data_ptr(),
           y.data_ptr(), M, N, K, bits, R.stream_handle())
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) <= TOL


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_skinny_gemm_one_hot_columns_exact(dev, bits):
    """Row r of x = e_k(r): y[r] is column k(r) of the dequantised weight,
    bit for bit (the in-register dequantisation equals the dequant kernel)."""
    g = S.gen(41 + bits)
    N, K, M = 300, 1024, 8
    w, sz = S.weight(N, K, bits, g)
    W = O.dequant(w.numpy(), None if sz is None else sz.numpy(), bits)
    ks = [0, 1, 4, 31, 32, 517, 1000, 1023]
    x = torch.zeros(M, K, dtype=torch.float16)
    for r, k in enumerate(ks):
        x[r, k] = 1.0
    y = int4_hip.dbg_gemm(x.to(dev), w.to(dev), None if sz is None else sz.to(dev), M, N, K)
    y = y.cpu().numpy()
    for r, k in enumerate(ks):
        assert np.array_equal(y[r], W[:, k]), k


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("M,N,K", [(300, 1000, 2048), (257, 520, 32), (600, 256, 4096),
                                   (512, 7168, 5120), (256, 255, 96)])
def test_ring_gemm_ragged_and_split(dev, bits, M, N, K):
    """M >= 256: the 256 x 256 LDS-ring kernel, with ragged M / N tiles,
    K loops shorter than the copy ring (K = 32, 96), and split-K over a
    workspace (few tiles, long K)."""
    got, want = _run(dev, bits, M, N, K, seed=M + 3 * N + K + bits)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) <= TOL
    for r in (0, M // 2, M - 1):
        assert rel_l2(got[r], want[r]) <= TOL, r


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("N,K", [(700, 1024), (300, 8192)])
def test_ring_gemm_one_hot_columns_exact(dev, bits, N, K):
    """Row r of x = e_k(r) over 300 rows: y[r] is column k(r) of the
    dequantised weight, bit for bit -- in one pass and with the K loop split
    (fp32 partials of zeros and one exact product)."""
    g = S.gen(43 + bits + K)
    M = 300
    w, sz = S.weight(N, K, bits, g)
    W = O.dequant(w.numpy(), None if sz is None else sz.numpy(), bits)
    ks = [(r * 997 + r // 7) % K for r in range(M)]
    x = torch.zeros(M, K, dtype=torch.float16)
    for r, k in enumerate(ks):
        x[r, k] = 1.0
    y = int4_hip.dbg_gemm(x.to(dev), w.to(dev), None if sz is None else sz.to(dev), M, N, K)
    y = y.cpu().numpy()
    for r, k in enumerate(ks):
        assert np.array_equal(y[r], W[:, k]), (r, k)


def test_ring_gemm_split_matches_unsplit(dev):
    """The split-K result equals the one-pass result within fp32 rounding."""
    import ctypes as C
    import r4q_lib as R
    g = S.gen(77)
    M, N, K = 512, 768, 8192
    w, sz = S.int4_weight(N, K, g)
    x = torch.randn(M, K, generator=g).half()
    X, Wd, SZ = x.to(dev), w.to(dev), sz.to(dev)
    nws = C.c_size_t(0)
    R.call("r4q_gemm_workspace_bytes", M, N, K, 4, C.byref(nws))
    assert nws.value > 0  # this shape splits
    ws = torch.empty(nws.value, dtype=torch.uint8, device=dev)
    y1 = torch.empty(M, N, dtype=torch.float16, device=dev)
    y2 = torch.empty(M, N, dtype=torch.float16, device=dev)
    R.call("r4q_gemm", X.data_ptr(), Wd.data_ptr(), SZ.data_ptr(), y1.data_ptr(), M, N, K, 4,
           R.stream_handle())
    R.call("r4q_gemm_ws", X.data_ptr(), Wd.data_ptr(), SZ.data_ptr(), y2.data_ptr(), M, N, K, 4,
           ws.data_ptr(), nws.value, R.stream_handle())
    a, b = y1.float().cpu().numpy(), y2.float().cpu().numpy()
    assert rel_l2(b, a) <= 1e-3
    want = O.gemm(x.numpy(), w.numpy(), sz.numpy(), 4)
    assert rel_l2(b, want) <= TOL


def test_small_m_path_matches_gemv(dev):
    """M <= 16 rows agree with the batch-1 GEMV row by row (different
    accumulation order: tolerance, not bits)."""
    g = S.gen(5)
    N, K = 1000, 5120
    w, sz = S.int4_weight(N, K, g)
    x = torch.randn(8, K, generator=g).half()
    W, SZ, X = w.to(dev), sz.to(dev), x.to(dev)
    y = int4_hip.dbg_gemm(X, W, SZ, 8, N, K)
    for r in range(8):
        assert rel_l2(y[r], int4_hip.dbg_gemv(X[r].contiguous(), W, SZ, N, K)) <= 1e-3


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("bits,M,I,K", [(4, 8, 17408, 5120), (8, 8, 17408, 5120), (4, 2, 512, 5120),
                                        (8, 16, 2048, 1024), (16, 4, 1024, 2048)])
def test_gemm_silu_fwht_matches_gemm_then_silu(dev, bits, M, I, K, split):
    """r4q_gemm_silu_fwht_ws equals r4q_gemm_ws with the same workspace into
    [M, 2I] followed by r4q_silu_mul_fwht, bit for bit, over two calls: with
    a workspace that splits K (split sum + SiLU gate + FWHT-32 in the reduce)
    and, for M <= 8, without one (the unsplit GEMM over tiles of 32 gate rows
    and the 32 up rows of the same indices, the gate in its epilogue)."""
    import r4q_lib as R
    g = S.gen(7 * M + I + K + bits)
    w, sz = S.weight(2 * I, K, bits, g)
    wd = w.to(dev)
    sd = None if sz is None else sz.to(dev)
    b = C.c_size_t(0)
    R.call("r4q_gemm_workspace_bytes", M, 2 * I, K, bits, C.byref(b))
    assert b.value > 0
    ws = torch.empty(b.value if split else 0, dtype=torch.uint8, device=dev)
    wsp = ws.data_ptr() if split else None
    st = R.stream_handle()
    if not split and M > 8:  # above 8 rows the gate needs the split path: rejected
        x = torch.zeros(M, K, dtype=torch.float16, device=dev)
        y = torch.empty(M, I, dtype=torch.float16, device=dev)
        with pytest.raises(RuntimeError):
            R.call("r4q_gemm_silu_fwht_ws", x.data_ptr(), wd.data_ptr(),
                   None if sd is None else sd.data_ptr(), y.data_ptr(), M, I, K, bits, None, 0,
                   st)
        return
    for rep in range(2):
        x = (torch.randn(M, K, generator=g) * (0.5 + rep)).half().to(dev)
        gu = torch.empty(M, 2 * I, dtype=torch.float16, device=dev)
        want = torch.empty(M, I, dtype=torch.float16, device=dev)
        R.call("r4q_gemm_ws", x.data_ptr(), wd.data_ptr(), None if sd is None else sd.data_ptr(),
               gu.data_ptr(), M, 2 * I, K, bits, wsp, ws.numel(), st)
        R.call("r4q_silu_mul_fwht", gu.data_ptr(), gu.data_ptr() + 2 * I, want.data_ptr(),
               M, I, 2 * I, I, st)
        got = torch.full((M, I), float("nan"), dtype=torch.float16, device=dev)
        R.call("r4q_gemm_silu_fwht_ws", x.data_ptr(), wd.data_ptr(),
               None if sd is None else sd.data_ptr(), got.data_ptr(), M, I, K, bits,
               wsp, ws.numel(), st)
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (bits, M, I, K, rep)


def test_gemm_silu_fwht_rejects_unsplit_shapes(dev):
    """One row, I off the 32-chunk grid, or more than 8 rows with a workspace
    too small to split K are errors (the caller uses r4q_gemm_ws +
    r4q_silu_mul_fwht there)."""
    import r4q_lib as R
    I, K = 512, 5120
    w, sz = S.weight(2 * I, K, 4, S.gen(5))
    wd, sd = w.to(dev), sz.to(dev)
    x = torch.zeros(16, K, dtype=torch.float16, device=dev)
    y = torch.empty(16, I, dtype=torch.float16, device=dev)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
    st = R.stream_handle()
    for (M, II, nbytes) in ((1, I, ws.numel()), (8, I - 16, ws.numel()), (16, I, 256)):
        with pytest.raises(RuntimeError):
            R.call("r4q_gemm_silu_fwht_ws", x.data_ptr(), wd.data_ptr(), sd.data_ptr(),
                   y.data_ptr(), M, II, K, 4, ws.data_ptr(), nbytes, st)


def _ref32(x, w, sz, bits):
    """x @ deq(W)^T in float32 on the CPU: the oracle's dequantisation (bit-exact
    to the kernels') and a library matmul, for shapes too large for the
    float64 oracle GEMM to finish in seconds."""
    W = torch.from_numpy(O.dequant(w.numpy(), None if sz is None else sz.numpy(), bits)).float()
    return (x.float() @ W.T).numpy()


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_ring_gemm_whole_tile_rounds_then_stream_k(dev, bits):
    """576 tiles of 256 x 256 (more than two rounds of 256 workgroups): the
    first two rounds' 512 tiles are computed whole, the remaining 64 tiles'
    K units are shared by 256 stream-K workgroups (pieces of tiles as fp32
    partials, summed in segment order)."""
    import ctypes as C
    import r4q_lib as R
    M, N, K = 2304, 16384, 768
    g = S.gen(91 + bits)
    w, sz = S.weight(N, K, bits, g)
    x = (torch.randn(M, K, generator=g) * 0.5).half()
    nws = C.c_size_t(0)
    R.call("r4q_gemm_workspace_bytes", M, N, K, bits, C.byref(nws))
    assert nws.value > 0
    SZ = None if sz is None else sz.to(dev)
    got = int4_hip.dbg_gemm(x.to(dev), w.to(dev), SZ, M, N, K).float().cpu().numpy()
    want = _ref32(x, w, sz, bits)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) <= TOL
    for r in (0, 255, 256, 1023, 2047, 2048, 2200, M - 1):  # whole-tile and shared rows
        assert rel_l2(got[r], want[r]) <= TOL, r


@pytest.mark.parametrize("splits", [2, 5])
def test_ring_gemm_forced_split_counts(dev, splits):
    """The gemm_splits override shares every tile among about `splits`
    workgroups; results equal the default plan's within fp32 rounding and
    the oracle's within the GEMM tolerance."""
    import ctypes as C
    import r4q_lib as R
    M, N, K = 512, 1280, 4096
    g = S.gen(17 + splits)
    w, sz = S.int4_weight(N, K, g)
    x = torch.randn(M, K, generator=g).half()
    X, Wd, SZ = x.to(dev), w.to(dev), sz.to(dev)
    base = int4_hip.dbg_gemm(X, Wd, SZ, M, N, K).float().cpu().numpy()
    try:
        R.tune("gemm_splits", splits)
        nws = C.c_size_t(0)
        R.call("r4q_gemm_workspace_bytes", M, N, K, 4, C.byref(nws))
        assert nws.value > 0
        got = int4_hip.dbg_gemm(X, Wd, SZ, M, N, K).float().cpu().numpy()
    finally:
        R.tune("gemm_splits", 0)
    assert rel_l2(got, base) <= 1e-3
    assert rel_l2(got, O.gemm(x.numpy(), w.numpy(), sz.numpy(), 4)) <= TOL


def _spec(fn):
    """Runs fn with the specialised-wave GEMM kernel selected."""
    import r4q_lib as R
    R.tune("gemm_kernel", 2)
    try:
        return fn()
    finally:
        R.tune("gemm_kernel", 0)


@pytest.mark.parametrize("M,N,K", [(512, 17408, 5120), (512, 5120, 17408), (600, 256, 4096),
                                   (512, 7168, 5120), (300, 1280, 2048)])
def test_spec_gemm_vs_oracle_and_ring(dev, M, N, K):
    """The specialised-wave kernel (INT4, N % 128 == 0, K % 256 == 0): config
    3 shapes, a ragged M and split-K shapes against the oracle, and against
    the ring kernel within fp32 / fp16-partial rounding."""
    g = S.gen(M + 5 * N + K)
    w, sz = S.int4_weight(N, K, g)
    x = torch.randn(M, K, generator=g).half()
    X, Wd, SZ = x.to(dev), w.to(dev), sz.to(dev)
    ring = int4_hip.dbg_gemm(X, Wd, SZ, M, N, K).float().cpu().numpy()
    got = _spec(lambda: int4_hip.dbg_gemm(X, Wd, SZ, M, N, K)).float().cpu().numpy()
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ring) <= 1e-3
    want = _ref32(x, w, sz, 4) if N * K > 4e7 else O.gemm(x.numpy(), w.numpy(), sz.numpy(), 4)
    assert rel_l2(got, want) <= TOL
    for r in (0, M // 2, M - 1):
        assert rel_l2(got[r], want[r]) <= TOL, r


def test_spec_gemm_whole_tiles_bit_identical_to_ring(dev):
    """With whole tiles only (gemm_splits 1) every output element sees the same
    MFMA sequence in both kernels: bit-identical results."""
    import r4q_lib as R
    M, N, K = 512, 1024, 2048
    g = S.gen(123)
    w, sz = S.int4_weight(N, K, g)
    x = torch.randn(M, K, generator=g).half()
    X, Wd, SZ = x.to(dev), w.to(dev), sz.to(dev)
    R.tune("gemm_splits", 1)
    try:
        ring = int4_hip.dbg_gemm(X, Wd, SZ, M, N, K).cpu().numpy()
        got = _spec(lambda: int4_hip.dbg_gemm(X, Wd, SZ, M, N, K)).cpu().numpy()
    finally:
        R.tune("gemm_splits", 0)
    assert np.array_equal(got.view(np.uint16), ring.view(np.uint16))


@pytest.mark.parametrize("splits", [0, 3])
def test_spec_gemm_one_hot_columns_exact(dev, splits):
    """Row r of x = e_k(r): y[r] is column k(r) of the dequantised weight, bit
    for bit, through the specialised-wave kernel's B stages -- in the default
    plan and with every tile shared by about 3 workgroups (fp16 partials of
    zeros and one exact product, summed by its reduce)."""
    import r4q_lib as R
    g = S.gen(211 + splits)
    M, N, K = 300, 384, 2048
    w, sz = S.int4_weight(N, K, g)
    W = O.dequant(w.numpy(), sz.numpy(), 4)
    ks = [(r * 631 + r // 5) % K for r in range(M)]
    x = torch.zeros(M, K, dtype=torch.float16)
    for r, k in enumerate(ks):
        x[r, k] = 1.0
    R.tune("gemm_splits", splits)
    try:
        y = _spec(lambda: int4_hip.dbg_gemm(x.to(dev), w.to(dev), sz.to(dev), M, N, K)).cpu().numpy()
    finally:
        R.tune("gemm_splits", 0)
    for r, k in enumerate(ks):
        assert np.array_equal(y[r], W[:, k]), (r, k)
