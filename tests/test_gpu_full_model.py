"""Config 4 at its full size: the 40-layer Qwen3-14B-shaped model (32 of 160
matrices INT8, FP16 LM head over vocab 151936) with FP8 caches filled to
ctx 2048, at batch 1 and batch 8.  The oracle cannot run 40 full-width layers
in test time (the 2-layer full-width step tests pin the arithmetic); here the
size-independent properties hold at full size:
  * the captured decode loop (one hipGraph per step, the position in device
    memory) produces the same tokens and KV bytes as the eager loop;
  * decode_step_logits through its captured graph equals the eager step bit
    for bit (logits and KV bytes);
  * logits are finite and each step writes exactly its own cache position."""
import numpy as np
import pytest
import torch

import int4_hip
import r4q_synth as S

pytestmark = pytest.mark.gpu
CTX, N_TOK = 2048, 4


@pytest.fixture(scope="module")
def model(dev):
    print("[full-model] generating 40 layers, batch 8, ctx 2048", flush=True)
    m = S.qwen3_model(CTX, 16, 8, dev)
    torch.cuda.synchronize()
    yield m
    del m
    torch.cuda.empty_cache()


def _tail(m, B):
    """Caches of the first B sequences (contiguous views) and the argument
    tail of decode_loop at CTX."""
    a = list(S.qwen3_bench_args(m, CTX))
    a[25] = [t[:B] for t in m["kc"]]
    a[26] = [t[:B] for t in m["vc"]]
    return a


def _written(m, B, lo, hi):
    return [t[:B, :, lo:hi].cpu().clone() for t in m["kc"] + m["vc"]]


def _clear(m, lo, hi):
    for t in m["kc"] + m["vc"]:
        t[:, :, lo:hi] = 0


@pytest.mark.parametrize("B", [1, 8])
def test_full_model_graph_loop_equals_eager(dev, model, B):
    m = model
    print(f"[full-model] decode loop B={B}", flush=True)
    h = (torch.randn(B, 1, m["D"], generator=S.gen(B)) * 0.5).half().to(dev)
    a = _tail(m, B)
    before = _written(m, B, 0, CTX)
    toks = {}
    kv = {}
    for use_graph in (False, True):
        _clear(m, CTX, CTX + N_TOK)
        (e, fn, lw, ls, V, K) = (m["embed"], m["final_norm"], m["lm_w"], None, m["V"], m["D"])
        toks[use_graph] = int4_hip.decode_loop(e, fn, lw, ls, V, K, h, N_TOK, *a[:25], a[25],
                                               a[26], a[32], use_graph=use_graph)
        torch.cuda.synchronize()
        kv[use_graph] = _written(m, B, CTX, CTX + N_TOK + 1)
    assert torch.equal(toks[False], toks[True])
    t = toks[True].reshape(N_TOK, -1)
    assert int(t.min()) >= 0 and int(t.max()) < m["V"]
    for x, y in zip(kv[False], kv[True]):
        assert torch.equal(x, y)
        assert int(x[:, :, :N_TOK].ne(0).sum()) > 0      # each step wrote its position
        assert int(x[:, :, N_TOK:].ne(0).sum()) == 0      # and nothing past the last
    after = _written(m, B, 0, CTX)
    for x, y in zip(before, after):
        assert torch.equal(x, y)                           # the prompt's positions untouched
    _clear(m, CTX, CTX + N_TOK)


def test_full_model_graph_step_equals_eager_step(dev, model):
    m = model
    print("[full-model] decode_step_logits graph vs eager", flush=True)
    h = (torch.randn(1, 1, m["D"], generator=S.gen(7)) * 0.5).half().to(dev)
    a = _tail(m, 1)
    res = {}
    for use_graph in (False, True):
        _clear(m, CTX, CTX + 2)
        lg = [int4_hip.decode_step_logits(h, *a[:18], CTX + i, *a[19:25], a[25], a[26], a[27],
                                          a[28], a[29], a[30], a[31], a[32],
                                          use_graph=use_graph).cpu() for i in range(2)]
        torch.cuda.synchronize()
        res[use_graph] = (lg, _written(m, 1, CTX, CTX + 2))
    for x, y in zip(res[False][0], res[True][0]):
        assert x.shape == (1, 1, m["V"])
        assert torch.isfinite(x.float()).all()
        assert torch.equal(x, y)
    for x, y in zip(res[False][1], res[True][1]):
        assert torch.equal(x, y)
    _clear(m, CTX, CTX + 2)
