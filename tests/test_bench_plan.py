"""Host-side plan of bench.py (no GPU): the KV cache capacity covers every
position the decode legs write, for the driver's (steps, warmup) and others,
and a failing secondary leg is recorded instead of ending the run."""
import importlib.util

import pytest

from conftest import ROOT


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


B = load_bench()

# (steps, warmup): the driver's command (20, 5), the defaults, and edges
PAIRS = [(20, 5), (128, 16), (1, 0), (1, 1), (5, 40), (3, 2), (200, 3), (36, 36)]


@pytest.mark.parametrize("steps,warmup", PAIRS)
@pytest.mark.parametrize("ctx", [1, 10, 128, 2048, 32768])
def test_capacity_covers_every_decode_leg(ctx, steps, warmup):
    cap = B.cache_capacity(ctx, steps, warmup)
    ranges = B.decode_ranges(ctx, steps, warmup)
    B.check_capacity(cap, ranges, "plan")  # raises on an overrun
    # the timed steps start at ctx, the engine leg decodes its tokens from ctx
    assert (ctx, steps) in ranges
    assert (ctx, B.ENGINE_WARM + B.ENGINE_TOKENS) in ranges
    assert cap >= ctx + max(steps, B.ENGINE_WARM + B.ENGINE_TOKENS)
    # the warm-up ends where the timed steps start (or starts at 0)
    if warmup:
        first, count = [r for r in ranges if r not in ((ctx, steps),
                                                       (ctx, B.ENGINE_WARM + B.ENGINE_TOKENS))][0]
        assert first == max(0, ctx - warmup) and count == warmup


def test_driver_command_engine_leg_fits():
    # the round's driver runs --steps 20 --warmup 5; the engine leg then
    # decodes 36 positions from ctx = 2048, past ctx + steps + warmup
    cap = B.cache_capacity(2048, 20, 5)
    assert 2048 + B.ENGINE_WARM + B.ENGINE_TOKENS <= cap
    with pytest.raises(RuntimeError):
        B.check_capacity(2048 + 33, [(2048, B.ENGINE_WARM + B.ENGINE_TOKENS)], "engine leg")


def test_guarded_records_failure_and_continues():
    errors = {}

    def boom():
        raise RuntimeError("librdna4q: status -1: positions exceed the KV cache")

    assert B.guarded("leg", errors, boom) is None
    assert "leg" in errors and "KV cache" in errors["leg"]
    assert B.guarded("ok", errors, lambda x: x + 1, 1) == 2
    assert "ok" not in errors


def test_matrix_covers_config4():
    assert set(B.MATRIX_CTX) == {128, 2048} and set(B.MATRIX_BATCH) == {1, 8}
