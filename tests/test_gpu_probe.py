"""The HBM read-floor measurement entry point (r4q_hbm_read): argument
checks on the host, and a run over a ragged byte count that leaves the sink
untouched."""
import pytest
import torch

import r4q_lib as R

pytestmark = pytest.mark.gpu


def test_hbm_read_runs_and_checks(dev):
    n = 55_705_600 + 7  # the config-0 GEMV's weight + scale bytes, plus a ragged tail
    src = torch.full((n + 9,), 3, dtype=torch.uint8, device=dev)
    sink = torch.zeros(8192, dtype=torch.uint8, device=dev)
    R.call("r4q_hbm_read", src.data_ptr(), n, sink.data_ptr(), sink.numel(), R.stream_handle())
    torch.cuda.synchronize()
    assert int(sink.count_nonzero()) == 0
    with pytest.raises(RuntimeError, match="sink must hold"):
        R.call("r4q_hbm_read", src.data_ptr(), n, sink.data_ptr(), 4096, R.stream_handle())
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        R.call("r4q_hbm_read", src.data_ptr() + 1, 64, sink.data_ptr(), sink.numel(),
               R.stream_handle())
