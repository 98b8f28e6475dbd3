"""The row-gather probe (va_probe_gather, tests/numerics/gather_probe.hip)
behind bench.py's gather ceiling: its copies land in LDS and every work-group
reports the first byte it read."""
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "numerics"))
import gather_probe  # noqa: E402

from vecattention_amd import _native as nat  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("sequential", [0, 1])
def test_probe_copies_rows_into_lds(device, sequential):
    rows, wgs, steps = 4096, 16, 32
    table = torch.full((rows * 256,), 3, dtype=torch.uint8, device=device)
    sink = torch.zeros(wgs, dtype=torch.int32, device=device)
    gather_probe.gather(nat.ptr(table), rows, wgs, steps, sequential, nat.ptr(sink),
                        torch.cuda.current_stream(device).cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(sink.cpu(), torch.full((wgs,), 3, dtype=torch.int32))
