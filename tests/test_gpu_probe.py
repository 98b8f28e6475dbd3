"""The row-gather probe (va_probe_gather) behind bench.py's gather ceiling:
its copies land in LDS and every work-group reports the first byte it read."""
import pytest
import torch

from vecattention_amd import _native as nat

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("sequential", [0, 1])
def test_probe_copies_rows_into_lds(device, sequential):
    rows, wgs, steps = 4096, 16, 32
    table = torch.full((rows * 256,), 3, dtype=torch.uint8, device=device)
    sink = torch.zeros(wgs, dtype=torch.int32, device=device)
    rc = nat.lib().va_probe_gather(nat.ptr(table), rows, wgs, steps, sequential, nat.ptr(sink),
                                   torch.cuda.current_stream(device).cuda_stream)
    nat.check("va_probe_gather", rc)
    torch.cuda.synchronize()
    assert torch.equal(sink.cpu(), torch.full((wgs,), 3, dtype=torch.int32))
