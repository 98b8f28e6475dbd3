"""Host-side logic of the drop-in: argument checks that mirror the reference's
assertions, the threshold -> gap conversion, and the synthetic generator."""
import math

import numpy as np
import pytest
import torch

from vecattention_amd import VecAttention_prefill, threshold_to_gap
from vecattention_amd.synth import WORKLOADS, make_inputs
from vecattention_amd.vecattention import reference_block_size_q


def _cpu_inputs():
    return (torch.zeros(1, 2, 128, 64), torch.zeros(1, 2, 128, 64), torch.zeros(1, 2, 128, 64))


def test_reference_assertions_come_first():
    q, k, v = _cpu_inputs()
    with pytest.raises(AssertionError, match="multiple of q_pooling_size"):
        VecAttention_prefill(q, k, v, 0.9, q_pooling_size=64, chunk_size=100)
    with pytest.raises(AssertionError, match="64 or 128"):
        VecAttention_prefill(q, k, v, 0.9, q_pooling_size=32, chunk_size=128)
    with pytest.raises(TypeError):
        VecAttention_prefill(q, k, v, None, q_pooling_size=64, chunk_size=128)
    with pytest.raises(RuntimeError, match="device tensors"):
        VecAttention_prefill(q, k, v, 0.9, q_pooling_size=64, chunk_size=128)


def test_gap_float_matches_reference_expression():
    gap, gaps = threshold_to_gap(0.8, 1, 4, "cpu")
    assert gaps is None
    assert gap == -math.log(0.8 + 1e-9, math.e)
    assert np.float32(gap) == np.float32(0.2231435477733612)


def test_gap_tensor_shapes():
    th = torch.tensor([0.8, 0.9, 0.5], dtype=torch.float32)
    _, g = threshold_to_gap(th, 2, 3, "cpu")
    assert g.shape == (2, 3) and g.dtype == torch.float32
    want = -torch.log(th + 1e-9)
    assert torch.equal(g[1], want)
    _, g = threshold_to_gap(torch.full((2, 3), 0.7), 2, 3, "cpu")
    assert torch.allclose(g, torch.full((2, 3), -math.log(0.7 + 1e-9)))
    with pytest.raises(AssertionError):
        threshold_to_gap(torch.ones(4), 2, 3, "cpu")


def test_block_size_q_of_reference_configs():
    for key in [(64, 16, 16, 128, True), (64, 16, 8192, 128, True)]:
        assert reference_block_size_q(*key) == 64


def test_generator_structure_and_determinism():
    q, k, v = make_inputs(1, 4, 2, 512, 32, torch.float32, seed=1)
    q2, k2, v2 = make_inputs(1, 4, 2, 512, 32, torch.float32, seed=1)
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
    assert q.shape == (1, 4, 512, 32) and k.shape == (1, 2, 512, 32)
    # Sinks carry the +4u vertical direction: their keys score high against q.
    s = (q[0, 0] @ k[0, 0].T).mean(0)
    assert s[:64].mean() > s[64:].mean() + 3.0


def test_workload_table_matches_plan():
    assert WORKLOADS["B"].S == 32768 and WORKLOADS["B"].Hq == 28 and WORKLOADS["B"].Hk == 4
    assert WORKLOADS["C"].S == 131072 and WORKLOADS["C"].keep == 0.05
    assert WORKLOADS["D"].S == 21 * 1560 and not WORKLOADS["D"].causal
    assert WORKLOADS["E"].S == 33 * 3600 + 256


def test_bench_refuses_more_than_one_gpu():
    # bench.py measures one GPU: asked for more it exits with status 2 and says
    # so, before touching a device (runs on the CPU-only host too).
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=root)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and r.stdout == ""
