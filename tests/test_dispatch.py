"""Host logic of the caller glue (no GPU): the DiT threshold files, the CFG
threshold switch, the dispatcher's config defaults and its error paths."""
import json

import pytest
import torch

from vecattention_amd import dispatch
from vecattention_amd.dispatch import (DiffusionStepContext, FastPrefillConfig,
                                       customize_prefill_attention, select_cfg_threshold)


def test_config_defaults_follow_the_reference():
    c = FastPrefillConfig()
    assert (c.metric, c.block_size_q, c.block_size_k, c.group_k_block, c.chunk_size) == \
        ("xattn", 64, 16, 1, 8 * 1024)
    assert c.vision_start_position is None and c.vision_end_position is None
    assert not hasattr(c, "threshold")
    assert FastPrefillConfig(threshold=0.9).threshold == 0.9


def test_threshold_matrix_round_trip(tmp_path):
    mat = [[0.1 * (i + 1) + 0.01 * j for j in range(3)] for i in range(2)]
    p = tmp_path / "thr.json"
    p.write_text(json.dumps(mat))
    t = dispatch._load_threshold_pt(str(p), num_layers=2, num_heads=3)
    assert t.dtype == torch.float32 and tuple(t.shape) == (2, 3)
    assert torch.equal(t, torch.tensor(mat, dtype=torch.float32))


@pytest.mark.parametrize("content,layers,heads", [
    ({"a": 1}, 2, 3),                  # not a list
    ([[0.1, 0.2, 0.3]], 2, 3),         # wrong layer count
    ([[0.1, 0.2], [0.3, 0.4]], 2, 3),  # wrong head count
    ([[0.1, 0.2, 0.3], [0.4]], 2, 3),  # a later layer with the wrong head count
    ([[0.1, 0.2, 0.3], 0.5], 2, 3),    # a layer that is not a list
])
def test_threshold_matrix_errors(tmp_path, content, layers, heads):
    p = tmp_path / "bad.json"
    p.write_text(json.dumps(content))
    with pytest.raises(RuntimeError):
        dispatch._load_threshold_pt(str(p), num_layers=layers, num_heads=heads)
    with pytest.raises(RuntimeError):
        dispatch._load_threshold_pt(str(tmp_path / "missing.json"), 2, 3)


def test_threshold_vector_save(tmp_path):
    p = str(tmp_path / "t.pt")
    dispatch._save_threshold_pt(p, 0.25, num_layers=4)
    assert torch.equal(torch.load(p, weights_only=True), torch.full((4,), 0.25))
    dispatch._save_threshold_pt(p, torch.tensor([0.5]), num_layers=3)
    assert torch.equal(torch.load(p, weights_only=True), torch.full((3,), 0.5))
    with pytest.raises(ValueError):
        dispatch._save_threshold_pt(p, torch.ones(2, 2), num_layers=3)
    with pytest.raises(TypeError):
        dispatch._save_threshold_pt(p, 3, num_layers=3)


def test_cfg_threshold_switch():
    cfg = FastPrefillConfig(metric="vecattention", threshold=0.0)
    cfg.pos_threshold, cfg.neg_threshold = 0.9, 0.7
    ctx = DiffusionStepContext(is_cfg=True)
    seen = []
    for ts in [999.0, 999.0, 980.0, 980.0, 961.0]:
        select_cfg_threshold(cfg, ctx, 5, torch.tensor([ts]))   # other layers: no change
        assert cfg.threshold == (seen[-1][1] if seen else 0.0)
        select_cfg_threshold(cfg, ctx, 0, torch.tensor([ts]))
        seen.append((ctx.current_rel_step, cfg.threshold))
    assert seen == [(0, 0.9), (0, 0.7), (1, 0.9), (1, 0.7), (2, 0.9)]
    plain = FastPrefillConfig(metric="vecattention", threshold=0.3)
    ctx2 = DiffusionStepContext(is_cfg=False)
    for ts in [5.0, 4.0]:
        select_cfg_threshold(plain, ctx2, 0, [ts])
    assert plain.threshold == 0.3 and ctx2.current_rel_step == 1


def test_dispatcher_error_paths():
    class L:
        layer_idx = 0
    q = torch.zeros(1, 1, 8, 64)
    with pytest.raises(AssertionError):
        customize_prefill_attention(L(), q, q, q, causal=False,
                                    config=FastPrefillConfig(metric="flex", output_time=False))
    with pytest.raises(NotImplementedError):
        customize_prefill_attention(L(), q, q, q, causal=True,
                                    config=FastPrefillConfig(metric="anchor", output_time=False))
