"""Caller glue of the prefill path: the attention dispatcher, dense prefill and
the DiT threshold helpers, on top of the HIP kernels.

- ``FastPrefillConfig``: the dispatcher's configuration
  (spattn/src/models/config_args.py:6-75), same fields and defaults.
- ``Full_prefill``: dense attention (spattn/src/Fullprefill.py:4-16, which
  calls flashinfer's single_prefill_with_kv_cache), here the MFMA attention
  kernel over every key (``va_dense_attn``).
- ``customize_prefill_attention``: the per-layer dispatcher
  (spattn/src/models/utils.py:47-162) for the 'vecattention' and 'full'
  metrics, including the vision-span slicing (text before the span and after
  it in dense attention, the span in VecAttention), the per-layer threshold of
  a (layers, heads) threshold tensor, the latency record and the Q/K dump.
- ``DiffusionStepContext`` and ``select_cfg_threshold``: the positive/negative
  threshold switch of classifier-free guidance
  (eval/DiTEvalKit/models/diffusion_context.py:4-40,
  eval/DiTEvalKit/models/wan/attention.py:647-666).
- ``_load_threshold_pt`` / ``_save_threshold_pt``: the DiT threshold matrix
  file helpers (eval/DiTEvalKit/utils/misc.py:44-93).

The other metrics of the reference dispatcher ('xattn', 'flex', 'anchor')
are other attention methods, not part of this path; they raise
NotImplementedError here.
"""
import json
import os
import threading
from typing import Optional, Union

import torch

from . import stages
from .vecattention import VecAttention_prefill

SPARSITY_RECORD = threading.local()

NUM_LAYERS = 60
NUM_HEADS = 24


class FastPrefillConfig(dict):
    """Prefill attention configuration (spattn/src/models/config_args.py:6-75).

    ``metric``: 'vecattention' or 'full' here.  ``threshold``: MinP threshold,
    a float or a per-head / (layers, heads) tensor.  ``vision_start_position``
    / ``vision_end_position``: the vision span of a VLM prompt (causal only).
    """

    def __init__(self, metric: str = "xattn", threshold: float = None, block_size_q: int = 64,
                 block_size_k: int = 16, group_k_block: int = 1, chunk_size: int = 8 * 1024,
                 vision_start_position: Optional[int] = None,
                 vision_end_position: Optional[int] = None, stride: int = 16,
                 gamma: float = 0.9, tau: float = 0.1, theta: float = 12, step: int = 16,
                 output_time: bool = True, dump_qk_dir: Optional[str] = None,
                 input_id: str = "input"):
        super().__init__()
        self.metric = metric
        self.output_time = output_time
        self.block_size_q = block_size_q
        self.block_size_k = block_size_k
        self.group_k_block = group_k_block
        self.chunk_size = chunk_size
        self.vision_start_position = vision_start_position
        self.vision_end_position = vision_end_position
        self.stride = stride
        self.gamma = gamma
        self.tau = tau
        self.theta = theta
        self.step = step
        self.dump_qk_dir = dump_qk_dir
        self.input_id = input_id
        if threshold is not None:
            self.threshold = threshold


def Full_prefill(query_states: torch.Tensor, key_states: torch.Tensor,
                 value_states: torch.Tensor, causal: bool = True) -> torch.Tensor:
    """Dense attention, (B, Hq, Sq, D) -> (B, Hq, Sq, D) in the input dtype.

    Causal rows see keys up to ``i + Sk - Sq`` (the last query aligned with the
    last key, flashinfer's convention for Sq < Sk).  Key/value heads may divide
    the query heads (GQA).  bf16/fp16/fp32, head_dim 64 or 128.
    """
    if query_states.dim() != 4 or key_states.dim() != 4 or value_states.dim() != 4:
        raise AssertionError("query/key/value must be (batch, heads, seq, head_dim)")
    if not query_states.is_cuda:
        raise RuntimeError("Full_prefill runs on the GPU")
    return stages.dense_attention(query_states, key_states, value_states, causal=causal)


def customize_prefill_attention(self, query_states, key_states, value_states,
                                attention_mask=None, position_ids=None, causal=True,
                                config=None):
    """Per-layer prefill attention dispatch (spattn/src/models/utils.py:47-162).

    ``self`` is the attention layer (its ``layer_idx`` picks the row of a
    (layers, heads) threshold tensor).  Returns (B, H, S, D).
    """
    if config is None:
        config = FastPrefillConfig()
    assert causal or config.metric in ["full", "xattn", "vecattention"], (
        f"Non-causal attention only supports full, xattn, or vecattention metrics. Got: {config.metric}.")
    start_evt = end_evt = None
    if config.output_time and query_states.is_cuda:
        start_evt = torch.cuda.Event(enable_timing=True)
        end_evt = torch.cuda.Event(enable_timing=True)
        start_evt.record(stream=torch.cuda.current_stream(device=query_states.device))

    if config.metric == "vecattention":
        threshold = config.threshold[self.layer_idx] if isinstance(config.threshold, torch.Tensor) \
            else config.threshold
        vs, ve = config.vision_start_position, config.vision_end_position
        kw = dict(threshold=threshold, q_pooling_size=config.block_size_q,
                  k_local_size=config.block_size_k, group_k_block=config.group_k_block,
                  causal=causal, chunk_size=config.chunk_size)
        if vs is None and ve is None:
            attn_output = VecAttention_prefill(query_states, key_states, value_states, **kw)
        else:
            assert causal, "Only causal attention is supported when vision positions are set"
            if vs is not None:  # dense attention on the text before the vision span
                before = Full_prefill(query_states[:, :, :vs, :], key_states[:, :, :vs, :],
                                      value_states[:, :, :vs, :], causal=causal)
            attn_va = VecAttention_prefill(query_states[:, :, :ve, :], key_states[:, :, :ve, :],
                                           value_states[:, :, :ve, :], **kw)
            if vs is not None:
                attn_va[:, :, :vs, :] = before
            if ve is not None:  # dense attention on the text after it, over every key
                after = Full_prefill(query_states[:, :, ve:, :], key_states, value_states,
                                     causal=causal)
                attn_output = torch.cat([attn_va, after], dim=2)
            else:
                attn_output = attn_va
    elif config.metric == "full":
        attn_output = Full_prefill(query_states, key_states, value_states, causal=causal)
    else:
        raise NotImplementedError(f"Unknown attention metric: {config.metric}")

    if start_evt is not None:
        end_evt.record(stream=torch.cuda.current_stream(device=query_states.device))
        if not hasattr(SPARSITY_RECORD, "attention_latency_list"):
            SPARSITY_RECORD.attention_latency_list = []
        SPARSITY_RECORD.attention_latency_list.append((start_evt, end_evt))

    if config.dump_qk_dir:
        dir_name = os.path.join(config.dump_qk_dir, config.input_id)
        os.makedirs(dir_name, exist_ok=True)
        path = os.path.join(dir_name, f"layer_{self.layer_idx}_qk.pt")
        if not os.path.exists(path):
            torch.save({"query_states": query_states, "key_states": key_states}, path)
    return attn_output


class DiffusionStepContext:
    """Runtime state shared by a DiT's attention layers across diffusion steps
    (eval/DiTEvalKit/models/diffusion_context.py:4-40)."""

    def __init__(self, is_cfg: bool = False, dump_qk_negative: bool = False):
        self.current_rel_step: int = -1
        self.pre_time_step: Optional[float] = None
        self.is_cfg: bool = is_cfg
        self.dump_qk_negative: bool = dump_qk_negative
        self.dump_qk_started: bool = False
        self.dump_qk_done: bool = False


def select_cfg_threshold(config, step_ctx: DiffusionStepContext, layer_idx: int, timestep) -> None:
    """Layer 0's step bookkeeping (eval/DiTEvalKit/models/wan/attention.py:647-666).

    A new timestep value starts a diffusion step.  Under classifier-free
    guidance each step runs twice: the first pass uses ``config.pos_threshold``
    and the second (same timestep) ``config.neg_threshold``.  Other layers and
    other metrics leave the config unchanged.
    """
    if config.metric != "vecattention" or layer_idx != 0:
        return
    cur = timestep[0].item() if isinstance(timestep, torch.Tensor) else float(timestep[0])
    change_step = step_ctx.pre_time_step is None or step_ctx.pre_time_step != cur
    if change_step:
        step_ctx.current_rel_step += 1
    if step_ctx.is_cfg:
        config.threshold = config.pos_threshold if change_step else config.neg_threshold
    step_ctx.pre_time_step = cur


def _read_matrix_rows(path: str, num_layers: int, num_heads: int):
    """Rows of a threshold matrix file: JSON holding one list of num_heads
    numbers per layer.  Every row is checked, not only the first."""
    with open(path, "r") as f:
        doc = json.load(f)
    if not isinstance(doc, list):
        raise ValueError(f"expected a JSON list of layers, found {type(doc).__name__}")
    if len(doc) != num_layers:
        raise ValueError(f"{len(doc)} layers in the file, {num_layers} expected")
    for layer, row in enumerate(doc):
        if not isinstance(row, list) or len(row) != num_heads:
            got = len(row) if isinstance(row, list) else type(row).__name__
            raise ValueError(f"layer {layer}: {got} heads, {num_heads} expected")
    return doc


def _load_threshold_pt(thr_path: Optional[str], num_layers: int = NUM_LAYERS,
                       num_heads: int = NUM_HEADS,
                       device: torch.device = torch.device("cpu")) -> torch.Tensor:
    """Per-layer, per-head thresholds of a DiT model as a contiguous
    (num_layers, num_heads) float32 tensor on `device`.

    File format (the one eval/DiTEvalKit/utils/misc.py:44-64 reads): a JSON
    list with one entry per layer, each a list of one threshold per head.
    A missing or unreadable file, or one of another shape, raises
    RuntimeError naming the file.
    """
    try:
        rows = _read_matrix_rows(thr_path, num_layers, num_heads)
        mat = torch.tensor(rows, dtype=torch.float32)
    except (OSError, ValueError, TypeError) as err:
        raise RuntimeError(f"threshold file {thr_path!r} unusable: {err}") from err
    return mat.to(device).contiguous()


def _save_threshold_pt(thr_path: str, thr_mat: Union[torch.Tensor, float],
                       num_layers: int = NUM_LAYERS) -> str:
    """Write one threshold per layer with torch.save, as a (num_layers,)
    float32 tensor (the file eval/DiTEvalKit/utils/misc.py:67-93 writes).

    `thr_mat` is a Python float (the same value for every layer), a
    one-element tensor (likewise) or a (num_layers,) tensor.  Other types
    raise TypeError, other shapes ValueError.  Returns the path.
    """
    if isinstance(thr_mat, float):
        vec = torch.full((num_layers,), thr_mat, dtype=torch.float32)
    elif isinstance(thr_mat, torch.Tensor):
        if thr_mat.dim() != 1 or thr_mat.numel() not in (1, num_layers):
            raise ValueError(f"a threshold tensor of shape {tuple(thr_mat.shape)} does not give "
                             f"one value per layer for {num_layers} layers")
        vec = thr_mat.expand(num_layers).clone() if thr_mat.numel() == 1 else thr_mat
    else:
        raise TypeError(f"thresholds must be a float or a tensor, not {type(thr_mat).__name__}")
    torch.save(vec, thr_path)
    return thr_path


load_threshold_matrix = _load_threshold_pt
save_threshold_vector = _save_threshold_pt
