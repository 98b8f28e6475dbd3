"""MI355X-native VecAttention prefill (selection + vector-sparse attention).

Drop-in for ``spattn.src.VecAttention.VecAttention_prefill`` and the
selection-stage helpers its threshold tuner calls.
"""
from .vecattention import VecAttention_prefill, threshold_to_gap
from .stages import average_vector, fuse_qk_softmax_minp_wo_causal
from .dispatch import (DiffusionStepContext, FastPrefillConfig, Full_prefill,
                       customize_prefill_attention, select_cfg_threshold)
from .tuner import seg_pr_perHead
from .decode import single_decode_with_kv_cache

__all__ = [
    "VecAttention_prefill",
    "average_vector",
    "fuse_qk_softmax_minp_wo_causal",
    "threshold_to_gap",
    "Full_prefill",
    "FastPrefillConfig",
    "customize_prefill_attention",
    "DiffusionStepContext",
    "select_cfg_threshold",
    "seg_pr_perHead",
    "single_decode_with_kv_cache",
]
