"""mini_trainer_amd: MI355X-native (gfx950) fused LM-head linear + per-token
cross-entropy for mini_trainer-style padding-free training.

The compute lives in libmt_flce.so (hand-written HIP, C ABI in
include/mt_flce.h); this package is the PyTorch-facing host side.
"""
from .causal_lm import (
    causal_lm_loss,
    cu_seqlens_from_lengths,
    cu_seqlens_from_minibatch,
    cu_seqlens_from_position_ids,
    patch_causal_lm,
    sample_loss_sums,
)
from .flce import (
    backward_plan,
    path_of,
    cross_entropy_none,
    fused_linear_cross_entropy,
    per_sample_loss_sums,
    prepare_targets,
)
from .none_reduction_losses import (
    hf_fixed_cross_entropy_none_reduction,
    liger_fixed_fused_linear_cross_entropy_none_reduction,
)
from .utils import patch_target_module

__all__ = [
    "causal_lm_loss",
    "cu_seqlens_from_lengths",
    "cu_seqlens_from_minibatch",
    "cu_seqlens_from_position_ids",
    "sample_loss_sums",
    "patch_causal_lm",
    "backward_plan",
    "path_of",
    "cross_entropy_none",
    "fused_linear_cross_entropy",
    "per_sample_loss_sums",
    "prepare_targets",
    "hf_fixed_cross_entropy_none_reduction",
    "liger_fixed_fused_linear_cross_entropy_none_reduction",
    "patch_target_module",
]
