"""Drop-in replacements for the reference's per-token loss functions.

Same names, signatures and semantics as none_reduction_losses.py:5-36 of
mini_trainer; installed the same way (utils.patch_target_module, called
before model construction as in setup_model_for_training.py:93-105).  The
arithmetic runs in libmt_flce.so on the ROCm device.
"""
from __future__ import annotations

from typing import Optional

import torch

from .flce import cross_entropy_none, fused_linear_cross_entropy

# The one keyword of **kwargs the drop-in reads (see its docstring).
GRAD_SCALE_KWARG = "mt_grad_scale"


def liger_fixed_fused_linear_cross_entropy_none_reduction(
    hidden_states: torch.Tensor,
    lm_head_weight: torch.Tensor,
    target: torch.Tensor,
    num_items_in_batch: Optional[int] = None,
    ignore_index: int = -100,
    final_logit_softcapping: Optional[float] = None,
    **kwargs,
) -> torch.Tensor:
    """Per-token fused LM-head + cross-entropy loss, reduction 'none'.

    Reference: none_reduction_losses.py:5-25, which forwards reduction='none',
    ignore_index and softcap=final_logit_softcapping to Liger's fused kernel
    and ignores num_items_in_batch and **kwargs (:9,12).  Returns fp32 [T]
    with +0.0 at ignored positions, differentiable in hidden_states and
    lm_head_weight.  Of **kwargs only `mt_grad_scale` is read (absent from
    the reference's callers, and named for this package so that no other
    caller's keyword selects it): a caller that knows the upstream gradient
    of the loss before the forward passes it to promise that gradient to the
    fused path (flce.fused_linear_cross_entropy's grad_scale).
    """
    return fused_linear_cross_entropy(hidden_states, lm_head_weight, target,
                                      ignore_index=ignore_index, softcap=final_logit_softcapping,
                                      grad_scale=kwargs.get(GRAD_SCALE_KWARG))


def hf_fixed_cross_entropy_none_reduction(
    source: torch.Tensor,
    target: torch.Tensor,
    num_items_in_batch: Optional[int] = None,
    ignore_index: int = -100,
    **kwargs,
) -> torch.Tensor:
    """Per-token cross-entropy over materialised logits, reduction 'none'.

    Reference: none_reduction_losses.py:27-36 (F.cross_entropy(source, target,
    ignore_index=ignore_index, reduction='none') at :35).
    """
    return cross_entropy_none(source, target, ignore_index=ignore_index)
