"""Model-side caller of the fused loss: a causal LM's final hidden states and
lm_head weight go to the kernel path without materialising [T, V] logits.

This stands in for Liger's lce_forward + LigerForCausalLMLoss, which the
reference installs with AutoLigerKernelForCausalLM
(setup_model_for_training.py:93-99) and which reach
none_reduction_losses.py:5-25 through fixed_fused_linear_cross_entropy; Liger
is not part of this build.  Label handling follows transformers'
ForCausalLMLoss (TF/loss/loss_utils.py:49-71): `shift_labels` when given,
otherwise `labels` padded with ignore_index and shifted by one position per
row, then flattened.  The returned loss is per token (reduction 'none'), as
train.py:97-104 consumes it: output.loss.float().sum().
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch
import torch.nn.functional as F

from .flce import fused_linear_cross_entropy, per_sample_loss_sums

__all__ = ["causal_lm_loss", "patch_causal_lm", "sample_loss_sums", "cu_seqlens_from_position_ids",
           "cu_seqlens_from_lengths", "cu_seqlens_from_minibatch"]


def causal_lm_loss(hidden_states: torch.Tensor, lm_head_weight: torch.Tensor,
                   labels: Optional[torch.Tensor] = None,
                   shift_labels: Optional[torch.Tensor] = None, ignore_index: int = -100,
                   final_logit_softcapping: Optional[float] = None, grad_scale=None,
                   dw_accumulator: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-token loss [B * T] fp32 of a causal LM head over hidden_states [B, T, H].

    A single packed row (B = 1, mini_trainer's layout) is shifted on the
    device inside the valid-row compaction; B > 1 rows are padded and shifted
    per row first, so no row takes the next row's first label.
    """
    H = hidden_states.shape[-1]
    hidden = hidden_states.reshape(-1, H)
    if shift_labels is not None:
        target, shift = shift_labels.reshape(-1), False
    elif labels is None:
        raise ValueError("causal_lm_loss needs labels or shift_labels")
    elif labels.dim() >= 2 and labels.shape[0] > 1:
        target = F.pad(labels, (0, 1), value=ignore_index)[..., 1:].reshape(-1)
        shift = False
    else:
        target, shift = labels.reshape(-1), True
    if target.numel() != hidden.shape[0]:
        raise ValueError(f"{target.numel()} labels for {hidden.shape[0]} hidden states")
    return fused_linear_cross_entropy(hidden, lm_head_weight, target, ignore_index=ignore_index,
                                      softcap=final_logit_softcapping, shift_labels=shift,
                                      dw_accumulator=dw_accumulator, grad_scale=grad_scale)


_OUTPUT_CLS = None


def _output_cls():
    """CausalLMOutputWithPast plus the per-sample sums (built on first use, so
    that importing this module does not import transformers)."""
    global _OUTPUT_CLS
    if _OUTPUT_CLS is None:
        from dataclasses import dataclass

        from transformers.modeling_outputs import CausalLMOutputWithPast

        @dataclass
        class CausalLMOutputWithSampleSums(CausalLMOutputWithPast):
            """seg_loss fp32 [S]: per-sample sum of the per-token loss over
            cu_seqlens; seg_cnt int32 [S]: its counted (non-ignored) tokens."""
            seg_loss: Optional[torch.FloatTensor] = None
            seg_cnt: Optional[torch.IntTensor] = None

        _OUTPUT_CLS = CausalLMOutputWithSampleSums
    return _OUTPUT_CLS


def patch_causal_lm(model: torch.nn.Module,
                    dw_accumulator: Optional[torch.Tensor] = None) -> torch.nn.Module:
    """Give a transformers *ForCausalLM model a forward that, when labels (or
    shift_labels) are passed, runs the decoder, hands its last hidden states
    and the output-embedding weight to causal_lm_loss and returns a
    CausalLMOutputWithPast (loss = per-token loss, logits = None).  Without
    labels the model's own forward runs unchanged.

    Extra keywords of the patched forward: `mt_grad_scale` (the upstream gradient
    of the per-token loss, known before the forward in train.py:97-104:
    world_size / batch_num_loss_counted_tokens) promises the gradient to the
    fused path; `cu_seqlens` (int32 [S + 1], the packed minibatch's sample
    boundaries, e.g. from cu_seqlens_from_minibatch in the collator) adds
    `seg_loss` / `seg_cnt`, the per-sample loss sums and counted tokens of
    the shifted targets, to the output without a host sync (a malformed
    cu_seqlens gives zeros there); `num_items_in_batch` is accepted and
    ignored, as by the reference's loss (none_reduction_losses.py:9).  With
    dw_accumulator (fp32 [V, H]) the lm_head gradient is added there in fp32
    instead of reaching autograd.
    """
    decoder = model.get_decoder()
    head = model.get_output_embeddings()
    if head is None or getattr(head, "bias", None) is not None:
        raise ValueError("patch_causal_lm needs an output embedding without bias")
    original = model.forward
    softcap = getattr(model.config, "final_logit_softcapping", None)

    def forward(input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                inputs_embeds=None, labels=None, use_cache=None, logits_to_keep=0,
                shift_labels=None, mt_grad_scale=None, cu_seqlens=None,
                ignore_index: int = -100, **kwargs):
        kwargs.pop("num_items_in_batch", None)
        if labels is None and shift_labels is None:
            return original(input_ids=input_ids, attention_mask=attention_mask,
                            position_ids=position_ids, past_key_values=past_key_values,
                            inputs_embeds=inputs_embeds, use_cache=use_cache,
                            logits_to_keep=logits_to_keep, **kwargs)
        out = decoder(input_ids=input_ids, attention_mask=attention_mask,
                      position_ids=position_ids, past_key_values=past_key_values,
                      inputs_embeds=inputs_embeds, use_cache=use_cache, **kwargs)
        hidden = out.last_hidden_state
        if hidden.dtype != head.weight.dtype:
            # a decoder kept in another precision than its output embedding:
            # the head sees its own dtype, as F.linear under autocast would
            hidden = hidden.to(head.weight.dtype)
        loss = causal_lm_loss(hidden, head.weight, labels=labels,
                              shift_labels=shift_labels, ignore_index=ignore_index,
                              final_logit_softcapping=softcap, grad_scale=mt_grad_scale,
                              dw_accumulator=dw_accumulator)
        seg_loss = seg_cnt = None
        if cu_seqlens is not None:
            seg_loss, seg_cnt = sample_loss_sums(loss, cu_seqlens, labels=labels,
                                                 shift_labels=shift_labels,
                                                 ignore_index=ignore_index)
        return _output_cls()(loss=loss, logits=None, past_key_values=out.past_key_values,
                             hidden_states=out.hidden_states, attentions=out.attentions,
                             seg_loss=seg_loss, seg_cnt=seg_cnt)

    model.forward = forward
    return model


def sample_loss_sums(loss: torch.Tensor, cu_seqlens: torch.Tensor,
                     labels: Optional[torch.Tensor] = None,
                     shift_labels: Optional[torch.Tensor] = None, ignore_index: int = -100):
    """Per-sample (loss sum fp32 [S], counted tokens int32 [S]) of a per-token
    loss produced by causal_lm_loss with the same labels / shift_labels:
    counted tokens are those whose shifted target is not ignore_index.  No
    host sync (cu_seqlens is moved to the loss's device if needed)."""
    cu = cu_seqlens.to(device=loss.device, dtype=torch.int32, non_blocking=True)
    if shift_labels is not None:
        tgt, shift = shift_labels.reshape(-1), False
    elif labels is None:
        raise ValueError("sample_loss_sums needs labels or shift_labels")
    elif labels.dim() >= 2 and labels.shape[0] > 1:
        tgt, shift = F.pad(labels, (0, 1), value=ignore_index)[..., 1:].reshape(-1), False
    else:
        tgt, shift = labels.reshape(-1), True
    return per_sample_loss_sums(loss.detach(), tgt, cu, ignore_index=ignore_index,
                                validate=False, shift=shift)


def cu_seqlens_from_minibatch(minibatch: Sequence[dict]) -> torch.Tensor:
    """int32 cu_seqlens [S + 1] of the packed row a collator builds from
    `minibatch`, the list of sample dicts it concatenates (sampler.py:144-208:
    input_ids of every sample, dummy padding samples included, one after the
    other).  Built on the host from the sample lengths, in the collator's
    worker process, so it costs the training step no device sync; a dummy
    sample (all labels ignore_index, not counted by sampler.py:193-194) gets
    its own segment, whose loss sum and count come out 0 and 0."""
    return cu_seqlens_from_lengths([len(item["input_ids"]) for item in minibatch])


def cu_seqlens_from_position_ids(position_ids: torch.Tensor) -> torch.Tensor:
    """int32 cu_seqlens [S + 1] of a packed row whose position_ids restart at 0
    at every sample start (the layout of sampler.py:182-188; transformers
    derives the same boundaries in TF/modeling_flash_attention_utils.py:458-481).
    Runs where position_ids lives (one host sync for the sample count)."""
    pos = position_ids.reshape(-1)
    T = pos.numel()
    if T == 0:
        return torch.zeros(1, dtype=torch.int32, device=pos.device)
    starts = torch.nonzero(pos == 0).flatten()
    if starts.numel() == 0 or int(starts[0]) != 0:
        starts = torch.cat([torch.zeros(1, dtype=starts.dtype, device=pos.device), starts])
    end = torch.full((1,), T, dtype=starts.dtype, device=pos.device)
    return torch.cat([starts, end]).to(torch.int32)


def cu_seqlens_from_lengths(lengths) -> torch.Tensor:
    """int32 cu_seqlens [S + 1] from the sample lengths a collator packs."""
    L = torch.as_tensor(lengths, dtype=torch.int64).reshape(-1)
    return torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(L, 0)]).to(torch.int32)
