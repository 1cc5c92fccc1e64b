"""The drop-in boundary on the CPU: same signatures as the reference's loss
functions (none_reduction_losses.py:5-13, :27-33), the reference's plugin
mechanism (utils.py:36-46), and no silent CPU fallback."""
from __future__ import annotations

import inspect
import sys
import types

import pytest
import torch

import mini_trainer_amd as mt
from mini_trainer_amd import none_reduction_losses as nrl
from mini_trainer_amd.utils import patch_target_module

# (name, kind, default) of each parameter, as written in the reference
REF_LIGER = [
    ("hidden_states", "POSITIONAL_OR_KEYWORD", inspect._empty),
    ("lm_head_weight", "POSITIONAL_OR_KEYWORD", inspect._empty),
    ("target", "POSITIONAL_OR_KEYWORD", inspect._empty),
    ("num_items_in_batch", "POSITIONAL_OR_KEYWORD", None),
    ("ignore_index", "POSITIONAL_OR_KEYWORD", -100),
    ("final_logit_softcapping", "POSITIONAL_OR_KEYWORD", None),
    ("kwargs", "VAR_KEYWORD", inspect._empty),
]
REF_HF = [
    ("source", "POSITIONAL_OR_KEYWORD", inspect._empty),
    ("target", "POSITIONAL_OR_KEYWORD", inspect._empty),
    ("num_items_in_batch", "POSITIONAL_OR_KEYWORD", None),
    ("ignore_index", "POSITIONAL_OR_KEYWORD", -100),
    ("kwargs", "VAR_KEYWORD", inspect._empty),
]


def params(fn):
    return [(p.name, p.kind.name, p.default) for p in inspect.signature(fn).parameters.values()]


def test_signatures_match_reference():
    assert params(nrl.liger_fixed_fused_linear_cross_entropy_none_reduction) == REF_LIGER
    assert params(nrl.hf_fixed_cross_entropy_none_reduction) == REF_HF
    assert mt.liger_fixed_fused_linear_cross_entropy_none_reduction is \
        nrl.liger_fixed_fused_linear_cross_entropy_none_reduction


def test_patch_target_module_semantics(monkeypatch):
    mod = types.ModuleType("mt_fake_loss_utils")
    mod.fixed_cross_entropy = lambda *a, **k: "original"
    monkeypatch.setitem(sys.modules, "mt_fake_loss_utils", mod)
    patch_target_module("mt_fake_loss_utils.fixed_cross_entropy", nrl.hf_fixed_cross_entropy_none_reduction)
    assert mod.fixed_cross_entropy is nrl.hf_fixed_cross_entropy_none_reduction
    with pytest.raises(AssertionError, match="must have an object to patch"):
        patch_target_module("nodots", None)
    with pytest.raises(ModuleNotFoundError):
        patch_target_module("mt_no_such_module.x", None)


def test_cpu_tensors_fail_loudly():
    X = torch.randn(4, 64, dtype=torch.bfloat16)
    W = torch.randn(10, 64, dtype=torch.bfloat16)
    y = torch.tensor([1, 2, -100, 3])
    with pytest.raises(RuntimeError, match="ROCm device"):
        nrl.liger_fixed_fused_linear_cross_entropy_none_reduction(X, W, y)
    with pytest.raises(RuntimeError, match="ROCm device"):
        nrl.hf_fixed_cross_entropy_none_reduction(torch.randn(4, 10), y)


def test_hf_loss_dispatch_reaches_the_patched_function(monkeypatch):
    """transformers' ForCausalLMLoss resolves fixed_cross_entropy from module
    globals at call time (TF/loss/loss_utils.py:70), so the patch installed by
    patch_target_module (setup_model_for_training.py:100-103) is what runs."""
    lu = pytest.importorskip("transformers.loss.loss_utils")
    seen = {}

    def spy(source, target, num_items_in_batch=None, ignore_index=-100, **kwargs):
        seen["args"] = (tuple(source.shape), tuple(target.shape), ignore_index)
        return nrl.hf_fixed_cross_entropy_none_reduction(source, target, num_items_in_batch,
                                                         ignore_index, **kwargs)

    monkeypatch.setattr(lu, "fixed_cross_entropy", lu.fixed_cross_entropy)
    patch_target_module("transformers.loss.loss_utils.fixed_cross_entropy", spy)
    logits = torch.randn(1, 6, 11)
    labels = torch.tensor([[1, 2, -100, 4, 5, 6]])
    with pytest.raises(RuntimeError, match="ROCm device"):
        lu.ForCausalLMLoss(logits, labels, vocab_size=11)
    assert seen["args"] == ((6, 11), (6,), -100)


def test_drop_in_reads_only_its_own_keyword(monkeypatch):
    """Of **kwargs the drop-in reads `mt_grad_scale` alone: an unrelated
    `grad_scale` a caller passes through the loss kwargs selects nothing."""
    seen = []

    def spy(hidden, weight, target, ignore_index=-100, softcap=None, grad_scale=None, **kw):
        seen.append((ignore_index, softcap, grad_scale))
        return "out"

    monkeypatch.setattr(nrl, "fused_linear_cross_entropy", spy)
    X, W, y = torch.zeros(2, 8), torch.zeros(3, 8), torch.zeros(2, dtype=torch.long)
    nrl.liger_fixed_fused_linear_cross_entropy_none_reduction(X, W, y, 7, -5, 30.0,
                                                               grad_scale=0.5)
    nrl.liger_fixed_fused_linear_cross_entropy_none_reduction(X, W, y, mt_grad_scale=0.25)
    assert seen == [(-5, 30.0, None), (-100, None, 0.25)]
    assert nrl.GRAD_SCALE_KWARG == "mt_grad_scale"
