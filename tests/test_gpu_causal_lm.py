"""The model-side caller on a transformers LlamaForCausalLM (bf16, on the
GPU): the patched forward returns per-token losses from the last hidden
states without logits, and its gradients reach the model's parameters.

The reference side is the torch path on the CPU over the same hidden states
(F.linear in bf16 -> .float() -> F.cross_entropy(reduction='none'), labels
shifted as transformers' ForCausalLMLoss does, TF/loss/loss_utils.py:61-64),
with the north-star tolerances.  The decoder has no attention layers (an
embedding and the final RMSNorm), which keeps the check on the loss path and
keeps batched bf16 products out of the test.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from mini_trainer_amd import cu_seqlens_from_position_ids, patch_causal_lm, per_sample_loss_sums
from oracle.torch_path import rel_fro, torch_path

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def tiny_llama(vocab=1500, hidden=128, seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=256,
                      num_hidden_layers=0, num_attention_heads=4, num_key_value_heads=4,
                      max_position_embeddings=4096, tie_word_embeddings=False)
    m = LlamaForCausalLM(cfg)
    with torch.no_grad():
        m.lm_head.weight.normal_(0, 0.05)
    return m.to(torch.bfloat16)


def packed_batch(lengths, vocab, seed=1, prompt_frac=0.4):
    g = torch.Generator().manual_seed(seed)
    ids, labels, pos = [], [], []
    for L in lengths:
        x = torch.randint(0, vocab, (L,), generator=g)
        y = x.clone()
        y[: int(L * prompt_frac)] = -100  # masked prompt (process_data.py:43-65)
        ids.append(x), labels.append(y), pos.append(torch.arange(L))
    return torch.cat(ids)[None], torch.cat(labels)[None], torch.cat(pos)[None]


def reference(model_cpu, input_ids, labels, grad_scale):
    """Per-token loss and lm_head / embedding grads of the unpatched model on the CPU."""
    model_cpu.zero_grad(set_to_none=True)
    hidden = model_cpu.model(input_ids=input_ids).last_hidden_state
    shifted = F.pad(labels, (0, 1), value=-100)[..., 1:].reshape(-1)
    logits = F.linear(hidden.reshape(-1, hidden.shape[-1]), model_cpu.lm_head.weight).float()
    loss = F.cross_entropy(logits, shifted, ignore_index=-100, reduction="none")
    (loss.sum() * grad_scale).backward()
    return (loss.detach(), model_cpu.lm_head.weight.grad.float(),
            model_cpu.model.embed_tokens.weight.grad.float(), hidden.detach(), shifted)


@pytest.mark.parametrize("fused", [False, True])
def test_patched_llama_matches_reference(gpu, fused):
    import copy

    model = tiny_llama()
    ref_model = copy.deepcopy(model)  # CPU, bf16, unpatched
    lengths = [37, 120, 5, 64, 90]
    ids, labels, pos = packed_batch(lengths, 1500)
    n = int((F.pad(labels, (0, 1), value=-100)[..., 1:] != -100).sum())
    scale = 1.0 / n
    rl, rdW, rdE, hidden, shifted = reference(ref_model, ids, labels, scale)

    model = patch_causal_lm(model.to(gpu))
    out = model(input_ids=ids.to(gpu), labels=labels.to(gpu), position_ids=pos.to(gpu),
                mt_grad_scale=scale if fused else None, num_items_in_batch=n)
    assert out.logits is None
    loss = out.loss
    assert loss.shape == (ids.numel(),) and loss.dtype == torch.float32
    (loss.float().sum() * scale).backward()  # the train.py:97-104 chain
    torch.cuda.synchronize()

    valid = shifted != -100
    l = loss.detach().cpu()
    assert torch.equal(l[~valid], torch.zeros(int((~valid).sum())))
    err = ((l[valid] - rl[valid]).abs() / rl[valid].abs()).max().item()
    assert err <= 2e-3, f"loss rel err {err:.3e}"
    # the oracle restated over the same hidden states
    ol, _, _ = torch_path(hidden.reshape(-1, hidden.shape[-1]), ref_model.lm_head.weight.detach(),
                          shifted, need_grads=False)
    assert ((l[valid] - ol[valid]).abs() / ol[valid].abs()).max().item() <= 2e-3
    assert rel_fro(model.lm_head.weight.grad.float().cpu(), rdW) <= 1e-2
    assert rel_fro(model.model.embed_tokens.weight.grad.float().cpu(), rdE) <= 1e-2

    # per-sample metrics over the same packed row
    cu = cu_seqlens_from_position_ids(pos).to(gpu)
    seg_loss, seg_cnt = per_sample_loss_sums(loss.detach(), shifted.to(gpu), cu)
    assert int(seg_cnt.sum()) == n
    assert abs(seg_loss.sum().item() - l.double().sum().item()) <= 1e-4 * l.double().sum().item()


def test_batch_rows_shift_per_row(gpu):
    # two rows: each row's last position is ignored, no row takes the next row's label
    model = patch_causal_lm(tiny_llama(seed=3).to(gpu))
    ids = torch.randint(0, 1500, (2, 40), generator=torch.Generator().manual_seed(4))
    labels = ids.clone()
    out = model(input_ids=ids.to(gpu), labels=labels.to(gpu))
    loss = out.loss.detach().cpu().view(2, 40)
    assert loss[0, -1].item() == 0.0 and loss[1, -1].item() == 0.0
    assert bool((loss[:, :-1] > 0).all())
    # shift_labels passes through unchanged
    sl = torch.full((2, 40), -100)
    sl[:, 3] = 7
    out2 = model(input_ids=ids.to(gpu), shift_labels=sl.to(gpu))
    l2 = out2.loss.detach().cpu().view(2, 40)
    assert torch.count_nonzero(l2[:, [i for i in range(40) if i != 3]]) == 0
    assert bool((l2[:, 3] > 0).all())


def one_layer_llama(vocab=1500, hidden=128, seed=0):
    """A Llama with one real decoder layer (attention + MLP) kept in fp32 and
    a bf16 lm_head: attention's batched products stay in fp32."""
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=256,
                      num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2,
                      max_position_embeddings=4096, tie_word_embeddings=False,
                      attn_implementation="eager")
    m = LlamaForCausalLM(cfg).float()
    with torch.no_grad():
        m.lm_head.weight.normal_(0, 0.05)
    m.lm_head.to(torch.bfloat16)
    return m


@pytest.mark.parametrize("world_size", [1, 3])
def test_decoder_layer_train_py_chain_with_sample_sums(gpu, world_size, monkeypatch):
    """A packed minibatch with a dummy sample (all labels ignored, as the
    collator pads with, sampler.py:193-194) through a model with a real
    decoder layer, driven as train.py:97-104 drives it (no grad_scale): the
    fused kernels run (path fused_unit), the loss, the lm_head gradient and a
    decoder weight's gradient match the unpatched model on the CPU, and the
    per-sample sums over the collator's cu_seqlens match the C restatement,
    with exactly 0 / 0 for the dummy sample."""
    import copy

    import numpy as np

    from mini_trainer_amd import cu_seqlens_from_minibatch, path_of
    from mini_trainer_amd.flce import FUSED_ENV
    from oracle import ref

    monkeypatch.setenv(FUSED_ENV, "1")
    model = one_layer_llama()
    ref_model = copy.deepcopy(model)
    lengths = [37, 120, 5, 64, 90]
    ids, labels, pos = packed_batch(lengths, 1500)
    labels[0, 157:162] = -100  # the 5-token dummy sample
    minibatch = [{"input_ids": ids[0, a:a + L].tolist()}
                 for a, L in zip(np.cumsum([0] + lengths[:-1]), lengths)]
    cu = cu_seqlens_from_minibatch(minibatch)
    assert cu.tolist() == [0, 37, 157, 162, 226, 316]

    shifted = F.pad(labels, (0, 1), value=-100)[..., 1:].reshape(-1)
    n = int((shifted != -100).sum())
    # unpatched model on the CPU: hidden (fp32) -> bf16 -> F.linear -> .float() -> CE
    hidden = ref_model.model(input_ids=ids, position_ids=pos).last_hidden_state
    logits = F.linear(hidden.reshape(-1, 128).to(torch.bfloat16), ref_model.lm_head.weight).float()
    rl = F.cross_entropy(logits, shifted, ignore_index=-100, reduction="none")
    (rl.sum() * world_size / n).backward()

    model = patch_causal_lm(model.to(gpu))
    out = model(input_ids=ids.to(gpu), labels=labels.to(gpu), position_ids=pos.to(gpu),
                cu_seqlens=cu)
    assert path_of(out.loss) == "fused_unit"
    loss = out.loss.float().sum()
    loss.detach().item()
    (loss * world_size / n).backward()
    torch.cuda.synchronize()

    valid = shifted != -100
    l = out.loss.detach().cpu()
    r = rl.detach()
    assert torch.equal(l[~valid], torch.zeros(int((~valid).sum())))
    assert ((l[valid] - r[valid]).abs() / r[valid].abs()).max().item() <= 2e-3
    assert rel_fro(model.lm_head.weight.grad.float().cpu(),
                   ref_model.lm_head.weight.grad.float()) <= 1e-2
    q_gpu = model.model.layers[0].self_attn.q_proj.weight.grad.cpu()
    q_ref = ref_model.model.layers[0].self_attn.q_proj.weight.grad
    assert rel_fro(q_gpu, q_ref) <= 1e-2

    want_l, want_c, st = ref.segment_sum(l.numpy(), shifted.numpy(), cu.numpy())
    assert st == 0
    seg_l, seg_c = out.seg_loss.cpu().numpy(), out.seg_cnt.cpu().numpy()
    assert np.array_equal(seg_c, want_c)
    assert np.allclose(seg_l, want_l, rtol=1e-6, atol=0)
    assert seg_c[2] == 0 and seg_l[2] == 0.0  # the dummy sample
    assert int(seg_c.sum()) == n
