"""Pins of the oracle itself (CPU only): the torch path and the C restatement
are checked against float64 closed forms, textbook special cases and
invariants chosen so that a dropped term, a wrong sign, a transposed operand
or a wrong index fails at least one check (see test_planted_mistakes_are_caught)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import brute, ref
from oracle.torch_path import rel_fro, torch_path


def case(T=40, H=24, V=97, seed=0, mask=0.25, w_std=0.3, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(T, H, generator=g).to(dtype)
    W = (torch.randn(V, H, generator=g) * w_std).to(dtype)
    y = torch.randint(0, V, (T,), generator=g)
    y[torch.rand(T, generator=g) < mask] = -100
    return X, W, y


def test_torch_path_matches_float64_closed_form():
    X, W, y = case()
    grad = torch.rand(40, generator=torch.Generator().manual_seed(1)) + 0.5
    l, dX, dW = torch_path(X, W, y, grad=grad)
    bl, bdX, bdW, _ = brute.flce_f64(X.numpy(), W.numpy(), y.numpy(), grad.numpy())
    np.testing.assert_allclose(l.numpy(), bl, rtol=1e-6, atol=1e-6)
    assert rel_fro(dX, torch.from_numpy(bdX)) < 1e-6
    assert rel_fro(dW, torch.from_numpy(bdW)) < 1e-6


def test_torch_path_softcap_matches_closed_form():
    X, W, y = case(seed=3, w_std=1.0)
    l, dX, dW = torch_path(X, W, y, softcap=2.5)
    bl, bdX, bdW, _ = brute.flce_f64(X.numpy(), W.numpy(), y.numpy(), softcap=2.5)
    np.testing.assert_allclose(l.numpy(), bl, rtol=1e-6, atol=1e-6)
    assert rel_fro(dX, torch.from_numpy(bdX)) < 1e-6
    assert rel_fro(dW, torch.from_numpy(bdW)) < 1e-6


def test_c_restatement_matches_float64_closed_form():
    X, W, y = case(seed=4)
    grad = np.linspace(0.2, 1.7, 40).astype(np.float32)
    loss, dX, dW = ref.backward(X.numpy(), W.numpy(), y.numpy(), grad, round_bf16=False)
    bl, bdX, bdW, _ = brute.flce_f64(X.numpy(), W.numpy(), y.numpy(), grad)
    np.testing.assert_allclose(loss, bl, rtol=1e-6, atol=1e-6)
    assert rel_fro(torch.from_numpy(dX), torch.from_numpy(bdX)) < 1e-6
    assert rel_fro(torch.from_numpy(dW), torch.from_numpy(bdW)) < 1e-6
    loss_c, _, _ = ref.backward(X.numpy(), W.numpy(), y.numpy(), 1.0, False, softcap=2.0)
    bl_c, _, _, _ = brute.flce_f64(X.numpy(), W.numpy(), y.numpy(), softcap=2.0)
    np.testing.assert_allclose(loss_c, bl_c, rtol=1e-6, atol=1e-6)


def test_c_restatement_bf16_matches_torch_path_bf16():
    # bf16 inputs: both round the logits and the logit gradient to bf16
    X, W, y = case(T=64, H=64, V=300, seed=6, w_std=0.05, dtype=torch.bfloat16)
    l, dX, dW = torch_path(X, W, y)
    cl, cdX, cdW = ref.backward(X.float().numpy(), W.float().numpy(), y.numpy(), 1.0,
                                round_bf16=True)
    v = (y != -100).numpy()
    assert np.max(np.abs(cl[v] - l.numpy()[v]) / np.abs(l.numpy()[v])) < 2e-3
    assert rel_fro(torch.from_numpy(cdX), dX.float()) < 1e-2
    assert rel_fro(torch.from_numpy(cdW), dW) < 1e-2


def test_zero_weight_gives_log_vocab():
    X, W, y = case(seed=7)
    W.zero_()
    l, dX, dW = torch_path(X, W, y)
    v = y != -100
    np.testing.assert_allclose(l[v].numpy(), math.log(97), rtol=1e-6)
    assert torch.count_nonzero(dX) == 0
    cl, cdX, _ = ref.backward(X.numpy(), W.numpy(), y.numpy(), 1.0, False)
    np.testing.assert_allclose(cl[v.numpy()], math.log(97), rtol=1e-7)
    assert not cdX.any()


def test_two_class_softplus_closed_form():
    # V = 2: loss = softplus(s_other - s_y)
    X = torch.tensor([[1.5], [-0.25], [3.0]])
    W = torch.tensor([[0.5], [-1.0]])
    y = torch.tensor([0, 1, 1])
    l, _, _ = torch_path(X, W, y)
    s = (X @ W.T).double()
    exp = [math.log1p(math.exp(float(s[i, 1 - y[i]] - s[i, y[i]]))) for i in range(3)]
    np.testing.assert_allclose(l.double().numpy(), exp, rtol=1e-6)


def test_dominant_label_gives_zero_loss():
    X = torch.tensor([[1.0, 0.0]])
    W = torch.tensor([[200.0, 0.0], [0.0, 1.0], [-3.0, 0.0]])
    l, _, _ = torch_path(X, W, torch.tensor([0]))
    assert float(l[0]) < 1e-30 + 1e-6


def test_weight_gradient_rows_sum_to_zero():
    # sum_v G[t, v] = 0 for every valid row, hence sum_v dW[v, :] = 0
    X, W, y = case(seed=8)
    _, _, dW = torch_path(X, W, y)
    assert dW.sum(0).abs().max() < 1e-5 * dW.abs().max()
    _, _, cdW = ref.backward(X.numpy(), W.numpy(), y.numpy(), 1.0, False)
    assert np.abs(cdW.sum(0)).max() < 1e-6 * np.abs(cdW).max()


def test_all_masked_gives_zeros():
    X, W, y = case(seed=9)
    y[:] = -100
    l, dX, dW = torch_path(X, W, y)
    assert torch.count_nonzero(l) == 0 and torch.count_nonzero(dX) == 0
    assert torch.count_nonzero(dW) == 0
    cl, cdX, cdW = ref.backward(X.numpy(), W.numpy(), y.numpy(), 1.0, False)
    assert not cl.any() and not cdX.any() and not cdW.any()


def test_row_permutation_and_chunking_invariance():
    X, W, y = case(T=50, seed=10)
    l, dX, dW = torch_path(X, W, y, chunk_rows=1024)
    perm = torch.randperm(50, generator=torch.Generator().manual_seed(2))
    lp, dXp, dWp = torch_path(X[perm], W, y[perm], chunk_rows=7)
    torch.testing.assert_close(lp, l[perm], rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(dXp, dX[perm], rtol=1e-5, atol=1e-6)
    assert rel_fro(dWp, dW) < 1e-6
    l1, _, _ = torch_path(X, W, y, chunk_rows=1)
    torch.testing.assert_close(l1, l, rtol=1e-6, atol=1e-6)


def test_upstream_grad_is_linear():
    X, W, y = case(seed=11)
    g = torch.rand(40, generator=torch.Generator().manual_seed(4))
    _, dX1, dW1 = torch_path(X, W, y, grad=g)
    _, dX2, dW2 = torch_path(X, W, y, grad=3.0 * g)
    assert rel_fro(dX2, 3.0 * dX1) < 1e-6 and rel_fro(dW2, 3.0 * dW1) < 1e-6


def test_prepare_restatement_against_numpy():
    rng = np.random.default_rng(0)
    for T in (0, 1, 5, 1000):
        lab = rng.integers(-3, 60, T)
        lab[rng.random(T) < 0.3] = -100
        for shift in (False, True):
            tgt = np.concatenate([lab[1:], [-100]]) if (shift and T) else lab
            ri, rl, counts = ref.prepare(lab, 50, -100, shift)
            valid = (tgt != -100) & (tgt >= 0) & (tgt < 50)
            idx = np.nonzero(valid)[0]
            assert counts[0] == idx.size
            assert np.array_equal(ri[:idx.size], idx)
            assert np.array_equal(rl[:idx.size], tgt[idx])
            assert np.array_equal(np.sort(ri[idx.size:]), np.nonzero(~valid)[0])
            bad = (tgt != -100) & ~valid
            assert counts[1] == bad.sum()
            assert counts[2] == (np.nonzero(bad)[0][0] if bad.any() else -1)


def test_segment_sum_restatement():
    rng = np.random.default_rng(1)
    L = rng.integers(0, 20, 30)
    cu = np.concatenate([[0], np.cumsum(L)]).astype(np.int32)
    T = int(cu[-1])
    loss = rng.random(T).astype(np.float32)
    tgt = rng.integers(0, 5, T)
    tgt[rng.random(T) < 0.5] = -100
    sl, sc, st = ref.segment_sum(loss, tgt, cu)
    assert st == 0
    c = np.concatenate([[0.0], np.cumsum(loss.astype(np.float64))])
    np.testing.assert_allclose(sl, c[cu[1:]] - c[cu[:-1]], rtol=1e-6, atol=1e-6)
    assert np.array_equal(sc, np.add.reduceat(np.append(tgt != -100, 0), cu[:-1])[:30] * (L > 0))
    assert abs(sl.sum() - loss.sum()) < 1e-3
    bad = cu.copy()
    bad[-1] += 1
    assert ref.segment_sum(loss, tgt, bad)[2] == 1


def test_ce_restatement_matches_torch():
    g = torch.Generator().manual_seed(12)
    logits = torch.randn(30, 50, generator=g) * 4
    y = torch.randint(0, 50, (30,), generator=g)
    y[::4] = -100
    l, lse, st = ref.ce_forward(logits.numpy(), y.numpy())
    ref_l = torch.nn.functional.cross_entropy(logits, y, reduction="none")
    np.testing.assert_allclose(l, ref_l.numpy(), rtol=1e-6, atol=1e-6)
    y[3] = 50
    assert ref.ce_forward(logits.numpy(), y.numpy())[2] == 1


def test_round_bf16_matches_torch():
    x = torch.randn(10000, generator=torch.Generator().manual_seed(0)) * 100
    a = ref.round_bf16(x.numpy())
    b = x.to(torch.bfloat16).float().numpy()
    assert np.array_equal(a, b)
    assert all(ref.lib().ref_round_bf16(float(v)) == float(w) for v, w in zip(x[:50], b[:50]))


@pytest.mark.parametrize("mistake", ["drop_label_term", "flip_grad_sign", "transpose_dw",
                                     "label_off_by_one", "no_bf16_rounding"])
def test_planted_mistakes_are_caught(mistake):
    """Each plausible slip in an oracle restatement fails the checks used above."""
    X, W, y = case(seed=13, T=32, H=16, V=16, mask=0.2, w_std=1.0)
    l, dX, dW = torch_path(X, W, y)
    bl, bdX, bdW, _ = brute.flce_f64(X.numpy(), W.numpy(), y.numpy())
    if mistake == "drop_label_term":
        _, _, _, lse = brute.flce_f64(X.numpy(), W.numpy(), y.numpy())
        bad = np.where(y.numpy() != -100, lse, 0.0)
        assert not np.allclose(bad, l.numpy(), rtol=1e-3)
    elif mistake == "flip_grad_sign":
        assert rel_fro(-dX, torch.from_numpy(bdX)) > 1e-2
    elif mistake == "transpose_dw":
        assert rel_fro(dW.t().contiguous(), torch.from_numpy(bdW)) > 1e-2
    elif mistake == "label_off_by_one":
        y2 = torch.where(y == -100, y, (y + 1) % 16)
        l2, _, _ = torch_path(X, W, y2)
        assert not np.allclose(l2.numpy(), bl, rtol=1e-3)
    elif mistake == "no_bf16_rounding":
        Xb, Wb = X.to(torch.bfloat16), (W * 4).to(torch.bfloat16)
        lb, _, _ = torch_path(Xb, Wb, y)
        cl, _, _ = ref.backward(Xb.float().numpy(), Wb.float().numpy(), y.numpy(), 1.0,
                                round_bf16=False)
        v = (y != -100).numpy()
        # unrounded logits differ from the bf16 torch path by more than rounding noise of fp32
        assert np.max(np.abs(cl[v] - lb.numpy()[v])) > 1e-4


def _bf16_case(seed, T=96, H=200, V=700, w_std=0.2, mask=0.3):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(T, H, generator=g).to(torch.bfloat16)
    W = (torch.randn(V, H, generator=g) * w_std).to(torch.bfloat16)
    y = torch.randint(0, V, (T,), generator=g)
    y[torch.rand(T, generator=g) < mask] = -100
    grad = torch.rand(T, generator=g) + 0.25
    return X, W, y, grad


@pytest.mark.parametrize("softcap", [None, 15.0])
@pytest.mark.parametrize("seed", [0, 1])
def test_upcast_branch_pinned(softcap, seed):
    """torch_path(upcast=True) -- the full-size GPU checker -- against the
    default branch (F.linear in bf16, pinned through the C restatement) and
    against the float64 closed form, bf16 inputs, softcap and a per-token
    upstream gradient.  The logits of both branches are the bf16 rounding of
    the same fp32 products, so the losses agree to fp32 noise; the closed
    form does not round the logits, hence its looser bound."""
    X, W, y, grad = _bf16_case(seed)
    v = y != -100
    l0, dX0, dW0 = torch_path(X, W, y, grad=grad, softcap=softcap, chunk_rows=40)
    l1, dX1, dW1 = torch_path(X, W, y, grad=grad, softcap=softcap, chunk_rows=40, upcast=True)
    assert dX1.dtype == torch.bfloat16 and dW1.dtype == torch.float32
    assert torch.equal(l1[~v], torch.zeros(int((~v).sum())))
    assert ((l1 - l0).abs() / l0.abs())[v].max().item() <= 1e-5
    assert rel_fro(dX1.float(), dX0.float()) <= 1e-3
    assert rel_fro(dW1, dW0) <= 1e-5
    bl, bdX, bdW, _ = brute.flce_f64(X.float().numpy(), W.float().numpy(), y.numpy(),
                                     grad.numpy(), softcap=softcap)
    vn = v.numpy()
    assert np.max(np.abs(l1.numpy()[vn] - bl[vn]) / np.abs(bl[vn])) < 1e-2
    assert rel_fro(dX1.float(), torch.from_numpy(bdX)) < 1e-2
    assert rel_fro(dW1, torch.from_numpy(bdW)) < 1e-2


def test_upcast_branch_planted_missing_rounding_is_caught():
    """The upcast branch with its `.to(X.dtype)` rounding of the logits
    dropped -- planted here by handing it fp32 copies of the bf16 inputs,
    which skips exactly that rounding -- fails the default-branch bound of
    test_upcast_branch_pinned."""
    X, W, y, grad = _bf16_case(0)
    v = y != -100
    l0, _, _ = torch_path(X, W, y, grad=grad, chunk_rows=40)
    bad, _, _ = torch_path(X.float(), W.float(), y, grad=grad, chunk_rows=40, upcast=True)
    assert ((bad - l0).abs() / l0.abs())[v].max().item() > 1e-5
