"""Parity of the HIP path (through the C ABI via the PyTorch host layer)
against the oracle: the reference's torch path (oracle/torch_path.py) and the
C restatement (oracle/ref.py).

Tolerances (north star): per-token loss 2e-3 relative in bf16 and 1e-5 in
fp32; dX and dW 1e-2 relative Frobenius error; ignored positions exactly
+0.0 (loss) and 0 (dX rows).  Integer outputs (row compaction, counts) are
compared bit-exactly.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from mini_trainer_amd import (cross_entropy_none, fused_linear_cross_entropy,
                              per_sample_loss_sums, prepare_targets)
from mini_trainer_amd.flce import BACKWARD_BUDGET_ENV
from oracle import ref
from oracle.torch_path import rel_fro, torch_path

pytestmark = pytest.mark.gpu

LOSS_RTOL = {torch.bfloat16: 2e-3, torch.float32: 1e-5}
GRAD_RFRO = 1e-2


def make_case(T, H, V, dtype, mask_frac=0.3, seed=0, w_std=0.02, label_hi=None):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(T, H, generator=g).to(dtype)
    W = (torch.randn(V, H, generator=g) * w_std).to(dtype)
    y = torch.randint(0, label_hi or V, (T,), generator=g)
    y[torch.rand(T, generator=g) < mask_frac] = -100
    return X, W, y


def run_ours(dev, X, W, y, grad=None, softcap=None, shift=False):
    Xd = X.to(dev).requires_grad_(True)
    Wd = W.to(dev).requires_grad_(True)
    acc = torch.zeros(W.shape, dtype=torch.float32, device=dev)
    loss = fused_linear_cross_entropy(Xd, Wd, y.to(dev), softcap=softcap, shift_labels=shift,
                                      dw_accumulator=acc)
    gl = torch.ones_like(loss) if grad is None else grad.to(dev)
    loss.backward(gl)
    torch.cuda.synchronize()
    return loss.detach().cpu(), Xd.grad.detach().cpu(), acc.cpu()


def check_parity(X, W, y, loss, dX, dW, grad=None, softcap=None):
    rl, rdX, rdW = torch_path(X, W, y, grad=grad, softcap=softcap)
    valid = y != -100
    # ignored rows: exactly +0.0 loss (sign included) and zero dX rows
    assert torch.equal(loss[~valid], torch.zeros(int((~valid).sum())))
    assert not torch.signbit(loss[~valid]).any()
    assert torch.count_nonzero(dX[~valid]) == 0
    rtol = LOSS_RTOL[X.dtype]
    if valid.any():
        err = ((loss[valid] - rl[valid]).abs() / rl[valid].abs().clamp_min(1e-3)).max().item()
        assert err <= rtol, f"loss max rel err {err:.3e} > {rtol}"
    assert rel_fro(dX.float(), rdX.float()) <= GRAD_RFRO
    assert rel_fro(dW, rdW) <= GRAD_RFRO
    return rl, rdX, rdW


@pytest.mark.parametrize("T,H,V,dtype", [
    (300, 128, 1000, torch.bfloat16),       # V tail (1000 = 3*256 + 232), T tail
    (513, 192, 2065, torch.bfloat16),       # H not a multiple of 256
    (257, 64, 777, torch.float32),          # fp32 path
    (64, 896, 4096, torch.bfloat16),        # Qwen2.5-0.5B hidden size
    (200, 1536, 2304, torch.bfloat16),      # config 2's hidden size (6 H tiles)
    (160, 3584, 1100, torch.bfloat16),      # config 4's hidden size (14 H tiles), V tail
    (96, 8192, 800, torch.bfloat16),        # config 5's hidden size: 128-stage logits K loop
])
def test_parity_small(gpu, T, H, V, dtype):
    print(f"case T={T} H={H} V={V} {dtype}", flush=True)
    X, W, y = make_case(T, H, V, dtype, seed=T + H)
    loss, dX, dW = run_ours(gpu, X, W, y)
    check_parity(X, W, y, loss, dX, dW)


def test_parity_fp32_tight(gpu):
    # fp32 inputs against the float64 closed form through the C restatement
    X, W, y = make_case(200, 96, 1500, torch.float32, seed=5, w_std=0.05)
    loss, dX, dW = run_ours(gpu, X, W, y)
    rloss, rdX, rdW = ref.backward(X.numpy(), W.numpy(), y.numpy(), 1.0, round_bf16=False)
    v = (y != -100).numpy()
    err = np.abs(loss.numpy()[v] - rloss[v]) / np.abs(rloss[v])
    assert err.max() <= 1e-5
    assert rel_fro(dX, torch.from_numpy(rdX)) <= 1e-5
    assert rel_fro(dW, torch.from_numpy(rdW)) <= 1e-5


@pytest.mark.parametrize("V", [3000, 2560])  # vocabulary tail / whole 256-column tiles
def test_per_token_grad_and_softcap(gpu, V):
    X, W, y = make_case(400, 128, V, torch.bfloat16, seed=11, w_std=0.2)
    grad = torch.rand(400, generator=torch.Generator().manual_seed(3)) * 2 - 0.5
    loss, dX, dW = run_ours(gpu, X, W, y, grad=grad, softcap=3.0)
    check_parity(X, W, y, loss, dX, dW, grad=grad, softcap=3.0)


def test_scalar_broadcast_grad(gpu):
    # loss.sum() * c then backward(): the upstream grad is an expanded scalar
    X, W, y = make_case(256, 128, 1024, torch.bfloat16, seed=2)
    Xd, Wd = X.to(gpu).requires_grad_(True), W.to(gpu).requires_grad_(True)
    acc = torch.zeros(W.shape, dtype=torch.float32, device=gpu)
    loss = fused_linear_cross_entropy(Xd, Wd, y.to(gpu), dw_accumulator=acc)
    n = int((y != -100).sum())
    (loss.float().sum() * (1.0 / n)).backward()
    g = torch.full((256,), 1.0 / n)
    check_parity(X, W, y, loss.detach().cpu(), Xd.grad.cpu(), acc.cpu(), grad=g)


def test_multi_block_backward(gpu, monkeypatch):
    # tiny workspace budget -> 256-row x 256-vocab blocks: several token and
    # vocabulary chunks, every dX accumulation mode and dW accumulation
    monkeypatch.setenv(BACKWARD_BUDGET_ENV, "1")
    X, W, y = make_case(1100, 128, 1300, torch.bfloat16, seed=7, mask_frac=0.2)
    grad = torch.rand(1100, generator=torch.Generator().manual_seed(1))
    loss, dX, dW = run_ours(gpu, X, W, y, grad=grad)
    check_parity(X, W, y, loss, dX, dW, grad=grad)


def test_one_row_block_vocabulary_blocks_reference_chain(gpu, monkeypatch):
    """The general path without dw_accumulator under a budget that fits one
    row block and several vocabulary blocks (mt_flce_backward_narrow: dW
    written in bf16 by its GEMM, dX's fp32 accumulator in the dW buffer).
    Loss, dX and the bf16 weight gradient against the torch path."""
    from mini_trainer_amd.flce import FUSED_ENV, backward_plan

    T, H, V = 1100, 128, 13000
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=17, mask_frac=0.2)
    n = int((y != -100).sum())
    budget = 1024 * 4096 * 2 + H * 1024 * 2 + (1 << 16)
    C, Cv, _ = backward_plan(T, n, H, V, torch.bfloat16, budget_bytes=budget, narrow=True)
    assert n <= C and Cv < V, (n, C, Cv)
    monkeypatch.setenv(BACKWARD_BUDGET_ENV, str(budget))
    monkeypatch.setenv(FUSED_ENV, "0")
    grad = torch.rand(T, generator=torch.Generator().manual_seed(3))
    Xd = X.to(gpu).requires_grad_(True)
    Wd = W.to(gpu).requires_grad_(True)
    loss = fused_linear_cross_entropy(Xd, Wd, y.to(gpu))
    loss.backward(grad.to(gpu))
    torch.cuda.synchronize()
    assert Wd.grad.dtype == torch.bfloat16
    check_parity(X, W, y, loss.detach().cpu(), Xd.grad.cpu(), Wd.grad.float().cpu(), grad=grad)


def _keep_case_budget():
    # one 1024-row block and 512-entry vocabulary blocks for T = 900, V = 2600
    return 1024 * 512 * 2 + 4096


def test_general_forward_keeps_first_block(gpu, monkeypatch):
    """General path, one row block, softcap off: the forward keeps the first
    vocabulary block's exponentials (mt_flce_forward_keep) and the narrowing
    backward turns them into G instead of recomputing that block (the last
    block a 40-column tail).  Loss, dX and the bf16 weight gradient against
    the torch path; the forward launch with the kept block is on record."""
    from mini_trainer_amd.flce import FUSED_ENV, backward_plan, profile_enable, profile_report

    T, H, V = 900, 64, 2600
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=23, mask_frac=0.0, w_std=0.1)
    n = T
    C, Cv, _ = backward_plan(T, n, H, V, torch.bfloat16, budget_bytes=_keep_case_budget(),
                             narrow=True)
    assert (C, Cv) == (1024, 512)
    monkeypatch.setenv(BACKWARD_BUDGET_ENV, str(_keep_case_budget()))
    monkeypatch.setenv(FUSED_ENV, "0")
    grad = torch.rand(T, generator=torch.Generator().manual_seed(4))
    Xd = X.to(gpu).requires_grad_(True)
    Wd = W.to(gpu).requires_grad_(True)
    profile_enable(True)
    try:
        loss = fused_linear_cross_entropy(Xd, Wd, y.to(gpu))
        loss.backward(grad.to(gpu))
        torch.cuda.synchronize()
    finally:
        profile_enable(False)
    rep = profile_report()
    assert any("fwd_bf16_kernel<keep>" in k for k in rep), list(rep)
    check_parity(X, W, y, loss.detach().cpu(), Xd.grad.cpu(), Wd.grad.float().cpu(), grad=grad)


def test_general_kept_block_second_backward(gpu, monkeypatch):
    """A second backward through the same loss (retain_graph) cannot reuse the
    kept exponentials (the first backward turned them into G): it recomputes
    every block and gives the same gradients within the tolerance, and the
    first backward's gradients match the torch path."""
    from mini_trainer_amd.flce import FUSED_ENV

    monkeypatch.setenv(BACKWARD_BUDGET_ENV, str(_keep_case_budget()))
    monkeypatch.setenv(FUSED_ENV, "0")
    T, H, V = 900, 64, 2600
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=29, mask_frac=0.0, w_std=0.1)
    grad = torch.rand(T, generator=torch.Generator().manual_seed(5))
    Xd = X.to(gpu).requires_grad_(True)
    Wd = W.to(gpu).requires_grad_(True)
    loss = fused_linear_cross_entropy(Xd, Wd, y.to(gpu))
    loss.backward(grad.to(gpu), retain_graph=True)
    gx1, gw1 = Xd.grad.clone(), Wd.grad.clone()
    Xd.grad = None
    Wd.grad = None
    loss.backward(grad.to(gpu))
    torch.cuda.synchronize()
    check_parity(X, W, y, loss.detach().cpu(), gx1.cpu(), gw1.float().cpu(), grad=grad)
    assert rel_fro(Xd.grad.float().cpu(), gx1.float().cpu()) <= 1e-2
    assert rel_fro(Wd.grad.float().cpu(), gw1.float().cpu()) <= 1e-2


@pytest.mark.parametrize("shift", [56.0, -56.0])
def test_general_kept_block_out_of_range_recomputes(gpu, monkeypatch, shift):
    """The kept exponentials hold their terms while every row's largest logit
    lies in [-48, 48]; here the first 256 rows' logits all move by `shift`, so
    the guard is raised and the first vocabulary block is recomputed.  Logits
    are exact multiples of 1/4 below 64 in magnitude (X in {-1, 0, 1}, W in
    quarters), so every path rounds them the same way."""
    from mini_trainer_amd.flce import FUSED_ENV

    monkeypatch.setenv(BACKWARD_BUDGET_ENV, str(_keep_case_budget()))
    monkeypatch.setenv(FUSED_ENV, "0")
    g = torch.Generator().manual_seed(47)
    T, H, V = 900, 64, 2600
    X = torch.zeros(T, H)
    W = torch.zeros(V, H)
    X[:, 1:16] = torch.randint(-1, 2, (T, 15), generator=g).float()
    W[:, 1:16] = torch.randint(-1, 2, (V, 15), generator=g).float() / 4
    X[:256, 0] = shift
    W[:, 0] = 1.0
    X, W = X.to(torch.bfloat16), W.to(torch.bfloat16)
    y = torch.randint(0, V, (T,), generator=g)
    grad = torch.full((T,), 1.0 / T)
    Xd = X.to(gpu).requires_grad_(True)
    Wd = W.to(gpu).requires_grad_(True)
    loss = fused_linear_cross_entropy(Xd, Wd, y.to(gpu))
    loss.backward(grad.to(gpu))
    torch.cuda.synchronize()
    check_parity(X, W, y, loss.detach().cpu(), Xd.grad.cpu(), Wd.grad.float().cpu(), grad=grad)


def test_accumulate_into_fp32_dw(gpu):
    X, W, y = make_case(300, 128, 700, torch.bfloat16, seed=9)
    X2, _, y2 = make_case(200, 128, 700, torch.bfloat16, seed=10)
    acc = torch.zeros(W.shape, dtype=torch.float32, device=gpu)
    Wd = W.to(gpu)
    for Xi, yi in ((X, y), (X2, y2)):
        fused_linear_cross_entropy(Xi.to(gpu), Wd.requires_grad_(True), yi.to(gpu),
                                   dw_accumulator=acc).sum().backward()
    _, _, r1 = torch_path(X, W, y)
    _, _, r2 = torch_path(X2, W, y2)
    assert rel_fro(acc.cpu(), r1 + r2) <= GRAD_RFRO


def test_all_masked_and_degenerate_sizes(gpu):
    X, W, y = make_case(100, 64, 500, torch.bfloat16, seed=4)
    y[:] = -100
    loss, dX, dW = run_ours(gpu, X, W, y)
    assert torch.equal(loss, torch.zeros(100)) and not torch.signbit(loss).any()
    assert torch.count_nonzero(dX) == 0 and torch.count_nonzero(dW) == 0
    # T = 1
    X1, W1, y1 = make_case(1, 64, 300, torch.bfloat16, seed=1, mask_frac=0.0)
    loss, dX, dW = run_ours(gpu, X1, W1, y1)
    check_parity(X1, W1, y1, loss, dX, dW)
    # T = 0
    X0 = torch.zeros(0, 64, dtype=torch.bfloat16)
    loss, dX, dW = run_ours(gpu, X0, W1, torch.zeros(0, dtype=torch.int64))
    assert loss.shape == (0,) and dX.shape == (0, 64) and torch.count_nonzero(dW) == 0


def test_shift_labels_on_device(gpu):
    X, W, lab = make_case(333, 128, 900, torch.bfloat16, seed=12)
    shifted = torch.cat([lab[1:], torch.tensor([-100])])
    a = run_ours(gpu, X, W, lab, shift=True)
    b = run_ours(gpu, X, W, shifted, shift=False)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_bad_label_raises(gpu):
    X, W, y = make_case(50, 64, 300, torch.bfloat16, seed=3)
    y[17] = 300
    with pytest.raises(IndexError):
        fused_linear_cross_entropy(X.to(gpu), W.to(gpu), y.to(gpu))
    y[17] = -5
    with pytest.raises(IndexError):
        fused_linear_cross_entropy(X.to(gpu), W.to(gpu), y.to(gpu))


@pytest.mark.parametrize("shift", [False, True])
def test_prepare_bit_exact(gpu, shift):
    rng = np.random.default_rng(5)
    for T in (0, 1, 4095, 4096, 4097, 70001):
        lab = rng.integers(0, 5000, T)
        lab[rng.random(T) < 0.4] = -100
        ri, rl, n = prepare_targets(torch.from_numpy(lab).to(gpu), 5000, -100, shift=shift)
        eri, erl, counts = ref.prepare(lab, 5000, -100, shift=shift)
        assert n == counts[0]
        assert np.array_equal(ri.cpu().numpy(), eri)
        assert np.array_equal(rl.cpu().numpy()[:n], erl[:n])


def test_segment_sums(gpu):
    rng = np.random.default_rng(6)
    L = rng.integers(1, 300, 77)
    L[[3, 40, 76]] = 0  # empty samples, the last one included
    T = int(L.sum())
    cu = np.concatenate([[0], np.cumsum(L)]).astype(np.int32)
    loss = rng.random(T).astype(np.float32)
    tgt = rng.integers(0, 10, T)
    tgt[rng.random(T) < 0.5] = -100
    tgt[cu[10]:cu[11]] = -100  # a fully masked sample (config 5 has five)
    loss[tgt == -100] = 0.0
    sl, sc = per_sample_loss_sums(torch.from_numpy(loss).to(gpu), torch.from_numpy(tgt).to(gpu),
                                  torch.from_numpy(cu).to(gpu))
    esl, esc, st = ref.segment_sum(loss, tgt, cu)
    assert st == 0
    assert np.array_equal(sc.cpu().numpy(), esc)
    np.testing.assert_allclose(sl.cpu().numpy(), esl, rtol=1e-5)
    assert sc[3].item() == 0 and sc[40].item() == 0 and sc[76].item() == 0 and sc[10].item() == 0
    assert sl[10].item() == 0.0
    # a checksum of checksums: the per-sample sums add up to the whole-batch sum
    np.testing.assert_allclose(sl.sum().item(), float(loss.astype(np.float64).sum()), rtol=1e-5)
    assert int(sc.sum().item()) == int((tgt != -100).sum())
    bad = cu.copy()
    bad[5], bad[6] = bad[6], bad[5]
    with pytest.raises(ValueError):
        per_sample_loss_sums(torch.from_numpy(loss).to(gpu), torch.from_numpy(tgt).to(gpu),
                             torch.from_numpy(bad).to(gpu))


@pytest.mark.parametrize("V", [1031, 2048])  # rows mostly misaligned / all 16-byte aligned
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cross_entropy_none_materialised(gpu, dtype, V):
    g = torch.Generator().manual_seed(8)
    logits = (torch.randn(333, V, generator=g) * 3).to(dtype)
    y = torch.randint(0, V, (333,), generator=g)
    y[::5] = -100
    src = logits.to(gpu).requires_grad_(True)
    out = cross_entropy_none(src, y.to(gpu))
    gr = torch.rand(333, generator=g)
    out.float().backward(gr.to(gpu))
    # torch's own call on the same dtype (bf16 logits give a bf16 loss there too)
    ref_src = logits.clone().requires_grad_(True)
    ref_out = torch.nn.functional.cross_entropy(ref_src, y, reduction="none")
    ref_out.float().backward(gr)
    assert out.dtype == ref_out.dtype
    if dtype == torch.float32:
        torch.testing.assert_close(out.cpu(), ref_out, rtol=1e-5, atol=1e-5)
    else:  # both round an fp32 result to bf16: at most one bf16 ulp apart
        torch.testing.assert_close(out.float().cpu(), ref_out.float(), rtol=2 ** -7, atol=1e-3)
    assert torch.equal(out.float().cpu()[::5], torch.zeros(67))
    assert torch.count_nonzero(src.grad[::5]) == 0
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel_fro(src.grad.float().cpu(), ref_src.grad.float()) <= tol


def test_real_vocab_tail_qwen(gpu):
    # V = 151936 (= 593 * 256 + 128), H = 1536
    X, W, y = make_case(384, 1536, 151936, torch.bfloat16, seed=21, mask_frac=0.5)
    loss, dX, dW = run_ours(gpu, X, W, y)
    check_parity(X, W, y, loss, dX, dW)


@pytest.mark.parametrize("fused,cap", [(False, "3"), (True, "3"), (False, "2"), (True, "2")])
def test_persistent_multi_tile(gpu, monkeypatch, fused, cap):
    # A grid of 3 workgroups makes the persistent bf16 GEMMs (logits,
    # recompute, dW) walk several tiles per workgroup: tile-to-tile
    # pipelining through the LDS ring, the next tile's fragments re-read after
    # each epilogue, and dW's fp32 tile preload (interior and edge tiles) are
    # all exercised at small sizes (dX keeps one workgroup per tile).  The
    # multi-block backward budget adds dX accumulation modes, and with the
    # cap standing in for a 3-CU GPU the general path runs dX and the
    # persistent dW one after the other instead of side by side.  V = 2300
    # leaves a partial last vocabulary tile: its 3 row tiles run first in the
    # workgroups with one full tile fewer, under a 2-workgroup grid two of
    # them in one workgroup.
    print(f"case persistent multi-tile fused={fused} cap={cap}", flush=True)
    monkeypatch.setenv("MT_FLCE_GRID_CAP", cap)
    if fused:
        monkeypatch.setenv("MT_FLCE_FUSED", "1")
    else:
        monkeypatch.setenv(BACKWARD_BUDGET_ENV, "1")
    X, W, y = make_case(700, 384, 2300, torch.bfloat16, seed=21, w_std=0.05)
    grad = torch.rand(700, generator=torch.Generator().manual_seed(4)) + 0.5
    Xd = X.to(gpu).requires_grad_(True)
    Wd = W.to(gpu).requires_grad_(True)
    acc = torch.zeros(W.shape, dtype=torch.float32, device=gpu)
    n = int((y != -100).sum())
    if fused:
        g = torch.full((700,), 1.0 / n)
        loss = fused_linear_cross_entropy(Xd, Wd, y.to(gpu), dw_accumulator=acc, grad_scale=1.0 / n)
        (loss.float().sum() * (1.0 / n)).backward()
    else:
        g = grad
        loss = fused_linear_cross_entropy(Xd, Wd, y.to(gpu), dw_accumulator=acc)
        loss.backward(grad.to(gpu))
    torch.cuda.synchronize()
    check_parity(X, W, y, loss.detach().cpu(), Xd.grad.cpu(), acc.cpu(), grad=g)
