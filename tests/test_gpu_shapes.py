"""Shapes beyond the tuned ones, against the reference's torch path with the
north-star tolerances (loss 2e-3 relative in bf16 and 1e-5 in fp32, dX and dW
1e-2 relative Frobenius, ignored rows exactly +0.0):

  * H not a multiple of the 64-element (bf16) or 32-element (fp32) K stage:
    the last K stage is partial and masked inside the kernels (H = 1000, 72,
    40 bf16; H = 100 fp32), on the general, fused and unit-gradient paths;
  * H not a whole 16-byte chunk (H = 1001 bf16, 1002 fp32): zero columns
    appended on the host;
  * V below one 256-column tile (V = 200, 37): every logits tile is a tail
    tile;
  * a weight beyond one buffer's reach (vocabulary blocks on the forward and
    the general backward; the fused planner declines it) and X beyond it
    (row ranges on the host), under the MT_FLCE_MAX_BUFFER_BYTES test hook
    that lowers the 4 GiB reach so that small problems take those paths.
"""
from __future__ import annotations

import pytest
import torch

from mini_trainer_amd import _lib, fused_linear_cross_entropy, path_of
from mini_trainer_amd.flce import FUSED_ENV
from mini_trainer_amd.none_reduction_losses import (
    liger_fixed_fused_linear_cross_entropy_none_reduction as drop_in)

from test_gpu_parity import check_parity, make_case

pytestmark = pytest.mark.gpu

REACH_ENV = "MT_FLCE_MAX_BUFFER_BYTES"


def run(dev, X, W, y, how, grad_scale=None, softcap=None):
    """how: "general" / "fused" (promised scalar gradient, fp32 accumulator) /
    "unit" (the reference's call chain).  Returns (path, loss, dX, dW)."""
    Xd, Wd, yd = X.to(dev).requires_grad_(True), W.to(dev).requires_grad_(True), y.to(dev)
    n = max(int((y != -100).sum()), 1)
    if how == "unit":
        out = drop_in(Xd, Wd, yd, None, -100, softcap)
        path = path_of(out)
        (out.float().sum() / n).backward()
        dW = Wd.grad.float()
    else:
        acc = torch.zeros(W.shape, dtype=torch.float32, device=dev)
        out = fused_linear_cross_entropy(Xd, Wd, yd, softcap=softcap, dw_accumulator=acc,
                                         grad_scale=(1.0 / n) if how == "fused" else None)
        path = path_of(out)
        (out.float().sum() / n).backward()
        dW = acc
    torch.cuda.synchronize()
    return path, out.detach().cpu(), Xd.grad.cpu(), dW.cpu()


@pytest.mark.parametrize("H", [1000, 72, 40])
@pytest.mark.parametrize("how", ["general", "fused", "unit"])
def test_partial_last_k_stage_bf16(gpu, monkeypatch, H, how):
    print(f"case K tail bf16 H={H} {how}", flush=True)
    monkeypatch.setenv(FUSED_ENV, "0" if how == "general" else "1")
    X, W, y = make_case(600, H, 1300, torch.bfloat16, seed=H)
    path, loss, dX, dW = run(gpu, X, W, y, how)
    assert path == {"general": "general", "fused": "fused", "unit": "fused_unit"}[how]
    n = int((y != -100).sum())
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((600,), 1.0 / n))


@pytest.mark.parametrize("V", [200, 37])
@pytest.mark.parametrize("how", ["general", "fused", "unit"])
def test_vocabulary_below_one_tile(gpu, monkeypatch, V, how):
    """V < 256: no full vocabulary tile at all, so every logits tile is a
    tail tile, run by the workgroups of the tail loop alone."""
    print(f"case vocabulary below one tile V={V} {how}", flush=True)
    monkeypatch.setenv(FUSED_ENV, "0" if how == "general" else "1")
    X, W, y = make_case(700, 128, V, torch.bfloat16, seed=V, w_std=0.2)
    path, loss, dX, dW = run(gpu, X, W, y, how)
    assert path == {"general": "general", "fused": "fused", "unit": "fused_unit"}[how]
    n = int((y != -100).sum())
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((700,), 1.0 / n))


def test_partial_last_k_stage_softcap(gpu, monkeypatch):
    monkeypatch.setenv(FUSED_ENV, "1")
    X, W, y = make_case(300, 200, 1000, torch.bfloat16, seed=5, w_std=0.2)
    _, loss, dX, dW = run(gpu, X, W, y, "unit", softcap=3.0)
    n = int((y != -100).sum())
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((300,), 1.0 / n), softcap=3.0)


def test_partial_last_k_stage_fp32(gpu):
    X, W, y = make_case(257, 100, 777, torch.float32, seed=3)
    _, loss, dX, dW = run(gpu, X, W, y, "general")
    n = int((y != -100).sum())
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((257,), 1.0 / n))


@pytest.mark.parametrize("H,dtype", [(1001, torch.bfloat16), (1002, torch.float32)])
def test_h_not_whole_chunks_is_padded(gpu, monkeypatch, H, dtype):
    monkeypatch.setenv(FUSED_ENV, "1")
    X, W, y = make_case(300, H, 900, dtype, seed=H)
    _, loss, dX, dW = run(gpu, X, W, y, "unit")
    assert dX.shape == (300, H) and dW.shape == (900, H)
    n = int((y != -100).sum())
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((300,), 1.0 / n))
    with pytest.raises(ValueError, match="multiple of"):
        fused_linear_cross_entropy(X.to(gpu).requires_grad_(True), W.to(gpu), y.to(gpu),
                                   dw_accumulator=torch.zeros(W.shape, device=gpu))


@pytest.mark.parametrize("how", ["general", "unit"])
def test_weight_beyond_one_buffer_runs_in_vocabulary_blocks(gpu, monkeypatch, how):
    # 3000 x 128 bf16 = 768 KB against a 128 KiB reach: vocabulary blocks of
    # 512 rows (the last one 440); the fused planner declines such a weight
    monkeypatch.setenv(REACH_ENV, str(128 << 10))
    monkeypatch.setenv(FUSED_ENV, "auto")
    assert _lib.load().mt_flce_max_buffer_bytes() == 128 << 10
    X, W, y = make_case(400, 128, 3000, torch.bfloat16, seed=17)
    path, loss, dX, dW = run(gpu, X, W, y, how)
    assert path == "general"
    n = int((y != -100).sum())
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((400,), 1.0 / n))


def test_weight_beyond_one_buffer_softcap_and_tail(gpu, monkeypatch):
    # blocks whose last one is not a whole tile (V = 2900), a partial K stage
    # (H = 200) and softcap together
    monkeypatch.setenv(REACH_ENV, str(160 << 10))
    X, W, y = make_case(300, 200, 2900, torch.bfloat16, seed=19, w_std=0.2)
    _, loss, dX, dW = run(gpu, X, W, y, "general", softcap=2.0)
    n = int((y != -100).sum())
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((300,), 1.0 / n), softcap=2.0)


@pytest.mark.parametrize("how", ["general", "unit", "fused"])
def test_hidden_beyond_one_buffer_runs_over_row_ranges(gpu, monkeypatch, how):
    # X of 1200 x 128 bf16 (300 KB) against a 128 KiB reach: row ranges of
    # 512 rows; the weight (1300 x 128, 325 KB) runs in vocabulary blocks
    monkeypatch.setenv(REACH_ENV, str(128 << 10))
    X, W, y = make_case(1200, 128, 1300, torch.bfloat16, seed=23)
    _, loss, dX, dW = run(gpu, X, W, y, how)
    n = int((y != -100).sum())
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((1200,), 1.0 / n))


def test_row_ranges_with_a_fitting_weight_keep_the_fused_path(gpu, monkeypatch):
    # reach 320 KiB: W (300 x 128 bf16 = 75 KB) and a 256-row logits chunk
    # (256 KiB) fit, X (1500 rows, 375 KB) does not -- both row ranges run
    # the fused kernels; the causal shift crosses the range boundary
    monkeypatch.setenv(REACH_ENV, str(320 << 10))
    monkeypatch.setenv(FUSED_ENV, "1")
    X, W, labels = make_case(1500, 128, 300, torch.bfloat16, seed=29)
    shifted = torch.cat([labels[1:], torch.tensor([-100])])
    Xd, Wd = X.to(gpu).requires_grad_(True), W.to(gpu).requires_grad_(True)
    out = fused_linear_cross_entropy(Xd, Wd, labels.to(gpu), shift_labels=True)
    n = int((shifted != -100).sum())
    (out.sum() / n).backward()
    torch.cuda.synchronize()
    check_parity(X, W, shifted, out.detach().cpu(), Xd.grad.cpu(), Wd.grad.float().cpu(),
                 grad=torch.full((1500,), 1.0 / n))


@pytest.mark.parametrize("fused", ["1", "0"])
def test_three_row_ranges_hold_one_weight_gradient(gpu, monkeypatch, fused):
    """X beyond one buffer's reach in three row ranges (2000 x 128 bf16
    against a 192 KiB reach: 768 + 768 + 464 rows), the reference's call
    chain, on the fused kernels ("1") or the general path ("0"): one
    autograd node whose ranges add into one weight gradient, so the peak
    beyond inputs and outputs (loss, dX, the fp32 dW the kernels accumulate)
    is at most one range's workspace; W.grad then owns exactly V x H bf16.
    Parity against the torch path as everywhere."""
    print(f"case three row ranges fused={fused}", flush=True)
    from mini_trainer_amd.flce import backward_plan, fused_plan

    monkeypatch.setenv(REACH_ENV, str(192 << 10))
    monkeypatch.setenv(FUSED_ENV, fused)
    T, H, V = 2000, 128, 256
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=31)
    n = int((y != -100).sum())
    Xd, Wd, yd = X.to(gpu).requires_grad_(True), W.to(gpu).requires_grad_(True), y.to(gpu)
    lib = _lib.load()
    rng = [(0, 768), (768, 1536), (1536, 2000)]
    ns = [int((y[a:b] != -100).sum()) for a, b in rng]
    if fused == "1":
        ws = max(fused_plan(b - a, k, H, V)[1] for (a, b), k in zip(rng, ns))
    else:
        ws = max(backward_plan(b - a, k, H, V, torch.bfloat16, narrow=True)[2] +
                 lib.mt_flce_forward_workspace_bytes(b - a, k, H, V, _lib.MT_DTYPE_BF16)
                 for (a, b), k in zip(rng, ns))
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(gpu)
    base = torch.cuda.memory_allocated(gpu)
    out = drop_in(Xd, Wd, yd)
    assert path_of(out) == ("fused_unit" if fused == "1" else "general")
    (out.float().sum() / n).backward()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(gpu)
    Hp = -(-H // 256) * 256
    dw_fp32 = Hp * 256 * 2 + (-(-V // 256)) * Hp * 256 * 4 + Hp * 256 * 4  # + one tile row
    outputs = T * 4 + T * H * 2 + dw_fp32
    assert peak - base - outputs <= ws + (256 << 10), (peak - base - outputs, ws)
    assert Wd.grad.dtype == torch.bfloat16 and Wd.grad.untyped_storage().nbytes() == V * H * 2
    check_parity(X, W, y, out.detach().cpu(), Xd.grad.cpu(), Wd.grad.float().cpu(),
                 grad=torch.full((T,), 1.0 / n))
