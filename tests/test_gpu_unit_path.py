"""The reference's unchanged caller reaches the fused kernels.

train.py:97-104 calls the drop-in with the reference's own arguments
(none_reduction_losses.py:5-13, no extra keyword), sums the per-token loss,
syncs with .item(), scales by world_size / batch_num_loss_counted_tokens and
calls backward().  Where the fused path pays, the forward forms dX and dW
for a unit upstream gradient (path "fused_unit", the structure of the
reference's Liger call at none_reduction_losses.py:16-23) and the backward
rescales them on the device (mt_flce_scale_grads).  Checked against the
reference's torch path with the north-star tolerances (loss 2e-3 relative,
dX and dW 1e-2 relative Frobenius, ignored rows exactly +0.0 / 0), for
world sizes that make the scale a non-power of two, for a per-token
gradient (recompute fallback), softcap, several chunks, and the C-ABI pieces
this path adds: the tiled dW (bit for bit the row-major one, tile layout
unscrambled in torch), the rescale kernels (bit-exact against torch's fp32
multiply and round-to-nearest-even), the shifted per-sample sums (against
the C restatement) and the per-launch timing hook.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from mini_trainer_amd import _lib, fused_linear_cross_entropy, path_of, per_sample_loss_sums
from mini_trainer_amd.flce import (BACKWARD_BUDGET_ENV, FUSED_ENV, PROMISE_ULPS, _p, _stream,
                                   fused_plan, prepare_targets, profile_enable, profile_report)
from mini_trainer_amd.none_reduction_losses import (
    liger_fixed_fused_linear_cross_entropy_none_reduction as drop_in)
from oracle import ref
from oracle.torch_path import rel_fro

from test_gpu_parity import check_parity, make_case

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _fused(monkeypatch):
    # the fused kernels whatever the planner prefers at these small sizes
    monkeypatch.setenv(FUSED_ENV, "1")


def train_py_chain(dev, X, W, y, world_size, n_counted, softcap=None):
    """train.py:97-104, literally, over the drop-in."""
    Xd = X.to(dev).requires_grad_(True)
    Wd = W.to(dev).requires_grad_(True)
    out = drop_in(Xd, Wd, y.to(dev), None, -100, softcap)
    path = path_of(out)
    loss = out.float().sum()
    loss.detach().item()
    loss = loss * world_size / n_counted
    loss.backward()
    torch.cuda.synchronize()
    return path, out.detach().cpu(), Xd.grad.cpu(), Wd.grad.float().cpu()


@pytest.mark.parametrize("world_size", [1, 3, 6])
@pytest.mark.parametrize("T,H,V", [(300, 128, 1000), (513, 192, 2065), (700, 256, 2560)])
def test_reference_chain_takes_the_fused_kernels(gpu, world_size, T, H, V):
    print(f"case unit path T={T} H={H} V={V} world_size={world_size}", flush=True)
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=T + world_size)
    n = int((y != -100).sum())
    path, loss, dX, dW = train_py_chain(gpu, X, W, y, world_size, n)
    assert path == "fused_unit"
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((T,), world_size / n))


def test_unit_path_softcap_and_many_chunks(gpu, monkeypatch):
    # tiny budget -> 256-row chunks (uneven last one), dW accumulated across
    # chunks before the rescale
    monkeypatch.setenv(BACKWARD_BUDGET_ENV, "1")
    X, W, y = make_case(1100, 128, 1300, torch.bfloat16, seed=7, mask_frac=0.2, w_std=0.2)
    n = int((y != -100).sum())
    assert fused_plan(1100, n, 128, 1300)[0] == 256
    path, loss, dX, dW = train_py_chain(gpu, X, W, y, 3, n, softcap=3.0)
    assert path == "fused_unit"
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((1100,), 3.0 / n), softcap=3.0)


@pytest.mark.parametrize("softcap", [None, 2.5])
def test_unit_path_per_token_gradient_recomputes(gpu, softcap):
    # a gradient that differs per token cannot be a rescale of the unit one:
    # the backward recomputes with the saved lse
    X, W, y = make_case(400, 128, 3000, torch.bfloat16, seed=11, w_std=0.2)
    grad = torch.rand(400, generator=torch.Generator().manual_seed(3)) * 2 - 0.5
    Xd, Wd = X.to(gpu).requires_grad_(True), W.to(gpu).requires_grad_(True)
    out = drop_in(Xd, Wd, y.to(gpu), None, -100, softcap)
    assert path_of(out) == "fused_unit"
    out.backward(grad.to(gpu))
    torch.cuda.synchronize()
    check_parity(X, W, y, out.detach().cpu(), Xd.grad.cpu(), Wd.grad.float().cpu(), grad=grad,
                 softcap=softcap)


def test_unit_path_only_when_the_weight_gradient_is_wanted(gpu):
    X, W, y = make_case(256, 64, 512, torch.bfloat16, seed=22)
    Xd = X.to(gpu).requires_grad_(True)
    out = drop_in(Xd, W.to(gpu), y.to(gpu))  # frozen lm_head: dW would be waste
    assert path_of(out) == "general"
    acc = torch.zeros(W.shape, dtype=torch.float32, device=gpu)
    out2 = fused_linear_cross_entropy(Xd, W.to(gpu).requires_grad_(True), y.to(gpu),
                                      dw_accumulator=acc)
    assert path_of(out2) == "general"  # an accumulator needs the scale at the forward


def test_unit_path_second_backward_raises(gpu):
    X, W, y = make_case(256, 64, 512, torch.bfloat16, seed=24)
    Xd, Wd = X.to(gpu).requires_grad_(True), W.to(gpu).requires_grad_(True)
    out = drop_in(Xd, Wd, y.to(gpu))
    (out.sum() * 0.5).backward(retain_graph=True)
    with pytest.raises(RuntimeError, match="second backward"):
        (out.sum() * 0.5).backward()


@pytest.mark.parametrize("world_size", [3, 6])
def test_promise_accepts_train_py_rounding(gpu, world_size):
    # grad_scale = world_size / n promised, the literal train.py expression
    # back-propagated: fl32(fl32(1 / n) * world_size) may differ from
    # fl32(world_size / n) by an ulp -- accepted; a 1e-3 relative miss is not
    X, W, y = make_case(300, 128, 1000, torch.bfloat16, seed=31)
    n = int((y != -100).sum())
    Xd, Wd = X.to(gpu).requires_grad_(True), W.to(gpu).requires_grad_(True)
    out = fused_linear_cross_entropy(Xd, Wd, y.to(gpu), grad_scale=world_size / n)
    assert path_of(out) == "fused"
    loss = out.float().sum()
    (loss * world_size / n).backward()
    torch.cuda.synchronize()
    check_parity(X, W, y, out.detach().cpu(), Xd.grad.cpu(), Wd.grad.float().cpu(),
                 grad=torch.full((300,), world_size / n))
    out = fused_linear_cross_entropy(Xd, Wd, y.to(gpu), grad_scale=world_size / n)
    with pytest.raises(RuntimeError, match=f"{PROMISE_ULPS} fp32 ulp"):
        (out.float().sum() * (world_size / n * (1 + 1e-3))).backward()


@pytest.mark.parametrize("H,ld", [(64, 64), (66, 72)])
def test_scale_grads_bit_exact(gpu, H, ld):
    """mt_flce_scale_grads against torch: bf16 dX in place, fp32 dW in place
    and fp32 dW -> bf16; columns between H and the pitch are left alone."""
    lib = _lib.load()
    g = torch.Generator(device=gpu).manual_seed(5)
    T, V = 333, 517
    dX = torch.randn(T, ld, device=gpu, generator=g).to(torch.bfloat16)
    dW = torch.randn(V, ld, device=gpu, generator=g)
    scale = torch.tensor([0.37], device=gpu)
    want_x = dX.clone()
    want_x[:, :H] = (dX[:, :H].float() * 0.37).to(torch.bfloat16)
    want_w32 = dW.clone()
    want_w32[:, :H] = dW[:, :H] * scale
    out16 = torch.full((V, ld), 7.0, device=gpu, dtype=torch.bfloat16)
    want_w16 = out16.clone()
    want_w16[:, :H] = (dW[:, :H] * scale).to(torch.bfloat16)
    s = _stream(gpu)
    _lib.check(lib.mt_flce_scale_grads(_p(scale), _p(dX), T, H, ld, _lib.MT_DTYPE_BF16, _p(dW),
                                       V, ld, _p(out16), ld, _lib.MT_DTYPE_BF16, s), "scale")
    _lib.check(lib.mt_flce_scale_grads(_p(scale), None, 0, H, ld, _lib.MT_DTYPE_BF16, _p(dW),
                                       V, ld, _p(dW), ld, _lib.MT_DTYPE_F32, s), "scale")
    torch.cuda.synchronize()
    assert torch.equal(dX, want_x)
    assert torch.equal(out16, want_w16)
    assert torch.equal(dW, want_w32)


@pytest.mark.parametrize("V,H,ld", [(1, 64, 64), (517, 66, 72), (1031, 4096, 4096)])
def test_narrow_in_place_bit_exact(gpu, V, H, ld):
    """fp32 dW -> bf16 scaled, written into the first bytes of dW's own
    allocation (row r at bf16 offset r * ld): every row, including those whose
    bytes are reused, equals torch's fp32 multiply rounded to nearest even."""
    lib = _lib.load()
    g = torch.Generator(device=gpu).manual_seed(V)
    dW = torch.randn(V, ld, device=gpu, generator=g)
    scale = torch.tensor([1.7], device=gpu)
    want = (dW[:, :H] * scale).to(torch.bfloat16)
    _lib.check(lib.mt_flce_scale_grads(_p(scale), None, 0, H, ld, _lib.MT_DTYPE_BF16, _p(dW), V,
                                       ld, _p(dW), ld, _lib.MT_DTYPE_BF16, _stream(gpu)), "narrow")
    torch.cuda.synchronize()
    got = dW.view(torch.uint8).view(-1)[: V * ld * 2].view(torch.bfloat16).view(V, ld)[:, :H]
    assert torch.equal(got, want)


def _tiled_buffers(V, H, dev, fill=float("nan")):
    """The two buffers of mt_flce_dw_tiles_layout, filled with `fill`:
    (lo: bf16 [V, H], hi: fp32, tile rows held in lo)."""
    lib = _lib.load()
    lo_b, rows, hi_b = ctypes.c_size_t(), ctypes.c_int64(), ctypes.c_size_t()
    _lib.check(lib.mt_flce_dw_tiles_layout(V, H, ctypes.byref(lo_b), ctypes.byref(rows),
                                           ctypes.byref(hi_b)), "mt_flce_dw_tiles_layout")
    assert lo_b.value == V * H * 2
    lo = torch.empty(V, H, dtype=torch.bfloat16, device=dev)
    lo.view(torch.float32).fill_(fill)
    hi = torch.full((hi_b.value // 4,), fill, dtype=torch.float32, device=dev)
    return lo, hi, rows.value


def _targs(lo, hi):
    """(lo, lo bytes, hi, hi bytes) as the C ABI takes them."""
    return (_p(lo), lo.numel() * 2, _p(hi), hi.numel() * 4)


def _fused_abi(dev, X, W, ri, rl, n, C, wsb, tiled):
    """One mt_flce_fused (row-major dW) or mt_flce_fused_tiles call for a
    unit upstream gradient; returns (loss, lse, dX, dW) with dW the
    row-major fp32 tensor or the (lo, hi, lo_rows) tiles."""
    lib = _lib.load()
    T, H = X.shape
    V = W.shape[0]
    g = torch.ones(1, device=dev)
    loss = torch.empty(T, device=dev)
    lse = torch.empty(max(n, 1), device=dev)
    dX = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    if tiled:
        dW = _tiled_buffers(V, H, dev)
        _lib.check(lib.mt_flce_fused_tiles(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                           _p(ri), _p(rl), n, _p(g), 0, _p(loss), _p(lse),
                                           _p(dX), H, *_targs(dW[0], dW[1]), 0, C, _p(ws), wsb,
                                           _stream(dev)), "mt_flce_fused_tiles")
    else:
        dW = torch.empty(V, H, device=dev)
        _lib.check(lib.mt_flce_fused(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                     _p(ri), _p(rl), n, _p(g), 0, _p(loss), _p(lse), _p(dX), H,
                                     _p(dW), H, 0, C, _p(ws), wsb, _stream(dev)), "mt_flce_fused")
    torch.cuda.synchronize()
    return loss, lse[:n], dX, dW


def _untile(tiles, V, H):
    """Row-major fp32 [V, H] from the tiled layout (lo, hi, lo_rows): tile
    rows [0, lo_rows) in lo after a pad of 256 * Hp bf16, the rest in hi;
    tile (tm, tn) at index tm * tiles_n + tn of that sequence, 256 KiB each,
    ordered (wave row wm, wave column wn, fragment row fm, fragment column
    fn, lane / 16, lane % 16, element r) for the element at row
    wm * 128 + fm * 16 + lane % 16, column wn * 128 + fn * 16 + 4 (lane / 16) + r."""
    lo, hi, rows = tiles
    vt, tn = -(-V // 256), -(-H // 256)
    pad = 128 * tn * 256
    flat = torch.cat([lo.view(torch.float32).reshape(-1)[pad:pad + rows * tn * 65536], hi])
    t = flat.view(vt, tn, 2, 2, 8, 8, 4, 16, 4)
    #       dims: tm tn wm wn fm fn lq li r -> rows (tm wm fm li), cols (tn wn fn lq r)
    t = t.permute(0, 2, 4, 7, 1, 3, 5, 6, 8).reshape(vt * 256, tn * 256)
    return t[:V, :H]


@pytest.mark.parametrize("T,H,V,budget", [(700, 1056, 65600, 1), (513, 192, 2065, 0),
                                          (300, 64, 256, 0), (200, 72, 100, 0)])
def test_fused_tiles_match_rows_bit_exact(gpu, T, H, V, budget):
    """mt_flce_fused_tiles against mt_flce_fused on the same inputs: loss,
    lse and dX the same bits; the tiles, unscrambled from their two buffers,
    the row-major fp32 dW bit for bit (tails in V and H; budget 1: 256-row
    chunks accumulating, and at 65600 x 1056 dW over its work queue).
    mt_flce_narrow_tiles in place (the bf16 gradient filling lo) against
    torch's fp32 multiply rounded to nearest even.  The last case is one
    partial tile (V < 256, H < 256) with a partial last K stage (H % 64 = 8),
    held wholly in hi."""
    print(f"case tiles T={T} H={H} V={V}", flush=True)
    lib = _lib.load()
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=T + 3)
    X, W, y = X.to(gpu), W.to(gpu), y.to(gpu)
    ri, rl, n = prepare_targets(y, V)
    C, wsb, _ = fused_plan(T, n, H, V, budget_bytes=budget)
    l0, s0, x0, d0 = _fused_abi(gpu, X, W, ri, rl, n, C, wsb, tiled=False)
    l1, s1, x1, d1 = _fused_abi(gpu, X, W, ri, rl, n, C, wsb, tiled=True)
    assert torch.equal(l0, l1) and torch.equal(s0, s1) and torch.equal(x0, x1)
    assert torch.equal(_untile(d1, V, H), d0)
    scale = torch.tensor([0.37], device=gpu)
    want = (d0 * scale).to(torch.bfloat16)
    _lib.check(lib.mt_flce_narrow_tiles(_p(scale), *_targs(d1[0], d1[1]), V, H, _stream(gpu)),
               "narrow in place")
    torch.cuda.synchronize()
    assert torch.equal(d1[0], want)


@pytest.mark.parametrize("C,Cv,cap", [(256, 52736, None), (256, 16384, "3"), (512, 65600 + 192, None),
                                      (768, 16384, None), (768, 16384, "3")])
def test_backward_tiles_match_rows_bit_exact(gpu, monkeypatch, C, Cv, cap):
    """mt_flce_backward_tiles against mt_flce_backward on the same inputs and
    blocks (per-token upstream gradient): dX the same bits, the tiles,
    unscrambled, the row-major fp32 dW bit for bit.  Blocks of (C, Cv):
    two row blocks and a vocabulary split whose first block runs dW beside dX
    over the work queue; under a 3-CU grid cap dW runs after dX, three
    persistent workgroups carrying tiles; one block over the whole
    vocabulary; one row block and five vocabulary blocks.  V = 65600, H = 1056
    (tails in both)."""
    print(f"case backward tiles C={C} Cv={Cv} cap={cap}", flush=True)
    if cap:
        monkeypatch.setenv("MT_FLCE_GRID_CAP", cap)
    lib = _lib.load()
    T, H, V = 700, 1056, 65600
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=61)
    X, W, y = X.to(gpu), W.to(gpu), y.to(gpu)
    ri, rl, n = prepare_targets(y, V)
    s = _stream(gpu)
    loss = torch.empty(T, device=gpu)
    lse = torch.empty(n, device=gpu)
    fwb = int(lib.mt_flce_forward_workspace_bytes(T, n, H, V, _lib.MT_DTYPE_BF16))
    fws = torch.empty(fwb, dtype=torch.uint8, device=gpu)
    _lib.check(lib.mt_flce_forward(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0, _p(ri),
                                   _p(rl), n, _p(loss), _p(lse), _p(fws), fwb, s), "forward")
    g = torch.rand(T, device=gpu, generator=torch.Generator(device=gpu).manual_seed(8)) - 0.3
    al = lambda b: (b + 255) // 256 * 256  # noqa: E731
    wsb = al(C * Cv * 2) + (al(C * H * 4) if Cv < V else 0) + al(H * C * 2) + al(32)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    dX0 = torch.empty(T, H, dtype=torch.bfloat16, device=gpu)
    dW0 = torch.empty(V, H, device=gpu)
    _lib.check(lib.mt_flce_backward(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0, _p(ri),
                                    _p(rl), n, _p(lse), _p(g), 1, _p(dX0), H, _p(dW0), H, 0, C, Cv,
                                    _p(ws), wsb, s), "backward")
    dX1 = torch.empty(T, H, dtype=torch.bfloat16, device=gpu)
    dW1 = _tiled_buffers(V, H, gpu)
    _lib.check(lib.mt_flce_backward_tiles(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                          _p(ri), _p(rl), n, _p(lse), _p(g), 1, _p(dX1), H,
                                          *_targs(dW1[0], dW1[1]), 0, C, Cv, _p(ws), wsb, s),
               "backward_tiles")
    torch.cuda.synchronize()
    assert torch.equal(dX0, dX1)
    assert torch.equal(_untile(dW1, V, H), dW0)
    if C < n:
        return
    # one row block: mt_flce_backward_narrow (dW narrowed in its epilogue
    # into a bf16 [V, H] of its own size, dX's accumulator and X^T in the
    # scratch buffer, only the G block in the workspace) against the tiles
    # narrowed by mt_flce_narrow_tiles
    one = torch.ones(1, device=gpu)
    _lib.check(lib.mt_flce_narrow_tiles(_p(one), *_targs(dW1[0], dW1[1]), V, H, s), "narrow_tiles")
    want = dW1[0]
    nwsb = al(C * Cv * 2) + al(32)  # the G block and the counters
    nws = torch.empty(nwsb, dtype=torch.uint8, device=gpu)
    sb = int(lib.mt_flce_narrow_scratch_bytes(V, H, C))
    assert sb > 0
    scratch = torch.full((sb,), 255, dtype=torch.uint8, device=gpu)
    dX2 = torch.empty(T, H, dtype=torch.bfloat16, device=gpu)
    dW2 = torch.full((V, H), float("nan"), dtype=torch.bfloat16, device=gpu)
    _lib.check(lib.mt_flce_backward_narrow(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                           _p(ri), _p(rl), n, _p(lse), _p(g), 1, _p(dX2), H,
                                           _p(dW2), V * H * 2, _p(scratch), sb, C, Cv, _p(nws),
                                           nwsb, None, s), "backward_narrow")
    torch.cuda.synchronize()
    assert torch.equal(dX2, dX0)
    assert torch.equal(dW2, want)


def test_backward_narrow_accumulator_in_workspace(gpu):
    """One row block and three vocabulary blocks where a bf16 gradient leaves
    no room of the fp32 one for dX's accumulator and X^T (V = 1300 < 3 C):
    mt_flce_backward_narrow keeps both in the workspace (the accumulator
    row-major) and still matches mt_flce_backward_tiles + mt_flce_narrow_tiles
    bit for bit, with the workspace mt_flce_backward_narrow_plan reports."""
    from mini_trainer_amd.flce import backward_plan

    print("case backward narrow, accumulator in the workspace", flush=True)
    lib = _lib.load()
    T, H, V = 900, 256, 1300
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=83, mask_frac=0.0)
    X, W, y = X.to(gpu), W.to(gpu), y.to(gpu)
    ri, rl, n = prepare_targets(y, V)
    s = _stream(gpu)
    loss = torch.empty(T, device=gpu)
    lse = torch.empty(n, device=gpu)
    fwb = int(lib.mt_flce_forward_workspace_bytes(T, n, H, V, _lib.MT_DTYPE_BF16))
    fws = torch.empty(fwb, dtype=torch.uint8, device=gpu)
    _lib.check(lib.mt_flce_forward(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0, _p(ri),
                                   _p(rl), n, _p(loss), _p(lse), _p(fws), fwb, s), "forward")
    al = lambda b: (b + 255) // 256 * 256  # noqa: E731
    budget = al(1024 * 512 * 2) + al(1024 * H * 4) + al(H * 1024 * 2) + al(32)
    C, Cv, wsb = backward_plan(T, n, H, V, torch.bfloat16, budget_bytes=budget, narrow=True)
    assert (C, Cv, wsb) == (1024, 512, budget)
    g = torch.rand(T, device=gpu, generator=torch.Generator(device=gpu).manual_seed(9))
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    dX1 = torch.empty(T, H, dtype=torch.bfloat16, device=gpu)
    dW1 = _tiled_buffers(V, H, gpu)
    _lib.check(lib.mt_flce_backward_tiles(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                          _p(ri), _p(rl), n, _p(lse), _p(g), 1, _p(dX1), H,
                                          *_targs(dW1[0], dW1[1]), 0, C, Cv, _p(ws), wsb, s),
               "backward_tiles")
    one = torch.ones(1, device=gpu)
    _lib.check(lib.mt_flce_narrow_tiles(_p(one), *_targs(dW1[0], dW1[1]), V, H, s), "narrow_tiles")
    assert int(lib.mt_flce_narrow_scratch_bytes(V, H, C)) == 0  # no room: all in the workspace
    dX2 = torch.empty(T, H, dtype=torch.bfloat16, device=gpu)
    dW2 = torch.full((V, H), float("nan"), dtype=torch.bfloat16, device=gpu)
    _lib.check(lib.mt_flce_backward_narrow(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                           _p(ri), _p(rl), n, _p(lse), _p(g), 1, _p(dX2), H,
                                           _p(dW2), V * H * 2, None, 0, C, Cv, _p(ws), wsb, None,
                                           s), "backward_narrow")
    torch.cuda.synchronize()
    assert torch.equal(dX2, dX1)
    assert torch.equal(dW2, dW1[0])


@pytest.mark.parametrize("shift,H", [(0.0, 192), (56.0, 192), (0.0, 200)])
def test_forward_keep_matches_forward(gpu, shift, H):
    """mt_flce_forward_keep against mt_flce_forward: loss and lse the same
    bits; the kept block holds exp of the bf16 logits of vocabulary columns
    [0, 512) for every valid row (within bf16 rounding of exp); the guard is 0
    while every row's largest logit lies in [-48, 48] and 1 when the first
    rows' logits are shifted by 56 (X column of 56 against a weight column of
    ones).  H = 200: a partial last K stage."""
    print(f"case forward_keep shift={shift} H={H}", flush=True)
    lib = _lib.load()
    T, V, K = 600, 1500, 512
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=71)
    if shift:
        X[:100, 0] = shift
        W[:, 0] = 1.0
    X, W, y = X.to(gpu), W.to(gpu), y.to(gpu)
    ri, rl, n = prepare_targets(y, V)
    s = _stream(gpu)
    fwb = int(lib.mt_flce_forward_workspace_bytes(T, n, H, V, _lib.MT_DTYPE_BF16))
    fws = torch.empty(fwb, dtype=torch.uint8, device=gpu)
    loss0, lse0 = torch.empty(T, device=gpu), torch.empty(n, device=gpu)
    _lib.check(lib.mt_flce_forward(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0, _p(ri),
                                   _p(rl), n, _p(loss0), _p(lse0), _p(fws), fwb, s), "forward")
    rows = (n + 255) // 256 * 256
    keep = torch.full((rows, K), float("nan"), dtype=torch.bfloat16, device=gpu)
    guard = torch.full((1,), 7, dtype=torch.int32, device=gpu)
    loss1, lse1 = torch.empty(T, device=gpu), torch.empty(n, device=gpu)
    _lib.check(lib.mt_flce_forward_keep(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                        _p(ri), _p(rl), n, _p(loss1), _p(lse1), _p(fws), fwb,
                                        _p(keep), K, keep.numel() * 2, _p(guard), s),
               "forward_keep")
    torch.cuda.synchronize()
    assert torch.equal(loss0, loss1) and torch.equal(lse0, lse1)
    assert int(guard.item()) == (1 if shift else 0)
    if not shift:
        z = (X[ri[:n].long()] @ W[:K].T).float()  # bf16 logits, as F.linear gives them
        want = torch.exp(z)
        got = keep[:n].float()
        assert ((got - want).abs() <= want * 2e-2 + 1e-30).all()


def test_fused_tiles_all_masked_and_narrow_phases(gpu):
    """No valid row: the tiles hold zeros (written over garbage).  In-place
    narrowing over 9 tile rows (launches {0}, {1}, [2, 4), [4, 8), {8}) of a
    random tile buffer: every row equals torch's scaled rounding of the
    unscrambled tiles, those whose bytes the bf16 rows reuse included."""
    lib = _lib.load()
    T, H, V = 64, 320, 2100
    X = torch.randn(T, H, device=gpu).to(torch.bfloat16)
    W = torch.randn(V, H, device=gpu).to(torch.bfloat16)
    y = torch.full((T,), -100, device=gpu)
    ri, rl, n = prepare_targets(y, V)
    assert n == 0
    dW = _tiled_buffers(V, H, gpu)
    assert dW[2] > 0  # tile rows in both buffers
    loss = torch.empty(T, device=gpu)
    dX = torch.empty(T, H, dtype=torch.bfloat16, device=gpu)
    _lib.check(lib.mt_flce_fused_tiles(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                       _p(ri), _p(rl), 0, None, 0, _p(loss), None, _p(dX), H,
                                       *_targs(dW[0], dW[1]), 0, 0, None, 0, _stream(gpu)),
               "all masked")
    torch.cuda.synchronize()
    assert torch.count_nonzero(_untile(dW, V, H)) == 0 and torch.count_nonzero(dX) == 0
    assert torch.equal(loss, torch.zeros(T, device=gpu))
    g = torch.Generator(device=gpu).manual_seed(2)
    lo, hi, rows = dW
    lo.view(torch.float32).copy_(torch.randn(lo.numel() // 2, device=gpu, generator=g).view(V, H // 2))
    hi.copy_(torch.randn(hi.numel(), device=gpu, generator=g))
    scale = torch.tensor([-2.5], device=gpu)
    want = (_untile(dW, V, H) * scale).to(torch.bfloat16)
    _lib.check(lib.mt_flce_narrow_tiles(_p(scale), *_targs(lo, hi), V, H, _stream(gpu)),
               "narrow in place")
    torch.cuda.synchronize()
    assert torch.equal(lo, want)


def test_reference_chain_extra_memory(gpu):
    """The reference chain on the fused kernels allocates, beyond its inputs
    and required outputs (loss, dX, the fp32 dW tiles -- half a tile row and
    the tile grid's padding more than V x H fp32), only the fused workspace;
    W.grad afterwards owns exactly V x H bf16 (the tiles' second buffer is
    gone)."""
    T, H, V = 4096, 512, 32000
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=51)
    n = int((y != -100).sum())
    C, ws, _ = fused_plan(T, n, H, V)
    Xd, Wd, yd = X.to(gpu).requires_grad_(True), W.to(gpu).requires_grad_(True), y.to(gpu)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(gpu)
    base = torch.cuda.memory_allocated(gpu)
    out = drop_in(Xd, Wd, yd)
    assert path_of(out) == "fused_unit"
    (out.float().sum() / n).backward()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(gpu)
    outputs = T * 4 + T * H * 2 + V * H * 4
    assert peak - base - outputs <= ws + (4 << 20), (peak - base - outputs, ws)
    assert Wd.grad.dtype == torch.bfloat16 and Wd.grad.is_contiguous()
    assert Wd.grad.untyped_storage().nbytes() == V * H * 2
    live = torch.cuda.memory_allocated(gpu) - base
    assert live <= T * 4 + 2 * T * H * 2 + V * H * 2 + (1 << 20), live  # loss, dX, X.grad, W.grad


def test_segment_sums_of_shifted_labels(gpu):
    """mt_segment_sum with shift counts position t when labels[t + 1] is
    valid; against the C restatement over the shifted target."""
    rng = np.random.default_rng(4)
    lengths = [5, 40, 1, 77, 5, 20]  # the 5-token samples are dummies
    T = sum(lengths)
    labels = rng.integers(0, 50, T).astype(np.int64)
    labels[rng.random(T) < 0.3] = -100
    labels[:5] = -100
    labels[123:128] = -100
    loss = rng.random(T).astype(np.float32)
    shifted = np.concatenate([labels[1:], [-100]])
    loss[shifted == -100] = 0.0
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    want_l, want_c, st = ref.segment_sum(loss, shifted, cu)
    assert st == 0
    sl, sc = per_sample_loss_sums(torch.from_numpy(loss).to(gpu), torch.from_numpy(labels).to(gpu),
                                  torch.from_numpy(cu).to(gpu), shift=True)
    assert np.array_equal(sc.cpu().numpy(), want_c)
    assert np.allclose(sl.cpu().numpy(), want_l, rtol=1e-6, atol=0)


@pytest.mark.parametrize("split", ["0", "1"])
def test_profile_hook_reports_the_fused_step(gpu, monkeypatch, split):
    """The per-launch events of the reference step: dX and dW in one launch
    (the phase), or (split = 1, the measurement hook) as two kernels inside
    the phase, each with its own event."""
    monkeypatch.setenv("MT_FLCE_SPLIT_PHASE", split)
    X, W, y = make_case(700, 128, 2560, torch.bfloat16, seed=41)
    n = int((y != -100).sum())
    profile_enable(True)
    try:
        path, *_ = train_py_chain(gpu, X, W, y, 1, n)
    finally:
        profile_enable(False)
    rep = profile_report()
    assert path == "fused_unit"
    # (3 dX tiles: the fused dX is split over the vocabulary)
    gemms = ("dx_bf16_kernel<split>", "dw_bf16_kernel") if split == "1" else ()
    for k in ("fwd_bf16_kernel<store_e>", "dx_dw_phase", "scale_rows_kernel<dX>",
              "narrow_tiles_kernel<dW>") + gemms:
        assert k in rep and rep[k]["launches"] >= 1 and rep[k]["ms_total"] > 0, k
    if split == "0":
        assert not any(k.startswith(("dx_bf16_kernel", "dw_bf16_kernel")) for k in rep)
    # algorithmic work: 2 H V n for each GEMM over all chunks, their sum for the phase
    f = 2.0 * 128 * 2560 * n
    for k in ("fwd_bf16_kernel<store_e>",) + gemms:
        assert rep[k]["flops"] == pytest.approx(f, rel=1e-9)
    assert rep["dx_dw_phase"]["flops"] == pytest.approx(2 * f, rel=1e-9)
    if split == "1":
        assert rep["dx_dw_phase"]["ms_total"] >= rep["dw_bf16_kernel"]["ms_total"] * 0.5
    # the report released its records; a disabled hook records nothing
    assert profile_report() == {}
    train_py_chain(gpu, X, W, y, 1, n)
    assert profile_report() == {}
    # a too-small buffer is an error that names the size it needs and keeps
    # the records for the retry
    profile_enable(True)
    try:
        train_py_chain(gpu, X, W, y, 1, n)
    finally:
        profile_enable(False)
    lib = _lib.load()
    need = ctypes.c_size_t(0)
    assert lib.mt_flce_profile_report(None, 0, ctypes.byref(need)) == 1 and need.value > 100
    assert "dx_dw_phase" in profile_report()


@pytest.mark.parametrize("kernel", ["dx_dw_bf16_kernel", "narrow_tiles_kernel",
                                    "recompute_kernel"])
def test_injected_launch_failure_raises_and_recovers(gpu, monkeypatch, kernel):
    """A launch reported failed (the test hook MT_FLCE_TEST_FAIL_LAUNCH; the
    kernel itself runs) surfaces from the reference chain as FlceError, a
    RuntimeError naming the kernel: in the fused forward (dx_dw), in the
    backward's narrowing, or in the general path's backward (recompute).
    Without the hook the next call on the same device runs and matches the
    torch path."""
    print(f"case injected failure {kernel}", flush=True)
    X, W, y = make_case(700, 128, 2560, torch.bfloat16, seed=43)
    n = int((y != -100).sum())
    monkeypatch.setenv(FUSED_ENV, "0" if kernel == "recompute_kernel" else "1")
    monkeypatch.setenv("MT_FLCE_TEST_FAIL_LAUNCH", kernel)
    with pytest.raises(_lib.FlceError, match=f"{kernel}: injected launch failure"):
        train_py_chain(gpu, X, W, y, 1, n)
    torch.cuda.synchronize()
    monkeypatch.delenv("MT_FLCE_TEST_FAIL_LAUNCH")
    path, loss, dX, dW = train_py_chain(gpu, X, W, y, 1, n)
    assert path == ("general" if kernel == "recompute_kernel" else "fused_unit")
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((700,), 1.0 / n))
