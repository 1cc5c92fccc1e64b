"""Memory safety of every entry point: each output, workspace and status
word sits between 64 KiB guard regions filled with a canary byte, and dX / dW
have row pitches wider than H whose padding columns hold the canary too.
The shapes are the tail cases -- T not a multiple of the 256-row tile, V not
a multiple of 256 (partial last vocabulary tile), H not a multiple of the
64-element K stage (partial last K stage), an uneven last fused chunk and
256 x 256 general-path blocks -- on the general and fused paths.  After each
call every guard byte and padding column must be intact, and the results
finite where defined."""
from __future__ import annotations

import pytest
import torch

from mini_trainer_amd import _lib, prepare_targets
from mini_trainer_amd.flce import _p, _stream, backward_plan, fused_plan

pytestmark = pytest.mark.gpu

CANARY = 0xA5
GUARD = 1 << 16


class Guarded:
    """nbytes of device memory between two GUARD-byte canary regions."""

    def __init__(self, dev, nbytes):
        self.n = int(nbytes)
        span = (self.n + 255) // 256 * 256
        self.buf = torch.full((GUARD + span + GUARD,), CANARY, dtype=torch.uint8, device=dev)

    @property
    def ptr(self):
        return self.buf.data_ptr() + GUARD

    def view(self, dtype, shape):
        return self.buf[GUARD:GUARD + self.n].view(dtype).view(shape)

    def intact(self):
        return bool((self.buf[:GUARD] == CANARY).all()) and bool((self.buf[GUARD + self.n:] == CANARY).all())


def matrix(dev, rows, cols, pitch, dtype):
    """A guarded [rows, pitch] matrix of which columns [0, cols) are used."""
    es = torch.finfo(dtype).bits // 8
    g = Guarded(dev, rows * pitch * es)
    return g, g.view(dtype, (rows, pitch))


def pad_intact(m, cols):
    pad = m[:, cols:].contiguous().view(torch.uint8)
    return bool((pad == CANARY).all())


T, H, V = 700, 200, 1300


@pytest.fixture
def case(gpu):
    g = torch.Generator(device=gpu).manual_seed(77)
    X = torch.randn(T, H, device=gpu, generator=g).to(torch.bfloat16)
    W = (torch.randn(V, H, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    y = torch.randint(0, V, (T,), device=gpu, generator=g)
    y[torch.rand(T, device=gpu, generator=g) < 0.3] = -100
    ri, rl, n = prepare_targets(y, V)
    return X, W, y, ri, rl, n


def test_prepare_and_forward_guards(gpu, case):
    X, W, y, _, _, _ = case
    lib = _lib.load()
    s = _stream(gpu)
    ri, rl, cnt = Guarded(gpu, T * 4), Guarded(gpu, T * 4), Guarded(gpu, 16)
    _lib.check(lib.mt_flce_prepare(_p(y), T, V, -100, 1, ri.ptr, rl.ptr, cnt.ptr, s), "prepare")
    torch.cuda.synchronize()
    assert ri.intact() and rl.intact() and cnt.intact()
    n = int(cnt.view(torch.int32, (4,))[0])
    wsb = lib.mt_flce_forward_workspace_bytes(T, n, H, V, _lib.MT_DTYPE_BF16)
    loss, lse, ws = Guarded(gpu, T * 4), Guarded(gpu, n * 4), Guarded(gpu, wsb)
    _lib.check(lib.mt_flce_forward(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0, ri.ptr,
                                   rl.ptr, n, loss.ptr, lse.ptr, ws.ptr, wsb, s), "forward")
    torch.cuda.synchronize()
    assert loss.intact() and lse.intact() and ws.intact()
    assert bool(torch.isfinite(loss.view(torch.float32, (T,))).all())
    loss2, lse2 = Guarded(gpu, T * 4), Guarded(gpu, n * 4)
    _lib.check(lib.mt_flce_forward_noalloc(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                           ri.ptr, rl.ptr, n, loss2.ptr, lse2.ptr, s), "noalloc")
    torch.cuda.synchronize()
    assert loss2.intact() and lse2.intact()
    assert torch.equal(loss.view(torch.float32, (T,)), loss2.view(torch.float32, (T,)))


@pytest.mark.parametrize("softcap", [0.0, 3.0])
def test_general_backward_guards(gpu, case, monkeypatch, softcap):
    X, W, y, ri, rl, n = case
    lib = _lib.load()
    s = _stream(gpu)
    wsb = lib.mt_flce_forward_workspace_bytes(T, n, H, V, _lib.MT_DTYPE_BF16)
    loss = torch.empty(T, device=gpu)
    lse = torch.empty(n, device=gpu)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    _lib.check(lib.mt_flce_forward(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, softcap,
                                   _p(ri), _p(rl), n, _p(loss), _p(lse), _p(ws), wsb, s), "forward")
    C, Cv, bws = backward_plan(T, n, H, V, torch.bfloat16, budget_bytes=1)  # 256 x 256 blocks
    assert (C, Cv) == (256, 256)
    grad = torch.rand(T, device=gpu)
    gdx, dX = matrix(gpu, T, H, H + 8, torch.bfloat16)
    gdw, dW = matrix(gpu, V, H, H + 4, torch.float32)
    gws = Guarded(gpu, bws)
    _lib.check(lib.mt_flce_backward(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, softcap,
                                    _p(ri), _p(rl), n, _p(lse), _p(grad), 1, gdx.ptr, H + 8,
                                    gdw.ptr, H + 4, 0, C, Cv, gws.ptr, bws, s), "backward")
    torch.cuda.synchronize()
    assert gdx.intact() and gdw.intact() and gws.intact()
    assert pad_intact(dX, H) and pad_intact(dW, H)
    assert bool(torch.isfinite(dX[:, :H].float()).all()) and bool(torch.isfinite(dW[:, :H]).all())


def test_backward_narrow_guards(gpu, case):
    """mt_flce_backward_narrow: one row block and several vocabulary blocks
    (dX's fp32 accumulator and X^T in the scratch buffer, dW written as bf16
    rows into a buffer of exactly V x H bf16), with exactly the workspace
    mt_flce_backward_narrow_plan and the scratch mt_flce_narrow_scratch_bytes
    report for that blocking."""
    X, W, y, ri, rl, n = case
    lib = _lib.load()
    s = _stream(gpu)
    wsb = lib.mt_flce_forward_workspace_bytes(T, n, H, V, _lib.MT_DTYPE_BF16)
    loss = torch.empty(T, device=gpu)
    lse = torch.empty(n, device=gpu)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    _lib.check(lib.mt_flce_forward(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                   _p(ri), _p(rl), n, _p(loss), _p(lse), _p(ws), wsb, s), "forward")
    C, Cv = 512, 512  # n < 512 rows; 1300 vocabulary entries in 3 blocks
    assert n <= C < V
    budget = C * Cv * 2 + H * C * 2 + 4096
    pc, pcv, bws = backward_plan(T, n, H, V, torch.bfloat16, budget_bytes=budget, narrow=True)
    assert (pc, pcv) == (C, Cv)
    assert bws < C * Cv * 2 + H * C * 2  # no accumulator or X^T in the workspace
    grad = torch.rand(T, device=gpu)
    gdx, dX = matrix(gpu, T, H, H + 8, torch.bfloat16)
    sb = int(lib.mt_flce_narrow_scratch_bytes(V, H, C))
    assert sb > 0
    gdw = Guarded(gpu, V * H * 2)
    gsc = Guarded(gpu, sb)
    gws = Guarded(gpu, bws)
    _lib.check(lib.mt_flce_backward_narrow(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0,
                                           _p(ri), _p(rl), n, _p(lse), _p(grad), 1, gdx.ptr,
                                           H + 8, gdw.ptr, V * H * 2, gsc.ptr, sb, C, Cv, gws.ptr,
                                           bws, None, s), "backward_narrow")
    torch.cuda.synchronize()
    assert gdx.intact() and gdw.intact() and gws.intact() and gsc.intact()
    assert pad_intact(dX, H)
    assert bool(torch.isfinite(dX[:, :H].float()).all())
    assert bool(torch.isfinite(gdw.view(torch.bfloat16, (V * H,)).float()).all())


def test_fused_and_rescale_guards(gpu, case):
    X, W, y, ri, rl, n = case
    lib = _lib.load()
    s = _stream(gpu)
    C, fws, _ = fused_plan(T, n, H, V, budget_bytes=1)  # 256-row chunks, uneven last one
    assert C == 256 and n % 256 != 0
    one = torch.ones(1, device=gpu)
    loss, lse = Guarded(gpu, T * 4), Guarded(gpu, n * 4)
    gdx, dX = matrix(gpu, T, H, H + 8, torch.bfloat16)
    gdw, dW = matrix(gpu, V, H, H + 4, torch.float32)
    gws = Guarded(gpu, fws)
    _lib.check(lib.mt_flce_fused(_p(X), _p(W), T, H, V, H, H, _lib.MT_DTYPE_BF16, 0.0, _p(ri),
                                 _p(rl), n, _p(one), 0, loss.ptr, lse.ptr, gdx.ptr, H + 8,
                                 gdw.ptr, H + 4, 0, C, gws.ptr, fws, s), "fused")
    torch.cuda.synchronize()
    assert loss.intact() and lse.intact() and gdx.intact() and gdw.intact() and gws.intact()
    assert pad_intact(dX, H) and pad_intact(dW, H)
    # rescale in place: dX scaled, dW narrowed to bf16 inside its own rows
    scale = torch.tensor([0.5], device=gpu)
    _lib.check(lib.mt_flce_scale_grads(_p(scale), gdx.ptr, T, H, H + 8, _lib.MT_DTYPE_BF16,
                                       gdw.ptr, V, H + 4, gdw.ptr, H + 4, _lib.MT_DTYPE_BF16, s),
               "scale")
    torch.cuda.synchronize()
    assert gdx.intact() and gdw.intact() and pad_intact(dX, H)


def test_segment_sum_and_materialised_ce_guards(gpu, case):
    X, W, y, _, _, _ = case
    lib = _lib.load()
    s = _stream(gpu)
    loss = torch.rand(T, device=gpu)
    cu = torch.tensor([0, 5, 300, 301, 699, T], dtype=torch.int32, device=gpu)
    sl, sc, st = Guarded(gpu, 5 * 4), Guarded(gpu, 5 * 4), Guarded(gpu, 4)
    _lib.check(lib.mt_segment_sum(_p(loss), _p(y), T, -100, 1, _p(cu), 5, sl.ptr, sc.ptr, st.ptr,
                                  s), "segment_sum")
    torch.cuda.synchronize()
    assert sl.intact() and sc.intact() and st.intact()
    logits = (X.float() @ W.float().t()).to(torch.bfloat16)  # [T, V], V % 8 != 0 rows
    ls, lse, st2 = Guarded(gpu, T * 4), Guarded(gpu, T * 4), Guarded(gpu, 4)
    _lib.check(lib.mt_ce_forward(_p(logits), T, V, V, _lib.MT_DTYPE_BF16, _p(y), -100, ls.ptr,
                                 lse.ptr, st2.ptr, s), "ce_forward")
    g = torch.rand(T, device=gpu)
    gd, dl = matrix(gpu, T, V, V + 4, torch.bfloat16)
    _lib.check(lib.mt_ce_backward(_p(logits), T, V, V, _lib.MT_DTYPE_BF16, _p(y), -100, lse.ptr,
                                  _p(g), 1, gd.ptr, V + 4, s), "ce_backward")
    torch.cuda.synchronize()
    assert ls.intact() and lse.intact() and st2.intact() and gd.intact() and pad_intact(dl, V)
