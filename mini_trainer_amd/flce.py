"""Host side of the fused LM-head linear + per-token cross-entropy.

Mirrors the reference's loss boundary (none_reduction_losses.py:5-36): the
functions here take PyTorch tensors on a ROCm device, hand raw pointers and
the current HIP stream to libmt_flce.so (include/mt_flce.h) and return
PyTorch tensors.  There is no CPU or eager-PyTorch fallback: non-device
tensors or a missing library raise.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import MT_DTYPE_BF16, MT_DTYPE_F32, check, load

__all__ = [
    "fused_linear_cross_entropy",
    "path_of",
    "profile_enable",
    "profile_report",
    "cross_entropy_none",
    "prepare_targets",
    "per_sample_loss_sums",
    "backward_plan",
    "fused_plan",
    "BACKWARD_BUDGET_ENV",
    "FUSED_ENV",
]

# Optional override of the backward workspace budget in bytes (default: 5% of
# the materialised-logits size T * V * sizeof(dtype)).
BACKWARD_BUDGET_ENV = "MT_FLCE_BWD_BUDGET_BYTES"
# With grad_scale given (bf16): "auto" (default) takes the fused path when the
# planner expects it to pay, "1" always, "0" never.
FUSED_ENV = "MT_FLCE_FUSED"


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return MT_DTYPE_BF16
    if dt == torch.float32:
        return MT_DTYPE_F32
    raise TypeError(f"fused linear cross-entropy supports bfloat16 and float32, got {dt}")


def _p(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_device(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{name} must be a ROCm device tensor; the fused linear cross-entropy has no CPU path"
        )


def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    """2-D view with unit stride along the last dim and a 16-byte row pitch."""
    t2 = t.reshape(-1, t.shape[-1])
    es = t2.element_size()
    if (t2.stride(1) != 1 or (t2.stride(0) * es) % 16 != 0 or t2.data_ptr() % 16 != 0
            or t2.stride(0) < t2.shape[1]):
        t2 = t2.contiguous()
    return t2


def prepare_targets(target: torch.Tensor, vocab_size: int, ignore_index: int = -100,
                    shift: bool = False) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """Valid-row compaction (mt_flce_prepare) plus the one host sync of a call.

    Returns (row_index int32 [T], row_label int32 [T], n_valid).  row_index
    lists the valid positions first (ascending), then every ignored one.
    Raises IndexError, like F.cross_entropy, for a target outside
    [0, vocab_size) that is not ignore_index.
    """
    _require_device("target", target)
    lib = load()
    tgt = target.reshape(-1)
    if tgt.dtype != torch.int64:
        tgt = tgt.to(torch.int64)
    tgt = tgt.contiguous()
    T = tgt.numel()
    dev = tgt.device
    row_index = torch.empty(T, dtype=torch.int32, device=dev)
    row_label = torch.empty(T, dtype=torch.int32, device=dev)
    counts = torch.empty(4, dtype=torch.int32, device=dev)
    check(lib.mt_flce_prepare(_p(tgt), T, int(vocab_size), int(ignore_index), int(bool(shift)),
                              _p(row_index), _p(row_label), _p(counts), _stream(dev)),
          "mt_flce_prepare")
    c = counts.cpu().tolist()
    if c[1] > 0:
        pos = c[2]
        src = pos + 1 if shift else pos
        bad = int(tgt[src].item())
        raise IndexError(f"Target {bad} is out of bounds (vocabulary size {vocab_size}, "
                         f"position {pos}, {c[1]} such targets).")
    return row_index, row_label, int(c[0])


def backward_plan(T: int, n_valid: int, H: int, V: int, dtype: torch.dtype,
                  budget_bytes: Optional[int] = None, narrow: bool = False) -> Tuple[int, int, int]:
    """(chunk_rows, chunk_vocab, workspace_bytes) of the backward blocking;
    narrow: the plan of a bf16 backward whose weight gradient is wanted in
    bf16 and added into nothing (mt_flce_backward_narrow_plan: chunk_rows >=
    n_valid means one row block through mt_flce_backward_narrow), else of
    mt_flce_backward."""
    lib = load()
    if budget_bytes is None:
        budget_bytes = int(os.environ.get(BACKWARD_BUDGET_ENV, "0"))
    c, cv, ws = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_size_t()
    fn = "mt_flce_backward_narrow_plan" if narrow else "mt_flce_backward_plan"
    check(getattr(lib, fn)(T, n_valid, H, V, _dtype_code(dtype), budget_bytes, ctypes.byref(c),
                           ctypes.byref(cv), ctypes.byref(ws)), fn)
    return c.value, cv.value, ws.value


def _default_budget(T: int, V: int, es: int) -> int:
    """The workspace budget the planners use when given 0: the override in
    MT_FLCE_BWD_BUDGET_BYTES, else 5% of the T x V logits in bytes."""
    env = int(os.environ.get(BACKWARD_BUDGET_ENV, "0"))
    return env if env > 0 else int(float(T) * V * es * 0.05)


def _grad_vector(grad: torch.Tensor, T: int) -> Tuple[torch.Tensor, int]:
    g = grad.reshape(-1) if grad.dim() != 1 else grad
    if g.dtype != torch.float32:
        g = g.float()
    if g.numel() == 1:
        return g, 0
    if g.stride(0) == 0:  # a scalar expanded over the tokens (sum().backward())
        return g, 0
    if g.stride(0) != 1:
        g = g.contiguous()
    if g.numel() != T:
        raise ValueError(f"grad of the loss has {g.numel()} elements, expected {T}")
    return g, 1


def _check_inputs(hidden, weight, target):
    _require_device("hidden_states", hidden)
    _require_device("lm_head_weight", weight)
    if weight.dim() != 2:
        raise ValueError(f"lm_head_weight must be [V, H], got {tuple(weight.shape)}")
    if hidden.dtype != weight.dtype:
        raise TypeError(f"hidden_states ({hidden.dtype}) and lm_head_weight ({weight.dtype}) "
                        "must have the same dtype")
    dt = _dtype_code(hidden.dtype)
    V, H = weight.shape
    if hidden.shape[-1] != H:
        raise ValueError(f"hidden size mismatch: hidden_states {tuple(hidden.shape)}, "
                         f"lm_head_weight {tuple(weight.shape)}")
    X = _rows(hidden, "hidden_states")
    W = _rows(weight, "lm_head_weight")
    T = X.shape[0]
    if target.numel() != T:
        raise ValueError(f"target has {target.numel()} elements, expected {T}")
    return X, W, T, H, V, dt


class _TiledDw:
    """The tiled fp32 weight gradient of mt_flce_fused_tiles /
    mt_flce_backward_tiles in the two buffers of mt_flce_dw_tiles_layout:
    `lo` is the bf16 [V, H] tensor the gradient is narrowed into in place
    (it holds the first tile rows until then), `hi` the other tile rows,
    dropped once narrowed -- so the weight gradient handed to autograd owns
    exactly V * H * 2 bytes."""

    def __init__(self, V: int, H: int, device: torch.device):
        lib = load()
        lo_b, rows, hi_b = ctypes.c_size_t(), ctypes.c_int64(), ctypes.c_size_t()
        check(lib.mt_flce_dw_tiles_layout(V, H, ctypes.byref(lo_b), ctypes.byref(rows),
                                          ctypes.byref(hi_b)), "mt_flce_dw_tiles_layout")
        self.V, self.H = V, H
        self.lo = torch.empty((V, H), dtype=torch.bfloat16, device=device)
        self.hi = torch.empty(hi_b.value // 4, dtype=torch.float32, device=device)

    def args(self) -> tuple:
        """(lo, lo bytes, hi, hi bytes) as the C ABI takes them."""
        return (_p(self.lo), self.lo.numel() * 2, _p(self.hi), self.hi.numel() * 4)

    def narrow(self, scale: torch.Tensor) -> torch.Tensor:
        """scale * the gradient in bf16, in place in `lo` (mt_flce_narrow_tiles);
        `hi` is released (the caching allocator reuses it only after the
        narrowing, on the same stream)."""
        check(load().mt_flce_narrow_tiles(_p(scale), *self.args(), self.V, self.H,
                                          _stream(self.lo.device)), "mt_flce_narrow_tiles")
        self.hi = None
        return self.lo


class _FusedLinearCrossEntropyNone(torch.autograd.Function):
    """Per-token loss; three paths over the same arithmetic (ctx.path).

    general     forward keeps lse (mt_flce_forward); the backward recomputes
                the logits for whatever upstream gradient arrives
                (mt_flce_backward; bf16 without dw_accumulator: one row
                block through mt_flce_backward_narrow, dW written in bf16 by
                its GEMM -- the forward then also keeps the first vocabulary
                block's exponentials for it, mt_flce_forward_keep, softcap
                off -- else mt_flce_backward_tiles, dW as 256 x 256 fp32
                tiles narrowed by mt_flce_narrow_tiles).
    fused       grad_scale promised the upstream gradient at the forward and
                the planner expects the fused path to pay (bf16,
                mt_flce_fused_plan): the forward also forms dX and dW for it
                (mt_flce_fused into dw_accumulator, else mt_flce_fused_tiles:
                dW as 256 x 256 fp32 tiles); the backward checks the gradient
                it receives against the promise and hands the stored
                gradients to autograd (tiles narrowed by mt_flce_narrow_tiles).
    fused_unit  no promise, no dw_accumulator, bf16, the planner expects the
                fused path to pay: the forward forms dX and dW for a unit
                upstream gradient -- the structure of the reference's fused
                loss (none_reduction_losses.py:16-23 -> Liger's
                fused_linear_cross_entropy_forward), which train.py:97-104
                drives unchanged (mt_flce_fused_tiles).  The backward
                multiplies them by the upstream gradient when it is one scalar
                for every token (stride 0, what sum() / mean() and train.py's
                scaling give; mt_flce_scale_grads for dX and
                mt_flce_narrow_tiles for dW read it on the device), and
                otherwise recomputes with the saved lse (the general path's
                bf16 backward into the same weight-gradient buffers), exact
                for any per-token gradient.

    `ranges` (row ranges [t0, t1) of X, each within one buffer's reach, in
    order) splits a large call: every range is compacted, run and (in the
    backward) recomputed on its own, into one dX and one weight gradient --
    dW of a later range adds into the tiles (or dw_accumulator) the earlier
    ones filled, so one weight-sized buffer serves the whole call.
    """

    @staticmethod
    def forward(ctx, hidden, weight, target, ignore_index, softcap, shift, dw_accumulator,
                grad_scale, allow_unit, ranges):
        X, W, T, H, V, dt = _check_inputs(hidden, weight, target)
        lib = load()
        dev = X.device
        tgt = target.reshape(-1)
        if ranges is None:
            ranges = [(0, T)]
        parts = []  # (t0, t1, row_index, row_label, n) per range
        for t0, t1 in ranges:
            ri, rl, n = prepare_targets(tgt[t0:t1], V, ignore_index, shift)
            parts.append((t0, t1, ri, rl, n))
        n_tot = sum(p[4] for p in parts)
        loss = torch.empty(T, dtype=torch.float32, device=dev)
        ctx.path = "general"
        ctx.ranges = [(p[0], p[1], p[4]) for p in parts]
        plans = None
        if dt == MT_DTYPE_BF16 and n_tot > 0 and (grad_scale is not None or allow_unit):
            plans = [fused_plan(t1 - t0, n, H, V, accumulator=dw_accumulator is not None)
                     if n > 0 else (0, 0, True) for t0, t1, _, _, n in parts]
            live = [pl for pl, p in zip(plans, parts) if p[4] > 0]
            # C = 0: the fused path cannot run that shape
            if all(pl[0] > 0 for pl in live) and _use_fused(all(pl[2] for pl in live)):
                ctx.path = "fused" if grad_scale is not None else "fused_unit"
        ctx.dw_accumulator = dw_accumulator
        ctx.meta = (float(softcap), hidden.shape, dt)
        lses = []
        if ctx.path != "general":
            if ctx.path == "fused":
                g, gstride = _promised_grad(grad_scale, T, dev)
            else:
                g, gstride = torch.ones(1, dtype=torch.float32, device=dev), 0
            dX = torch.empty((T, H), dtype=X.dtype, device=dev)
            dW = dw_accumulator if dw_accumulator is not None else _TiledDw(V, H, dev)
            for r, ((t0, t1, ri, rl, n), (C, ws_bytes, _)) in enumerate(zip(parts, plans)):
                ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
                lse = torch.empty(n, dtype=torch.float32, device=dev)
                Xr, gr = X[t0:t1], (g[t0:t1] if gstride else g)
                dXr, lr = dX[t0:t1], loss[t0:t1]
                if dw_accumulator is not None:
                    check(lib.mt_flce_fused(_p(Xr), _p(W), t1 - t0, H, V, X.stride(0),
                                            W.stride(0), dt, float(softcap), _p(ri), _p(rl), n,
                                            _p(gr), gstride, _p(lr), _p(lse), _p(dXr),
                                            dX.stride(0), _p(dW), dW.stride(0), 1, C, _p(ws),
                                            ws_bytes, _stream(dev)), "mt_flce_fused")
                else:
                    # dW as 256 x 256 tiles in the weight gradient's own bf16
                    # buffer and a second one, narrowed into the first later
                    check(lib.mt_flce_fused_tiles(_p(Xr), _p(W), t1 - t0, H, V, X.stride(0),
                                                  W.stride(0), dt, float(softcap), _p(ri), _p(rl),
                                                  n, _p(gr), gstride, _p(lr), _p(lse), _p(dXr),
                                                  dX.stride(0), *dW.args(), int(r > 0), C,
                                                  _p(ws), ws_bytes, _stream(dev)),
                          "mt_flce_fused_tiles")
                del ws
                lses.append(lse)
            if ctx.path == "fused":
                ctx.save_for_backward(g, *[p[2] for p in parts])
                ctx.gstride = gstride
            else:  # kept for the recompute fallback of a per-token gradient
                ctx.save_for_backward(X, W, *[t for p, lse in zip(parts, lses)
                                              for t in (p[2], p[3], lse)])
            ctx.w_shape = (V, H)
            ctx.dX = dX
            ctx.dW = None if dw_accumulator is not None else dW
            ctx.fused_consumed = False
            return loss.view(hidden.shape[:-1])
        ctx.keep = None
        for t0, t1, ri, rl, n in parts:
            lse = torch.empty(n, dtype=torch.float32, device=dev)
            lses.append(lse)
            Xr, lr = X[t0:t1], loss[t0:t1]
            plan = None
            ws_bytes = lib.mt_flce_forward_workspace_bytes(t1 - t0, n, H, V, dt)
            if (dt == MT_DTYPE_BF16 and allow_unit and float(softcap) == 0.0 and n > 0
                    and len(parts) == 1):
                # the kept block sits beside the forward's own workspace: plan
                # it under what the budget leaves of that
                left = _default_budget(T, V, 2) - ws_bytes
                if left > 0:
                    plan = backward_plan(T, n, H, V, X.dtype, budget_bytes=left, narrow=True)
            if plan is not None and plan[0] >= n and plan[1] < V:
                # one row block in the backward: the forward keeps the first
                # vocabulary block's exponentials in that backward's G block,
                # which lives from here to the backward (or until the loss's
                # graph is freed, when no backward follows)
                C, Cv, bws_bytes = plan
                bws = torch.empty(bws_bytes, dtype=torch.uint8, device=dev)
                guard = torch.empty(1, dtype=torch.int32, device=dev)
                ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
                check(lib.mt_flce_forward_keep(_p(Xr), _p(W), t1 - t0, H, V, X.stride(0),
                                               W.stride(0), dt, 0.0, _p(ri), _p(rl), n, _p(lr),
                                               _p(lse), _p(ws), ws_bytes, _p(bws), Cv, bws_bytes,
                                               _p(guard), _stream(dev)), "mt_flce_forward_keep")
                ctx.keep = (C, Cv, bws, guard)
            else:
                ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
                check(lib.mt_flce_forward(_p(Xr), _p(W), t1 - t0, H, V, X.stride(0), W.stride(0),
                                          dt, float(softcap), _p(ri), _p(rl), n, _p(lr), _p(lse),
                                          _p(ws), ws_bytes, _stream(dev)), "mt_flce_forward")
            del ws
        ctx.save_for_backward(X, W, *[t for p, lse in zip(parts, lses) for t in (p[2], p[3], lse)])
        return loss.view(hidden.shape[:-1])

    @staticmethod
    def _range_tensors(ctx):
        """X, W and [(t0, t1, n, row_index, row_label, lse)] per range."""
        saved = ctx.saved_tensors
        X, W, rest = saved[0], saved[1], saved[2:]
        out = []
        for i, (t0, t1, n) in enumerate(ctx.ranges):
            out.append((t0, t1, n, rest[3 * i], rest[3 * i + 1], rest[3 * i + 2]))
        return X, W, out

    @staticmethod
    def backward(ctx, grad_loss):
        if ctx.path == "fused":
            return _FusedLinearCrossEntropyNone._backward_fused(ctx, grad_loss)
        if ctx.path == "fused_unit":
            return _FusedLinearCrossEntropyNone._backward_fused_unit(ctx, grad_loss)
        X, W, rngs = _FusedLinearCrossEntropyNone._range_tensors(ctx)
        softcap, hshape, dt = ctx.meta
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        acc = ctx.dw_accumulator
        none = (None,) * 8
        if not need_x and not need_w and acc is None:
            return (None, None) + none
        lib = load()
        T, H = X.shape
        V = W.shape[0]
        dev = X.device
        g, gstride = _grad_vector(grad_loss, T)
        dX = torch.empty((T, H), dtype=X.dtype, device=dev)
        if acc is None and dt == MT_DTYPE_BF16:
            # dW in bf16; the first backward takes the exponentials its
            # forward kept
            keep, ctx.keep = getattr(ctx, "keep", None), None
            grad_w = _backward_bf16_weight(lib, X, W, rngs, g, gstride, softcap, dX, keep=keep)
            grad_w = grad_w if need_w else None
        else:
            dW = acc if acc is not None else torch.empty((V, H), dtype=torch.float32, device=dev)
            for r, (t0, t1, n, ri, rl, lse) in enumerate(rngs):
                C, Cv, ws_bytes = backward_plan(t1 - t0, n, H, V, X.dtype)
                ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
                gr = g[t0:t1] if gstride else g
                check(lib.mt_flce_backward(_p(X[t0:t1]), _p(W), t1 - t0, H, V, X.stride(0),
                                           W.stride(0), dt, softcap, _p(ri), _p(rl), n, _p(lse),
                                           _p(gr), gstride, _p(dX[t0:t1]), dX.stride(0), _p(dW),
                                           dW.stride(0), int(acc is not None or r > 0), C, Cv,
                                           _p(ws), ws_bytes, _stream(dev)), "mt_flce_backward")
                del ws
            grad_w = _weight_grad_in_dtype(dW, W.dtype) if (need_w and acc is None) else None
        grad_x = dX.view(hshape) if need_x else None
        return (grad_x, grad_w) + none

    @staticmethod
    def _backward_fused(ctx, grad_loss):
        saved = ctx.saved_tensors
        g, ris = saved[0], saved[1:]
        gstride = ctx.gstride
        _, hshape, _ = ctx.meta
        T = sum(t1 - t0 for t0, t1, _ in ctx.ranges)
        gl = grad_loss.reshape(-1)
        if gl.numel() == 1:
            gl = gl.expand(T)
        for (t0, t1, n), ri in zip(ctx.ranges, ris):
            if n == 0:
                continue
            if gl.stride(0) == 0 and gstride == 0:  # one scalar against one scalar
                got, want = gl[:1].float(), g
            else:
                valid = ri[:n].long() + t0
                got, want = gl[valid].float(), (g.expand(n) if gstride == 0 else g[valid])
            if not _within_promise(got, want):
                raise RuntimeError(
                    "the upstream gradient of the loss differs from the grad_scale promised to "
                    "fused_linear_cross_entropy by more than "
                    f"{PROMISE_ULPS} fp32 ulp; the fused path has already formed dX and dW "
                    "for the promised one (and added dW into dw_accumulator, if one was given): "
                    "call without grad_scale for an arbitrary gradient")
        if ctx.fused_consumed:
            raise RuntimeError(
                "the fused path formed dX and dW once, at the forward, and has already handed "
                "them to autograd; a second backward through the same loss needs the general "
                "path (call without grad_scale)")
        dX, dW = ctx.dX, ctx.dW
        ctx.dX = ctx.dW = None
        ctx.fused_consumed = True
        grad_x = dX.view(hshape) if ctx.needs_input_grad[0] else None
        grad_w = None
        if ctx.needs_input_grad[1] and dW is not None:
            grad_w = dW.narrow(torch.ones(1, dtype=torch.float32, device=dX.device))
        return (grad_x, grad_w) + (None,) * 8

    @staticmethod
    def _backward_fused_unit(ctx, grad_loss):
        X, W, rngs = _FusedLinearCrossEntropyNone._range_tensors(ctx)
        softcap, hshape, dt = ctx.meta
        if ctx.fused_consumed:
            raise RuntimeError(
                "the fused path formed dX and dW once, at the forward, and has already handed "
                "them to autograd; a second backward through the same loss needs the general "
                "path (call under MT_FLCE_FUSED=0)")
        ctx.fused_consumed = True
        dX, dW = ctx.dX, ctx.dW
        ctx.dX = ctx.dW = None
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        T, H = X.shape
        dev = X.device
        lib = load()
        g, gstride = _grad_vector(grad_loss, T)
        if gstride == 0:
            # one upstream scalar for every token: rescale the unit-gradient
            # dX in place and narrow the tiled dW, times the scalar, into the
            # weight gradient's own bf16 buffer
            scale = g.reshape(-1)[:1]
            if need_x:
                check(lib.mt_flce_scale_grads(_p(scale), _p(dX), T, H, dX.stride(0), dt, None, 0,
                                              H, None, H, _dtype_code(W.dtype), _stream(dev)),
                      "mt_flce_scale_grads")
            dW_out = dW.narrow(scale) if need_w else None
            del dW
        else:
            # a per-token gradient: the unit-gradient results cannot be
            # rescaled; recompute into the same buffers
            dW_out = _backward_bf16_weight(lib, X, W, rngs, g, gstride, softcap, dX, dW)
        grad_x = dX.view(hshape) if need_x else None
        grad_w = dW_out if need_w else None
        return (grad_x, grad_w) + (None,) * 8


def _narrowed_view(dW: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """The [V, H] gradient in `dtype` that mt_flce_scale_grads narrowed into
    the first bytes of the fp32 dW's own storage (bf16 row r at element
    offset r * dW.stride(0)); fp32 is dW itself."""
    if dtype == torch.float32:
        return dW
    V, H = dW.shape
    out = torch.empty(0, dtype=dtype, device=dW.device)
    # storage offsets count elements: one fp32 element is two 16-bit ones
    out.set_(dW.untyped_storage(), 2 * dW.storage_offset(), (V, H), (dW.stride(0), 1))
    return out


def _backward_bf16_weight(lib, X, W, rngs, g, gstride, softcap, dX,
                          dWt: Optional[_TiledDw] = None, keep=None) -> torch.Tensor:
    """The bf16 backward into dX and a weight gradient in bf16 (nothing
    added into), returned as a bf16 [V, H] tensor of its own size: one row
    block through mt_flce_backward_narrow when its plan says so (one range),
    else tiles (dWt's buffers, or new ones; every range adding into them)
    and the narrowing pass.  rngs: [(t0, t1, n, row_index, row_label, lse)]
    per row range.  keep = (C, Cv, workspace, guard) of a forward that kept
    the first vocabulary block's exponentials in that workspace
    (mt_flce_forward_keep): its plan and workspace are used."""
    T, H = X.shape
    V = W.shape[0]
    dev = X.device
    guard = None
    one = len(rngs) == 1
    if one:
        n = rngs[0][2]
        plan = keep[:3] if keep is not None else backward_plan(T, n, H, V, X.dtype, narrow=True)
    if one and plan[0] >= n:
        (t0, t1, n, ri, rl, lse), (C, Cv, ws) = rngs[0], plan
        if keep is not None:
            guard = keep[3]
        else:
            ws = torch.empty(ws, dtype=torch.uint8, device=dev)
        out = dWt.lo if dWt is not None else torch.empty((V, H), dtype=torch.bfloat16, device=dev)
        need = int(lib.mt_flce_narrow_scratch_bytes(V, H, C))
        if dWt is not None and dWt.hi is not None and dWt.hi.numel() * 4 >= need:
            scratch = dWt.hi
        else:
            scratch = torch.empty(need, dtype=torch.uint8, device=dev)
        nbytes = scratch.numel() * scratch.element_size()
        check(lib.mt_flce_backward_narrow(_p(X), _p(W), T, H, V, X.stride(0), W.stride(0),
                                          MT_DTYPE_BF16, softcap, _p(ri), _p(rl), n, _p(lse),
                                          _p(g), gstride, _p(dX), dX.stride(0), _p(out),
                                          out.numel() * 2, _p(scratch), nbytes, C, Cv, _p(ws),
                                          ws.numel(), _p(guard), _stream(dev)),
              "mt_flce_backward_narrow")
        del ws, scratch
        if dWt is not None:
            dWt.hi = None
        return out
    if dWt is None:
        dWt = _TiledDw(V, H, dev)
    for r, (t0, t1, n, ri, rl, lse) in enumerate(rngs):
        # one range: the narrowing plan (several row blocks here); more: the
        # plan of mt_flce_backward_tiles itself (dX's accumulator and X^T in
        # the workspace)
        C, Cv, ws_bytes = (plan if one else backward_plan(t1 - t0, n, H, V, X.dtype))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        gr = g[t0:t1] if gstride else g
        check(lib.mt_flce_backward_tiles(_p(X[t0:t1]), _p(W), t1 - t0, H, V, X.stride(0),
                                         W.stride(0), MT_DTYPE_BF16, softcap, _p(ri), _p(rl), n,
                                         _p(lse), _p(gr), gstride, _p(dX[t0:t1]), dX.stride(0),
                                         *dWt.args(), int(r > 0), C, Cv, _p(ws), ws_bytes,
                                         _stream(dev)), "mt_flce_backward_tiles")
        del ws
    return dWt.narrow(torch.ones(1, dtype=torch.float32, device=dev))


def _weight_grad_in_dtype(dW: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """fp32 dW -> the weight's dtype inside dW's own allocation (autograd
    would otherwise cast it into a second buffer while dW is still alive)."""
    if dtype == torch.float32:
        return dW
    one = torch.ones(1, dtype=torch.float32, device=dW.device)
    V, H = dW.shape
    check(load().mt_flce_scale_grads(_p(one), None, 0, H, H, MT_DTYPE_F32, _p(dW), V,
                                     dW.stride(0), _p(dW), dW.stride(0), _dtype_code(dtype),
                                     _stream(dW.device)), "mt_flce_scale_grads")
    return _narrowed_view(dW, dtype)


# A promised gradient is accepted when every token's received gradient is
# within this many fp32 ulp of the promise: train.py:102's literal
# `loss * world_size / batch_num_loss_counted_tokens` back-propagates
# fl32(fl32(1 / n) * world_size), one or two ulp from fl32(world_size / n).
PROMISE_ULPS = 4


def _within_promise(got: torch.Tensor, want: torch.Tensor) -> bool:
    tol = want.abs() * (PROMISE_ULPS * 2.0 ** -23)
    return bool(((got - want).abs() <= tol).all())


def path_of(loss: torch.Tensor) -> Optional[str]:
    """The path ("general", "fused" or "fused_unit") that produced a loss
    returned by fused_linear_cross_entropy (looked up through its autograd
    node and the view / reshape nodes in front of it), or None."""
    fn = loss.grad_fn
    while fn is not None:
        if hasattr(fn, "path"):
            return fn.path
        nxt = [f for f, _ in fn.next_functions if f is not None]
        fn = nxt[0] if len(nxt) == 1 else None
    return None


def profile_enable(enable: bool = True) -> None:
    """Turn the library's per-launch timing events on or off (mt_flce_profile_enable)."""
    check(load().mt_flce_profile_enable(int(bool(enable))), "mt_flce_profile_enable")


def profile_report() -> dict:
    """Per-kernel timing of the launches recorded since the last report
    (synchronises; mt_flce_profile_report)."""
    import json

    lib = load()
    need = ctypes.c_size_t(0)
    lib.mt_flce_profile_report(None, 0, ctypes.byref(need))
    buf = ctypes.create_string_buffer(max(int(need.value), 2) + 256)
    check(lib.mt_flce_profile_report(buf, len(buf), ctypes.byref(need)), "mt_flce_profile_report")
    return json.loads(buf.value.decode())


def fused_plan(T: int, n_valid: int, H: int, V: int, budget_bytes: Optional[int] = None,
               accumulator: bool = False) -> Tuple[int, int, bool]:
    """(chunk_rows, workspace_bytes, pays) of the fused forward + backward
    (bf16); pays: the planner expects it to beat the general path that the
    same call would otherwise take (accumulator: the weight gradient added
    into an fp32 dw_accumulator; else wanted in bf16, the narrowing plan)."""
    lib = load()
    if budget_bytes is None:
        budget_bytes = int(os.environ.get(BACKWARD_BUDGET_ENV, "0"))
    c, ws, pays = ctypes.c_int64(), ctypes.c_size_t(), ctypes.c_int()
    check(lib.mt_flce_fused_plan(T, n_valid, H, V, MT_DTYPE_BF16, budget_bytes, int(accumulator),
                                 ctypes.byref(c), ctypes.byref(ws), ctypes.byref(pays)),
          "mt_flce_fused_plan")
    return c.value, ws.value, bool(pays.value)


def _use_fused(pays: bool) -> bool:
    mode = os.environ.get(FUSED_ENV, "auto").strip().lower()
    if mode in ("1", "on", "always"):
        return True
    if mode in ("0", "off", "never"):
        return False
    return pays


def _promised_grad(grad_scale, T: int, dev: torch.device) -> Tuple[torch.Tensor, int]:
    if isinstance(grad_scale, torch.Tensor):
        g = grad_scale.detach().reshape(-1).to(device=dev, dtype=torch.float32)
        if g.numel() == 1:
            return g.contiguous(), 0
        if g.numel() != T:
            raise ValueError(f"grad_scale has {g.numel()} elements, expected 1 or {T}")
        return g.contiguous(), 1
    return torch.full((1,), float(grad_scale), dtype=torch.float32, device=dev), 0


def fused_linear_cross_entropy(hidden_states: torch.Tensor, lm_head_weight: torch.Tensor,
                               target: torch.Tensor, ignore_index: int = -100,
                               softcap: Optional[float] = None, shift_labels: bool = False,
                               dw_accumulator: Optional[torch.Tensor] = None,
                               grad_scale=None) -> torch.Tensor:
    """Per-token loss of hidden_states @ lm_head_weight.T against target.

    loss[t] = logsumexp(logits[t]) - logits[t, target[t]], +0.0 where
    target[t] == ignore_index; logits are rounded to the input dtype as
    F.linear would produce them, then evaluated in fp32.  Differentiable in
    hidden_states and lm_head_weight; the gradient of the weight is formed in
    fp32.  With dw_accumulator (fp32 [V, H]) the weight gradient is added into
    that tensor instead of being returned to autograd.  shift_labels applies
    the causal shift (target[t] = labels[t + 1]) on the device; with target of
    shape [B, T'] and B > 1 every row is shifted on its own (its last
    position gets ignore_index), as transformers' ForCausalLMLoss does.

    bf16 inputs whose shapes make the fused path pay (mt_flce_fused_plan: each
    logits tile computed once, dX and dW formed during the forward) take it
    without any promise when no dw_accumulator is given: the forward forms
    the gradients for a unit upstream gradient and the backward rescales
    them when the gradient it receives is one scalar for every token (what
    train.py:97-104's sum and scaling produce), or recomputes for a per-token
    one -- see _FusedLinearCrossEntropyNone.

    grad_scale (a float, or a [T] tensor of per-token values) promises the
    upstream gradient of the returned loss -- train.py:97-104 knows it before
    the forward: world_size / batch_num_loss_counted_tokens for every token.
    The fused path then forms dX and dW for it directly (no rescaling pass)
    and may add dW into dw_accumulator during the forward; the backward
    checks that the gradient it receives is within PROMISE_ULPS fp32 ulp of
    the promise and raises otherwise.  dw_accumulator has then already been
    updated (at the forward), also when that check raises or when no
    backward follows.
    """
    if dw_accumulator is not None:
        V, H = lm_head_weight.shape
        if (dw_accumulator.dtype != torch.float32 or tuple(dw_accumulator.shape) != (V, H)
                or dw_accumulator.stride(1) != 1 or not dw_accumulator.is_cuda):
            raise ValueError("dw_accumulator must be a float32 device tensor of shape [V, H] "
                             "with unit stride along H")
    cap = 0.0 if softcap is None else float(softcap)
    if cap < 0:
        raise ValueError("softcap must be positive (or None)")
    # whole 16-byte chunks along H: zero columns appended (F.pad, whose
    # backward slices the gradients back) contribute nothing to the logits
    H = lm_head_weight.shape[-1]
    hmul = 16 // max(lm_head_weight.element_size(), 1)
    if H % hmul and lm_head_weight.dtype in (torch.bfloat16, torch.float32):
        if dw_accumulator is not None:
            raise ValueError(f"dw_accumulator needs H a multiple of {hmul} (H={H}): the weight "
                             "gradient is formed at a zero-padded width")
        Hp = -(-H // hmul) * hmul
        return fused_linear_cross_entropy(
            torch.nn.functional.pad(hidden_states, (0, Hp - H)),
            torch.nn.functional.pad(lm_head_weight, (0, Hp - H)), target,
            ignore_index=ignore_index, softcap=softcap, shift_labels=shift_labels,
            grad_scale=grad_scale)
    recording = torch.is_grad_enabled() and (hidden_states.requires_grad
                                             or lm_head_weight.requires_grad)
    if not recording:
        # no backward will follow (no_grad / evaluation): the fused path would
        # form dX and dW nobody asked for and add into dw_accumulator
        grad_scale = None
    # the unit-gradient fused path needs the weight's gradient to be wanted
    # (else dW is waste) and no accumulator (which would need the scale now)
    allow_unit = recording and lm_head_weight.requires_grad and dw_accumulator is None
    if shift_labels and target.dim() >= 2 and target.shape[0] > 1:
        target = torch.nn.functional.pad(target, (0, 1), value=int(ignore_index))[..., 1:]
        shift_labels = False
    # bf16 rows are addressed with 32-bit offsets: X beyond one buffer's
    # reach (mt_flce_max_buffer_bytes) runs over row ranges inside one
    # autograd node, whose lm_head gradient every range adds into
    T = target.numel()
    ranges = None
    if hidden_states.dtype == torch.bfloat16 and T > 0:
        limit = int(load().mt_flce_max_buffer_bytes())
        pitch = -(-H // 8) * 8 * 2
        rows = max(1, limit // pitch)
        if T > rows:
            if shift_labels:
                target = torch.nn.functional.pad(target.reshape(T), (0, 1),
                                                 value=int(ignore_index))[1:]
                shift_labels = False
            ranges = [(t0, min(T, t0 + rows)) for t0 in range(0, T, rows)]
    return _FusedLinearCrossEntropyNone.apply(hidden_states, lm_head_weight, target,
                                              int(ignore_index), cap, bool(shift_labels),
                                              dw_accumulator, grad_scale, allow_unit, ranges)


class _CrossEntropyNone(torch.autograd.Function):
    @staticmethod
    def forward(ctx, source, target, ignore_index):
        _require_device("source", source)
        _require_device("target", target)
        dt = _dtype_code(source.dtype)
        L = _rows(source, "source")
        T, V = L.shape
        tgt = target.reshape(-1).to(torch.int64).contiguous()
        if tgt.numel() != T:
            raise ValueError(f"target has {tgt.numel()} elements, expected {T}")
        lib = load()
        dev = L.device
        loss = torch.empty(T, dtype=torch.float32, device=dev)
        lse = torch.empty(T, dtype=torch.float32, device=dev)
        status = torch.empty(1, dtype=torch.int32, device=dev)
        check(lib.mt_ce_forward(_p(L), T, V, L.stride(0), dt, _p(tgt), int(ignore_index), _p(loss),
                                _p(lse), _p(status), _stream(dev)), "mt_ce_forward")
        if int(status.item()) != 0:
            bad = tgt[(tgt != ignore_index) & ((tgt < 0) | (tgt >= V))][0].item()
            raise IndexError(f"Target {bad} is out of bounds.")
        ctx.save_for_backward(L, tgt, lse)
        ctx.meta = (int(ignore_index), dt, source.shape, source.dtype)
        out = loss.view(source.shape[:-1])
        return out if source.dtype == torch.float32 else out.to(source.dtype)

    @staticmethod
    def backward(ctx, grad_loss):
        L, tgt, lse = ctx.saved_tensors
        ignore_index, dt, shape, dtype = ctx.meta
        if not ctx.needs_input_grad[0]:
            return None, None, None
        T, V = L.shape
        g, gstride = _grad_vector(grad_loss, T)
        d = torch.empty((T, V), dtype=dtype, device=L.device)
        check(load().mt_ce_backward(_p(L), T, V, L.stride(0), dt, _p(tgt), ignore_index, _p(lse),
                                    _p(g), gstride, _p(d), d.stride(0), _stream(L.device)),
              "mt_ce_backward")
        return d.view(shape), None, None


def cross_entropy_none(source: torch.Tensor, target: torch.Tensor,
                       ignore_index: int = -100) -> torch.Tensor:
    """F.cross_entropy(source, target, ignore_index, reduction='none') on the device."""
    return _CrossEntropyNone.apply(source, target, int(ignore_index))


def per_sample_loss_sums(loss: torch.Tensor, target: torch.Tensor, cu_seqlens: torch.Tensor,
                         ignore_index: int = -100, validate: bool = True,
                         shift: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-sample (sum of loss, number of counted tokens) over a packed batch.

    cu_seqlens (int32 [S+1]) partitions the T packed positions into samples.
    With shift, `target` holds the unshifted labels and position t counts when
    labels[t + 1] is not ignore_index (the causal shift the loss applied).
    With validate, a malformed cu_seqlens raises ValueError (one sync);
    without it nothing synchronises.
    """
    for name, t in (("loss", loss), ("target", target), ("cu_seqlens", cu_seqlens)):
        _require_device(name, t)
    lib = load()
    ls = loss.reshape(-1).float().contiguous()
    tgt = target.reshape(-1).to(torch.int64).contiguous()
    cu = cu_seqlens.reshape(-1).to(torch.int32).contiguous()
    T, S = ls.numel(), cu.numel() - 1
    if tgt.numel() != T or S < 0:
        raise ValueError("loss and target must have the same number of elements; "
                         "cu_seqlens needs at least one entry")
    dev = ls.device
    seg_loss = torch.empty(S, dtype=torch.float32, device=dev)
    seg_cnt = torch.empty(S, dtype=torch.int32, device=dev)
    status = torch.empty(1, dtype=torch.int32, device=dev)
    check(lib.mt_segment_sum(_p(ls), _p(tgt), T, int(ignore_index), int(bool(shift)), _p(cu), S,
                             _p(seg_loss), _p(seg_cnt), _p(status), _stream(dev)),
          "mt_segment_sum")
    if validate and int(status.item()) != 0:
        raise ValueError(f"cu_seqlens is not a partition of [0, {T}): must start at 0, be "
                         f"non-decreasing and end at {T}")
    return seg_loss, seg_cnt
