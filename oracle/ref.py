"""ctypes wrapper of the C restatement (test infrastructure only)."""
from __future__ import annotations

import ctypes
import os
from ctypes import c_double, c_int, c_int64, c_void_p

import numpy as np

from .build import LIB, build

_lib = None


def lib() -> ctypes.CDLL:
    """The C restatement; MT_ORACLE_LIB names another build of it (the
    sanitised one of oracle/build.py, for tests/test_oracle_asan.py)."""
    global _lib
    if _lib is None:
        path = os.environ.get("MT_ORACLE_LIB")
        if not path:
            if not LIB.exists():
                build()
            path = str(LIB)
        L = ctypes.CDLL(path)
        L.ref_prepare.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p, c_void_p, c_void_p]
        L.ref_forward.argtypes = [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_double,
                                  c_void_p, c_void_p, c_int64, c_void_p, c_void_p]
        L.ref_backward.argtypes = [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_double,
                                   c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
                                   c_void_p, c_int]
        L.ref_segment_sum.argtypes = [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64,
                                      c_void_p, c_void_p, c_void_p]
        L.ref_ce_forward.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p,
                                     c_void_p, c_void_p]
        L.ref_round_bf16.argtypes = [ctypes.c_float]
        L.ref_round_bf16.restype = ctypes.c_float
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def prepare(labels, V, ignore_index=-100, shift=False):
    lab = _c(labels, np.int64)
    T = lab.size
    ri = np.zeros(T, np.int32)
    rl = np.zeros(T, np.int32)
    counts = np.zeros(4, np.int32)
    lib().ref_prepare(lab.ctypes.data, T, V, ignore_index, int(shift), ri.ctypes.data,
                      rl.ctypes.data, counts.ctypes.data)
    return ri, rl, counts


def forward(X, W, labels, round_bf16, ignore_index=-100, softcap=0.0):
    X = _c(X, np.float32)
    W = _c(W, np.float32)
    T, H = X.shape
    V = W.shape[0]
    ri, rl, counts = prepare(labels, V, ignore_index)
    N = int(counts[0])
    loss = np.zeros(T, np.float32)
    lse = np.zeros(max(N, 1), np.float32)
    lib().ref_forward(X.ctypes.data, W.ctypes.data, T, H, V, int(round_bf16), float(softcap or 0.0),
                      ri.ctypes.data, rl.ctypes.data, N, loss.ctypes.data, lse.ctypes.data)
    return loss, lse[:N], ri, rl, N


def backward(X, W, labels, grad, round_bf16, ignore_index=-100, softcap=0.0, dW_init=None):
    X = _c(X, np.float32)
    W = _c(W, np.float32)
    T, H = X.shape
    V = W.shape[0]
    loss, lse, ri, rl, N = forward(X, W, labels, round_bf16, ignore_index, softcap)
    g = _c(np.broadcast_to(np.asarray(grad, np.float32), (T,)), np.float32)
    dX = np.zeros((T, H), np.float32)
    dW = np.zeros((V, H), np.float32) if dW_init is None else _c(dW_init, np.float32).copy()
    lib().ref_backward(X.ctypes.data, W.ctypes.data, T, H, V, int(round_bf16), float(softcap or 0.0),
                       ri.ctypes.data, rl.ctypes.data, N, lse.ctypes.data if N else None,
                       g.ctypes.data, 1, dX.ctypes.data, dW.ctypes.data, int(dW_init is not None))
    return loss, dX, dW


def segment_sum(loss, target, cu, ignore_index=-100):
    loss = _c(loss, np.float32)
    tgt = _c(target, np.int64)
    cu = _c(cu, np.int32)
    S = cu.size - 1
    sl = np.zeros(max(S, 1), np.float32)
    sc = np.zeros(max(S, 1), np.int32)
    st = np.zeros(1, np.int32)
    lib().ref_segment_sum(loss.ctypes.data, tgt.ctypes.data, loss.size, ignore_index, cu.ctypes.data,
                          S, sl.ctypes.data, sc.ctypes.data, st.ctypes.data)
    return sl[:S], sc[:S], int(st[0])


def ce_forward(logits, target, ignore_index=-100):
    L = _c(logits, np.float32)
    tgt = _c(target, np.int64)
    T, V = L.shape
    loss = np.zeros(T, np.float32)
    lse = np.zeros(T, np.float32)
    st = np.zeros(1, np.int32)
    lib().ref_ce_forward(L.ctypes.data, T, V, tgt.ctypes.data, ignore_index, loss.ctypes.data,
                         lse.ctypes.data, st.ctypes.data)
    return loss, lse, int(st[0])


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Vectorised round-to-nearest-even to bfloat16 values (as float32)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)
