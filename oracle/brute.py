"""float64 closed forms for tiny shapes (test infrastructure only).

loss_t = logsumexp_v(s_tv) - s_{t,y_t},  s = X W^T  (optionally softcapped),
G = g_t (softmax(s_t) - onehot(y_t)) * softcap', dX = G W, dW = G^T X;
all zero on ignored rows.  This is the textbook form of what
none_reduction_losses.py:35 (F.cross_entropy, reduction='none') and its
autograd compute; it pins torch_path.py and flce_ref.c.
"""
from __future__ import annotations

import numpy as np


def flce_f64(X, W, target, grad=None, ignore_index=-100, softcap=None):
    X = np.asarray(X, dtype=np.float64)
    W = np.asarray(W, dtype=np.float64)
    y = np.asarray(target, dtype=np.int64)
    T = X.shape[0]
    g = np.ones(T) if grad is None else np.broadcast_to(np.asarray(grad, np.float64), (T,))
    s = X @ W.T
    if softcap:
        th = np.tanh(s / softcap)
        z = softcap * th
        dz = 1.0 - th * th
    else:
        z, dz = s, np.ones_like(s)
    valid = y != ignore_index
    m = z.max(axis=1, keepdims=True)
    lse = (m + np.log(np.exp(z - m).sum(axis=1, keepdims=True)))[:, 0]
    yy = np.where(valid, y, 0)
    loss = np.where(valid, lse - z[np.arange(T), yy], 0.0)
    p = np.exp(z - lse[:, None])
    p[np.arange(T), yy] -= 1.0
    G = p * dz * (g * valid)[:, None]
    return loss, G @ W, G.T @ X, lse
