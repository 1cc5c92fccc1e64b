"""The reference's torch path (test infrastructure only).  It runs where its
inputs live: on the CPU, or on the GPU as the full-size checker of the
HIP kernels (never as the path under test).

Forward, per row chunk (rows are independent, so chunking is exact for the
loss and dX and only reorders the fp32 sum of dW):
    logits = F.linear(X_c, W)               model dtype (bf16-rounded for bf16),
                                            TF/models/llama/modeling_llama.py:480
    z      = logits.float()                 TF/loss/loss_utils.py:59
    z      = cap * tanh(z / cap)            only with a softcap
    loss   = F.cross_entropy(z, y, ignore_index=ignore_index, reduction='none')
                                            none_reduction_losses.py:35
Backward: autograd of the above w.r.t. the fp32 logits with the per-token
upstream gradient g (train.py:98-104 makes g uniform), cast to the model
dtype at the .float() boundary, then the F.linear backward:
    dX_c = G_c @ W            (model dtype, as torch autograd produces it)
    dW  += G_c^T @ X_c        (fp32 accumulation: the north-star dW)

Pinned by: oracle/brute.py (float64 closed forms, fp32 inputs), the
invariants in tests/test_oracle.py (W = 0 gives ln V, sum_v dW = 0, all-masked
gives zeros, row-permutation and chunking invariance) and the committed
golden vectors tests/golden/*.npz.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn.functional as F


def torch_path(X: torch.Tensor, W: torch.Tensor, target: torch.Tensor,
               grad: Optional[torch.Tensor] = None, ignore_index: int = -100,
               softcap: Optional[float] = None, chunk_rows: int = 1024,
               rows: Optional[int] = None, need_grads: bool = True, upcast: bool = False
               ) -> Tuple[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]:
    """Returns (loss fp32 [T], dX [T, H] in X.dtype, dW fp32 [V, H]).

    grad: per-token upstream gradient ([T] or scalar); default 1.
    rows: only process the first `rows` rows (bounded CPU samples).
    upcast: form the logits as an fp32 product rounded to X.dtype (what
      F.linear in bf16 computes, up to the fp32 summation order) and dX as
      an fp32 product of the rounded G -- the same arithmetic as the default,
      only faster on CPUs without a fast bf16 GEMM.
    """
    T, H = X.shape
    V = W.shape[0]
    dev = X.device
    n = T if rows is None else min(rows, T)
    y_all = target.reshape(-1).to(device=dev, dtype=torch.int64)
    if grad is None:
        g_all = torch.ones(T, dtype=torch.float32, device=dev)
    else:
        g_all = grad.reshape(-1).to(device=dev, dtype=torch.float32)
        if g_all.numel() == 1:
            g_all = g_all.expand(T)
    loss = torch.zeros(n, dtype=torch.float32, device=dev)
    dX = torch.zeros(n, H, dtype=X.dtype, device=dev) if need_grads else None
    dW = torch.zeros(V, H, dtype=torch.float32, device=dev) if need_grads else None
    Wf = W.float() if upcast else None
    for a in range(0, n, chunk_rows):
        b = min(a + chunk_rows, n)
        Xc, y = X[a:b], y_all[a:b]
        logits = (F.linear(Xc.float(), Wf).to(X.dtype) if upcast and X.dtype != torch.float32
                  else F.linear(Xc, W))
        z0 = logits.float().requires_grad_(need_grads)
        z = softcap * torch.tanh(z0 / softcap) if softcap else z0
        lc = F.cross_entropy(z, y, ignore_index=ignore_index, reduction="none")
        loss[a:b] = lc.detach()
        if need_grads:
            (G,) = torch.autograd.grad(lc, z0, g_all[a:b])
            Gd = G.to(X.dtype)
            dX[a:b] = (Gd.float() @ Wf).to(X.dtype) if upcast else Gd @ W
            dW += Gd.float().t() @ Xc.float()
    return loss, dX, dW


def rel_fro(a: torch.Tensor, b: torch.Tensor) -> float:
    """||a - b||_F / ||b||_F in float64 (0 when both are zero)."""
    a = a.double()
    b = b.double()
    nb = torch.linalg.vector_norm(b).item()
    nd = torch.linalg.vector_norm(a - b).item()
    if nb == 0.0:
        return 0.0 if nd == 0.0 else float("inf")
    return nd / nb
