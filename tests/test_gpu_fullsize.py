"""Config 3 at its full size (T=65536, H=4096, V=128256, bf16, Zipf labels,
30% masked, 128 packed samples): the HIP paths are checked where the oracle
can follow them at this size and through size-independent properties.

  * sampled rows: loss and dX of 24 valid and 8 ignored rows against the
    reference torch path on the CPU (loss 2e-3
    relative, dX 1e-2 relative Frobenius; ignored rows exactly 0);
  * sampled vocabulary rows of dW: sum_t g (exp(logit_tv - lse_t) - [y_t = v])
    x_t on the CPU from the returned lse (itself pinned by the loss check);
  * sum over the vocabulary of dW is ~0 (every row of softmax - onehot sums
    to zero);
  * the fused path (gradient promised at the forward) and the general path
    agree: identical loss bits, dX / dW within rounding;
  * per-sample segment sums add up to the batch sum and count the valid rows.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from mini_trainer_amd import fused_linear_cross_entropy, per_sample_loss_sums, synth
from mini_trainer_amd.flce import FUSED_ENV
from oracle.torch_path import rel_fro, torch_path

pytestmark = pytest.mark.gpu


def test_config3_full_size(gpu, monkeypatch):
    cfg = synth.CONFIGS[3]
    b = synth.make_batch(cfg, 0, with_tensors=False)
    T, H, V = cfg.T, cfg.H, cfg.V
    print(f"config 3 full size: T={T} H={H} V={V}", flush=True)
    gen = torch.Generator(device=gpu).manual_seed(3)
    X = torch.randn(T, H, device=gpu, generator=gen).to(torch.bfloat16)
    W = (torch.randn(V, H, device=gpu, generator=gen) * cfg.w_std).to(torch.bfloat16)
    y = b["target"].to(gpu)
    cu = b["cu_seqlens"].to(gpu)
    valid = y != -100
    n = int(valid.sum())
    scale = 1.0 / n

    def run(fused: bool):
        monkeypatch.setenv(FUSED_ENV, "1" if fused else "0")
        Xd = X.detach().requires_grad_(True)
        dW = torch.zeros(V, H, dtype=torch.float32, device=gpu)
        loss = fused_linear_cross_entropy(Xd, W, y, dw_accumulator=dW,
                                          grad_scale=scale if fused else None)
        (loss.sum() * scale).backward()
        torch.cuda.synchronize()
        return loss.detach(), Xd.grad, dW

    loss_f, dX_f, dW_f = run(True)
    loss_g, dX_g, dW_g = run(False)
    print("paths done", flush=True)

    # fused vs general: same forward arithmetic, gradients within rounding
    assert torch.equal(loss_f, loss_g)
    assert rel_fro(dX_f.float(), dX_g.float()) <= 1e-2
    assert rel_fro(dW_f, dW_g) <= 1e-3

    # ignored rows
    assert torch.count_nonzero(loss_f[~valid]) == 0 and not torch.signbit(loss_f[~valid]).any()
    assert torch.count_nonzero(dX_f[~valid]) == 0
    assert bool((loss_f[valid] > 0).all())

    # sampled rows against the reference torch path on the CPU
    rng = np.random.default_rng(33)
    vidx = torch.nonzero(valid).flatten().cpu().numpy()
    iidx = torch.nonzero(~valid).flatten().cpu().numpy()
    rows = np.concatenate([rng.choice(vidx, 24, replace=False), rng.choice(iidx, 8, replace=False)])
    rows_t = torch.from_numpy(rows).to(gpu)
    Wc = W.cpu()
    rl, rdX, _ = torch_path(X[rows_t].cpu(), Wc, y[rows_t].cpu(), grad=torch.tensor(scale),
                            upcast=True)
    sl, sdX = loss_f[rows_t].cpu(), dX_f[rows_t].cpu()
    v = y[rows_t].cpu() != -100
    err = ((sl[v] - rl[v]).abs() / rl[v].abs()).max().item()
    assert err <= 2e-3, f"sampled loss rel err {err:.3e}"
    assert torch.equal(sl[~v], torch.zeros(int((~v).sum())))
    assert rel_fro(sdX.float(), rdX.float()) <= 1e-2

    # sampled dW rows on the CPU, from the returned loss: lse_t = loss_t + logit_{t, y_t}
    vrows = torch.from_numpy(rng.choice(V, 6, replace=False))
    Xv = X[valid].float().cpu()
    yv = y[valid].cpu()
    Wf = Wc.float()
    ly = (Xv * Wf[yv]).sum(1).to(torch.bfloat16).float()
    lse_v = loss_f[valid].cpu() + ly
    logits = (Xv @ Wf[vrows].t()).to(torch.bfloat16).float()  # [n, 6]
    onehot = (yv[:, None] == vrows[None, :]).float()
    Gs = scale * (torch.exp(logits.double() - lse_v.double()[:, None]) - onehot.double())
    ref_rows = Gs.t() @ Xv.double()
    assert rel_fro(dW_f[vrows.to(gpu)].cpu().double(), ref_rows) <= 1e-2

    # every softmax - onehot row sums to zero, hence so does dW over the vocabulary
    col = dW_f.double().sum(0)
    assert (col.norm() / dW_f.double().norm()).item() <= 1e-2

    # segment sums: a checksum of checksums
    seg_loss, seg_cnt = per_sample_loss_sums(loss_f, y, cu)
    np.testing.assert_allclose(seg_loss.double().sum().item(), loss_f.double().sum().item(), rtol=1e-5)
    assert int(seg_cnt.sum()) == n
