"""Golden vectors (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle (torch path and C restatement) reproduces them.  GPU: the HIP
path matches them to the north-star tolerances."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import ref
from oracle.torch_path import rel_fro, torch_path

GOLDEN = Path(__file__).resolve().parent / "golden"
NAMES = ["fp32_small", "bf16_small", "bf16_softcap"]


def load(name):
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    dt = torch.bfloat16 if "bfloat16" in str(z["dtype"]) else torch.float32

    def t(a):
        if dt == torch.bfloat16 and a.dtype == np.uint16:
            return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        return torch.from_numpy(a.copy())

    cap = float(z["softcap"]) or None
    return dict(X=t(z["X"]), W=t(z["W"]), y=torch.from_numpy(z["target"].copy()),
                grad=torch.from_numpy(z["grad"].copy()), loss=torch.from_numpy(z["loss"].copy()),
                dX=t(z["dX"]), dW=torch.from_numpy(z["dW"].copy()), cap=cap, dt=dt)


@pytest.mark.parametrize("name", NAMES)
def test_torch_path_reproduces_golden(name):
    g = load(name)
    loss, dX, dW = torch_path(g["X"], g["W"], g["y"], grad=g["grad"], softcap=g["cap"])
    torch.testing.assert_close(loss, g["loss"], rtol=1e-6, atol=1e-6)
    assert rel_fro(dX.float(), g["dX"].float()) < 1e-3
    assert rel_fro(dW, g["dW"]) < 1e-5


@pytest.mark.parametrize("name", NAMES)
def test_c_restatement_matches_golden(name):
    g = load(name)
    bf = g["dt"] == torch.bfloat16
    loss, dX, dW = ref.backward(g["X"].float().numpy(), g["W"].float().numpy(), g["y"].numpy(),
                                g["grad"].numpy(), round_bf16=bf, softcap=g["cap"] or 0.0)
    v = (g["y"] != -100).numpy()
    tol = 2e-3 if bf else 1e-5
    assert np.max(np.abs(loss[v] - g["loss"].numpy()[v]) / np.abs(g["loss"].numpy()[v])) < tol
    assert not loss[~v].any()
    assert rel_fro(torch.from_numpy(dX), g["dX"].float()) < 1e-2
    assert rel_fro(torch.from_numpy(dW), g["dW"]) < 1e-2


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_path_matches_golden(gpu, name):
    from mini_trainer_amd import fused_linear_cross_entropy

    g = load(name)
    X = g["X"].to(gpu).requires_grad_(True)
    acc = torch.zeros(g["W"].shape, dtype=torch.float32, device=gpu)
    loss = fused_linear_cross_entropy(X, g["W"].to(gpu).requires_grad_(True), g["y"].to(gpu),
                                      softcap=g["cap"], dw_accumulator=acc)
    loss.backward(g["grad"].to(gpu))
    torch.cuda.synchronize()
    loss = loss.detach().cpu()
    v = g["y"] != -100
    tol = 2e-3 if g["dt"] == torch.bfloat16 else 1e-5
    err = ((loss[v] - g["loss"][v]).abs() / g["loss"][v].abs()).max().item()
    assert err <= tol
    assert torch.equal(loss[~v], torch.zeros(int((~v).sum())))
    assert rel_fro(X.grad.cpu().float(), g["dX"].float()) <= 1e-2
    assert rel_fro(acc.cpu(), g["dW"]) <= 1e-2
