"""Parity of the fused forward + backward (mt_flce_fused: the upstream
gradient promised at the forward, each logits tile computed once) against the
reference's torch path, with the north-star tolerances: per-token loss 2e-3
relative (bf16), dX and dW 1e-2 relative Frobenius error, ignored positions
exactly +0.0 / 0.  Also: its results agree with the general path's, the
backward rejects a gradient other than the promised one, the chunking
(several chunks, uneven last chunk) does not change the result, and a chunk
whose logits leave the range of the exponential scheme is redone from its
logits.
"""
from __future__ import annotations

import threading

import pytest
import torch

from mini_trainer_amd import fused_linear_cross_entropy, path_of
from mini_trainer_amd.flce import BACKWARD_BUDGET_ENV, FUSED_ENV, fused_plan
from mini_trainer_amd.none_reduction_losses import (
    liger_fixed_fused_linear_cross_entropy_none_reduction)
from oracle.torch_path import rel_fro

from test_gpu_parity import GRAD_RFRO, check_parity, make_case

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _always_fused(monkeypatch):
    # these tests exercise the fused path itself, whatever the planner prefers
    monkeypatch.setenv(FUSED_ENV, "1")


def run_fused(dev, X, W, y, grad_scale, softcap=None, acc=None, backward_grad=None):
    Xd = X.to(dev).requires_grad_(True)
    Wd = W.to(dev).requires_grad_(True)
    if acc is None:
        acc = torch.zeros(W.shape, dtype=torch.float32, device=dev)
    gs = grad_scale.to(dev) if isinstance(grad_scale, torch.Tensor) else grad_scale
    loss = fused_linear_cross_entropy(Xd, Wd, y.to(dev), softcap=softcap, dw_accumulator=acc,
                                      grad_scale=gs)
    if backward_grad is None:
        if isinstance(grad_scale, torch.Tensor):
            loss.backward(grad_scale.to(dev))
        else:
            (loss.float().sum() * grad_scale).backward()
    else:
        loss.backward(backward_grad.to(dev))
    torch.cuda.synchronize()
    return loss.detach().cpu(), Xd.grad.detach().cpu(), acc.cpu()


@pytest.mark.parametrize("T,H,V", [(300, 128, 1000), (513, 192, 2065), (64, 896, 4096)])
def test_fused_uniform_grad(gpu, T, H, V):
    print(f"case fused T={T} H={H} V={V}", flush=True)
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=T + V)
    n = int((y != -100).sum())
    loss, dX, dW = run_fused(gpu, X, W, y, 1.0 / n)
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((T,), 1.0 / n))


@pytest.mark.parametrize("V", [3000, 2560])  # vocabulary tail / whole 256-column tiles
def test_fused_per_token_grad_and_softcap(gpu, V):
    X, W, y = make_case(400, 128, V, torch.bfloat16, seed=11, w_std=0.2)
    grad = torch.rand(400, generator=torch.Generator().manual_seed(3)) * 2 - 0.5
    loss, dX, dW = run_fused(gpu, X, W, y, grad, softcap=3.0)
    check_parity(X, W, y, loss, dX, dW, grad=grad, softcap=3.0)


def test_fused_many_chunks_matches_general_path(gpu, monkeypatch):
    # tiny budget -> 256-row chunks: several chunks, an uneven last one, dW
    # accumulated across chunks
    monkeypatch.setenv(BACKWARD_BUDGET_ENV, "1")
    X, W, y = make_case(1100, 128, 1300, torch.bfloat16, seed=7, mask_frac=0.2)
    n = int((y != -100).sum())
    C, ws, _ = fused_plan(1100, n, 128, 1300)
    assert C == 256 and ws > 0
    loss, dX, dW = run_fused(gpu, X, W, y, 0.5)
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((1100,), 0.5))
    # the general path on the same inputs: same loss bits, gradients within rounding
    monkeypatch.setenv(FUSED_ENV, "0")
    Xd, Wd = X.to(gpu).requires_grad_(True), W.to(gpu).requires_grad_(True)
    acc = torch.zeros(W.shape, dtype=torch.float32, device=gpu)
    l2 = fused_linear_cross_entropy(Xd, Wd, y.to(gpu), dw_accumulator=acc)
    (l2.float().sum() * 0.5).backward()
    assert torch.equal(l2.detach().cpu(), loss)
    assert rel_fro(Xd.grad.cpu().float(), dX.float()) <= 1e-2
    # the fused dW is E^T (s X): one bf16 rounding more (of s X) than G^T X
    assert rel_fro(acc.cpu(), dW) <= 3e-3


@pytest.mark.parametrize("shift", [56.0, -56.0])
def test_fused_out_of_range_logits_recompute_their_chunk(gpu, monkeypatch, shift):
    # The fused forward keeps exp(logit) in bf16 while every row's largest
    # logit lies in [-48, 48]; a chunk with a row outside is redone from its
    # stored logits.  Here the first 256-row chunk's logits all move by
    # `shift` (an X column of `shift` against a weight column of ones: a
    # weight column of `shift` would multiply the bf16 rounding of G into dX)
    # and the other chunks stay near 0.  The logits are exact multiples of
    # 1/4 below 64 in magnitude (X in {-1, 0, 1}, W in quarters), so that
    # every path rounds them the same way.
    monkeypatch.setenv(BACKWARD_BUDGET_ENV, "1")  # 256-row chunks
    g = torch.Generator().manual_seed(43)
    T, H, V = 900, 64, 700
    X = torch.zeros(T, H)
    W = torch.zeros(V, H)
    X[:, 1:16] = torch.randint(-1, 2, (T, 15), generator=g).float()
    W[:, 1:16] = torch.randint(-1, 2, (V, 15), generator=g).float() / 4
    X[:256, 0] = shift
    W[:, 0] = 1.0
    X, W = X.to(torch.bfloat16), W.to(torch.bfloat16)
    y = torch.randint(0, V, (T,), generator=g)
    n = T
    assert fused_plan(T, n, H, V)[0] == 256
    loss, dX, dW = run_fused(gpu, X, W, y, 1.0 / n)
    check_parity(X, W, y, loss, dX, dW, grad=torch.full((T,), 1.0 / n))
    monkeypatch.setenv(FUSED_ENV, "0")
    l2 = fused_linear_cross_entropy(X.to(gpu), W.to(gpu), y.to(gpu))
    assert torch.equal(l2.cpu(), loss)


@pytest.mark.parametrize("split", ["0", "1"])
def test_fused_dw_work_queue_with_tails(gpu, monkeypatch, split):
    # 257 x 5 = 1285 dW tiles per chunk, at least 4 per CU: dW runs
    # persistent over its work queue; a vocabulary tail (V = 65600) and a
    # hidden tail (H = 1056: the fifth column of tiles 32 wide), 256-row
    # chunks.  dX and dW in one launch, and (split = 1, the measurement
    # hook) as two kernels on two streams.  Reference: the torch path on
    # the GPU in fp32.
    from mini_trainer_amd.flce import profile_enable, profile_report
    from oracle.torch_path import torch_path
    monkeypatch.setenv(BACKWARD_BUDGET_ENV, "1")
    monkeypatch.setenv("MT_FLCE_SPLIT_PHASE", split)
    T, H, V = 700, 1056, 65600
    X, W, y = make_case(T, H, V, torch.bfloat16, seed=51)
    n = int((y != -100).sum())
    assert fused_plan(T, n, H, V)[0] == 256
    profile_enable(True)
    try:
        loss, dX, dW = run_fused(gpu, X, W, y, 1.0 / n)
    finally:
        profile_enable(False)
    rep = profile_report()
    assert rep["dx_dw_phase"]["launches"] == -(-n // 256)  # one per chunk
    if split == "1":
        assert rep["dw_bf16_kernel<queue>"]["launches"] == -(-n // 256)
    g = torch.full((T,), 1.0 / n, device=gpu)
    rl, rdX, rdW = torch_path(X.to(gpu), W.to(gpu), y.to(gpu), grad=g, upcast=True)
    valid = y != -100
    assert torch.equal(loss[~valid], torch.zeros(int((~valid).sum())))
    err = ((loss[valid] - rl.cpu()[valid]).abs() / rl.cpu()[valid].abs()).max().item()
    assert err <= 2e-3, err
    assert rel_fro(dX.float(), rdX.cpu().float()) <= GRAD_RFRO
    assert rel_fro(dW, rdW.cpu()) <= GRAD_RFRO


def test_fused_accumulates_and_all_masked(gpu):
    X, W, y = make_case(300, 128, 700, torch.bfloat16, seed=9)
    X2, _, y2 = make_case(200, 128, 700, torch.bfloat16, seed=10)
    y3 = torch.full((50,), -100)
    X3 = torch.randn(50, 128).to(torch.bfloat16)
    acc = torch.zeros(W.shape, dtype=torch.float32, device=gpu)
    for Xi, yi in ((X, y), (X2, y2), (X3, y3)):
        loss, dX, _ = run_fused(gpu, Xi, W, yi, 1.0, acc=acc)
    assert torch.equal(loss, torch.zeros(50)) and torch.count_nonzero(dX) == 0
    from oracle.torch_path import torch_path
    _, _, r1 = torch_path(X, W, y)
    _, _, r2 = torch_path(X2, W, y2)
    assert rel_fro(acc.cpu(), r1 + r2) <= GRAD_RFRO


def test_fused_rejects_a_different_gradient(gpu):
    X, W, y = make_case(256, 64, 512, torch.bfloat16, seed=21)
    with pytest.raises(RuntimeError, match="promised"):
        run_fused(gpu, X, W, y, 1.0, backward_grad=torch.full((256,), 2.0))


def test_drop_in_reads_grad_scale_kwarg(gpu):
    X, W, y = make_case(256, 64, 512, torch.bfloat16, seed=22)
    Xd, Wd = X.to(gpu).requires_grad_(True), W.to(gpu).requires_grad_(True)
    loss = liger_fixed_fused_linear_cross_entropy_none_reduction(
        Xd, Wd, y.to(gpu), None, -100, None, mt_grad_scale=0.25)
    assert path_of(loss) == "fused"
    (loss.sum() * 0.25).backward()
    check_parity(X, W, y, loss.detach().cpu(), Xd.grad.cpu(), Wd.grad.cpu(),
                 grad=torch.full((256,), 0.25))


def test_fused_second_backward_raises(gpu):
    # dX and dW exist once (formed at the forward): a second backward through
    # the same graph must fail loudly rather than return no gradient
    X, W, y = make_case(256, 64, 512, torch.bfloat16, seed=24)
    Xd = X.to(gpu).requires_grad_(True)
    loss = fused_linear_cross_entropy(Xd, W.to(gpu), y.to(gpu), grad_scale=0.5)
    (loss.sum() * 0.5).backward(retain_graph=True)
    assert Xd.grad is not None
    with pytest.raises(RuntimeError, match="second backward"):
        (loss.sum() * 0.5).backward()


def test_grad_scale_ignored_without_autograd(gpu):
    # Under no_grad (or with inputs that do not require grad) no backward
    # follows, so the promise is not acted on: the loss is the same and the
    # dW accumulator is left untouched.
    X, W, y = make_case(300, 128, 1000, torch.bfloat16, seed=23)
    Xd, Wd, yd = X.to(gpu), W.to(gpu), y.to(gpu)
    acc = torch.full(W.shape, 0.5, dtype=torch.float32, device=gpu)
    ref = fused_linear_cross_entropy(Xd, Wd, yd)
    with torch.no_grad():
        a = fused_linear_cross_entropy(Xd.requires_grad_(True), Wd, yd, dw_accumulator=acc,
                                       grad_scale=0.01)
    b = fused_linear_cross_entropy(Xd.detach(), Wd, yd, dw_accumulator=acc, grad_scale=0.01)
    torch.cuda.synchronize()
    assert torch.equal(a, ref) and torch.equal(b, ref)
    assert bool((acc == 0.5).all())


@pytest.mark.parametrize("split", ["0", "1"])
def test_fused_concurrent_host_threads(gpu, monkeypatch, split):
    # Two host threads, each on its own stream: every call orders its dW
    # after its own G and its caller's stream after its own dW (split = 1:
    # the two share the library's per-device side stream and fork / join
    # events).  Results are bit-identical to the same calls made one after
    # the other.
    monkeypatch.setenv("MT_FLCE_SPLIT_PHASE", split)
    cases = []
    for seed in (31, 32):
        X, W, y = make_case(600, 128, 1500, torch.bfloat16, seed=seed)
        cases.append((X, W, y, 1.0 / int((y != -100).sum())))
    ref = [run_fused(gpu, X, W, y, s) for X, W, y, s in cases]
    streams = [torch.cuda.Stream(device=gpu) for _ in cases]
    out = [None] * len(cases)
    errors = []

    def work(i):
        try:
            X, W, y, s = cases[i]
            with torch.cuda.stream(streams[i]):
                out[i] = run_fused(gpu, X, W, y, s)
        except Exception as e:  # reported below, in the main thread
            errors.append(e)

    for _ in range(3):
        threads = [threading.Thread(target=work, args=(i,)) for i in range(len(cases))]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        assert not errors, errors
        for got, want in zip(out, ref):
            for g, w in zip(got, want):
                assert torch.equal(g, w)
