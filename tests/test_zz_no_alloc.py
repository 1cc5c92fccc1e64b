"""The forward without allocation (mt_flce_forward_noalloc, scratch in a
static device array) against the forward with a workspace
(mt_flce_forward), both through the C ABI: two calls in a row, the second
with a smaller input, the first spanning several scratch-sized row chunks.
bf16 results are bit-identical; fp32 (whose split of the vocabulary depends
on the row count) within 1e-6 relative.  The same call captured in a HIP
graph (torch.cuda.graph) and replayed: every replay bit-identical to the
workspace forward."""
from __future__ import annotations

import pytest
import torch

from mini_trainer_amd import _lib, prepare_targets
from mini_trainer_amd.flce import _dtype_code, _p, _stream

pytestmark = pytest.mark.gpu


def case(dev, T, H, V, dtype, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    X = torch.randn(T, H, device=dev, generator=g).to(dtype)
    W = (torch.randn(V, H, device=dev, generator=g) * 0.05).to(dtype)
    y = torch.randint(0, V, (T,), device=dev, generator=g)
    y[torch.rand(T, device=dev, generator=g) < 0.3] = -100
    return X, W, y


def forward_both(dev, X, W, y, softcap):
    lib = _lib.load()
    T, H = X.shape
    V = W.shape[0]
    dt = _dtype_code(X.dtype)
    ri, rl, n = prepare_targets(y, V)
    s = _stream(dev)
    loss_a = torch.full((T,), float("nan"), device=dev)
    lse_a = torch.full((n,), float("nan"), device=dev)
    wsb = lib.mt_flce_forward_workspace_bytes(T, n, H, V, dt)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    _lib.check(lib.mt_flce_forward(_p(X), _p(W), T, H, V, X.stride(0), W.stride(0), dt, softcap,
                                   _p(ri), _p(rl), n, _p(loss_a), _p(lse_a), _p(ws), wsb, s),
               "mt_flce_forward")
    loss_b = torch.full((T,), float("nan"), device=dev)
    lse_b = torch.full((n,), float("nan"), device=dev)
    _lib.check(lib.mt_flce_forward_noalloc(_p(X), _p(W), T, H, V, X.stride(0), W.stride(0), dt,
                                           softcap, _p(ri), _p(rl), n, _p(loss_b), _p(lse_b), s),
               "mt_flce_forward_noalloc")
    torch.cuda.synchronize()
    return (loss_a, lse_a), (loss_b, lse_b), n


def rows_per_chunk(V):
    """Valid rows whose forward partials (8 bytes per 256-wide vocabulary
    tile) and label logit (4 bytes) fit the static scratch."""
    scratch = _lib.load().mt_flce_noalloc_scratch_bytes()
    return scratch // (8 * ((V + 255) // 256) + 4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_forward_matches_workspace_forward(gpu, dtype):
    lib = _lib.load()
    assert lib.mt_flce_noalloc_scratch_bytes() == 16 << 20
    # first call: several scratch chunks (bf16: ~10.6k valid rows per chunk at
    # V = 50000); second call: smaller, one chunk, with a softcap
    for (T, H, V, cap, seed) in ((40000, 256, 50000, 0.0, 1), (3000, 128, 7001, 4.0, 2)):
        print(f"case noalloc T={T} H={H} V={V} {dtype} softcap={cap}", flush=True)
        X, W, y = case(gpu, T, H, V, dtype, seed)
        (la, sa), (lb, sb), n = forward_both(gpu, X, W, y, cap)
        if dtype == torch.bfloat16 and T == 40000:
            assert n > rows_per_chunk(V)  # really spans several chunks
        valid = y != -100
        assert torch.equal(lb[~valid], torch.zeros(int((~valid).sum()), device=gpu))
        assert not torch.isnan(lb).any() and not torch.isnan(sb).any()
        if dtype == torch.bfloat16:
            assert torch.equal(la, lb) and torch.equal(sa, sb)
        else:
            assert ((la[valid] - lb[valid]).abs() / la[valid].abs()).max().item() <= 1e-6
            assert ((sa - sb).abs() / sa.abs()).max().item() <= 1e-6


def test_noalloc_forward_under_graph_capture(gpu):
    """Warmed up once (the scratch's address is looked up on a device's first
    call), captured with torch.cuda.graph and replayed three times, with the
    outputs overwritten by NaN and eager work between the replays: each
    replay gives mt_flce_forward's loss and lse bit for bit (bf16; several
    scratch chunks)."""
    print("case noalloc graph capture", flush=True)
    lib = _lib.load()
    T, H, V = 30000, 128, 60000
    X, W, y = case(gpu, T, H, V, torch.bfloat16, 5)
    (la, sa), _, n = forward_both(gpu, X, W, y, 0.0)
    assert n > rows_per_chunk(V)
    ri, rl, n2 = prepare_targets(y, V)
    assert n2 == n
    loss = torch.empty(T, device=gpu)
    lse = torch.empty(n, device=gpu)
    args = (_p(X), _p(W), T, H, V, X.stride(0), W.stride(0), _lib.MT_DTYPE_BF16, 0.0, _p(ri),
            _p(rl), n, _p(loss), _p(lse))
    _lib.check(lib.mt_flce_forward_noalloc(*args, _stream(gpu)), "warm-up")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(lib.mt_flce_forward_noalloc(*args, _stream(gpu)), "captured")
    for i in range(3):
        loss.fill_(float("nan"))
        lse.fill_(float("nan"))
        junk = torch.randn(1 << 20, device=gpu).sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(loss, la) and torch.equal(lse, sa), i
