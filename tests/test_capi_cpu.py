"""C-ABI surface without a GPU: the library loads, exports every symbol the
header declares, and its host-only logic (argument checks, planners) behaves.
No call here launches a kernel."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from mini_trainer_amd import _lib, backward_plan, synth

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mt_flce.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mt_\w+)\s*\(", text)))


def test_header_symbols_exported():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/mt_flce.h but not exported"
    assert sorted(_lib.SIGNATURES) == names, "ctypes signatures must mirror the header"


def test_integration_stub_matches_binding():
    # the ctypes stub shown to maintainers declares the same argument and
    # result types as the package's own binding (which mirrors the header)
    text = (ROOT / "INTEGRATION.md").read_text()
    stub = text.split("```python\nimport ctypes\n", 1)[1].split("assert lib.mt_flce_abi_version", 1)[0]
    stub = stub.replace('lib = ctypes.CDLL("/path/to/libmt_flce.so")', "")

    class Fn:
        pass

    class Lib:
        def __getattr__(self, name):
            f = Fn()
            object.__setattr__(self, name, f)
            return f

    ns = {"lib": Lib()}
    exec("import ctypes\n" + stub, ns)
    declared = {n: f for n, f in vars(ns["lib"]).items() if hasattr(f, "argtypes")}
    assert len(declared) >= 7
    for name, f in declared.items():
        restype, argtypes = _lib.SIGNATURES[name]
        assert list(f.argtypes) == list(argtypes), name
        assert getattr(f, "restype", None) == restype, name


def test_abi_version_matches_header():
    m = re.search(r"#define MT_FLCE_ABI_VERSION (\d+)", HEADER.read_text())
    assert _lib.load().mt_flce_abi_version() == int(m.group(1)) == _lib.ABI_VERSION


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(_lib.FlceError):
        _lib.load()


def call_forward(**kw):
    lib = _lib.load()
    a = dict(X=16, W=16, T=8, H=64, V=100, ldx=64, ldw=64, dtype=1, softcap=0.0, ri=16, rl=16,
             n=4, loss=16, lse=16, ws=16, wsb=1 << 20, stream=None)
    a.update(kw)
    return lib.mt_flce_forward(a["X"], a["W"], a["T"], a["H"], a["V"], a["ldx"], a["ldw"],
                               a["dtype"], a["softcap"], a["ri"], a["rl"], a["n"], a["loss"],
                               a["lse"], a["ws"], a["wsb"], a["stream"])


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=7), 1),            # unknown dtype
    (dict(H=100, ldx=104, ldw=104), 3),  # H not whole 16-byte chunks (bf16: multiple of 8)
    (dict(ldx=32), 1),             # ldx < H
    (dict(ldx=68), 1),             # row pitch not a multiple of 16 bytes
    (dict(X=18), 1),               # misaligned X
    (dict(n=9), 1),                # n_valid > T
    (dict(T=-1), 1),
    (dict(V=0), 1),
    (dict(softcap=-1.0), 1),
    (dict(wsb=0), 2),              # workspace too small
    (dict(W=None), 1),
])
def test_forward_host_checks(kw, code):
    assert call_forward(**kw) == code
    assert _lib.load().mt_flce_last_error()


def test_backward_and_misc_host_checks():
    lib = _lib.load()
    args = [16, 16, 8, 64, 100, 64, 64, 1, 0.0, 16, 16, 4, 16, 16, 1, 16, 64, 16, 64, 0]
    # chunk sizes must be positive multiples of 256
    assert lib.mt_flce_backward(*args, 100, 256, 16, 1 << 30, None) == 1
    # workspace too small for the requested blocks
    assert lib.mt_flce_backward(*args, 256, 256, 16, 10, None) == 2
    # a bf16 G block beyond the 4 GiB reach of 32-bit buffer offsets
    assert lib.mt_flce_backward(*args, 65536, 65536, 16, 1 << 62, None) == 3
    assert "4 GiB" in lib.mt_flce_last_error().decode()
    # negative grad stride
    bad = list(args)
    bad[14] = -1
    assert lib.mt_flce_backward(*bad, 256, 256, 16, 1 << 30, None) == 1
    assert lib.mt_flce_prepare(None, -1, 10, -100, 0, None, None, None, None) == 1
    assert lib.mt_segment_sum(None, None, 4, -100, 0, None, 1, None, None, None, None) == 1
    # scale_grads: null scale; in place with another pitch; in-place narrowing
    # beyond the row width one workgroup holds
    assert lib.mt_flce_scale_grads(None, None, 0, 64, 64, 1, None, 0, 64, None, 64, 0, None) == 1
    assert lib.mt_flce_scale_grads(16, None, 0, 64, 64, 1, 16, 4, 64, 16, 72, 1, None) == 1
    assert "ldo == lddw" in lib.mt_flce_last_error().decode()
    assert lib.mt_flce_scale_grads(16, None, 0, 20000, 20000, 1, 16, 4, 20000, 16, 20000, 1,
                                   None) == 3
    assert "H <= 16384" in lib.mt_flce_last_error().decode()
    assert lib.mt_ce_forward(None, 4, 10, 5, 1, None, -100, None, None, None, None) == 1


def dw_layout(V, H):
    lib = _lib.load()
    lo, rows, hi = ctypes.c_size_t(), ctypes.c_int64(), ctypes.c_size_t()
    st = lib.mt_flce_dw_tiles_layout(V, H, ctypes.byref(lo), ctypes.byref(rows), ctypes.byref(hi))
    return st, lo.value, rows.value, hi.value


def test_dw_tiles_layout_and_host_checks():
    """Tiled dW over two buffers: `lo` is exactly the bf16 [V, H] gradient
    (V H 2 bytes) and holds, after a pad of half a tile row, as many whole
    tile rows as fit; `hi` holds the rest.  Together they hold at least the
    fp32 gradient; the narrowing's in-place order is safe (the bf16 rows of
    tile row r end before tile row floor((r + 1) / 2) starts, and every tile
    row it writes over comes earlier).  Argument checks return before any
    launch."""
    lib = _lib.load()
    for V, H in [(100, 64), (256, 256), (65600, 1056), (128256, 4096), (1, 8), (151936, 1536),
                 (768, 256), (767, 256), (300, 1000)]:
        st, lo, rows, hi = dw_layout(V, H)
        assert st == 0 and lo == V * H * 2
        Hp, R = -(-H // 256) * 256, -(-V // 256)
        tr, pad = Hp * 256 * 4, Hp * 256 * 2
        if rows > 0:
            assert pad + rows * tr <= lo < pad + (rows + 1) * tr or rows == R
        else:
            assert lo < pad + tr
        assert hi == (R - rows) * tr
        assert lo + hi >= V * H * 4
        for r in range(R):  # narrowing tile row r writes bf16 bytes [256 r H 2, ...)
            end = min(V, 256 * (r + 1)) * H * 2
            q = (r + 1) // 2  # first fp32 tile row not yet read when row r is narrowed
            assert q >= rows or end <= pad + q * tr
    assert dw_layout(0, 64)[0] == 1 and dw_layout(10, -1)[0] == 1
    st, lo, rows, hi = dw_layout(100, 64)
    p = 1 << 20  # aligned dummy addresses, never dereferenced
    # fused_tiles: lo below V H 2, hi below the layout's, fp32 operands
    def fused(dt=1, lo_b=lo, hi_ptr=p + (1 << 16), hi_b=hi):
        return lib.mt_flce_fused_tiles(16, 16, 8, 64, 100, 64, 64, dt, 0.0, 16, 16, 4, 16, 0, 16,
                                       16, 16, 64, p, lo_b, hi_ptr, hi_b, 0, 256, 16, 1 << 30, None)
    assert fused(lo_b=lo - 2) == 1
    assert "V H 2" in lib.mt_flce_last_error().decode()
    assert fused(hi_b=hi - 16) == 1
    assert "mt_flce_dw_tiles_layout" in lib.mt_flce_last_error().decode()
    assert fused(hi_ptr=p + 4096) == 1                 # hi overlaps lo
    assert "overlap" in lib.mt_flce_last_error().decode()
    assert fused(dt=0) == 3                            # the fused path is bf16 only
    # backward_tiles: fp32 unsupported, buffers below the layout's sizes
    bargs = [16, 16, 8, 64, 100, 64, 64]
    rest = [0.0, 16, 16, 4, 16, 16, 1, 16, 64]

    def btiles(dt=1, lo_b=lo, hi_b=hi, C=256):
        return lib.mt_flce_backward_tiles(*bargs, dt, *rest, p, lo_b, p + (1 << 16), hi_b, 0, C,
                                          256, 16, 1 << 30, None)
    assert btiles(dt=0) == 3
    assert btiles(hi_b=hi - 16) == 1
    assert btiles(lo_b=0) == 1
    assert btiles(C=100) == 1                          # blocks: positive multiples of 256

    def narrow(**kw):
        a = dict(scale=16, lo=p, lo_b=lo, hi=p + (1 << 16), hi_b=hi, V=100, H=64)
        a.update(kw)
        return lib.mt_flce_narrow_tiles(a["scale"], a["lo"], a["lo_b"], a["hi"], a["hi_b"],
                                        a["V"], a["H"], None)
    H60 = dw_layout(100, 60)
    assert narrow(H=60, lo_b=H60[1], hi_b=H60[3]) == 3  # H % 8
    assert narrow(lo_b=lo - 1) == 1                    # buffers too small
    assert narrow(hi_b=hi - 1) == 1
    assert narrow(lo=p + 8) == 1                       # misaligned
    assert narrow(scale=None) == 1
    assert narrow(V=0) == 1


@pytest.mark.parametrize("key", [1, 2, 3, 4, 5])
def test_backward_plan_fits_budget(key):
    cfg = synth.CONFIGS[key]
    n = int((synth.make_batch(cfg, 0, with_tensors=False)["target"] != -100).sum())
    C, Cv, ws = backward_plan(cfg.T, n, cfg.H, cfg.V, cfg.dtype)
    es = 2 if cfg.dtype == torch.bfloat16 else 4
    assert C % 256 == 0 and Cv % 256 == 0 and C >= 256 and Cv >= 256
    assert ws <= 0.05 * cfg.T * cfg.V * es
    # the workspace formula: G block + fp32 dX accumulator (if V is split) + X^T block
    # + (bf16) the 8 counters of dW's work queue
    al = lambda b: (b + 255) // 256 * 256  # noqa: E731
    expect = (al(C * Cv * es) + (al(C * cfg.H * 4) if Cv < cfg.V else 0) + al(cfg.H * C * es) +
              (al(8 * 4) if es == 2 else 0))
    assert ws == expect


@pytest.mark.parametrize("key", [2, 3, 4, 5])
def test_backward_narrow_plan_fits_budget(key):
    """The narrowing plan: within the budget; one row block (C >= n) keeps
    dX's accumulator and X^T in the narrowing scratch (the workspace holds
    the G block and the counters only); more row blocks have mt_flce_backward's
    workspace.  Config 5 (H = 8192, a 210 MB budget) takes one row block per
    minibatch; fp32 has no narrowing path."""
    cfg = synth.CONFIGS[key]
    n = int((synth.make_batch(cfg, 0, with_tensors=False)["target"] != -100).sum())
    C, Cv, ws = backward_plan(cfg.T, n, cfg.H, cfg.V, cfg.dtype, narrow=True)
    assert C % 256 == 0 and Cv % 256 == 0 and ws <= 0.05 * cfg.T * cfg.V * 2
    al = lambda b: (b + 255) // 256 * 256  # noqa: E731
    one = C >= n
    if one:
        expect = al(C * Cv * 2) + al(8 * 4)
    else:
        expect = (al(C * Cv * 2) + (al(C * cfg.H * 4) if Cv < cfg.V else 0) +
                  al(cfg.H * C * 2) + al(8 * 4))
    assert ws == expect
    if key == 5:
        assert one
    with pytest.raises(_lib.FlceError):
        backward_plan(cfg.T, n, cfg.H, cfg.V, torch.float32, narrow=True)


def test_backward_narrow_plan_workspace_formula():
    """Over random shapes and budgets: the narrowing plan's blocks are
    multiples of 256 and its workspace is the formula mt_flce_backward_narrow
    checks -- the G block and the counters when one row block's accumulator
    (as 256 x 256 tiles) and X^T fit in what a bf16 gradient leaves of the
    fp32 one (they then go to the scratch of mt_flce_narrow_scratch_bytes),
    else the G block, the row-major accumulator (several vocabulary blocks),
    X^T and the counters; within the budget unless nothing fits (the 256 x
    256 fallback)."""
    lib = _lib.load()
    rng = np.random.default_rng(3)
    al = lambda b: (b + 255) // 256 * 256  # noqa: E731
    cd = lambda a, b: -(-a // b)  # noqa: E731
    for _ in range(300):
        T = int(rng.integers(1, 40000))
        n = int(rng.integers(1, T + 1))
        H = int(rng.integers(1, 80)) * 64
        V = int(rng.integers(256, 160000))
        budget = int(rng.choice([0, 1, int(rng.integers(1, 1 << 30))]))
        C, Cv, ws = backward_plan(T, n, H, V, torch.bfloat16, budget_bytes=budget, narrow=True)
        assert C % 256 == 0 and Cv % 256 == 0 and C > 0 and Cv > 0
        Hp = cd(H, 256) * 256
        tb = Hp * 256 * 2 + cd(V, 256) * Hp * 256 * 4  # the fp32 gradient the budget counts
        need = al(cd(C, 256) * cd(H, 256) * 65536 * 4) + al(H * C * 2)
        fits = C >= n and tb >= al(V * H * 2) + need
        # the scratch that holds dX's accumulator and X^T outside the workspace
        assert int(lib.mt_flce_narrow_scratch_bytes(V, H, C)) == \
            (need if tb >= al(V * H * 2) + need else 0)
        if fits:
            expect = al(C * Cv * 2) + al(32)
        else:
            expect = al(C * Cv * 2) + (al(C * H * 4) if Cv < V else 0) + al(H * C * 2) + al(32)
        assert ws == expect, (T, n, H, V, budget, C, Cv)
        b = budget or int(0.05 * T * V * 2)
        assert ws <= b or (C, Cv) == (256, 256)


def test_forward_keep_host_checks():
    """mt_flce_forward_keep refuses fp32, a softcap, keep_cols not a multiple
    of 256 or not below V, and a keep buffer below round_up(n_valid, 256) x
    keep_cols bf16, before touching any pointer."""
    lib = _lib.load()
    T, H, V, n = 1000, 128, 5000, 700
    p = 16

    def call(dtype=1, cap=0.0, K=512, kb=768 * 512 * 2, guard=16):
        return lib.mt_flce_forward_keep(p, p, T, H, V, H, H, dtype, cap, p, p, n, p, p, p,
                                        1 << 30, p, K, kb, guard, None)
    assert call(dtype=0) == 3
    assert call(cap=5.0) == 3
    assert call(K=500) == 1
    assert call(K=5120) == 1
    assert call(kb=768 * 512 * 2 - 2) == 1
    assert call(guard=None) == 1


def test_backward_narrow_host_checks():
    """mt_flce_backward_narrow refuses fp32, H not a multiple of 8, an output
    below V H 2 bytes, a scratch below mt_flce_narrow_scratch_bytes and more
    than one row block, before touching any pointer."""
    lib = _lib.load()
    T, H, V, n = 1000, 128, 5000, 700
    need = int(lib.mt_flce_narrow_scratch_bytes(V, H, 768))
    assert need > 0
    p = 16  # a dummy, aligned, never-dereferenced address

    def call(dtype=1, h=H, ld=H, ob=V * H * 2, sp=p, sb=need, C=768, Cv=1024):
        return lib.mt_flce_backward_narrow(p, p, T, h, V, ld, ld, dtype, 0.0, p, p, n, p, p, 0, p,
                                           ld, p, ob, sp, sb, C, Cv, p, 1 << 40, None, None)
    assert call(dtype=0) == 3
    assert call(h=100, ld=104) == 3
    assert call(ob=V * H * 2 - 1) == 1
    assert call(sb=need - 16) == 1
    assert "mt_flce_narrow_scratch_bytes" in lib.mt_flce_last_error().decode()
    assert call(sp=None) == 1
    assert call(C=512) == 1
    assert lib.mt_flce_narrow_scratch_bytes(V, H, 0) == 0


def test_backward_plan_budget_override_and_degenerate():
    C, Cv, ws = backward_plan(1000, 700, 128, 5000, torch.bfloat16, budget_bytes=1)
    assert (C, Cv) == (256, 256)  # smallest blocks when nothing fits
    C, Cv, ws = backward_plan(1000, 0, 128, 5000, torch.bfloat16)
    assert (C, Cv, ws) == (0, 0, 0)
    C, Cv, ws = backward_plan(4096, 3000, 128, 5000, torch.bfloat16, budget_bytes=1 << 40)
    assert Cv >= 5000 and C >= 3000  # everything in one block


def test_forward_workspace_is_small():
    lib = _lib.load()
    for key in (2, 3, 4, 5):
        cfg = synth.CONFIGS[key]
        ws = lib.mt_flce_forward_workspace_bytes(cfg.T, cfg.T, cfg.H, cfg.V, 1)
        # one (max, sum) fp32 pair per (row, 256-wide vocabulary tile) plus the
        # label logit: at most 1/64 + 1/(2V) of the bf16 logits it replaces
        per_row = -(-cfg.V // 256) * 8 + 4
        assert 0 < ws <= cfg.T * per_row + 512
        assert ws < 0.02 * cfg.T * cfg.V * 2
    assert lib.mt_flce_forward_workspace_bytes(10, 0, 64, 100, 1) == 0


def test_fused_planner_prefers_the_faster_path():
    """Routing of configs 2-5, against the general path each call would
    otherwise take.  With the weight gradient wanted in bf16 (the reference's
    call chain, no accumulator) that is the narrowing plan -- one row block
    through mt_flce_backward_narrow after mt_flce_forward_keep, or tiles and
    the narrowing pass -- and with an fp32 accumulator it is
    mt_flce_backward.  Either way the fused path pays at configs 2, 3 and 4
    (same-box steps, fused against general: 21.8 vs 25.3 ms at config 2,
    111-113 vs 143-145 ms at config 3, 173-177 ms against a modelled 226 at
    config 4) and not at config 5, whose 5% budget forces 512-row chunks
    (182-189 vs 163-167 ms)."""
    lib = _lib.load()
    want = {2: 1, 3: 1, 4: 1, 5: 0}
    for key, pays_expected in want.items():
        cfg = synth.CONFIGS[key]
        n = int((synth.make_batch(cfg, 0, with_tensors=False)["target"] != -100).sum())
        for acc in (0, 1):
            c, ws, pays = ctypes.c_int64(), ctypes.c_size_t(), ctypes.c_int()
            assert lib.mt_flce_fused_plan(cfg.T, n, cfg.H, cfg.V, 1, 0, acc, ctypes.byref(c),
                                          ctypes.byref(ws), ctypes.byref(pays)) == 0
            assert pays.value == pays_expected, (key, acc)
            assert c.value % 256 == 0 and 0 < ws.value <= 0.05 * cfg.T * cfg.V * 2
    c, ws, pays = ctypes.c_int64(), ctypes.c_size_t(), ctypes.c_int()
    assert lib.mt_flce_fused_plan(100, 50, 64, 100, 0, 0, 0, ctypes.byref(c), ctypes.byref(ws),
                                  ctypes.byref(pays)) == 3  # fp32: unsupported


def test_buffer_reach_hook(monkeypatch):
    """MT_FLCE_MAX_BUFFER_BYTES lowers the reach of one bf16 buffer: X beyond it
    is rejected (the host layer splits rows), 256 weight rows beyond it too,
    and the fused path rejects a weight beyond it (no kernel is launched)."""
    lib = _lib.load()
    assert lib.mt_flce_max_buffer_bytes() == 0xFFFFFFFF
    monkeypatch.setenv("MT_FLCE_MAX_BUFFER_BYTES", "4096")
    assert lib.mt_flce_max_buffer_bytes() == 4096
    # X of 8 rows x 64 bf16 = 1 KiB fits; 64 rows = 8 KiB does not
    assert call_forward(T=64, n=4) == 3
    assert "row ranges" in lib.mt_flce_last_error().decode()
    # fused: W of 100 x 64 bf16 = 12.8 KB beyond 4 KiB
    assert lib.mt_flce_fused(16, 16, 8, 64, 100, 64, 64, 1, 0.0, 16, 16, 4, 16, 0, 16, 16, 16, 64,
                             16, 64, 0, 256, 16, 1 << 30, None) == 3
    assert "one buffer" in lib.mt_flce_last_error().decode()
    monkeypatch.setenv("MT_FLCE_MAX_BUFFER_BYTES", "1000")
    # 256 weight rows of 128 bytes exceed 1000 bytes
    assert call_forward(T=4, n=2) == 3
    assert "256 of them" in lib.mt_flce_last_error().decode()


def test_launch_failure_surfaces_as_flce_error(monkeypatch):
    """A launch the HIP runtime refuses (here: no GPU in this process) comes
    back as MT_ERR_HIP with the kernel's name and the runtime's text, which
    the binding raises as FlceError (a RuntimeError); the test hook
    MT_FLCE_TEST_FAIL_LAUNCH reports the same for a named launch.  CPU only:
    the call's pointers are dummies that a GPU would fault on."""
    if torch.cuda.is_available():
        pytest.skip("launches with dummy pointers: a process without a GPU only")
    lib = _lib.load()
    p = 1 << 20
    rc = lib.mt_flce_prepare(p, 10, 100, -100, 0, p, p, p, None)
    assert rc == 4
    with pytest.raises(_lib.FlceError, match="mt_flce_prepare: MT_ERR_HIP: prepare_kernel: "):
        _lib.check(rc, "mt_flce_prepare")
    assert issubclass(_lib.FlceError, RuntimeError)
    monkeypatch.setenv("MT_FLCE_TEST_FAIL_LAUNCH", "prepare")
    rc = lib.mt_flce_prepare(p, 10, 100, -100, 0, p, p, p, None)
    assert rc == 4 and "injected launch failure" in lib.mt_flce_last_error().decode()
