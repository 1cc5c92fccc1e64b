"""Benchmark of the fused LM-head linear + per-token cross-entropy on one MI355X.

One step = the hot path of one optimizer step's minibatches exactly as
train.py:97-104 drives it, through the drop-in
liger_fixed_fused_linear_cross_entropy_none_reduction with the reference's
own arguments: forward, `output.loss.float().sum()`, the `.item()` sync,
`loss * world_size / batch_num_loss_counted_tokens`, `backward()`; the
lm_head gradient accumulates into `W.grad` across the minibatches (config 5:
four) and is cleared after the step, as the optimizer's zero_grad does.
bf16 shapes where the fused path pays take it without any promise (dX and dW
formed at the forward for a unit upstream gradient, rescaled in the
backward).  Inputs are seeded synthetic tensors of the named configuration,
resident in HBM before timing starts.

Prints ONE JSON line (driver contract) with, in addition:
  roofline      the dominant unit of the timed step (the side-by-side dX and
                dW GEMMs of each fused chunk, one launch: 2*C*V*H flops
                each), timed live with the library's per-launch HIP events on
                the stream the kernel runs on, against the bf16 dense peak;
                `kernels` lists every kernel of the step the same way (with
                the GEMMs' calibrated counter bytes per dispatch);
                traffic = HBM bytes per launch from the committed rocprofv3
                FETCH_SIZE / WRITE_SIZE summary (profiles/)
  cpu_baseline  the reference torch path (oracle/torch_path.py) on the host
                cores over a bounded prefix of the same batch
  north_star    6*H*V*N / t_step against the same peak, extra HBM, the
                promised-gradient and general paths, the other configurations
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from typing import Optional

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from mini_trainer_amd import _lib, synth  # noqa: E402
from mini_trainer_amd.flce import (FUSED_ENV, _dtype_code, _p, _stream,  # noqa: E402
                                   backward_plan, fused_linear_cross_entropy, path_of,
                                   prepare_targets, profile_enable, profile_report)
from mini_trainer_amd.none_reduction_losses import (  # noqa: E402
    liger_fixed_fused_linear_cross_entropy_none_reduction as drop_in)

PEAK_BF16 = 2.5166e15  # MI355X dense bf16 MFMA, 256 CU x 2.4 GHz x 4096 flop/clk
PEAK_FP32 = 157.3e12
PEAK_HBM = 8.0e12
METRIC = "fused linear-CE fwd+bwd tokens/s on 1 GPU; MFMA util % of peak; extra HBM GB"
WORLD_SIZE = 1  # train.py:102's world_size on one GPU


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(cfg, budget_s: float):
    """Reference torch path on the CPU over a bounded prefix of the batch."""
    from oracle.torch_path import torch_path

    threads = torch.get_num_threads()
    b = synth.make_batch(cfg, 0, with_tensors=False)
    g = torch.Generator().manual_seed(cfg.key)
    rows = 128
    X = torch.randn(4096, cfg.H, generator=g).to(cfg.dtype)
    W = synth.make_weight(cfg)
    y = b["target"][:4096]
    grad = torch.full((4096,), 1.0)
    spent, done_rows, t_total = 0.0, 0, 0.0
    while True:
        t0 = time.perf_counter()
        torch_path(X[:rows], W, y[:rows], grad=grad[:rows], chunk_rows=1024)
        dt = time.perf_counter() - t0
        done_rows, t_total = rows, dt
        spent += dt
        if dt * 2.5 > budget_s - spent or rows >= 4096:
            break
        rows *= 2
    return {
        "value": done_rows / t_total,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"reference torch path (F.linear {str(cfg.dtype).replace('torch.', '')} -> "
                   f".float() -> F.cross_entropy(reduction='none') + autograd backward, "
                   f"none_reduction_losses.py:35) on the first {done_rows} packed rows of "
                   f"config {cfg.key} (T x V logits in 1024-row chunks), {t_total:.1f} s, "
                   f"torch threads={threads}, host cpus={os.cpu_count()}"),
    }


def torch_gpu_path(data, W, scale: float, steps: int = 2):
    """The reference's torch path on the GPU as a comparator: per minibatch
    F.linear in the model dtype (TF/models/llama/modeling_llama.py:480), the
    fp32 upcast (TF/loss/loss_utils.py:59), F.cross_entropy(reduction='none')
    (none_reduction_losses.py:35), sum, .item(), backward with the uniform
    scale (train.py:98-104).  It materialises T x V logits, their fp32 copy,
    the saved log-softmax and its gradient (~16 bytes per logit), so it runs
    only where that fits beside what is already allocated."""
    dev = W.device
    T, V = data[0][0].shape[0], W.shape[0]
    need = 16 * T * V + (8 << 30)
    free, total = torch.cuda.mem_get_info(dev)
    if need > free:
        return {"skipped": f"needs ~{need / 1e9:.0f} GB of device memory, {free / 1e9:.0f} GB free"}
    Wr = W.detach().requires_grad_(True)

    def step():
        for X, y in data:
            Xr = X.detach().requires_grad_(True)
            logits = torch.nn.functional.linear(Xr, Wr).float()
            loss = torch.nn.functional.cross_entropy(logits, y, ignore_index=-100, reduction="none")
            s = loss.sum()
            s.item()
            (s * scale).backward()
            del logits, loss, s, Xr
        Wr.grad = None

    try:
        step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
    except torch.cuda.OutOfMemoryError as e:  # reported, not fatal: a comparator only
        Wr.grad = None
        torch.cuda.empty_cache()
        return {"skipped": f"out of memory ({str(e).splitlines()[0][:80]})"}
    ms = e0.elapsed_time(e1) / steps
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "tokens_per_s": T * len(data) / (ms / 1e3), "steps": steps,
            "path": "F.linear -> .float() -> F.cross_entropy(reduction='none') -> backward (torch on the GPU)"}


def traffic_summary(key: int):
    """The committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of this
    workload (bytes calibrated against a 1 GiB device copy), or None."""
    path = os.path.join(ROOT, "profiles", f"flce_cfg{key}_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def measured_traffic(key: int, unit: str):
    """HBM bytes per launch of the roofline unit from that summary, or None
    when no summary covers it."""
    t = traffic_summary(key)
    if not t or t.get("unit") != unit:
        return None
    return t.get("traffic_bytes")


def add_counter_bytes(kernels: dict, key: int) -> None:
    """Per-dispatch read / written bytes of the summary's kernels (same
    names as the event report) beside their event timings, and, where the
    summary has them, the kernel's MFMA counters from a pass that runs each
    dispatch alone: busy fraction per busy-CU cycle, clock, whole-chip
    utilisation."""
    t = traffic_summary(key) or {}
    for name, b in t.get("per_kernel", {}).items():
        if name in kernels:
            kernels[name]["counter_read_GB_per_launch"] = b["read_bytes"] / 1e9
            kernels[name]["counter_write_GB_per_launch"] = b["write_bytes"] / 1e9
            for k in ("mfma_busy", "clock_GHz", "mfma_util"):
                if k in b:
                    kernels[name]["counter_" + k + "_alone"] = b[k]
    # dX and dW of the phase as two kernels (MT_FLCE_SPLIT_PHASE=1), counted
    # apart: their MFMA busy fractions inside the one launch the step runs
    for name, b in t.get("split_parts", {}).items():
        kernels.setdefault("dx_dw_phase", {}).setdefault("parts_launched_apart", {})[name] = b


def copy_calibration():
    """One device-to-device copy of exactly 1 GiB: under rocprofv3 --pmc its
    FETCH_SIZE / WRITE_SIZE readings (KiB per dispatch) against 1048576 KiB
    give the factor that turns those counters into bytes."""
    n = 1 << 28
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": 4 * n}), flush=True)


def mfma_ceiling(dev, shapes=(0, 1), cu_counts=None, launches: int = 3) -> dict:
    """The register-only bf16 MFMA stream (mt_flce_probe_mfma) on P CUs:
    achieved TFLOP/s and its fraction of the dense peak of the P CUs and of
    the chip, timed with HIP events on the current stream (the stream it is
    launched on).  Operands: random bf16 in N(0, 1)."""
    lib = _lib.load()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    Ps = cu_counts or sorted({max(1, cus // 4), cus // 2, 3 * cus // 4, cus})
    g = torch.Generator(device=dev).manual_seed(7)
    ops = torch.randn(max(Ps) * 256 * 16 * 8, device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty(max(Ps) * 256, device=dev)
    stream = _stream(dev)
    res = {}
    for shape in shapes:
        name = ("v_mfma_f32_16x16x32_bf16", "v_mfma_f32_32x32x16_bf16")[shape]
        fl_it = float(1 << 20) if shape == 0 else float(1 << 19)
        iters = 60000 if shape == 0 else 120000
        rows = {}
        for P in Ps:
            call = lambda: _lib.check(lib.mt_flce_probe_mfma(shape, P, iters, _p(ops), _p(out),
                                                             stream), "mt_flce_probe_mfma")
            call()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(launches):
                call()
            e1.record()
            torch.cuda.synchronize()
            s = e0.elapsed_time(e1) / launches / 1e3
            rate = fl_it * iters * 4 * P / s
            rows[str(P)] = {"ms_per_launch": s * 1e3, "TFLOPs": rate / 1e12,
                            "frac_of_P_CU_peak": rate / (PEAK_BF16 * P / cus),
                            "frac_of_chip_peak": rate / PEAK_BF16}
        res[name] = rows
    return res


class ForcedPath:
    """Sets MT_FLCE_FUSED for the duration of a block ("0": general path)."""

    def __init__(self, value):
        self.value, self.old = value, None

    def __enter__(self):
        self.old = os.environ.get(FUSED_ENV)
        if self.value is not None:
            os.environ[FUSED_ENV] = self.value

    def __exit__(self, *exc):
        if self.old is None:
            os.environ.pop(FUSED_ENV, None)
        else:
            os.environ[FUSED_ENV] = self.old


def reference_minibatch(X, y, Wl, n_counted: int, paths=None):
    """train.py:97-104 for one minibatch through the drop-in; W.grad
    accumulates."""
    Xl = X.detach().requires_grad_(True)
    out_loss = drop_in(Xl, Wl, y)
    if paths is not None:
        paths.append(path_of(out_loss))
    loss = out_loss.float().sum()
    loss.item()  # train.py:99
    loss = loss * WORLD_SIZE / n_counted  # train.py:102
    loss.backward()  # train.py:104


def reference_step(data, Wl, n_counted: int, paths=None):
    """train.py:97-104 for each minibatch through the drop-in, W.grad
    accumulating across them, cleared at the end (the optimizer's zero_grad)."""
    for X, y in data:
        reference_minibatch(X, y, Wl, n_counted, paths)
    Wl.grad = None


def promise_step(data, Wl, n_counted: int, dW):
    """The same chain with the scale promised at the forward (grad_scale) and
    the lm_head gradient accumulated in fp32 into dW (no rescaling pass)."""
    scale = WORLD_SIZE / n_counted
    for X, y in data:
        Xl = X.detach().requires_grad_(True)
        loss = fused_linear_cross_entropy(Xl, Wl, y, dw_accumulator=dW, grad_scale=scale)
        s = loss.float().sum()
        s.item()
        (s * WORLD_SIZE / n_counted).backward()


def timed(step, steps: int, warmup: int, stats: Optional[dict] = None) -> float:
    """Median ms per step (BASELINE.md's statistic) over `steps` steps after
    `warmup` untimed ones, between device synchronisations: one event after
    each step on the current stream, each step's time the difference of
    consecutive events.  stats, if given, receives the mean, min and max."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record()
    for i in range(steps):
        step()
        evs[i + 1].record()
    torch.cuda.synchronize()
    per = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(steps))
    mid = len(per) // 2
    median = per[mid] if len(per) % 2 else 0.5 * (per[mid - 1] + per[mid])
    if stats is not None:
        stats.update(mean=evs[0].elapsed_time(evs[-1]) / steps, min=per[0], max=per[-1])
    return median


def extra_hbm(data, Wl, n_counted: int, dtype) -> dict:
    """Device memory of the whole reference step, minibatch by minibatch
    with W.grad accumulating across them: each minibatch's allocator peak
    minus what is live when it starts (inputs, and W.grad so far) minus its
    required outputs -- loss [T] fp32, dX [T, H] and the weight gradient in
    the fp32 form the kernels accumulate it in (V H 4 bytes; a path that
    never forms it, the narrowing backward, comes out below zero); the worst
    minibatch is reported.  `..._over_bf16_outputs` counts the weight
    gradient at its own dtype instead.  w_grad_storage_GB: the bytes
    W.grad's storage holds after the step, against its nominal V H es."""
    V, H = Wl.shape
    es = torch.finfo(dtype).bits // 8
    dev = Wl.device
    Wl.grad = None
    worst, worst_own, peak_all = -float("inf"), -float("inf"), 0
    for X, y in data:
        T = X.shape[0]
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        reference_minibatch(X, y, Wl, n_counted)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated(dev)
        peak_all = max(peak_all, peak)
        common = T * 4 + T * H * es
        worst = max(worst, peak - base - common - V * H * 4)
        worst_own = max(worst_own, peak - base - common - V * H * es)
    storage = Wl.grad.untyped_storage().nbytes()
    Wl.grad = None
    T = data[0][0].shape[0]
    return {"extra_hbm_GB": worst / 1e9,
            "extra_hbm_budget_GB": 0.05 * T * V * es / 1e9,
            "extra_hbm_over_bf16_outputs_GB": worst_own / 1e9,
            "w_grad_storage_GB": storage / 1e9,
            "w_grad_nominal_GB": V * H * es / 1e9,
            "peak_memory_GB": peak_all / 1e9}


def roofline_of(report: dict, peak_flops: float, steps: int) -> tuple:
    """(roofline entry of the dominant unit, per-kernel table) from a
    mt_flce_profile_report over `steps` steps."""
    kernels = {}
    for name, r in report.items():
        n, ms = r["launches"], r["ms_total"]
        if r["flops"] > 0:
            ach = r["flops"] / (ms / 1e3)
            kernels[name] = {"launches_per_step": n / steps, "ms_per_launch": ms / n,
                             "ms_per_step": ms / steps, "achieved_TFLOPs": ach / 1e12,
                             "frac": ach / peak_flops, "bound": "mfma"}
        elif r["bytes"] > 0:
            ach = r["bytes"] / (ms / 1e3)
            kernels[name] = {"launches_per_step": n / steps, "ms_per_launch": ms / n,
                             "ms_per_step": ms / steps, "achieved_GBs": ach / 1e9,
                             "frac": ach / PEAK_HBM, "bound": "hbm"}
        else:  # a launch that works only if a device flag says so (time only)
            kernels[name] = {"launches_per_step": n / steps, "ms_per_launch": ms / n,
                             "ms_per_step": ms / steps, "bound": None}
    if "dx_dw_phase" in report:
        unit = "dx_dw_phase"
        # dX and dW share the chip inside the phase: each one's span runs
        # from its own start to its own end, so its frac is not its rate
        for name in kernels:
            if name.startswith(("dx_bf16_kernel", "dw_bf16_kernel")):
                kernels[name]["span_inside"] = "dx_dw_phase"
    else:
        gemms = {k: v for k, v in report.items() if v["flops"] > 0}
        unit = max(gemms, key=lambda k: gemms[k]["ms_total"]) if gemms else None
    if unit is None:
        return None, kernels
    r = report[unit]
    per_launch_s = r["ms_total"] / r["launches"] / 1e3
    flops_per_launch = r["flops"] / r["launches"]
    ach = flops_per_launch / per_launch_s
    return {"bound": "mfma", "kernel": unit, "achieved": ach / 1e12, "peak": peak_flops / 1e12,
            "unit": "TFLOP/s", "frac": ach / peak_flops, "traffic": None,
            "ms_per_launch": per_launch_s * 1e3, "flops_per_launch": flops_per_launch,
            "launches_per_step": r["launches"] / steps,
            "share_of_step": r["ms_total"] / steps}, kernels


def general_forward_roofline(X, W, y, peak_flops: float, reps: int) -> dict:
    """The general path's logits GEMM alone (fwd_bf16_kernel through
    mt_flce_forward, one launch over all valid rows), HIP events on the
    current stream, which is the stream it is launched on."""
    lib = _lib.load()
    dev = X.device
    T, H = X.shape
    V = W.shape[0]
    ri, rl, n = prepare_targets(y, V)
    dt = _dtype_code(X.dtype)
    loss = torch.empty(T, dtype=torch.float32, device=dev)
    lse = torch.empty(n, dtype=torch.float32, device=dev)
    wsb = lib.mt_flce_forward_workspace_bytes(T, n, H, V, dt)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    stream = _stream(dev)

    def fwd_call():
        _lib.check(lib.mt_flce_forward(_p(X), _p(W), T, H, V, X.stride(0), W.stride(0), dt, 0.0,
                                       _p(ri), _p(rl), n, _p(loss), _p(lse), _p(ws), wsb, stream),
                   "mt_flce_forward")

    fwd_call()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(reps):
        fwd_call()
    ev1.record()
    torch.cuda.synchronize()
    s = ev0.elapsed_time(ev1) / reps / 1e3
    flops = 2.0 * H * V * n
    return {"kernel": "fwd_bf16_kernel (mt_flce_forward)", "ms_per_launch": s * 1e3,
            "achieved": flops / s / 1e12, "frac": flops / s / peak_flops,
            "flops_per_launch": flops}


def device_inputs(cfg, dev):
    """Seeded inputs generated on the device (fast for the extra
    configurations): labels, masks and packing from synth (CPU numpy), X and
    W from a device generator in fp32, cast to the config dtype."""
    data = []
    g = torch.Generator(device=dev).manual_seed(1000 + cfg.key)
    W = (torch.randn(cfg.V, cfg.H, device=dev, generator=g) * cfg.w_std).to(cfg.dtype)
    for j in range(cfg.minibatches):
        b = synth.make_batch(cfg, j, with_tensors=False)
        gx = torch.Generator(device=dev).manual_seed(cfg.key if cfg.minibatches == 1 else 50 + j)
        X = torch.empty(cfg.T, cfg.H, dtype=cfg.dtype, device=dev)
        for r0 in range(0, cfg.T, 8192):  # fp32 draws in slabs keep the peak low
            r1 = min(cfg.T, r0 + 8192)
            X[r0:r1] = torch.randn(r1 - r0, cfg.H, device=dev, generator=gx).to(cfg.dtype)
        data.append((X, b["target"].to(dev)))
    return W, data


def other_config(key: int, dev, steps: int, warmup: int) -> dict:
    cfg = synth.CONFIGS[key]
    W, data = device_inputs(cfg, dev)
    Wl = W.requires_grad_(True)
    n_counted = sum(int((y != -100).sum().item()) for _, y in data)
    paths = []
    reference_step(data[:1], Wl, n_counted, paths)
    ms = timed(lambda: reference_step(data, Wl, n_counted), steps, warmup)
    mem = extra_hbm(data, Wl, n_counted, cfg.dtype)
    peak = PEAK_BF16 if cfg.dtype == torch.bfloat16 else PEAK_FP32
    T_total = cfg.T * len(data)
    out = {"workload": cfg.name, "T": cfg.T, "H": cfg.H, "V": cfg.V, "minibatches": len(data),
           "n_valid": n_counted, "path": paths[0], "steps": steps, "ms_per_step": ms,
           "tokens_per_s": T_total / (ms / 1e3),
           "frac_of_peak_6HVN": 6.0 * cfg.H * cfg.V * n_counted / (ms / 1e3) / peak, **mem}
    del W, Wl, data
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--cpu-budget-s", type=float, default=25.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-torch-gpu", action="store_true",
                    help="skip the reference torch path on the GPU (a comparator, not the metric)")
    ap.add_argument("--no-variants", action="store_true",
                    help="time the reference step only (no promised-gradient / general path)")
    ap.add_argument("--other-configs", default="2,4,5",
                    help="comma-separated configurations also timed (reference step, 3 steps "
                         "on device-generated inputs) when --config is 3; '' for none")
    ap.add_argument("--step-only", action="store_true",
                    help="only the reference step (timed, then profiled): no variants, no "
                         "general-forward roofline, no other configurations or comparators "
                         "(what the committed rocprofv3 summaries run)")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="only run the register-only MFMA stream (mt_flce_probe_mfma) on 1/4, "
                         "1/2, 3/4 and all of the CUs, both MFMA shapes, and print its rates")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device copy (the reference point that scales "
                         "FETCH_SIZE / WRITE_SIZE counter readings to bytes) and exit")
    args = ap.parse_args()
    if args.step_only:
        args.no_variants = args.no_torch_gpu = args.no_cpu_baseline = True
        args.other_configs = ""
    if args.copy_calibration:
        copy_calibration()
        return
    if args.mfma_ceiling:
        _lib.load()
        print(json.dumps({"mfma_ceiling": mfma_ceiling(torch.device("cuda", 0))}), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the dW reduce-scatter across ranks is design-only). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    cfg = synth.CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    _lib.load()
    t0 = time.perf_counter()
    mbs = [synth.make_batch(cfg, j) for j in range(cfg.minibatches)]
    log(f"inputs for config {cfg.key} generated in {time.perf_counter() - t0:.1f}s")
    W = mbs[0]["W"].to(dev)
    data = [(m["X"].to(dev), m["target"].to(dev)) for m in mbs]
    del mbs
    V, H = W.shape
    T = data[0][0].shape[0]
    Wl = W.requires_grad_(True)
    n_valid = [int((y != -100).sum().item()) for _, y in data]
    N_total = sum(n_valid)
    T_total = T * len(data)
    peak_flops = PEAK_BF16 if cfg.dtype == torch.bfloat16 else PEAK_FP32
    alg_flops = 6.0 * H * V * N_total

    paths = []
    reference_step(data, Wl, N_total, paths)
    torch.cuda.synchronize()
    mem = extra_hbm(data, Wl, N_total, cfg.dtype)
    log(f"reference step: path {paths[0]}, extra HBM {mem['extra_hbm_GB']:.3f} GB")

    step_stats = {}
    ms = timed(lambda: reference_step(data, Wl, N_total), args.steps, args.warmup, step_stats)
    t_step = ms / 1e3
    log(f"reference step: median {ms:.2f} ms, mean {step_stats['mean']:.2f} ms")

    # the same steps again with the library's per-launch events: the roofline
    # unit and the per-kernel table of the timed step
    profile_enable(True)
    ms_prof = timed(lambda: reference_step(data, Wl, N_total), args.steps, 0)
    profile_enable(False)
    report = profile_report()
    roof, kernels = roofline_of(report, peak_flops, args.steps)
    if roof is not None:
        roof["traffic"] = measured_traffic(cfg.key, roof["kernel"])
    add_counter_bytes(kernels, cfg.key)
    log(f"profiled step: {ms_prof:.2f} ms; roofline unit {roof and roof['kernel']}")

    north = {
        "alg_flops_6HVN": alg_flops,
        "achieved_TFLOPs": alg_flops / t_step / 1e12,
        "frac_of_peak": alg_flops / t_step / peak_flops,
        "dense_convention_frac": 6.0 * H * V * T_total / t_step / peak_flops,
        "path": paths[0],
        "call": ("liger_fixed_fused_linear_cross_entropy_none_reduction(hidden, W, target) -> "
                 ".float().sum() -> .item() -> * world_size / batch_num_loss_counted_tokens -> "
                 "backward(), W.grad accumulated across minibatches (train.py:97-104)"),
        "profiled_ms_per_step": ms_prof,
        **mem,
    }
    if not args.no_variants and cfg.dtype == torch.bfloat16:
        dW = torch.zeros(V, H, dtype=torch.float32, device=dev)
        ms_p = timed(lambda: promise_step(data, Wl, N_total, dW), args.steps, 1)
        Wl.grad = None
        del dW
        with ForcedPath("0"):
            ms_g = timed(lambda: reference_step(data, Wl, N_total), args.steps, 1)
        north["promised_grad_ms_per_step"] = ms_p
        north["promised_grad_frac_of_peak"] = alg_flops / (ms_p / 1e3) / peak_flops
        north["general_path_ms_per_step"] = ms_g
        north["general_path_frac_of_peak"] = alg_flops / (ms_g / 1e3) / peak_flops
        log(f"promised-gradient step {ms_p:.2f} ms, general path {ms_g:.2f} ms")
        torch.cuda.empty_cache()
    C, Cv, _ = backward_plan(T, n_valid[0], H, V, cfg.dtype, narrow=cfg.dtype == torch.bfloat16)
    gen_fwd = None
    if not args.step_only:
        gen_fwd = general_forward_roofline(data[0][0], W.detach(), data[0][1], peak_flops,
                                           max(3, min(args.steps, 5)))
        torch.cuda.empty_cache()

    out = {
        "metric": METRIC,
        "value": T_total / t_step,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "ms_per_step_stat": "median of the timed steps (per-step HIP events)",
        "ms_per_step_mean": step_stats["mean"],
        "ms_per_step_min": step_stats["min"],
        "ms_per_step_max": step_stats["max"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (seeded; X~N(0,1), W~N(0,%g), packed lognormal samples)" % cfg.w_std,
        "config": {
            "workload": f"config {cfg.key}: {cfg.name} fused LM-head linear + CE fwd+bwd",
            "T": T, "H": H, "V": V, "minibatches": len(data), "n_valid": N_total,
            "general_bwd_chunk_rows": C, "general_bwd_chunk_vocab": Cv,
        },
        "roofline": roof,
        "kernels": kernels,
        "roofline_general_forward": gen_fwd,
        "north_star": north,
    }
    if args.config == 3 and args.other_configs.strip():
        others = {}
        for k in [int(x) for x in args.other_configs.split(",") if x.strip()]:
            t1 = time.perf_counter()
            others[f"config {k}"] = other_config(k, dev, steps=3, warmup=1)
            log(f"config {k}: {others[f'config {k}']['ms_per_step']:.2f} ms "
                f"({others[f'config {k}']['path']}) in {time.perf_counter() - t1:.1f}s")
        out["other_configs"] = others
    if not args.step_only:
        # the chip's ceiling for the GEMMs' MFMA instruction on this box, this run
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        c = mfma_ceiling(dev, shapes=(0,), cu_counts=[cus])["v_mfma_f32_16x16x32_bf16"][str(cus)]
        out["mfma_ceiling"] = {"what": "register-only v_mfma_f32_16x16x32_bf16 stream on every CU "
                                       "(mt_flce_probe_mfma)", **c}
    if not args.no_torch_gpu:
        torch.cuda.empty_cache()
        tg = torch_gpu_path(data, W.detach(), WORLD_SIZE / N_total)
        if "ms_per_step" in tg:
            tg["speedup_of_value"] = out["value"] / tg["tokens_per_s"]
        out["torch_gpu_path"] = tg
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_budget_s)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
