"""Benchmark of the fused LM-head linear + per-token cross-entropy on one MI355X.

One step = the hot path of one training minibatch as train.py:97-104 drives
it: forward, the caller's sum + .item() sync, and the backward with the
uniform upstream gradient 1/N into an fp32 dW accumulator.  train.py knows
that scale before the forward, so the step passes it as grad_scale and bf16
runs the fused path (each logits tile computed once; dX and dW formed during
the forward, the backward checks the gradient it receives); the general path
(forward keeps lse only, backward recomputes the logits) is timed beside it.
Inputs are seeded synthetic tensors of the named configuration, resident in
HBM before timing starts.

Prints ONE JSON line (driver contract) with, in addition:
  roofline      the logits GEMM (fwd_bf16_kernel: 2*H*V*N MFMA flops per
                launch, one launch over all valid rows through
                mt_flce_forward) timed with HIP events through the C ABI on
                the stream it is launched on, against the bf16 dense peak;
                traffic = HBM bytes per launch from the committed rocprofv3
                FETCH_SIZE / WRITE_SIZE summary (profiles/)
  cpu_baseline  the reference torch path (oracle/torch_path.py) on the host
                cores over a bounded prefix of the same batch
  north_star    6*H*V*N / t_step against the same peak, extra HBM, etc.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from mini_trainer_amd import _lib, synth  # noqa: E402
from mini_trainer_amd.flce import (_dtype_code, _p, _stream, backward_plan,  # noqa: E402
                                   fused_linear_cross_entropy, fused_plan, prepare_targets)

PEAK_BF16 = 2.5166e15  # MI355X dense bf16 MFMA, 256 CU x 2.4 GHz x 4096 flop/clk
PEAK_FP32 = 157.3e12
METRIC = "fused linear-CE fwd+bwd tokens/s on 1 GPU; MFMA util % of peak; extra HBM GB"


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


def measured_traffic(key: int, kernel: str):
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary of this workload (calibrated
    against a 1 GiB device copy), or None when no summary covers it."""
    path = os.path.join(ROOT, "profiles", f"flce_cfg{key}_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("kernel") != kernel:
        return None
    return t.get("traffic_bytes")


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
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device copy (the reference point that scales "
                         "FETCH_SIZE / WRITE_SIZE counter readings to bytes) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the dW reduce-scatter across ranks is design-only). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    cfg = synth.CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    lib = _lib.load()
    t0 = time.perf_counter()
    mbs = [synth.make_batch(cfg, j) for j in range(cfg.minibatches)]
    log(f"inputs for config {cfg.key} generated in {time.perf_counter() - t0:.1f}s")
    W = mbs[0]["W"].to(dev)
    data = [(m["X"].to(dev), m["target"].to(dev)) for m in mbs]
    del mbs
    V, H = W.shape
    T = data[0][0].shape[0]
    dW = torch.zeros(V, H, dtype=torch.float32, device=dev)
    Wl = W.requires_grad_(True)
    n_valid = [int((y != -100).sum().item()) for _, y in data]
    N_total = sum(n_valid)
    T_total = T * len(data)

    scale = 1.0 / N_total  # train.py:102 with world_size 1: known before the forward

    def make_step(fused: bool):
        def step():
            # one optimizer step's worth of minibatches (config 5: 4 grad-accum minibatches)
            for X, y in data:
                Xl = X.detach().requires_grad_(True)
                loss = fused_linear_cross_entropy(Xl, Wl, y, dw_accumulator=dW,
                                                  grad_scale=scale if fused else None)
                s = loss.float().sum()
                s.item()  # the caller's sync (train.py:99)
                torch.autograd.grad(s * scale, (Xl,))
        return step

    def timed(step):
        for _ in range(args.warmup):
            step()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(args.steps):
            step()
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / args.steps

    fused = cfg.dtype == torch.bfloat16
    step = make_step(fused)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # extra HBM of one step: allocator peak - live inputs/outputs
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(dev)
    es = torch.finfo(cfg.dtype).bits // 8
    outputs = T * 4 + T * H * es  # loss + dX of the live minibatch (dW fp32 is preallocated)
    extra = peak - base - outputs
    budget = 0.05 * T * V * es

    ms = timed(step)
    t_step = ms / 1e3
    # the general path (gradient not known at the forward: recompute in the backward)
    ms_general = timed(make_step(False)) if fused else ms
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    # dominant kernel: fwd_kernel via mt_flce_forward on the current stream
    X, y = data[0]
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
    reps = max(3, args.steps)
    ev0.record()
    for _ in range(reps):
        fwd_call()
    ev1.record()
    torch.cuda.synchronize()
    fwd_s = ev0.elapsed_time(ev1) / reps / 1e3
    fwd_flops = 2.0 * H * V * n
    peak_flops = PEAK_BF16 if cfg.dtype == torch.bfloat16 else PEAK_FP32
    C, Cv, bws = backward_plan(T, n, H, V, cfg.dtype)

    fwd_kernel_name = "fwd_bf16_kernel" if cfg.dtype == torch.bfloat16 else "fwd_kernel"
    fused_taken = fused and fused_plan(T, n_valid[0], H, V)[2]
    traffic = measured_traffic(cfg.key, fwd_kernel_name)

    alg_flops = 6.0 * H * V * N_total
    out = {
        "metric": METRIC,
        "value": T_total / t_step,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (seeded; X~N(0,1), W~N(0,%g), packed lognormal samples)" % cfg.w_std,
        "config": {
            "workload": f"config {cfg.key}: {cfg.name} fused LM-head linear + CE fwd+bwd",
            "T": T, "H": H, "V": V, "minibatches": len(data), "n_valid": N_total,
            "bwd_chunk_rows": C, "bwd_chunk_vocab": Cv,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": f"{fwd_kernel_name} (mt_flce_forward)",
            "achieved": fwd_flops / fwd_s / 1e12,
            "peak": peak_flops / 1e12,
            "unit": "TFLOP/s",
            "frac": fwd_flops / fwd_s / peak_flops,
            "traffic": traffic,
            "ms_per_launch": fwd_s * 1e3,
            "flops_per_launch": fwd_flops,
        },
        "north_star": {
            "alg_flops_6HVN": alg_flops,
            "achieved_TFLOPs": alg_flops / t_step / 1e12,
            "frac_of_peak": alg_flops / t_step / peak_flops,
            "dense_convention_frac": 6.0 * H * V * T_total / t_step / peak_flops,
            "path": ("fused: grad_scale = 1/N passed at the forward (mt_flce_fused, 6HVN)"
                     if fused_taken else
                     "general (mt_flce_forward + mt_flce_backward, 8HVN)"
                     + ("; the planner declined the fused path for this budget" if fused else "")),
            "general_path_ms_per_step": ms_general,
            "general_path_frac_of_peak": alg_flops / (ms_general / 1e3) / peak_flops,
            "extra_hbm_GB": extra / 1e9,
            "extra_hbm_budget_GB": budget / 1e9,
            "peak_memory_GB": peak / 1e9,
        },
    }
    if not args.no_torch_gpu:
        del ws
        torch.cuda.empty_cache()
        tg = torch_gpu_path(data, W, scale)
        if "ms_per_step" in tg:
            tg["speedup_of_value"] = out["value"] / tg["tokens_per_s"]
        out["torch_gpu_path"] = tg
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_budget_s)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
