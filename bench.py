"""Benchmark of the fused causal self-attention forward on one MI355X.

A step is one forward call (pmkl_attn_fwd through the C ABI) over one batch of
the workload, inputs already resident in HBM.  Default workload: C3, bf16
B=4 H=32 S=4096 D=128, causal, scale 1/sqrt(D) - the configuration the
headline metric is quoted on.  Prints one JSON line.

  value      whole-job TFLOP/s = causal FLOPs per step * steps / elapsed,
             FLOPs = 2*B*H*D*S*(S+1) (QK^T and PV multiply-adds of the visible
             pairs; softmax not counted)
  roofline   the attention kernel against the dense bf16 MFMA peak
             (2,516.6 TFLOP/s): achieved = FLOPs per launch / average launch
             duration from HIP events on the launch stream; kernel = the one the
             library's dispatcher chose (pmkl_attn_fwd_kernel_name); launches =
             median / min / max of 64 launches timed one by one after the timed
             region; traffic = HBM bytes per launch from the committed
             rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by a
             copy-kernel calibration), or null; profile = the committed
             rocprofv3 kernel-trace means of this kernel (one per lease, with
             the shader clock of that lease) and the fraction they give
  cpu_baseline  the reference's own CPU operator (oracle/_ref, compiled from
             pmkl_pytorch_ext/fused_self_attention.cpp) on a bounded sample:
             one head per core on all usable cores at once (value), and one
             head alone on one core (single_core), with the host CPU named

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C3] [--no-cpu] [--sdpa]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_TFLOPS = {"bf16": 2516.6, "fp16": 2516.6, "fp32": 157.3}   # dense MFMA, MI355X public spec
PEAK_HBM_GBS = 8000.0
METRIC = "causal-attn TFLOP/s on 1 MI355X, bf16 B4 H32 S4096 D128; % of MFMA peak"


WARMUP_MIN_S = 1.0
LAUNCH_SAMPLES = 64


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="C3", choices=["C1", "C2", "C3", "C4", "C5"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--warmup-seconds", type=float, default=WARMUP_MIN_S,
                    help="minimum seconds of back-to-back warm-up launches (clock ramp; default 1.0). "
                         "Counter runs (rocprofv3 --pmc serialises every dispatch) may lower it.")
    ap.add_argument("--sdpa", action="store_true",
                    help="also time torch's scaled_dot_product_attention on the same tensors (reference point; "
                         "restricted to its flash / memory-efficient backends: the math fallback runs "
                         "transposed bf16 batched products)")
    ap.add_argument("--op", default="fwd", choices=["fwd", "bwd", "softmax"],
                    help="fwd: the headline forward (default); bwd: the backward (pmkl_attn_bwd), "
                         "its own JSON line")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 512 MiB device copy (torch copy kernel) so that rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE can be scaled against a known byte count")
    return ap.parse_args()


def calibrate_copy():
    """One device-to-device copy of 512 MiB: reads 512 MiB, writes 512 MiB."""
    import torch

    n = 512 * 1024 * 1024 // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": n * 4, "bytes_written": n * 4, "launches": 3}))


def read_traffic(config: str, kernel: str, name: str | None = None):
    """HBM bytes per launch from profiles/pmc_attn_fwd_<config>.txt (or
    profiles/<name>) when that summary was measured on `kernel` (its
    "kernel_id:" line equals the kernel's name up to its launch shape), else
    None."""
    path = ROOT / "profiles" / (name or f"pmc_attn_fwd_{config}.txt")
    if not path.exists():
        return None
    txt = path.read_text()
    k = re.search(r"^kernel_id:\s*(.+?)\s*$", txt, re.M)
    if k is None or k.group(1) != kernel.split(" grid")[0]:
        return None
    m = re.search(r"^hbm_bytes_per_launch:\s*([0-9.eE+]+)", txt, re.M)
    return float(m.group(1)) if m else None


def read_profile(config: str, kernel: str, work: float, peak: float, unit_scale: float = 1e12):
    """The committed kernel traces of `kernel` at `config`
    (profiles/<family>_<config>_kernel_trace.txt, family = the kernel's name
    without "_kernel<...>", e.g. attn_fwd_w64): one "lease:" line per fresh
    GPU lease with the trace mean of the timed dispatches (us) and the
    shader clock of that lease; returns them with the fraction of peak they
    give (work per launch / trace mean / unit_scale / peak: FLOP and 1e12 for
    TFLOP/s, bytes and 1e9 for GB/s), or None when no summary was taken on
    this kernel."""
    family = kernel.split("<")[0].removesuffix("_kernel")
    path = ROOT / "profiles" / f"{family}_{config}_kernel_trace.txt"
    if not path.exists():
        return None
    txt = path.read_text()
    k = re.search(r"^kernel_id:\s*(.+?)\s*$", txt, re.M)
    if k is None or k.group(1) != kernel.split(" grid")[0]:
        return None
    # shader_clock_GHz is "n/a" where the counter window cannot give a clock (kernels of a few us).
    leases = [{"lease": m.group(1), "trace_mean_us": float(m.group(2)),
               "shader_clock_GHz": None if m.group(3) == "n/a" else float(m.group(3))}
              for m in re.finditer(r"^lease:\s*(\S+)\s+trace_mean_us\s+([0-9.]+)\s+shader_clock_GHz\s+([0-9.]+|n/a)",
                                   txt, re.M)]
    if not leases:
        return None
    best = min(x["trace_mean_us"] for x in leases)
    mean = sum(x["trace_mean_us"] for x in leases) / len(leases)
    return {"file": str(path.relative_to(ROOT)), "leases": leases,
            "frac_best_lease": round(work / (best / 1e6) / unit_scale / peak, 4),
            "frac_mean_of_leases": round(work / (mean / 1e6) / unit_scale / peak, 4)}


def _host_cpu():
    """Model name of the host CPU (/proc/cpuinfo), its logical CPU count and
    the CPUs this process may run on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"model": model, "nproc": os.cpu_count(), "usable_cpus": usable}


# A GPU box gives one GPU's job a share of 16 CPUs, whatever nproc shows.
CPU_WORKERS_MAX = 16
CPU_WORKER_TIMEOUT_S = 240


def _run_cpu_workers(npz: str, heads):
    """One oracle.cpu_baseline worker per head (child processes that never
    touch the GPU), released together once all have loaded their head.
    Returns (per-worker seconds, wall seconds from release to the last
    result), or None if a worker failed."""
    import subprocess

    import queue
    import threading

    procs = [subprocess.Popen([sys.executable, "-m", "oracle.cpu_baseline", npz, str(h)], cwd=str(ROOT),
                              stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True) for h in heads]
    # Each worker's lines arrive through a reader thread, so that every wait
    # has a deadline: a worker that hangs costs the CPU leg, never the line.
    lines = [queue.Queue() for _ in procs]

    def reader(p, q):
        for ln in p.stdout:
            q.put(ln)
        q.put(None)

    for p, q in zip(procs, lines):
        threading.Thread(target=reader, args=(p, q), daemon=True).start()
    deadline = time.perf_counter() + CPU_WORKER_TIMEOUT_S

    def next_line(q):
        ln = q.get(timeout=max(0.0, deadline - time.perf_counter()))
        if ln is None:
            raise ValueError("worker ended")
        return ln

    try:
        for q in lines:
            if next_line(q).strip() != "ready":
                return None
        t0 = time.perf_counter()
        for p in procs:
            p.stdin.write("go\n")
            p.stdin.flush()
        secs = []
        for q in lines:
            r = json.loads(next_line(q))
            if "seconds" not in r:
                return None
            secs.append(r["seconds"])
        wall = time.perf_counter() - t0
        for p in procs:
            p.wait(timeout=max(1.0, deadline - time.perf_counter()))
        return secs, wall
    except (ValueError, OSError, queue.Empty, subprocess.TimeoutExpired):
        return None
    finally:
        for p in procs:
            if p.poll() is None:
                p.kill()
                p.wait()


def cpu_baseline(w):
    """The reference's own CPU operator (oracle/_ref) on a bounded sample of
    the workload: one head on one core (the operator as written walks heads
    on one thread), then one head per core on all usable cores at once (up to
    CPU_WORKERS_MAX), each worker on its own head.  `value` is the all-cores
    throughput, the single-core one is reported beside it; both count the
    same causal FLOPs as the GPU line."""
    import tempfile

    import numpy as np

    from oracle import oracle
    from pmkl_amd.workloads import causal_flops, host_inputs

    if oracle.reference_op() is None:
        return None
    host = _host_cpu()
    n = max(1, min(CPU_WORKERS_MAX, host["usable_cpus"], w.B * w.H))
    q, k, v = (a.reshape(w.B * w.H, w.S, w.D)[:n] for a in host_inputs(w))
    flops_head = causal_flops(1, 1, w.S, w.D)
    with tempfile.TemporaryDirectory() as tmp:
        npz = os.path.join(tmp, "heads.npz")
        np.savez(npz, q=q, k=k, v=v, dtype=np.array(w.dtype), causal=np.array(True))
        one = _run_cpu_workers(npz, [0])
        many = _run_cpu_workers(npz, list(range(n)))
    if one is None or many is None:
        return None
    single_s = one[0][0]
    secs, wall = many
    return {
        "value": flops_head * n / wall / 1e12,
        "unit": "TFLOP/s",
        "cores": n,
        "kind": "reference",
        "sample": f"{n} of {w.B * w.H} heads of {w.name} (S={w.S}, D={w.D}, {w.dtype}, causal), one head per "
                  f"process on {n} cores at once, through the reference fused_self_attention_fw CPU body "
                  f"(single-threaded per head as written); {wall:.3g} s wall (slowest head {max(secs):.3g} s, "
                  f"fastest {min(secs):.3g} s)",
        "single_core": {"value": flops_head / single_s / 1e12, "cores": 1, "seconds": float(f"{single_s:.4g}"),
                        "sample": f"head 0 of {w.name} alone on one core"},
        "host_cpu": host,
        "full_job_seconds_extrapolated": {"single_core": round(single_s * w.B * w.H, 1),
                                          "all_cores": round(wall * w.B * w.H / n, 1)},
    }


def bench_bwd(args):
    """Backward of the attention output (pmkl_attn_bwd) on the workload: one
    step is one call (two kernel launches), inputs resident in HBM.  FLOPs:
    10*D per visible (i, j) pair (the five products QK^T, dout V^T, P^T dout,
    dS^T Q, dS K), i.e. 2.5x the forward's count; the pass that forms
    sum_j P dP from the keys when O is not given is not counted."""
    import torch

    import pmkl_amd
    from pmkl_amd import capi
    from pmkl_amd.workloads import WORKLOADS, causal_flops, torch_inputs

    w = WORKLOADS[args.config]
    dev = torch.device("cuda:0")
    q, k, v = torch_inputs(w, dev)
    g = torch.Generator(device="cpu").manual_seed(w.seed + 1)
    do = torch.randn(q.shape, generator=g).to(q.dtype).to(dev)
    o, m, l = pmkl_amd.attn_fwd(q, k, v, is_causal=True)
    dq, dk, dv = (torch.empty_like(x) for x in (q, k, v))
    lib = capi.load()
    ws_bytes = int(lib.pmkl_attn_bwd_workspace_size(w.B, w.H, w.S))
    ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    dt = pmkl_amd.torch_dtype_to_pmkl(q.dtype)
    results = {}
    for with_o in (False, True):
        cargs = capi.make_bwd_args(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   o.data_ptr() if with_o else 0, m.data_ptr(), l.data_ptr(), dq.data_ptr(),
                                   dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes, dtype=dt, batch=w.B,
                                   heads=w.H, seq_len=w.S, head_dim=w.D, is_causal=True)

        def step():
            rc = capi.attn_bwd_raw(cargs, stream.cuda_stream)
            if rc != capi.PMKL_OK:
                raise capi.PmklError(rc, capi.last_error())

        t_w = time.perf_counter()
        while time.perf_counter() - t_w < args.warmup_seconds:
            for _ in range(max(args.warmup, 1)):
                step()
            torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record(stream)
        for _ in range(args.steps):
            step()
        ev1.record(stream)
        torch.cuda.synchronize()
        results[with_o] = ev0.elapsed_time(ev1) / args.steps
    flops = causal_flops(w.B, w.H, w.S, w.D) * 10 // 4
    peak = PEAK_TFLOPS[w.dtype]
    ms = results[False]
    line = {
        "metric": f"causal-attn backward TFLOP/s on 1 MI355X, {w.dtype} B{w.B} H{w.H} S{w.S} D{w.D}",
        "value": round(flops / (ms / 1e3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "dtype": w.dtype,
        "data": "synthetic: seeded PCG64 " + w.note + "; dout ~ N(0,1)",
        "config": {"workload": f"{w.name} causal self-attention bwd {w.dtype} B{w.B} H{w.H} S{w.S} D{w.D}",
                   "flops_per_step": flops, "flop_count": "10*D per visible pair (5 products)"},
        "pct_of_mfma_peak": round(100.0 * flops / (ms / 1e3) / 1e12 / peak, 2),
        "with_o": {"ms_per_step": round(results[True], 4),
                   "value": round(flops / (results[True] / 1e3) / 1e12, 2)},
        "kernels": ["attn_bwd_f32_dq_kernel", "attn_bwd_f32_dkdv_kernel"] if w.dtype == "fp32"
        else ["attn_bwd_dq_kernel", "attn_bwd_dkdv_kernel"],
        "torch_sdpa": torch_sdpa_bwd_reference(q, k, v, do, flops, min(args.steps, 20)) if args.sdpa else None,
    }
    print(json.dumps(line), flush=True)


def _sdpa_fused_backends_only():
    """Context that lets torch's scaled_dot_product_attention pick only its
    flash or memory-efficient backend.  Its math fallback runs batched bf16
    products on transposed views, which have faulted these GPU boxes; with
    this context a missing fused backend raises (and is reported in the
    line) instead of falling back."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    return sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION])


def torch_sdpa_bwd_reference(q, k, v, do, flops, steps):
    """Reference point, timed after the timed region: the backward of torch's
    scaled_dot_product_attention (causal) on the same tensors, i.e.
    torch.autograd.grad of its output with the forward graph kept, so only
    the backward kernels run per step."""
    import torch
    import torch.nn.functional as F

    what = ("backward of torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True): "
            "torch.autograd.grad(out, (q, k, v), dout) with the forward graph kept")
    try:
        qg, kg, vg = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
        with _sdpa_fused_backends_only():
            out = F.scaled_dot_product_attention(qg, kg, vg, is_causal=True)
        for _ in range(3):
            torch.autograd.grad(out, (qg, kg, vg), do, retain_graph=True)
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(steps):
            torch.autograd.grad(out, (qg, kg, vg), do, retain_graph=True)
        ev1.record()
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / steps
        return {"what": what, "ms": round(ms, 4), "TFLOP/s": round(flops / (ms / 1e3) / 1e12, 2), "steps": steps}
    except Exception as ex:  # a missing backend is reported, not fatal
        return {"what": what, "error": str(ex)[:200]}


SOFTMAX_ROWS, SOFTMAX_N = 131072, 1024


def bench_softmax(args):
    """Row softmax (pmkl_softmax_fwd, the replacement of
    pmkl::norm::warp_softmax_forward) over 131,072 rows x 1,024 fp32 elements:
    the score rows of C2 (B*H*S = 8*16*1024 rows of S = 1024 keys) at the
    reference's widest row and its tested dtype.  A step is one call (one
    launch), inputs resident in HBM.  Algorithmic bytes per call: every
    element read once and written once, rows * n * (4 + 4) = 1 GiB."""
    import torch

    from pmkl_amd import capi

    rows, n = SOFTMAX_ROWS, SOFTMAX_N
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(1006)
    x = torch.rand((rows, n), generator=g, device=dev) * 20.0 - 10.0
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream(dev)
    handle = stream.cuda_stream
    cargs = capi.make_softmax_args(y.data_ptr(), x.data_ptr(), out_dtype=capi.PMKL_DTYPE_F32,
                                   in_dtype=capi.PMKL_DTYPE_F32, elements=n, stride=n, batch=rows)

    def step():
        rc = capi.softmax_raw(cargs, handle)
        if rc != capi.PMKL_OK:
            raise capi.PmklError(rc, capi.last_error())

    t_w = time.perf_counter()
    while time.perf_counter() - t_w < args.warmup_seconds:
        for _ in range(max(args.warmup, 1)):
            step()
        torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    avg_ms = ev0.elapsed_time(ev1) / args.steps
    alg_bytes = rows * n * (4 + 4)
    achieved = alg_bytes / (avg_ms / 1e3) / 1e9
    kernel = "softmax_fwd_kernel<float,float,4,4,false>"
    # Reference point after the timed region: torch's device copy of the same
    # bytes (rows * n fp32 read, the same written) on the same stream.
    ycp = torch.empty_like(x)
    for _ in range(max(args.warmup, 1)):
        ycp.copy_(x)
    torch.cuda.synchronize()
    ev0.record(stream)
    for _ in range(args.steps):
        ycp.copy_(x)
    ev1.record(stream)
    torch.cuda.synchronize()
    copy_ms = ev0.elapsed_time(ev1) / args.steps
    del ycp
    cpu = None
    if not args.no_cpu:
        from oracle import oracle

        xh = x.cpu().numpy()
        t0 = time.perf_counter()
        oracle.softmax_host_f32(xh)
        cpu_s = time.perf_counter() - t0
        cpu = {"value": round(alg_bytes / cpu_s / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"the whole workload ({rows} x {n} fp32) through the reference's CPU softmax check "
                         f"host_softmax_forward (test/test_softmax.cpp:10-28) restated in C, single-threaded; "
                         f"{cpu_s:.2f} s"}
    line = {
        "metric": f"row softmax GB/s on 1 MI355X, fp32 {rows} rows x {n}",
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(avg_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: U(-10, 10) from torch's seeded device generator (seed 1006)",
        "config": {"workload": f"row softmax fp32 rows={rows} n={n} stride={n}", "rows": rows, "elements": n,
                   "alg_bytes_per_step": alg_bytes, "byte_count": "rows*n*(4 read + 4 written)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": read_traffic("", kernel, "pmc_softmax_fwd_fp32_131072x1024.txt"),
                     "kernel": kernel, "avg_launch_us": round(avg_ms * 1e3, 2)},
        "cpu_baseline": cpu,
        "device_copy": {"what": "torch copy_ of the same bytes (the input into a new tensor), same stream, "
                                "timed after the softmax", "ms": round(copy_ms, 4),
                        "GB/s": round(alg_bytes / (copy_ms / 1e3) / 1e9, 1)},
    }
    print(json.dumps(line), flush=True)


def torch_sdpa_reference(q, k, v, flops, steps):
    """Reference point, timed after the timed region: torch's own
    scaled_dot_product_attention (causal, default scale 1/sqrt(D)) on the
    same device tensors, with whichever backend torch picks on this image."""
    import torch
    import torch.nn.functional as F

    what = "torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True), same tensors and stream"
    try:
        with _sdpa_fused_backends_only():
            for _ in range(3):
                F.scaled_dot_product_attention(q, k, v, is_causal=True)
            torch.cuda.synchronize()
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            ev0.record()
            for _ in range(steps):
                F.scaled_dot_product_attention(q, k, v, is_causal=True)
            ev1.record()
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / steps
        return {"what": what, "ms": round(ms, 4), "TFLOP/s": round(flops / (ms / 1e3) / 1e12, 2), "steps": steps}
    except Exception as ex:  # a missing backend is reported, not fatal
        return {"what": what, "error": str(ex)[:200]}


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the attention path has no multi-GPU leg); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)

    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.op == "bwd":
        bench_bwd(args)
        return
    if args.op == "softmax":
        bench_softmax(args)
        return

    import torch

    import pmkl_amd
    from pmkl_amd import capi
    from pmkl_amd.workloads import WORKLOADS, causal_flops, torch_inputs

    w = WORKLOADS[args.config]
    dev = torch.device("cuda:0")
    q, k, v = torch_inputs(w, dev)
    o = torch.empty_like(q)
    m = torch.empty((w.B, w.H, w.S), dtype=q.dtype, device=dev)
    l = torch.empty_like(m)
    stream = torch.cuda.current_stream(dev)

    # The argument block is built once, as a serving caller would hold it; a
    # step is one pmkl_attn_fwd call (one kernel launch) on `stream`.
    pmkl_amd.attn_fwd(q, k, v, is_causal=True, out=o, out_m=m, out_l=l, stream=stream.cuda_stream)
    dt = pmkl_amd.torch_dtype_to_pmkl(q.dtype)
    cargs = capi.make_args(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), m.data_ptr(), l.data_ptr(),
                           dtype=dt, ml_dtype=dt, batch=w.B, heads=w.H, seq_len=w.S, head_dim=w.D,
                           is_causal=True)
    handle = stream.cuda_stream

    def step():
        rc = capi.attn_fwd_raw(cargs, handle)
        if rc != capi.PMKL_OK:
            raise capi.PmklError(rc, capi.last_error())

    # Warm-up: W steps, extended until WARMUP_MIN_S of back-to-back work has
    # run.  Launch durations settle only after ~50 ms of sustained load (the
    # clocks ramp: at C3 the first launches take 640-830 us, then 590-600 us).
    t_w = time.perf_counter()
    warm_run = 0
    while warm_run < args.warmup or time.perf_counter() - t_w < args.warmup_seconds:
        for _ in range(max(args.warmup, 1)):
            step()
        warm_run += max(args.warmup, 1)
        torch.cuda.synchronize()

    # Timed region: exactly K steps bracketed by device syncs, with HIP events
    # on the launch stream.  Each step is one launch of the attention kernel,
    # so the average launch duration is the event interval / K.
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    avg_launch_ms = gpu_ms / args.steps

    # Per-launch statistics, after the timed region: each of LAUNCH_SAMPLES
    # launches between its own pair of events on the launch stream.
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(LAUNCH_SAMPLES)]
    for e0, e1 in evs:
        e0.record(stream)
        step()
        e1.record(stream)
    torch.cuda.synchronize()
    per_launch_us = sorted(e0.elapsed_time(e1) * 1e3 for e0, e1 in evs)

    flops = causal_flops(w.B, w.H, w.S, w.D)
    esize = {"bf16": 2, "fp16": 2, "fp32": 4}[w.dtype]
    alg_bytes = (4 * w.B * w.H * w.S * w.D + 2 * w.B * w.H * w.S) * esize
    elapsed_s = max(gpu_ms / 1e3, 1e-12)
    value = flops * args.steps / elapsed_s / 1e12
    achieved = flops / (avg_launch_ms / 1e3) / 1e12
    peak = PEAK_TFLOPS[w.dtype]
    # The bound of the roofline: HBM where the arithmetic intensity times the
    # HBM peak is below the MFMA peak (C5), else the matrix cores.
    hbm_bound = flops / alg_bytes * PEAK_HBM_GBS / 1e3 < peak
    kernel = capi.attn_fwd_kernel_name(cargs)
    traffic = read_traffic(w.name, kernel)

    cpu = None if args.no_cpu else cpu_baseline(w)
    sdpa = torch_sdpa_reference(q, k, v, flops, min(args.steps, 20)) if args.sdpa else None

    line = {
        "metric": METRIC if w.name == "C3" else f"causal-attn TFLOP/s on 1 MI355X, {w.dtype} B{w.B} H{w.H} S{w.S} D{w.D}",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic: seeded PCG64 " + w.note,
        "config": {"workload": f"{w.name} causal self-attention fwd {w.dtype} B{w.B} H{w.H} S{w.S} D{w.D}",
                   "B": w.B, "H": w.H, "S": w.S, "D": w.D, "causal": True, "seed": w.seed,
                   "flops_per_step": flops, "flop_count": "2*B*H*D*S*(S+1)",
                   "alg_bytes_per_step": alg_bytes, "parallelism": "single GPU"},
        "pct_of_mfma_peak": round(100.0 * value / peak, 2),
        "roofline": {**({"bound": "hbm", "achieved": round(alg_bytes / (avg_launch_ms / 1e3) / 1e9, 1),
                         "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(alg_bytes / (avg_launch_ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4)} if hbm_bound else
                        {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                         "frac": round(achieved / peak, 4)}),
                     "traffic": traffic,
                     "kernel": kernel,
                     "avg_launch_us": round(avg_launch_ms * 1e3, 2),
                     "launches": {"n": len(per_launch_us),
                                  "median_us": round(per_launch_us[len(per_launch_us) // 2], 2),
                                  "min_us": round(per_launch_us[0], 2), "max_us": round(per_launch_us[-1], 2),
                                  "frac_at_median": round((alg_bytes / 1e9 / PEAK_HBM_GBS if hbm_bound else
                                                           flops / 1e12 / peak)
                                                          / (per_launch_us[len(per_launch_us) // 2] / 1e6), 4)},
                     "profile": (read_profile(w.name, kernel, alg_bytes, PEAK_HBM_GBS, 1e9) if hbm_bound else
                                 read_profile(w.name, kernel, flops, peak)),
                     "hbm_GBs_algorithmic": round(alg_bytes / (avg_launch_ms / 1e3) / 1e9, 1)},
        "cpu_baseline": cpu,
        "torch_sdpa": sdpa,
        "wall_s_timed": round(wall, 4),
        "warmup_steps_run": warm_run,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
