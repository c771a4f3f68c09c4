#!/usr/bin/env python3
"""Throughput of the fused PLE path on one MI355X.

A step is one forward (bin search + interpolated prefix table + bias) and one
backward (dx, dW, db) of the fused operators over one batch of the headline
workload (configs[1]: N=65536, F=128, 48 bins, d=32, fp32), inputs resident in
HBM before the timed region starts.  Prints ONE JSON line.

    python bench.py [--steps K] [--warmup W] [--config 1] [--mode fwdbwd|fwd|module|copy]
                    [--no-cpu-baseline]

``--mode copy`` times a plain 1 GiB device-to-device copy instead (the
reference kernel for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE counters to
bytes).  ``--mode module`` times the whole module in the reference
benchmark's configuration (version B, no activation; forward and
forward+backward), fused against the reference's op sequence (the forward
operator followed by PyTorch's linear0 and residual add); ``--compile`` adds
both under torch.compile as the reference harness compiles them.  ``--mode encode``
times the dense encoding kernels (``encode`` / ``encode_backward``).

Timing: W untimed warm-up steps; the forward and backward operators timed
alone (K calls each); K steps with each kernel's own start / end events (the
library's ``ple_timing_*``: hipExtLaunchKernelGGL records them at the
kernel's start and end), which give the per-kernel durations of ``kernels``
and ``roofline``; then the timed region -- K whole steps between two events on the launch
stream, synchronised on both sides (``value``, ``ms_per_step``) -- and the
reference harness's discipline, 10 repeats of 10 steps, median
(``ms_per_step_median_10x10``).  ``roofline`` prices the dominant kernel's
algorithmic bytes per launch against MI355X's 8 TB/s HBM peak;
``cpu_baseline`` times the dense upstream CPU algorithm
(``oracle/dense_torch.py``) on the job's host cores, on the whole batch where
its dense [N, F, Bmax] intermediate stays within 1.6 GB, plus config 0.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
REPO = os.path.dirname(os.path.abspath(__file__))


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=1)
    ap.add_argument("--mode", choices=("fwdbwd", "fwd", "module", "encode", "copy"), default="fwdbwd")
    ap.add_argument("--version", choices=("A", "B"), default="B", help="module version (--mode module)")
    ap.add_argument("--activation", action="store_true", help="ReLU in the module (--mode module)")
    ap.add_argument("--compile", action="store_true",
                    help="also time torch.compile(inductor, default mode, dynamic, fullgraph) (--mode module)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=None,
                    help="rows of the workload timed on the CPU (default: the whole batch, up to a 1.6 GB "
                         "dense intermediate)")
    return ap.parse_args()


def _traffic(kernel: str, workload: str):
    """HBM bytes per launch measured by rocprofv3 PMC runs, if committed, and
    the commit of the build they measured."""
    path = os.path.join(REPO, "profiles", f"traffic_{kernel}_{workload}.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as fh:
        rec = json.load(fh)
    return rec.get("bytes_per_launch"), rec.get("measured_commit")


# dense [rows, F, Bmax] elements the CPU baseline's sample may hold (c1 in full:
# 65536 x 128 x 48, a 1.6 GB fp32 intermediate)
CPU_SAMPLE_ELEMS = 65536 * 128 * 48


def _cpu_baseline(w, n_rows: int | None = None):
    """The dense upstream algorithm on the host cores: fwd+bwd samples/s."""
    import numpy as np
    import torch

    from oracle.dense_torch import DensePLE

    # every core the job has (torch's default: OMP_NUM_THREADS where it is
    # set -- 16 per GPU on the GPU boxes -- else all cores)
    threads = torch.get_num_threads()
    n, f, bmax, _ = w.shape
    rows = min(n, max(1, CPU_SAMPLE_ELEMS // (f * bmax))) if n_rows is None else min(n_rows, n)
    x = torch.from_numpy(np.ascontiguousarray(w.x[:rows]))
    g = torch.randn((rows, f, w.weight.shape[2]), generator=torch.Generator().manual_seed(0))
    m = DensePLE(w.bins, w.weight, w.bias)
    for _ in range(3):
        m.forward_backward(x, g)
    times = []
    t_end = time.perf_counter() + 30.0
    while len(times) < 10 and (time.perf_counter() < t_end or len(times) < 3):
        t0 = time.perf_counter()
        m.forward_backward(x, g)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {
        "value": rows / med,
        "unit": "samples/s",
        "cores": threads,
        "host_cpus": os.cpu_count(),
        "kind": "port",
        "sample": f"{rows} of {n} rows of {w.name}, dense upstream algorithm in torch fp32 "
                  f"(addcmul/clamp/cat/bmm/+bias, autograd fwd+bwd), 3 warm-up, median of {len(times)}",
        "median_s": med,
    }


def _copy_calibration(args):
    """1 GiB copy: what FETCH_SIZE / WRITE_SIZE read for known traffic."""
    import torch

    n = 256 * 1024 * 1024
    src = torch.ones(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(max(args.warmup, 1)):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    print(json.dumps({"metric": "device copy GB/s (read + write)", "value": 2 * n * 4 / (ms * 1e-3) / 1e9,
                      "unit": "GB/s", "bytes_read_per_copy": n * 4, "bytes_written_per_copy": n * 4,
                      "ms_per_copy": ms, "steps": args.steps}), flush=True)


def _module_bench(args):
    """Module fwd and fwd+bwd: fused tail vs the reference's op sequence."""
    import torch

    import rtdl_num_embeddings_cuda
    from piecewiselinearembeddings_optimized_amd import workloads

    dev = torch.device("cuda:0")
    w = workloads.make(args.config)
    n, f, bmax, d = w.shape
    bins = [torch.from_numpy(w.edges[i, : int(w.n_bins[i]) + 1].copy()) for i in range(f)]
    torch.manual_seed(0)
    m = rtdl_num_embeddings_cuda.CudaPiecewiseLinearEmbeddings(bins, d, activation=args.activation,
                                                                version=args.version).to(dev)
    torch.nn.init.uniform_(m.linear.weight, -0.2, 0.2)
    ops = torch.ops.rtdl_num_embeddings_cuda
    x_plain = torch.from_numpy(w.x).to(dev)
    x_grad = x_plain.clone().requires_grad_(True)
    g = torch.randn((n, f, d), device=dev, generator=torch.Generator(dev).manual_seed(0))

    def unfused(xx):
        x_ple, _ = ops.forward(xx, m._cuda_bin_edges, m._cuda_inv_bin_widths, m._cuda_n_bins, m.linear.weight,
                               torch.float32)
        if m.linear.bias is not None:
            x_ple = x_ple + m.linear.bias
        if m.activation is not None:
            x_ple = m.activation(x_ple)
        return x_ple if m.linear0 is None else m.linear0(xx) + x_ple

    # The reference harness's step (tests/test_ple_cuda_benchmark.py:646-657): gradients set to None, then
    # forward and backward; its x needs no gradient (:1372-1379).  `*_fwdbwd_dx_ms`: the same with x
    # requiring a gradient too (dx, and x.grad set to None each step).
    def timed(fn, backward, x):
        def step():
            if backward:
                m.zero_grad(set_to_none=True)
                x.grad = None
            out = fn(x)
            if backward:
                out.backward(g)
        for _ in range(max(args.warmup, 1)):
            step()
        torch.cuda.synchronize()
        # median of five regions of K steps (the GPU's clocks move between regions)
        t = []
        for _ in range(5):
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(args.steps):
                step()
            t1.record()
            torch.cuda.synchronize()
            t.append(t0.elapsed_time(t1) / args.steps)
        return sorted(t)[2]

    res = {}
    for name, fn in (("fused", m), ("reference_ops", unfused)):
        with torch.no_grad():
            res[f"{name}_fwd_ms"] = timed(fn, False, x_plain)
        res[f"{name}_fwdbwd_ms"] = timed(fn, True, x_plain)
        res[f"{name}_fwdbwd_dx_ms"] = timed(fn, True, x_grad)
    if args.compile:
        # The reference harness's compiled execution (tests/test_ple_cuda_benchmark.py:128-137,
        # 740-746): inductor, default mode, dynamic and fullgraph; compiled and stabilised before
        # timing at the benchmark shape, at half the batch (the dynamic shape) and three more calls
        # (:748-774).
        half = n // 2

        def stabilise(fn, backward):
            for xx, gg in ((x_plain, g), (x_plain[:half], g[:half]), (x_plain, g), (x_plain, g), (x_plain, g)):
                if backward:
                    m.zero_grad(set_to_none=True)
                    fn(xx).backward(gg)
                else:
                    fn(xx)
            torch.cuda.synchronize()

        for name, fn in (("fused", m), ("reference_ops", unfused)):
            cfn = torch.compile(fn, backend="inductor", mode="default", dynamic=True, fullgraph=True)
            with torch.no_grad():
                stabilise(cfn, False)
                res[f"compiled_{name}_fwd_ms"] = timed(cfn, False, x_plain)
            stabilise(cfn, True)
            res[f"compiled_{name}_fwdbwd_ms"] = timed(cfn, True, x_plain)
    line = {
        "metric": f"module fwd+bwd samples/s (version {args.version}, activation={args.activation}, {w.name})",
        "value": n / (res["fused_fwdbwd_ms"] * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": res["fused_fwdbwd_ms"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": w.name, "N": n, "F": f, "bins": bmax, "d": d, "version": args.version,
                   "activation": args.activation, "mode": "module"},
        **res,
        "speedup_fwd": res["reference_ops_fwd_ms"] / res["fused_fwd_ms"],
        "speedup_fwdbwd": res["reference_ops_fwdbwd_ms"] / res["fused_fwdbwd_ms"],
    }
    print(json.dumps(line), flush=True)


def _encode_bench(args):
    """Dense encoding output [N, sum n_f] and its dx, with HBM bytes per launch."""
    import numpy as np
    import torch

    import piecewiselinearembeddings_optimized_amd  # noqa: F401
    from piecewiselinearembeddings_optimized_amd import workloads

    dev = torch.device("cuda:0")
    ops = torch.ops.rtdl_num_embeddings_cuda
    w = workloads.make(args.config)
    n, f, bmax, d = w.shape
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    nbins = w.n_bins.astype(np.int64)
    offs = np.concatenate([[0], np.cumsum(nbins)[:-1]]).astype(np.int32)
    total = int(nbins.sum())
    x, e, iw, nb, of = t(w.x), t(w.edges), t(w.inv_widths), t(w.n_bins), t(offs)
    g = torch.randn((n, total), device=dev, generator=torch.Generator(dev).manual_seed(0))

    def tm(fn):
        for _ in range(max(args.warmup, 1)):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(args.steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / args.steps

    fwd_ms = tm(lambda: ops.encode(x, e, iw, nb, of, total))
    bwd_ms = tm(lambda: ops.encode_backward(g, x, e, iw, nb, of))
    fwd_bytes = n * total * 4 + n * f * 4                    # output + x
    bwd_bytes = n * f * (4 + 4) + n * f * 128                # x, dx, and one 128-byte line of g per pair
    print(json.dumps({
        "metric": f"dense encoding samples/s ({w.name}, {total} columns)", "value": n / (fwd_ms * 1e-3),
        "unit": "samples/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": fwd_ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": w.name, "N": n, "F": f, "total_bins": total, "mode": "encode"},
        "fwd_ms": fwd_ms, "fwd_GBps": fwd_bytes / (fwd_ms * 1e-3) / 1e9,
        "fwd_frac": fwd_bytes / (fwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "bwd_ms": bwd_ms, "bwd_GBps_line_bound": bwd_bytes / (bwd_ms * 1e-3) / 1e9,
    }), flush=True)


def main():
    args = _parse()
    if args.mode == "copy":
        _copy_calibration(args)
        return
    if args.mode == "module":
        _module_bench(args)
        return
    if args.mode == "encode":
        _encode_bench(args)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} (WORLD_SIZE={world}) is not supported: "
              "this path is a single-device operator and the run uses one GPU", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the HIP ops)
    from piecewiselinearembeddings_optimized_amd import capi, workloads

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    ops = torch.ops.rtdl_num_embeddings_cuda

    w = workloads.make(args.config)
    n, f, bmax, d = w.shape
    quant = torch.bfloat16 if w.quant == "bf16" else torch.float32
    out_bytes = 2 if w.quant == "bf16" else 4
    x = torch.from_numpy(w.x).to(dev)
    e = torch.from_numpy(w.edges).to(dev)
    iw = torch.from_numpy(w.inv_widths).to(dev)
    nb = torch.from_numpy(w.n_bins).to(dev)
    wt = torch.from_numpy(w.weight).to(dev)
    bt = torch.from_numpy(w.bias).to(dev)
    g = torch.randn((n, f, d), device=dev, generator=torch.Generator(dev).manual_seed(0)).to(quant)

    def fwd():
        if quant == torch.float32:
            return ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
        return ops.forward(x, e, iw, nb, wt, quant)

    def bwd(idx):
        if quant == torch.float32:
            return ops.backward_with_bias(g, x, e, iw, nb, wt, idx, torch.float32, True, True, True)
        return ops.backward(g, x, e, iw, nb, wt, idx, True, True)

    # warm-up (also populates the caching allocator)
    for _ in range(max(args.warmup, 1)):
        out, idx = fwd()
        if args.mode == "fwdbwd":
            bwd(idx)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()

    def region(steps, kernel_events):
        """`steps` whole steps between two events on the launch stream,
        synchronised on both sides; with kernel_events the library records an
        event pair around the forward and the backward gradient kernel of
        every step (ple_timing_*)."""
        torch.cuda.synchronize()
        if kernel_events:
            capi.timing_start(steps)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        a.record(stream)
        for _ in range(steps):
            o, i = fwd()
            if args.mode == "fwdbwd":
                bwd(i)
        b.record(stream)
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - w0
        kern = None
        if kernel_events:
            capi.timing_stop()
            kern = {name: capi.timing_read(t) for name, t in
                    (("fwd", capi.TIMER_FORWARD), ("bwd", capi.TIMER_BACKWARD))}
            capi.timing_start(0)
        return a.elapsed_time(b) / steps, wall_s, kern

    # operator-level passes (the backward op includes its finalize kernel)
    def time_pass(fn, reps):
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in ev:
            a.record(stream)
            fn()
            b.record(stream)
        torch.cuda.synchronize()
        ts = sorted(a.elapsed_time(b) for a, b in ev)
        return sum(ts) / len(ts), ts[len(ts) // 2]

    fwd_op_ms, fwd_op_med = time_pass(fwd, args.steps)
    _, idx = fwd()

    def peak_bytes(fn):
        """Device memory a call allocates at its peak beyond what is held
        before it (the reference benchmark's incremental peak,
        tests/test_ple_cuda_benchmark.py:935-971)."""
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        res = fn()
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated()
        del res
        return max(0, peak - base)

    memory = {"fwd_peak_bytes": peak_bytes(fwd)}
    if args.mode == "fwdbwd":
        memory["bwd_peak_bytes"] = peak_bytes(lambda: bwd(idx))
        memory["step_peak_bytes"] = peak_bytes(lambda: bwd(fwd()[1]))
        memory["bwd_workspace_bytes"] = capi.workspace_bytes(n, f, bmax, d)
    bwd_op_ms = bwd_op_med = 0.0
    if args.mode == "fwdbwd":
        bwd_op_ms, bwd_op_med = time_pass(lambda: bwd(idx), args.steps)

    # K steps with the kernels' own start / end events (hipExtLaunchKernelGGL)
    # -> per-kernel durations inside the step, for the roofline
    instr_ms, _, kern = region(args.steps, True)
    # the timed region: K whole steps, no kernel events -> value (after the
    # passes above, so the GPU's clocks have settled however short W is)
    step_ms, wall, _ = region(args.steps, False)
    value = n / (step_ms * 1e-3)
    # the reference harness's discipline: 10 repeats x 10 steps, median
    reps = sorted(region(10, False)[0] for _ in range(10))
    median_ms = 0.5 * (reps[4] + reps[5])

    fwd_bytes, bwd_bytes = workloads.algorithmic_bytes(n, f, bmax, d, out_bytes=out_bytes)
    # The backward's plan decides what its timed kernel writes: with one chunk
    # (and one bin window) the sorted path's and the matrix-core path's
    # gradient kernel writes dW / db itself, otherwise a finalize kernel does
    # (from chunk partials).  The fallback path's timer spans its dx and
    # histogram kernels.
    plan = capi.backward_plan(n, f, bmax, d, grad_dtype=g.dtype, quant_dtype=quant, grad_output=g)
    bwd_kernel_bytes = bwd_bytes
    single = (plan["sorted"] or plan["matrix_cores"]) and plan["chunks"] == 1 and plan["windows"] == 1
    if not single:
        bwd_kernel_bytes -= f * bmax * d * 4 + f * d * 4
    kernels = {}
    fwd_name = "ple_fwd_kernel"
    bwd_name = ("ple_bwd_mfma_kernel" if plan["matrix_cores"] else
                "ple_bwd_fused_kernel" if plan["sorted"] else "ple_bwd_simple_dx_kernel+ple_bwd_simple_hist_kernel")
    for name, key, nbytes in ((fwd_name, "fwd", fwd_bytes), (bwd_name, "bwd", bwd_kernel_bytes)):
        total_ms, launches = kern[key]
        if launches == 0:
            continue
        avg = total_ms / launches
        kernels[name] = {"ms": avg, "launches": launches, "bytes": nbytes,
                         "GB/s": nbytes / (avg * 1e-3) / 1e9,
                         "frac": nbytes / (avg * 1e-3) / 1e9 / HBM_PEAK_GBS}
    dom_name = max(kernels, key=lambda k: kernels[k]["ms"])
    dom = kernels[dom_name]
    traffic, traffic_commit = _traffic(dom_name, w.name)
    total_bytes = fwd_bytes + (bwd_bytes if args.mode == "fwdbwd" else 0)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_baseline(w, args.cpu_sample)
        if args.config != 0:
            # the reference's CPU-runnable case too
            c0 = _cpu_baseline(workloads.make(0))
            cpu["c0_plumbing"] = {k: c0[k] for k in ("value", "unit", "cores", "sample", "median_s")}

    metric = ("fwd+bwd samples/s (B=65536,F=128,48 bins,d=32) + achieved HBM GB/s" if args.config == 1
              else f"{'fwd+bwd' if args.mode == 'fwdbwd' else 'fwd'} samples/s ({w.name})")
    line = {
        "metric": metric if args.mode == "fwdbwd" else metric.replace("fwd+bwd", "fwd"),
        "value": value,
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.quant == "f32" else "bf16",
        "data": "synthetic",
        "config": {
            "workload": w.name, "N": n, "F": f, "bins": bmax, "d": d, "mode": args.mode,
            "path": "torch.ops.rtdl_num_embeddings_cuda.forward_with_bias/backward_with_bias -> C ABI -> HIP",
        },
        "achieved_GBps": total_bytes / (step_ms * 1e-3) / 1e9,
        "hbm_frac": total_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "ms_per_step_with_kernel_events": instr_ms,
        "ms_per_step_median_10x10": median_ms,
        "fwd_op_ms": fwd_op_ms,
        "fwd_op_median_ms": fwd_op_med,
        "bwd_op_ms": bwd_op_ms,
        "bwd_op_median_ms": bwd_op_med,
        "kernels": kernels,
        "memory": memory,
        "backward_plan": plan,
        "roofline": {
            "kernel": dom_name,
            "bound": "hbm",
            "achieved": dom["GB/s"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dom["frac"],
            "traffic": traffic,
            "traffic_measured_commit": traffic_commit,
            "algorithmic_bytes": dom["bytes"],
            "ms": dom["ms"],
        },
        "cpu_baseline": cpu,
        "wall_s_timed": wall,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
