"""Throughput benchmark of the INT8 vision path on one MI355X.

Workload (default): the MobileNetV4-Conv-Small-shaped int8 classifier,
224x224x3, batch 256 per step, random-init seeded weights, synthetic uniform
int8 images resident in HBM before timing starts. One step = one forward pass
of the batch through every op of the plan (ug_enqueue_device).

Prints ONE JSON line. Besides the headline images/s it reports:
  roofline      the op with the largest average launch time, its algorithmic
                bytes (or ops) per launch over its HIP-event duration
  network_roofline  the step's algorithmic bytes at 8 TB/s against the step
  cpu_baseline  the reference's portable C runtime (oracle/_ref, built from
                the reference sources) on this host's cores, batch-1 plans;
                cpu_baseline_other: the same for the secondary workloads
  secondary     YOLO26n-shaped detector images/s (320x320, batch 64), int8
                conv TOPS (1x1 head GEMM, 3x3 implicit GEMM, batch 512),
                batch-1 1x1 conv latency, host-buffer throughput and latency,
                depthwise HBM GB/s (four cases, batch 64); each with `frac`
                against its bound (5.0 POP/s dense int8, or 8 TB/s);
                mfma_ceiling: the int8 rate a register-only MFMA loop
                sustains for as long as each GEMM launch, against which the
                GEMMs also carry `frac_of_ceiling`
With --library-gemm it only prints the vendor library's int8 GEMM timings on
the same GEMM shapes.
"""
import argparse
import ctypes as C
import json
import multiprocessing as mp
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "unoq-dsp_amd"))

import uq_plan as P  # noqa: E402
import uq_workloads as W  # noqa: E402
from uq_native import DeviceBuffer, Graph, mfma_ceiling, open_library  # noqa: E402

METRIC = "images/sec @ batch 256, MobileNetV4-S int8 224²; conv int8 TOPS + DW HBM GB/s"
HBM_PEAK = 8.0e12          # bytes/s
INT8_PEAK = 5.0e15         # dense int8 MFMA ops/s
RIDGE = INT8_PEAK / HBM_PEAK
PER_OP_PASSES = 100        # least number of per-op timing passes before the warm-up steps
REF_RELEASE = ROOT / "oracle" / "_ref" / "libuq_ref_release.so"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_device(lib, graph, images, steps, warmup, seed=7):
    x = P.random_input(graph.plan, images, seed)
    din = DeviceBuffer(lib, x.nbytes)
    dout = DeviceBuffer(lib, images * graph.output_bytes)
    din.upload(x)
    # Per-op durations from HIP events stamped by the kernels' own dispatches
    # (first start to last end of each op's kernels), averaged over at least
    # PER_OP_PASSES passes (more when more steps are timed). They run first:
    # their passes also bring the GPU clock up, which otherwise keeps rising
    # over the first passes: MobileNetV4-S timed over 20 steps after 5
    # warm-up steps measured 0.441 ms/step after 20 such passes, 0.434 after
    # 100 with enqueued warm-up steps, against 0.421 over 200 steps after 50.
    graph.profile(1)
    for _ in range(max(steps, PER_OP_PASSES)):
        rc = lib.ug_run_device(din.ptr, dout.ptr, images)
        assert rc == 0, rc
    counters = graph.profile(2)
    graph.profile(0)
    # Warm-up steps exactly as the timed ones: enqueued back to back.
    for _ in range(warmup):
        rc = lib.ug_enqueue_device(din.ptr, dout.ptr, images)
        assert rc == 0, rc
    assert lib.ug_synchronize() == 0
    t0 = time.perf_counter()
    for _ in range(steps):
        rc = lib.ug_enqueue_device(din.ptr, dout.ptr, images)
        assert rc == 0, rc
    assert lib.ug_synchronize() == 0
    seconds = time.perf_counter() - t0
    din.free()
    dout.free()
    runs = max(int(counters[0]), 1)
    per_op_ns = counters[2:2 + lib.ug_op_count()].astype(np.float64) / runs
    return seconds, per_op_ns


def _cpu_worker(args):
    plan, seconds, seed = args
    lib = C.CDLL(str(REF_RELEASE))
    lib.ug_load.argtypes = [C.c_void_p, C.c_uint32]
    lib.ug_run.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32]
    buf = C.create_string_buffer(plan, len(plan))
    assert lib.ug_load(buf, len(plan)) == 0
    ib, ob = P.input_bytes(plan), P.output_bytes(plan)
    x = P.random_input(plan, 1, seed)
    y = np.empty(ob, np.int8)
    lib.ug_run(x.ctypes.data, ib, y.ctypes.data, ob)  # warm-up
    done, t0 = 0, time.perf_counter()
    while True:
        assert lib.ug_run(x.ctypes.data, ib, y.ctypes.data, ob) == 0
        done += 1
        if time.perf_counter() - t0 >= seconds:
            break
    return done, time.perf_counter() - t0


# CPU legs of the other workloads: batch-1 plans of the same layers (the
# reference runs one image per ug_run call; its plans hold a bounded tensor
# size, runtime/graph.h:7,9), timed the same way as the headline leg.
CPU_LEGS = ("dw3s1", "dw3s2", "dw5s1", "dw5s2", "yolo", "head", "conv3x3")


def cpu_legs(workload, seconds_per_worker=1.5, legs=CPU_LEGS):
    """Images/s of the reference's release build on this host's cores for
    `workload` (the cpu_baseline of the JSON line) and for each of `legs`:
    one batch-1 plan per worker process, at most 16 processes, all legs in
    one pool."""
    if not REF_RELEASE.exists():
        return None, {}
    workers = max(1, min(16, len(os.sched_getaffinity(0))))
    names = [workload] + [n for n in legs if n != workload]
    plans = {n: W.WORKLOADS[n](images=1)[0] for n in names}
    ctx = mp.get_context("spawn")
    with ctx.Pool(workers) as pool:
        res = {n: pool.map(_cpu_worker, [(plans[n], seconds_per_worker, 100 + i) for i in range(workers)])
               for n in names}
    out = {}
    for n in names:
        rate = sum(d / t for d, t in res[n])
        costs = P.op_costs(plans[n], 1)
        entry = {"value": round(rate, 2), "unit": "images/s", "cores": workers, "kind": "reference",
                 "sample": f"{sum(d for d, _ in res[n])} {n} batch-1 images via ug_run, {workers} processes x "
                           f"~{seconds_per_worker}s (reference runtime/graph.c+qnn.c+gemm.c, release macros, gcc -O3)"}
        ops, nbytes = sum(c["ops"] for c in costs), sum(c["bytes"] for c in costs)
        if n.startswith("dw"):
            entry["gbps"] = round(rate * nbytes / 1e9, 3)
        elif n in ("head", "conv3x3"):
            entry["tops"] = round(rate * ops / 1e12, 4)
        out[n] = entry
    head = out.pop(workload)
    return head, out


def roofline_entry(costs, per_op_ns):
    i = int(np.argmax(per_op_ns))
    c = costs[i]
    dur = per_op_ns[i] * 1e-9
    ai = c["ops"] / c["bytes"] if c["bytes"] else 0.0
    if c["ops"] and ai >= RIDGE:
        achieved, peak, unit, bound = c["ops"] / dur / 1e12, INT8_PEAK / 1e12, "TOP/s", "mfma"
    else:
        achieved, peak, unit, bound = c["bytes"] / dur / 1e9, HBM_PEAK / 1e9, "GB/s", "hbm"
    return i, {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
               "frac": round(achieved / peak, 4), "traffic": None, "op": i, "code": c["code"],
               "algorithmic_bytes": c["bytes"], "algorithmic_ops": c["ops"], "avg_ns": round(float(per_op_ns[i]), 1)}


def committed_traffic(workload, op):
    """HBM bytes per launch of `op`, from the rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary committed under profiles/ (None when no summary covers it)."""
    for path in sorted((ROOT / "profiles").glob("*traffic*.txt")):
        for line in path.read_text().splitlines():
            if line.startswith("machine:"):
                kv = dict(item.split("=", 1) for item in line.split()[1:])
                if kv.get("workload") == workload and int(kv.get("op", -1)) == op:
                    return int(kv["traffic_bytes"]), path.name
    return None, None


def host_transfer(lib, steps):
    """MobileNetV4-S from pinned host buffers, PCIe included: 1024 images as
    one blocking batch call against the pipelined call in 256-image chunks
    (host-to-device copies of one chunk under the compute of the previous),
    and batch-1 latency through the session ABI in its two modes."""
    plan, _ = W.WORKLOADS["mnv4"]()
    images = 1024
    g = Graph(plan, lib)
    ib, ob = g.input_bytes, g.output_bytes
    x = P.random_input(plan, images, 5)
    hin, hout = lib.ug_host_alloc(x.nbytes), lib.ug_host_alloc(images * ob)
    C.memmove(hin, x.ctypes.data, x.nbytes)
    res = {"images": images, "input_mb": round(x.nbytes / 1e6, 2)}

    def timed(fn):
        fn()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        return (time.perf_counter() - t0) / steps

    def blocking():
        assert lib.ug_run_batch(hin, x.nbytes, hout, images * ob, images) == 0

    def pipelined():
        assert lib.ug_run_batch_pipelined(hin, x.nbytes, hout, images * ob, images, 256) == 0

    for key, fn in (("blocking", blocking), ("pipelined", pipelined)):
        sec = timed(fn)
        res[key] = {"ms": round(sec * 1e3, 3), "images_per_s": round(images / sec, 1)}
    lib.ug_host_free(hin)
    lib.ug_host_free(hout)
    from uq_native import Session
    for mode in ("rpc", "mailbox"):
        with Session(plan, mode, lib) as s:
            one = x[:ib]
            res[f"latency_b1_{mode}_ms"] = round(timed(lambda: s.run(one)) * 1e3, 4)
    return res


def pointwise_latency(lib, steps):
    """The batch-1 1x1 conv (56x56x32 -> 64): microseconds per call through
    ug_run_device (device buffers, returns when the output is complete) and
    through a mailbox session (host buffers, copies included), and the
    kernel's own time from its HIP events."""
    plan, images = W.WORKLOADS["pointwise"]()
    g = Graph(plan, lib)
    x = P.random_input(plan, images, 3)
    din = DeviceBuffer(lib, x.nbytes)
    dout = DeviceBuffer(lib, images * g.output_bytes)
    din.upload(x)
    n = max(steps * 10, 50)
    for _ in range(20):
        assert lib.ug_run_device(din.ptr, dout.ptr, images) == 0
    t0 = time.perf_counter()
    for _ in range(n):
        assert lib.ug_run_device(din.ptr, dout.ptr, images) == 0
    run_us = (time.perf_counter() - t0) / n * 1e6
    g.profile(1)
    for _ in range(n):
        assert lib.ug_run_device(din.ptr, dout.ptr, images) == 0
    counters = g.profile(2)
    g.profile(0)
    kernel_us = float(counters[2:2 + lib.ug_op_count()].sum()) / max(int(counters[0]), 1) / 1e3
    din.free()
    dout.free()
    from uq_native import Session
    with Session(plan, "mailbox", lib) as s:
        for _ in range(20):
            s.run(x)
        t0 = time.perf_counter()
        for _ in range(n):
            s.run(x)
        mailbox_us = (time.perf_counter() - t0) / n * 1e6
    nbytes = sum(c["bytes"] for c in P.op_costs(plan, images))
    return {"images": images, "run_device_us": round(run_us, 2), "mailbox_us": round(mailbox_us, 2),
            "kernel_us": round(kernel_us, 2), "bytes": nbytes,
            "frac": round(nbytes / (kernel_us * 1e-6) / HBM_PEAK, 4), "bound": "hbm"}


def secondary(lib, steps):
    out = {}
    plan, images = W.WORKLOADS["yolo"]()
    g = Graph(plan, lib)
    sec, per_op = time_device(lib, g, images, steps, 2)
    costs = P.op_costs(plan, images)
    nbytes = sum(c["bytes"] for c in costs)
    out["yolo"] = {"images": images, "ms": round(sec / steps * 1e3, 4), "images_per_s": round(images * steps / sec, 1),
                   "gops": round(sum(c["ops"] for c in costs) / 1e9, 2),
                   "frac": round(nbytes / (sec / steps) / HBM_PEAK, 4), "bound": "hbm (network bytes)"}
    # The matrix cores' sustained rate on this device: a register-only MFMA
    # loop launched back to back for about as long as each GEMM launch
    # (short: the head's ~45 us; long: the 3x3's ~0.6 ms), so that the clock
    # it holds under that load is the GEMM's.
    ceiling = {}
    for label, iters in (("short", 180), ("long", 2400)):
        tops, us = mfma_ceiling(lib, iters, warmup=3, reps=steps)
        ceiling[label] = {"tops": round(tops, 1), "launch_us": round(us, 1), "frac": round(tops * 1e12 / INT8_PEAK, 4)}
    out["mfma_ceiling"] = ceiling
    for name, leg in (("head", "short"), ("conv3x3", "long")):
        plan, images = W.WORKLOADS[name]()
        g = Graph(plan, lib)
        sec, per_op = time_device(lib, g, images, steps, 2)
        ops = sum(c["ops"] for c in P.op_costs(plan, images))
        kernel_tops = ops / (per_op.sum() * 1e-9) / 1e12
        out[name] = {"images": images, "ms": round(sec / steps * 1e3, 4), "tops": round(ops / (sec / steps) / 1e12, 2),
                     "kernel_tops": round(kernel_tops, 2), "frac": round(kernel_tops * 1e12 / INT8_PEAK, 4),
                     "frac_of_ceiling": round(kernel_tops / ceiling[leg]["tops"], 4), "bound": "mfma"}
    out["pointwise_b1"] = pointwise_latency(lib, steps)
    out["host_transfer"] = host_transfer(lib, max(steps // 2, 3))
    for name in ("dw3s1", "dw3s2", "dw5s1", "dw5s2"):
        plan, images = W.WORKLOADS[name]()
        g = Graph(plan, lib)
        sec, per_op = time_device(lib, g, images, steps, 2)
        nbytes = sum(c["bytes"] for c in P.op_costs(plan, images))
        kernel_gbps = nbytes / (per_op.sum() * 1e-9) / 1e9
        out[name] = {"images": images, "ms": round(sec / steps * 1e3, 4),
                     "gbps": round(nbytes / (sec / steps) / 1e9, 1),
                     "kernel_gbps": round(kernel_gbps, 1), "frac": round(kernel_gbps * 1e9 / HBM_PEAK, 4),
                     "bound": "hbm"}
    return out


def library_gemm(reps=20):
    """The vendor library's int8 GEMM (torch._int_mm: int8 x int8 -> int32,
    no requantisation) on the head and 3x3 layers' GEMM shapes and on a
    large square one, random operands, for comparison with the large-tile
    kernels here."""
    import torch
    torch.manual_seed(0)
    res = {}
    for name, (m, k, n) in {"head": (25088, 960, 1280), "conv3x3_as_gemm": (3276800, 1152, 128),
                            "square_8192": (8192, 8192, 8192)}.items():
        a = torch.randint(-128, 128, (m, k), dtype=torch.int8, device="cuda")
        b = torch.randint(-128, 128, (n, k), dtype=torch.int8, device="cuda").t()
        for _ in range(5):
            torch._int_mm(a, b)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            torch._int_mm(a, b)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        res[name] = {"m": m, "k": k, "n": n, "us": round(us, 1), "tops": round(2 * m * k * n / us / 1e6, 1)}
        del a, b
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 50 warm-up steps (~30 ms for MNv4): the GPU clock keeps rising for the
    # first few tens of passes; 200 timed steps (~120 ms).
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="mnv4")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--per-op", action="store_true", help="print the per-op table to stderr")
    ap.add_argument("--images", type=int, default=0, help="batch size (default: the workload's own)")
    ap.add_argument("--library-gemm", action="store_true",
                    help="only time the vendor library's int8 GEMM on the same shapes and print it as JSON")
    ap.add_argument("--mfma-ceiling", type=int, default=0, metavar="ITERS",
                    help="only time the register-only int8 MFMA loop (ITERS rounds per wave, --steps launches "
                         "after --warmup) and print it as JSON")
    args = ap.parse_args()
    if args.library_gemm:
        print(json.dumps(library_gemm()), flush=True)
        return
    if args.mfma_ceiling:
        tops, us = mfma_ceiling(open_library(), args.mfma_ceiling, warmup=args.warmup, reps=args.steps)
        print(json.dumps({"mfma_ceiling": {"iters": args.mfma_ceiling, "tops": round(tops, 1), "launch_us": round(us, 1),
                                           "frac": round(tops * 1e12 / INT8_PEAK, 4)}}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); images are independent, so N GPUs "
              f"would each run this same per-GPU batch", file=sys.stderr)
        sys.exit(2)
    plan, images = W.WORKLOADS[args.workload]()
    images = args.images or images
    # The CPU baseline runs first, in child processes, before this process
    # touches the GPU.
    cpu, cpu_other = (None, {}) if args.no_cpu else cpu_legs(args.workload,
                                                              legs=() if args.no_secondary else CPU_LEGS)
    lib = open_library()
    graph = Graph(plan, lib)
    seconds, per_op_ns = time_device(lib, graph, images, args.steps, args.warmup)
    costs = P.op_costs(plan, images)
    if args.per_op:
        for i, (c, ns) in enumerate(zip(costs, per_op_ns)):
            log(f"op {i:3d} code {c['code']:2d} {ns / 1e3:9.2f} us  {c['bytes'] / ns:8.1f} GB/s  "
                f"{(c['ops'] / ns / 1e3 if c['ops'] else 0):8.1f} TOP/s")
        log(f"sum of op times {per_op_ns.sum() / 1e3:.1f} us, wall per step {seconds / args.steps * 1e6:.1f} us")
    op, roof = roofline_entry(costs, per_op_ns)
    traffic, source = committed_traffic(args.workload, op)
    if traffic:
        roof["traffic"] = traffic
        roof["traffic_source"] = f"profiles/{source}"
    ms = seconds / args.steps * 1e3
    result = {
        "metric": METRIC, "value": round(images * args.steps / seconds, 1), "unit": "images/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded uniform int8 images, random-init int8 weights)",
        "config": {"workload": f"{args.workload}: MobileNetV4-Conv-Small-shaped int8 classifier 224x224x3"
                               if args.workload == "mnv4" else args.workload,
                   "global_batch": images, "ops": len(costs),
                   "gops_per_step": round(sum(c["ops"] for c in costs) / 1e9, 3),
                   "gbytes_per_step": round(sum(c["bytes"] for c in costs) / 1e9, 4),
                   "parallelism": "single GPU, batch-outer"},
        "roofline": roof,
        "sum_kernel_us": round(float(per_op_ns.sum()) / 1e3, 2),
        # The whole step against HBM: every op's algorithmic bytes at 8 TB/s.
        "network_roofline": {"floor_us": round(sum(c["bytes"] for c in costs) / HBM_PEAK * 1e6, 1),
                             "frac": round(sum(c["bytes"] for c in costs) / HBM_PEAK / (seconds / args.steps), 4)},
    }
    if not args.no_secondary:
        result["secondary"] = secondary(lib, 10)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu
        if cpu_other:
            result["cpu_baseline_other"] = cpu_other
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
