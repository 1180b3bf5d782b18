#!/usr/bin/env python3
"""BFP8 W8A16 GEMV benchmark on one MI355X.

Workload (default, --workload sweep): the synthetic 24-layer decode-token
weight sweep at batch 1 -- per layer gate 3584x1024, up 3584x1024, down
1024x3584, in-projection 6144x1024, out-projection 1024x2048 -- followed by
the 65536x1024 lm_head with fused greedy argmax + top-40.  Mantissas uniform
in [-127, 127], exponents uniform in [124, 130] ([122, 128] for the lm_head),
a fresh N(0,1) activation per GEMV (silu(a)*b with 1% +-20 outliers for the
down projection).  One step = one persistent launch (bfp8_sweep_kernel, 3
five-wavefront workgroups per CU): each workgroup streams the lm_head's
tiles dealt to it, then takes the other 120 GEMVs' tiles from ticket
queues, quantizing every unit's activation itself; the last workgroup
merges the lm_head's per-tile top-k lists as they are published.  Weights
resident in HBM.  Weight copies rotate (2 sweeps = 1.08 GB) so the 256 MB
Infinity Cache cannot serve repeats.

roofline: the launch that moves the most bytes (for the sweep, its one
launch), timed alone with HIP events on its stream; its algorithmic bytes =
weights + int16 activations (2 B/element) + f32 block scales + f32 outputs.

value = algorithmic bytes per sweep (weights once + f32 x in + f32 y out; the
fused lm_head writes no logits) / wall time per step, in GB/s.

Extra workloads for the per-config numbers: --workload lm_head (65536x1024
fused top-40), gemv (3584x1024), down (1024x3584), batch16 (B=16 x 3584x1024 and
65536x1024), select (top-k above 64 at the lm_head),
lm_head_bf16 (the reference's bf16 tied-embedding lm_head, top-64),
forward_token (the reference's forward_token_c: 24 layers at the model's
shapes with distinct synthetic weights + bf16 lm_head argmax, per token).

    python bench.py [--steps K] [--warmup W] [--workload sweep] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import mmap
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
# the CPU baseline's OpenMP threads stay on neighbouring cores (read by
# libgomp when the reference library first loads it)
os.environ.setdefault("OMP_PROC_BIND", "close")
PKG = ROOT / "qwen35-ax7020-edge-llm_amd"
sys.path.insert(0, str(PKG))

PEAK_HBM_GBPS = 8000.0
PEAK_MFMA_I8_TOPS = 5000.0  # dense int8 MFMA, MI355X (the batch kernel's integer part)
VALU_LANE_OPS = 256 * 4 * 16 * 2.4e9  # 32-bit VALU lane operations per second, no packed math
LAYER = [("gate", 3584, 1024), ("up", 3584, 1024), ("down", 1024, 3584), ("in_proj", 6144, 1024),
         ("out_proj", 1024, 2048)]
N_LAYERS = 24
LM_HEAD = (65536, 1024)
TOPK = 40


def wbytes(M, K):
    return M * K + M * (K // 64)


def workload_items(name):
    """[(tag, M, K, e_lo, e_hi, topk)] for one step of a workload."""
    if name == "sweep":
        items = [("lm_head", *LM_HEAD, 122, 128, TOPK)]
        for layer in range(N_LAYERS):
            items += [(f"l{layer}.{t}", M, K, 124, 130, 0) for t, M, K in LAYER]
        return items
    if name == "layers":  # the sweep without the lm_head
        return [it for it in workload_items("sweep") if it[0] != "lm_head"]
    if name == "lm_head":
        return [("lm_head", *LM_HEAD, 122, 128, TOPK)]
    if name == "lm_head_plain":  # the lm_head GEMV without the fused top-k
        return [("lm_head", *LM_HEAD, 122, 128, 0)]
    if name == "gemv":
        return [("gemv", 3584, 1024, 124, 130, 0)]
    if name == "down":
        return [("down", 1024, 3584, 124, 130, 0)]
    raise ValueError(name)


def metric_bytes(items):
    """Weights once + f32 activations in + f32 outputs (none for the fused lm_head)."""
    return sum(wbytes(M, K) + 4 * K + (0 if tk else 4 * M) for _, M, K, _, _, tk in items)


def kernel_bytes(items):
    """Bytes the grouped GEMV kernel must move: weights, int16 activations
    (split form, 2 B/element) + f32 block scales, f32 outputs."""
    return sum(wbytes(M, K) + 2 * K + 4 * (K // 64) + (0 if tk else 4 * M) for _, M, K, _, _, tk in items)


def read_traffic(workload, kernel):
    """HBM bytes per dispatch of `kernel` from the committed rocprofv3 PMC
    summary of this workload, if any (a line `traffic_bytes_per_dispatch
    <kernel>: <bytes>`)."""
    p = ROOT / "profiles" / f"{workload}_pmc.md"
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_dispatch " + re.escape(kernel) + r":\s*([0-9.]+)", p.read_text())
    return float(m.group(1)) if m else None


def cpu_baseline(items, seconds=10.0, single_seconds=6.0, batch=1, nbytes=None):
    """The reference's host bfp8_gemv (float path, 04/qwen_kernels_opt.c:311-325)
    built from its own sources (oracle/_ref), timed on this host over the same
    synthetic GEMV list; falls back to the oracle's restatement of that path.
    Timed with the OpenMP default thread count, then with one thread.  With
    batch > 1 each GEMV is called once per activation vector (the reference
    has no batched GEMV) and a pass counts `nbytes` (default: the list's
    metric bytes)."""
    import numpy as np

    import qwen_kernels_gpu as qk

    ref = ROOT / "oracle" / "_ref" / "libref_qwen_kernels.so"
    port = ROOT / "oracle" / "liboracle.so"
    if ref.exists():
        lib = ctypes.CDLL(str(ref))
        lib.init_kernels()
        fn, kind = lib.bfp8_gemv, "reference"
    elif port.exists():
        lib = ctypes.CDLL(str(port))
        fn, kind = lib.orc_gemv_float, "port"
    else:
        return None
    fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 2
    fn.restype = None
    host = []
    for i, (tag, M, K, lo, hi, tk) in enumerate(items):
        mant, exps = qk.synth_planes(M, K, 7_000 + i, lo, hi)
        for b in range(batch):
            x = qk.synth_normal(K, 8_000 + 100 * i + b)
            host.append((mant, exps, x, np.empty(M, dtype=np.float32), M, K))
    if nbytes is None:
        nbytes = metric_bytes(items)

    def timed(limit):
        for mant, exps, x, y, M, K in host[:1]:  # first touch of the pages, untimed
            fn(y.ctypes.data, x.ctypes.data, mant.ctypes.data, exps.ctypes.data, M, K)
        t0 = time.perf_counter()
        sweeps = 0
        while True:
            for mant, exps, x, y, M, K in host:
                fn(y.ctypes.data, x.ctypes.data, mant.ctypes.data, exps.ctypes.data, M, K)
            sweeps += 1
            el = time.perf_counter() - t0
            if el >= limit:
                return sweeps, el

    gomp = None
    if kind == "reference":
        # libgomp.so.1 is the OpenMP runtime the reference library links:
        # its thread count is the one the timed calls use
        gomp = ctypes.CDLL("libgomp.so.1")
        gomp.omp_set_num_threads.argtypes = [ctypes.c_int]
        gomp.omp_get_max_threads.restype = ctypes.c_int
    sweeps, el = timed(seconds)
    threads = gomp.omp_get_max_threads() if gomp else 1
    out = {"value": round(nbytes * sweeps / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
           "sample": (f"{sweeps} passes over the same GEMV list ({len(items)} GEMVs, {nbytes / 1e6:.1f} MB per pass; "
                      f"the lm_head as a plain GEMV, the reference having no fused BFP8 lm_head)" if batch == 1 else
                      f"{sweeps} batches of {batch} bfp8_gemv calls on one {items[0][1]}x{items[0][2]} matrix "
                      f"({nbytes / 1e6:.2f} MB per batch counted as for the GPU: weights once + f32 x in + f32 y out)")
                     + f", host float path with OpenMP over rows (OMP_PROC_BIND={os.environ.get('OMP_PROC_BIND')}), "
                       f"{el:.1f} s"}
    if gomp:
        # the same library with one OpenMP thread
        gomp.omp_set_num_threads(1)
        s1, e1 = timed(single_seconds)
        gomp.omp_set_num_threads(threads)
        out["single_thread"] = {"value": round(nbytes * s1 / e1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                                "sample": f"{s1} {'batches' if batch > 1 else 'passes over the same list'}, {e1:.1f} s"}
    return out


def read_probe_same_bytes(lib, qk, torch, stream, nbytes, steps):
    """The read-bandwidth probe (`bfp8_read_probe_kernel`) over nbytes, as one
    launch reads them: windows of nbytes rotating through >= 1 GiB (so none is
    served from the 256 MB last-level cache), `steps` back-to-back launches
    between one event pair.  A streaming read of that size with its ramp-up and
    tail: what one launch of the kernel's bytes can reach here, beside the
    8 TB/s peak."""
    n = (nbytes + 15) // 16 * 16
    nwin = max(2, -(-(1 << 30) // n))
    buf = torch.empty(nwin * n, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    base = buf.data_ptr()
    for i in range(2):
        qk.check(lib.bfp8_dev_read_probe(base + (i % nwin) * n, n, sink.data_ptr(), stream.cuda_stream))
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(steps):
        qk.check(lib.bfp8_dev_read_probe(base + (i % nwin) * n, n, sink.data_ptr(), stream.cuda_stream))
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / steps
    del buf
    return {"bytes": n, "avg_us": round(us, 3), "GBps": round(n / (us * 1e-6) / 1e9, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # (200 timed steps: the wall clock's fixed cost around the loop, the first
    # launch's latency and the final synchronization, ~15-25 us and now and
    # then ~120 us with host jitter, spread over 200 steps instead of 50)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="sweep",
                    choices=["sweep", "layers", "lm_head", "lm_head_plain", "gemv", "down", "batch16", "lm_head_bf16",
                             "host_gemv", "select",
                             "forward_token"])
    ap.add_argument("--rotate-gb", type=float, default=1.0, help="rotating weight copies totalling >= this")
    ap.add_argument("--bf16-layout", choices=["tiles", "rows"], default="tiles",
                    help="lm_head_bf16: the library's cached tile layout or a row-major device table")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--callback", choices=["none", "gemv4"], default="none",
                    help="forward_token: the full-attention layers' host callback -- none, or the engine's "
                         "rmsnorm + q/k/v/o bfp8_gemv calls through the host ABI (attention itself stubbed)")
    ap.add_argument("--batch-shape", choices=["all", "3584x1024", "65536x1024"], default="all",
                    help="batch16: the matrix shapes to run")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py runs on one GPU only; the path shards by rows across GPUs "
              "(each GPU a contiguous slice of row tiles, the lm_head top-k merged across them), but "
              "multi-GPU runs are not part of it", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import qwen_kernels_gpu as qk

    torch.cuda.set_device(0)
    lib = qk.load()
    lib.init_kernels()
    if args.workload == "batch16":
        return bench_batch16(args, qk, torch, np)
    if args.workload == "lm_head_bf16":
        return bench_lm_head_bf16(args, qk, torch, np)
    if args.workload == "forward_token":
        return bench_forward_token(args, qk, torch, np)
    if args.workload == "host_gemv":
        return bench_host_gemv(args, qk, torch, np)
    if args.workload == "select":
        return bench_select(args, qk, torch, np)

    items = workload_items(args.workload)
    per_copy = sum(wbytes(M, K) for _, M, K, *_ in items)
    copies = max(1, int(np.ceil(args.rotate_gb * 1e9 / per_copy)))
    print(f"[bench] {args.workload}: {len(items)} GEMVs, {per_copy / 1e6:.1f} MB weights, {copies} copies",
          file=sys.stderr, flush=True)
    xs = []
    for i, (tag, M, K, lo, hi, tk) in enumerate(items):
        x = qk.synth_swiglu(K, 5_000 + i) if (K == 3584) else qk.synth_normal(K, 5_000 + i)
        xs.append(torch.from_numpy(x).cuda())
    plans, keep = [], []
    for c in range(copies):
        plan_items = []
        for i, (tag, M, K, lo, hi, tk) in enumerate(items):
            dm = qk.DeviceMatrix.synth(M, K, 1_000_003 * c + i, lo, hi)
            it = {"mat": dm, "x": xs[i]}
            if tk:
                it["topk"] = tk
            else:
                it["y"] = torch.empty(M, dtype=torch.float32, device="cuda")
            plan_items.append(it)
        plans.append(qk.SweepPlan(plan_items))
        keep.append(plan_items)
    torch.cuda.synchronize()

    # warmup, then the timed steps (plan.run(): every launch of one step)
    for i in range(args.warmup):
        plans[i % copies].run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        plans[i % copies].run()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    mbytes = metric_bytes(items)
    value = mbytes / (ms_per_step * 1e-3) / 1e9
    print(f"[bench] timed {args.steps} steps: {ms_per_step * 1e3:.1f} us/step", file=sys.stderr, flush=True)

    # each step alone between HIP events: median and min, cold (rotating
    # weight copies, as above) and warm (one copy again and again, so a
    # workload under the 256 MB last-level cache is served from it)
    stream = torch.cuda.current_stream()

    def per_step(pick):
        evs = []
        for i in range(args.steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            plans[pick(i)].run()
            b.record(stream)
            evs.append((a, b))
        torch.cuda.synchronize()
        us = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
        return {"us_median": round(us[len(us) // 2], 2), "us_min": round(us[0], 2),
                "GBps_median": round(mbytes / (us[len(us) // 2] * 1e-6) / 1e9, 1)}

    cold = per_step(lambda i: i % copies)
    for i in range(2):
        plans[0].run()
    warm = per_step(lambda i: 0)
    print(f"[bench] per step: cold {cold}, warm {warm}", file=sys.stderr, flush=True)

    # each GEMV launch alone, HIP events on the stream it is launched on:
    # stage 0 streams the lm_head's tiles, stage 1 every other GEMV's (its
    # workgroup 0 also merges the lm_head top-k; with no other GEMV, stage 1
    # is the stand-alone merge kernel)
    head = [it for it in items if it[5]]
    rest = [it for it in items if not it[5]]
    stages = []
    single = plans[0].kernel_name(0) == "bfp8_sweep_kernel"  # the whole plan in one launch
    for stage, its in (((0, items),) if single else ((0, head), (1, rest))):
        name = plans[0].kernel_name(stage)
        if not name:
            continue
        # `steps` back-to-back launches of this stage between one event pair
        # (rotating weight copies): per-launch time without the dispatch
        # latency of an isolated launch, as the kernel trace measures it
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for i in range(2):
            plans[i % copies].launch(stage)
        a.record(stream)
        for i in range(args.steps):
            plans[i % copies].launch(stage)
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / args.steps
        # algorithmic bytes of the launch: the single launch reads the float
        # activations (quantized in LDS), the two-launch path's layer launch
        # the quantized records
        nbytes = metric_bytes(its) if single else kernel_bytes(its)
        stages.append({"stage": stage, "name": name, "avg_us": us,
                       "bytes": nbytes if name != "bfp8_topk_merge_kernel" else 0})
    dom = max(stages, key=lambda st: st["bytes"])
    kernel_us = dom["avg_us"]
    achieved = dom["bytes"] / (kernel_us * 1e-6) / 1e9

    # a separate quantize launch (the two-launch path runs one when its plan
    # has no fused lm_head; the single launch quantizes in LDS)
    quant_us = None
    if not single:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(args.steps):
            plans[i % copies].quantize()
        b.record(stream)
        torch.cuda.synchronize()
        quant_us = a.elapsed_time(b) * 1e3 / args.steps

    # measured read-only ceiling over 1 GiB, and a copy of known size (the
    # PMC counter calibration kernel)
    buf = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    for _ in range(2):
        qk.check(lib.bfp8_dev_read_probe(buf.data_ptr(), buf.numel(), sink.data_ptr(), stream.cuda_stream))
    rev = []
    for _ in range(10):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        qk.check(lib.bfp8_dev_read_probe(buf.data_ptr(), buf.numel(), sink.data_ptr(), stream.cuda_stream))
        b.record(stream)
        rev.append((a, b))
    torch.cuda.synchronize()
    ceiling = buf.numel() / (np.mean([a.elapsed_time(b) for a, b in rev]) * 1e-3) / 1e9
    cpy = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    qk.check(lib.bfp8_dev_copy_probe(cpy.data_ptr(), buf.data_ptr(), cpy.numel(), stream.cuda_stream))
    torch.cuda.synchronize()
    del buf, cpy
    same = read_probe_same_bytes(lib, qk, torch, stream, dom["bytes"], args.steps)

    traffic = read_traffic(args.workload, dom["name"])
    result = {
        "metric": "BFP8 GEMV achieved HBM GB/s (% of peak); us per 24-layer decode sweep",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint16->int32, f32 epilogue",
        "data": "synthetic (seeded counter-hash mantissas/exponents, Box-Muller activations)",
        "config": {"workload": args.workload, "gemvs_per_step": len(items), "batch": 1,
                   "weight_bytes_per_step": per_copy, "metric_bytes_per_step": mbytes,
                   "rotating_copies": copies, "parallelism": "single GPU"},
        "us_per_step": round(ms_per_step * 1e3, 2),
        "pct_of_peak": round(100 * value / PEAK_HBM_GBPS, 2),
        "per_step_cold": cold,
        "per_step_warm": warm,
        "kernel": {"name": dom["name"], "stage": dom["stage"], "avg_us": round(kernel_us, 2),
                   "algorithmic_bytes": dom["bytes"]},
        "launches_us": {f"stage{st['stage']}:{st['name']}": round(st["avg_us"], 2) for st in stages}
                       | ({"quantize": round(quant_us, 2)} if quant_us is not None else {}),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": traffic},
        "hbm_read_ceiling_GBps": round(ceiling, 1),
        "frac_of_measured_ceiling": round(achieved / ceiling, 4),
        "read_probe_same_bytes": same,
        "frac_of_same_bytes_probe": round(achieved / same["GBps"], 4),
    }
    if not args.no_cpu:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(items)
    print(json.dumps(result), flush=True)
    for p in plans:
        p.close()


def batch_kernel(M, K):
    """The kernel the library's batch launch picks for B = 16 (M rows, K
    columns) while K <= 1024: a workgroup per four 64-row tiles from 512
    tiles on, below that a workgroup per half tile and half of the vectors
    with each residue's blocks split over four wavefronts; with larger K the
    per-tile / per-half matrix-core kernel."""
    if K // 64 > 16:
        return "bfp8_gemv_batch_mfma_kernel"
    return "bfp8_gemv_batch_cu_kernel" if (M + 63) // 64 >= 512 else "bfp8_gemv_batch_split_kernel"


def bench_batch16(args, qk, torch, np):
    """C4: B = 16 activation vectors against one weight matrix, weights read
    once per batch, at 3584 x 1024 and at 65536 x 1024, on the matrix-core
    batch kernel (int8 MFMA for the exact residue sums, the float epilogue on
    the VALU).  roofline: HBM, with the kernel's algorithmic bytes (weights +
    int16 activations + f32 block scales + f32 outputs) over its time between
    HIP events.  Its two floors beside it: hbm_floor_us (those bytes at
    8 TB/s) and epilogue_floor_us, the float epilogue on the VALU at its
    least -- per row, vector, block and residue an integer combine of the
    two int8 parts' sums, a conversion, a multiply and an add (the
    reference's order, no contraction), 4 lane-operations at 256 CUs x 4
    SIMDs x 16 lanes x 2.4 GHz.  binding_floor_us is the larger, and
    frac_of_binding_floor its ratio to the time.  mfma_tops: the int8 MFMA
    operations (2 per weight, vector and activation part) per second, against
    the 5.0 POP/s dense int8 peak.  3584 x 1024 is latency-bound (112 tiles:
    both floors are under 1 us).  Per call, `us_eager_calls` times `steps`
    calls issued one by one and `us_graph` the same calls replayed from a HIP
    graph (the 3584 x 1024 kernel is shorter than a host ctypes launch, so
    the eager loop times the host there); `us` is the faster of the two,
    named in `timing`."""
    B = 16
    lib = qk.load()
    s = torch.cuda.current_stream()
    shapes = []
    for M, K, e_lo, e_hi in ((3584, 1024, 124, 130), (65536, 1024, 122, 128)):
        if args.batch_shape not in ("all", f"{M}x{K}"):
            continue
        per_copy = wbytes(M, K)
        copies = max(1, int(np.ceil(args.rotate_gb * 1e9 / per_copy)))
        mats = [qk.DeviceMatrix.synth(M, K, 900 + c, e_lo, e_hi) for c in range(copies)]
        X = torch.from_numpy(np.stack([qk.synth_normal(K, 950 + b) for b in range(B)])).cuda()
        xsp = torch.empty(B * K // 64 * 32, dtype=torch.int32, device="cuda")
        xsc = torch.empty(B * K // 64, dtype=torch.float32, device="cuda")
        for b in range(B):
            qk.check(lib.bfp8_dev_quantize(None, xsc.data_ptr() + b * (K // 64) * 4, xsp.data_ptr() + b * (K // 64) * 128,
                                           X[b].data_ptr(), K, s.cuda_stream))
        Y = torch.empty((B, M), dtype=torch.float32, device="cuda")
        # the launches' arguments resolved beforehand: a loop of bare ctypes
        # calls keeps ahead of the GPU, so the events time the kernels
        fn = lib.bfp8_dev_gemv_batch
        call = [(Y.data_ptr(), xsp.data_ptr(), xsc.data_ptr(), m.mant.data_ptr(), m.exps.data_ptr(), M, K, B,
                 s.cuda_stream) for m in mats]
        for i in range(args.warmup):
            qk.check(fn(*call[i % copies]), "gemv_batch")
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        rcs = []
        a.record(s)
        for i in range(args.steps):
            rcs.append(fn(*call[i % copies]))
        b.record(s)
        torch.cuda.synchronize()
        if any(rcs):
            raise RuntimeError(f"bfp8_dev_gemv_batch failed: {set(rcs)}")
        us_eager = a.elapsed_time(b) * 1e3 / args.steps
        # The same calls replayed from a HIP graph: a 3584 x 1024 call runs
        # shorter than one ctypes launch takes on the host (~5-7 us), so the
        # eager loop above can time the host; the replay times the kernels.
        # Every replay's output is checked against the eager call's.
        cs = torch.cuda.Stream()
        cs.wait_stream(s)
        gcall = [c[:-1] + (cs.cuda_stream,) for c in call]
        with torch.cuda.stream(cs):
            qk.check(fn(*gcall[0]), "gemv_batch")
        s.wait_stream(cs)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cs):
            for i in range(args.steps):
                qk.check(fn(*gcall[i % copies]), "gemv_batch")
        torch.cuda.synchronize()
        qk.check(fn(*call[(args.steps - 1) % copies]), "gemv_batch")
        torch.cuda.synchronize()
        y_eager = Y.clone()
        reps = 5
        g.replay()
        torch.cuda.synchronize()
        if not torch.equal(Y, y_eager):
            raise RuntimeError("batch GEMV graph replay differs from the eager call")
        a.record(s)
        for _ in range(reps):
            g.replay()
        b.record(s)
        torch.cuda.synchronize()
        if not torch.equal(Y, y_eager):
            raise RuntimeError("batch GEMV graph replay differs from the eager call")
        us_graph = a.elapsed_time(b) * 1e3 / (reps * args.steps)
        del g
        # the faster of the two submissions (the same calls, the same work):
        # the graph where the host cannot keep ahead of the kernels, the eager
        # calls where a graph's per-node cost exceeds the launch gap
        us, timing = (us_graph, "hip graph") if us_graph < us_eager else (us_eager, "eager calls")
        gbs = (per_copy + B * 4 * K + B * 4 * M) / (us * 1e-6) / 1e9
        mfma_tops = 2.0 * 2 * M * K * B / (us * 1e-6) / 1e12
        kbytes = per_copy + B * (2 * K + 4 * (K // 64)) + B * 4 * M
        kgbs = kbytes / (us * 1e-6) / 1e9
        hbm_floor = kbytes / (PEAK_HBM_GBPS * 1e9) * 1e6
        epi_floor = 4.0 * M * B * (K // 64) * 4 / VALU_LANE_OPS * 1e6
        floor = max(hbm_floor, epi_floor)
        del mats, X, Y
        same = read_probe_same_bytes(lib, qk, torch, s, kbytes, args.steps)
        shapes.append({"M": M, "K": K, "B": B, "us": round(us, 3), "timing": timing,
                       "us_eager_calls": round(us_eager, 3), "us_graph": round(us_graph, 3),
                       "GBps": round(gbs, 2),
                       "mfma_tops": round(mfma_tops, 3), "mfma_frac": round(mfma_tops / PEAK_MFMA_I8_TOPS, 4),
                       "hbm_floor_us": round(hbm_floor, 3), "epilogue_floor_us": round(epi_floor, 3),
                       "binding_floor_us": round(floor, 3), "frac_of_binding_floor": round(floor / us, 4),
                       "rotating_copies": copies,
                       "roofline": {"bound": "hbm", "achieved": round(kgbs, 2), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                                    "frac": round(kgbs / PEAK_HBM_GBPS, 4), "algorithmic_bytes": kbytes,
                                    "traffic": read_traffic("batch16", f"{batch_kernel(M, K)}@{M}x{K}")},
                       "read_probe_same_bytes": same,
                       "frac_of_same_bytes_probe": round(kgbs / same["GBps"], 4)})
    # a copy of known size: the PMC counters' calibration kernel
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    cpy = torch.empty_like(src)
    qk.check(lib.bfp8_dev_copy_probe(cpy.data_ptr(), src.data_ptr(), cpy.numel(), s.cuda_stream))
    torch.cuda.synchronize()
    del src, cpy
    first = shapes[0]
    out = {"metric": "BFP8 GEMV B=16 achieved GB/s and int Tops/s", "value": first["GBps"],
           "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "us_per_step": first["us"], "mfma_tops": first["mfma_tops"],
           "epilogue_floor_us": first["epilogue_floor_us"], "frac_of_binding_floor": first["frac_of_binding_floor"],
           "higher_is_better": True,
           "dtype": "int8xint16->int32, f32 epilogue", "data": "synthetic",
           "config": {"workload": "batch16", "M": first["M"], "K": first["K"], "B": B},
           "roofline": first["roofline"], "shapes": shapes}
    if not args.no_cpu:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        M, K = first["M"], first["K"]
        out["cpu_baseline"] = cpu_baseline([("batch16", M, K, 124, 130, 0)], batch=B,
                                           nbytes=wbytes(M, K) + B * 4 * K + B * 4 * M)
    print(json.dumps(out), flush=True)


def bench_select(args, qk, torch, np):
    """k above 64 at the 65536 x 1024 lm_head (bfp8_dev_lm_head_topk): the
    scores (the plain GEMV into the stream's scratch), then the selection --
    32 blocks of 2048 keys sorted in LDS and registers, each block's first
    min(k, 2048) keys ranked against every block's -- for k = 65, 200 and
    vocab + 50.
    Per k: the call, and the GEMV alone on the same inputs (the difference is
    the selection's)."""
    V, H = 65536, 1024
    lib = qk.load()
    dm = qk.DeviceMatrix.synth(V, H, 777, 122, 128)
    x = torch.from_numpy(qk.synth_normal(H, 778)).cuda()
    _, xs, xsp = qk.quantize(x)
    y = torch.empty(V, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream
    ev = lambda: torch.cuda.Event(enable_timing=True)

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        a, b = ev(), ev()
        a.record(stream)
        for _ in range(args.steps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / args.steps

    gemv_us = timed(lambda: qk.check(lib.bfp8_dev_gemv(y.data_ptr(), xsp.data_ptr(), xs.data_ptr(), dm.mant.data_ptr(),
                                                       dm.exps.data_ptr(), V, H, None, s)))
    per_k = {}
    for k in (65, 200, V + 50):
        kk = min(k, V)
        ids = torch.empty(kk, dtype=torch.int32, device="cuda")
        sc = torch.empty(kk, dtype=torch.float32, device="cuda")
        cnt = torch.empty(2, dtype=torch.int32, device="cuda")
        us = timed(lambda: qk.check(lib.bfp8_dev_lm_head_topk(ids.data_ptr(), sc.data_ptr(), cnt.data_ptr(),
                                                               cnt.data_ptr() + 4, xsp.data_ptr(), xs.data_ptr(),
                                                               dm.mant.data_ptr(), dm.exps.data_ptr(), V, H, k, s)))
        per_k[str(k)] = {"us_per_call": round(us, 2), "selection_us": round(us - gemv_us, 2)}
    print(json.dumps({"metric": "lm_head top-k above 64: us per call", "value": per_k["200"]["us_per_call"],
                      "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                      "higher_is_better": False,
                      "config": {"workload": "select", "vocab": V, "hidden": H, "k": [65, 200, V + 50]},
                      "gemv_alone_us": round(gemv_us, 2), "per_k": per_k}), flush=True)


def bench_lm_head_bf16(args, qk, torch, np):
    """The reference's own lm_head: bf16 tied embedding 65536 x 1024 (134 MB)
    with the fused top-64 (the chat sampler's k), rotating table copies.
    --bf16-layout tiles (default): the 64-row tile layout the library keeps
    its cached tables in (lm_head_argmax / lm_head_topk / forward_token_c on
    the engine's read-only image), converted once before timing; rows: a
    caller's row-major device table (bf16_dev_lm_head)."""
    V, H, K = 65536, 1024, 64
    lib = qk.load()
    tiled = args.bf16_layout == "tiles"
    per_copy = V * H * 2
    copies = max(1, int(np.ceil(args.rotate_gb * 1e9 / per_copy)))
    tables = []
    for c in range(copies):
        g = torch.Generator(device="cuda").manual_seed(100 + c)
        t = (torch.randn((V, H), device="cuda", generator=g) * 0.05).to(torch.bfloat16).view(torch.int16)
        if tiled:
            tt = torch.empty(lib.bf16_dev_tiles_bytes(V, H) // 2, dtype=torch.int16, device="cuda")
            qk.check(lib.bf16_dev_tile_table(tt.data_ptr(), t.data_ptr(), V, H, None))
            torch.cuda.synchronize()
            del t
            t = tt
        tables.append(t)
    h = torch.randn(H, device="cuda", dtype=torch.float32)
    ids = torch.empty(K, dtype=torch.int32, device="cuda")
    sc = torch.empty(K, dtype=torch.float32, device="cuda")
    cnt = torch.empty(2, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    s = stream.cuda_stream

    def head(i, k, logits):
        if tiled:
            return lib.bf16_dev_lm_head_tiles(ids.data_ptr() if k else None, sc.data_ptr() if k else None,
                                              cnt.data_ptr() if k else None, cnt.data_ptr() + 4 if k else None,
                                              logits, h.data_ptr(), tables[i % copies].data_ptr(), V, H, k, s)
        return lib.bf16_dev_lm_head(ids.data_ptr() if k else None, sc.data_ptr() if k else None,
                                    cnt.data_ptr() if k else None, cnt.data_ptr() + 4 if k else None, logits,
                                    h.data_ptr(), tables[i % copies].data_ptr(), V, H, k, 1, s)

    def run(i, k):
        qk.check(head(i, k, None))

    for i in range(args.warmup):
        run(i, K)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        run(i, K)
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) * 1e6 / args.steps
    # the dot-product kernel alone (scores to a logits buffer, no selection)
    logits = torch.empty(V, dtype=torch.float32, device="cuda")
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(args.steps):
        qk.check(head(i, 0, logits.data_ptr()))
    b.record(stream)
    torch.cuda.synchronize()
    kus = a.elapsed_time(b) * 1e3 / args.steps
    kbytes = per_copy + H * 4 + V * 4
    step_bytes = per_copy + H * 4
    print(json.dumps({"metric": "bf16 lm_head achieved HBM GB/s", "value": round(step_bytes / us / 1e3, 2),
                      "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                      "us_per_step": round(us, 2), "higher_is_better": True,
                      "config": {"workload": "lm_head_bf16", "vocab": V, "hidden": H, "topk": K,
                                 "layout": args.bf16_layout, "rotating_copies": copies},
                      "kernel": {"name": "bf16_lm_head_tiles_kernel" if tiled else "bf16_lm_head_kernel",
                                 "avg_us": round(kus, 2), "algorithmic_bytes": kbytes},
                      "roofline": {"bound": "hbm", "achieved": round(kbytes / kus / 1e3, 1), "peak": PEAK_HBM_GBPS,
                                   "unit": "GB/s", "frac": round(kbytes / kus / 1e3 / PEAK_HBM_GBPS, 4)}}), flush=True)


class _SynthModel:
    """Model-shaped synthetic weights in host memory, the engine's layout:
    BFP8 planes (mantissas [M][K], exponents [M][K/64]) distinct per layer,
    float parameters, states, a bf16 embedding table, and the plan arrays
    forward_token_c takes."""

    GEMVS = {"qkv": (6144, 1024), "z": (2048, 1024), "o": (1024, 2048), "gate": (3584, 1024),
             "up": (3584, 1024), "down": (1024, 3584)}
    FULL = (3, 7, 11, 15, 19, 23)

    def __init__(self, qk, np, lin_type, mlp_type, seed=77):
        lib = qk.load()
        rng = np.random.default_rng(seed)
        self.keep = []
        self.is_full = np.array([1 if l in self.FULL else 0 for l in range(N_LAYERS)], dtype=np.int32)
        self.lin = (lin_type * 18)()
        self.mlp = (mlp_type * N_LAYERS)()
        self.weight_bytes = 0
        self.param_bytes = 0
        self.state_bytes = 0
        li, seed_i = 0, seed * 1000

        def arr(a):
            a = np.ascontiguousarray(a)
            self.keep.append(a)
            return a

        def vec(n, scale):
            self.param_bytes += 4 * n
            return arr((rng.standard_normal(n) * scale).astype(np.float32))

        def planes(plan, names):
            nonlocal seed_i
            for name in names:
                M, K = self.GEMVS[name]
                m = arr(np.empty(M * K, dtype=np.int8))
                e = arr(np.empty(M * (K // 64), dtype=np.uint8))
                lib.bfp8_synth_planes_host(m.ctypes.data, e.ctypes.data, M, K, seed_i, 122, 126)
                seed_i += 1
                self.weight_bytes += m.nbytes + e.nbytes
                setattr(plan, "mant_" + name, m.ctypes.data)
                setattr(plan, "exp_" + name, e.ctypes.data)
                setattr(plan, "M_" + name, M)
                setattr(plan, "K_" + name, K)

        for l in range(N_LAYERS):
            if self.is_full[l]:
                p = self.mlp[l]
                p.post_ln_w = vec(1024, 0.1).ctypes.data
                planes(p, ("gate", "up", "down"))
                continue
            p = self.lin[li]
            li += 1
            p.in_ln_w, p.post_ln_w = vec(1024, 0.1).ctypes.data, vec(1024, 0.1).ctypes.data
            p.conv_w = vec(6144 * 4, 0.5).ctypes.data
            p.wa, p.wb = vec(16 * 1024, 0.03).ctypes.data, vec(16 * 1024, 0.03).ctypes.data
            p.nea = arr((-rng.uniform(0.2, 3.0, 16)).astype(np.float32)).ctypes.data
            p.dt = arr(rng.uniform(-2, 2, 16).astype(np.float32)).ctypes.data
            p.norm_w = vec(128, 0.5).ctypes.data
            p.conv_s = arr(np.zeros(3 * 6144, dtype=np.float32)).ctypes.data
            p.state = arr(np.zeros(16 * 128 * 128, dtype=np.float32)).ctypes.data
            self.state_bytes += 4 * (3 * 6144 + 16 * 128 * 128)
            planes(p, ("qkv", "z", "o", "gate", "up", "down"))
        self.final_w = vec(1024, 0.1)
        # bf16 table: random sign, exponent 119..123, random 7-bit mantissa,
        # in read-only pages like the engine's mmap of its weight image
        # (04/qwen_real_engine.py:745-751), which the library caches on the
        # device in the lm_head's tile layout
        u = rng.integers(0, 2 ** 16, size=65536 * 1024, dtype=np.uint16)
        self._embed_map = mmap.mmap(-1, u.nbytes)
        self.embed = np.frombuffer(self._embed_map, dtype=np.uint16)
        self.embed[:] = (u & 0x807F) | ((119 + (u >> 7) % 5).astype(np.uint16) << 7)
        libc = ctypes.CDLL(None)
        libc.mprotect.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        if libc.mprotect(self.embed.ctypes.data, u.nbytes, mmap.PROT_READ) != 0:
            raise OSError("mprotect of the embedding table failed")
        self.h = arr(np.zeros(1024, dtype=np.float32))

    def token_bytes(self):
        """Algorithmic HBM bytes of one token: every BFP8 plane, the bf16
        table (the lm_head reads all of it), the float parameters, and the
        conv + recurrent states read and written once."""
        return self.weight_bytes + self.embed.nbytes + self.param_bytes + 2 * self.state_bytes

    def run(self, fn, token, cb=None):
        return fn(token, self.h.ctypes.data, ctypes.addressof(self.lin), ctypes.addressof(self.mlp),
                  self.is_full.ctypes.data, self.final_w.ctypes.data, self.embed.ctypes.data, cb, None)


# The full-attention callback's GEMVs (04/qwen_real_engine.py:1059-1087): q with
# its gate (16 heads x 256, interleaved), k and v (2 kv heads x 256), o.
CALLBACK_GEMVS = (("q", 4096, 1024), ("k", 512, 1024), ("v", 512, 1024), ("o", 1024, 2048))


class _ReadOnlyPlanes:
    """BFP8 planes (mantissas [M][K], exponents [M][K/64]) in a private mapping
    made read-only afterwards, as the engine's PROT_READ mmap of its weight
    image (04/qwen_real_engine.py:745-751): the library converts such weights
    once and keeps the device copy."""

    def __init__(self, lib, np, M, K, seed):
        self.M, self.K = M, K
        nm, ne = M * K, M * (K // 64)
        self.map = mmap.mmap(-1, nm + ne)
        buf = np.frombuffer(self.map, dtype=np.uint8)
        self.mant, self.exps = buf[:nm].view(np.int8), buf[nm:]
        lib.bfp8_synth_planes_host(self.mant.ctypes.data, self.exps.ctypes.data, M, K, seed, 122, 126)
        libc = ctypes.CDLL(None)
        libc.mprotect.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        page = mmap.PAGESIZE
        base = buf.ctypes.data & ~(page - 1)
        if libc.mprotect(base, (buf.ctypes.data + nm + ne - base + page - 1) // page * page, mmap.PROT_READ) != 0:
            raise OSError("mprotect of the weight planes failed")


def bench_host_gemv(args, qk, torch, np):
    """The engine's own bfp8_gemv calls through the host ABI (host pointers,
    synchronous: x copied in, y copied back), at the full-attention
    callback's shapes, weights in read-only pages (converted once, cached on
    the device).  Per-call latency, median and mean over --steps calls each,
    and the callback's four GEMVs per full-attention layer and per token (6
    such layers)."""
    lib = qk.load()
    mats = {n: _ReadOnlyPlanes(lib, np, M, K, 4100 + i) for i, (n, M, K) in enumerate(CALLBACK_GEMVS)}
    shapes = []
    for n, M, K in CALLBACK_GEMVS:
        w = mats[n]
        x = qk.synth_normal(K, 4200)
        y = np.empty(M, dtype=np.float32)
        for _ in range(max(3, args.warmup)):
            lib.bfp8_gemv(y.ctypes.data, x.ctypes.data, w.mant.ctypes.data, w.exps.ctypes.data, M, K)
        ts = []
        for _ in range(max(20, args.steps)):
            t0 = time.perf_counter()
            lib.bfp8_gemv(y.ctypes.data, x.ctypes.data, w.mant.ctypes.data, w.exps.ctypes.data, M, K)
            ts.append(time.perf_counter() - t0)
        ts.sort()
        shapes.append({"gemv": n, "M": M, "K": K, "us_median": round(ts[len(ts) // 2] * 1e6, 2),
                       "us_mean": round(sum(ts) / len(ts) * 1e6, 2), "us_min": round(ts[0] * 1e6, 2)})
    per_layer = sum(sh["us_median"] for sh in shapes)
    wb = sum(wbytes(M, K) for _, M, K in CALLBACK_GEMVS)
    print(json.dumps({"metric": "host-ABI bfp8_gemv latency per call (engine callback shapes)",
                      "value": round(per_layer, 2), "unit": "us per full-attention layer (4 GEMVs)",
                      "n_gpus": 1, "steps": max(20, args.steps), "warmup": max(3, args.warmup),
                      "higher_is_better": False, "dtype": "int8xint16->int32, f32 epilogue", "data": "synthetic",
                      "config": {"workload": "host_gemv", "weights": "read-only mapping (device copy cached)",
                                 "weight_bytes_per_layer": wb},
                      "us_per_token_6_layers": round(6 * per_layer, 1), "shapes": shapes}), flush=True)


def _callback_gemv4(qk, np, lib):
    """The full-attention callback of 04/qwen_real_engine.py:1059-1087 through
    this library's host ABI: rmsnorm of h, q/k/v GEMVs, the attention step
    (libqwen_attn.so's, not part of this library: stubbed as the first 2048
    q outputs), o GEMV, h += o.  Returns (callback, keepalive)."""
    mats = {n: _ReadOnlyPlanes(lib, np, M, K, 4300 + i) for i, (n, M, K) in enumerate(CALLBACK_GEMVS)}
    ln = (np.random.default_rng(5).standard_normal(1024) * 0.1).astype(np.float32)
    normed = np.empty(1024, dtype=np.float32)
    ys = {n: np.empty(M, dtype=np.float32) for n, M, _ in CALLBACK_GEMVS}
    gated = np.empty(2048, dtype=np.float32)

    def gemv(n, y, x):
        w = mats[n]
        lib.bfp8_gemv(y.ctypes.data, x.ctypes.data, w.mant.ctypes.data, w.exps.ctypes.data, w.M, w.K)

    def cb(layer, h_ptr, ctx):
        h = np.ctypeslib.as_array(ctypes.cast(h_ptr, ctypes.POINTER(ctypes.c_float)), shape=(1024,))
        lib.rmsnorm(normed.ctypes.data, h_ptr, ln.ctypes.data, 1024, 1e-6)
        gemv("q", ys["q"], normed)
        gemv("k", ys["k"], normed)
        gemv("v", ys["v"], normed)
        gated[:] = ys["q"][:2048] * np.float32(1e-3)
        gemv("o", ys["o"], gated)
        np.add(h, ys["o"], out=h)

    return qk.FULL_ATTN_CALLBACK(cb), (mats, ln, normed, ys, gated, cb)


def bench_forward_token(args, qk, torch, np):
    """forward_token_c (04/qwen_kernels_opt.c:1008-1049) called exactly as the
    engine calls it (host pointers, synchronous): 18 linear-attention layers +
    6 MLP-only layers (the full-attention layers' attention is the engine's
    host callback and is not part of the library: none here), final rmsnorm,
    bf16 lm_head argmax over 65536 x 1024.  Timed with the conv / recurrent
    states resident on the device (qwen_forward_state_resident(1)) and, as a
    second figure, with the reference's copy-in / copy-out of the states on
    every call."""
    lib = qk.load()
    m = _SynthModel(qk, np, qk.LinearLayerPlan, qk.MlpPlan)
    print(f"[bench] forward_token: {m.weight_bytes / 1e6:.1f} MB BFP8 + {m.embed.nbytes / 1e6:.1f} MB bf16 table "
          f"+ {m.param_bytes / 1e6:.1f} MB params, {m.state_bytes / 1e6:.1f} MB states", flush=True)

    if args.callback == "gemv4":
        cb, cb_keep = _callback_gemv4(qk, np, lib)
    else:
        cb = qk.FULL_ATTN_CALLBACK()  # NULL: no full-attention callback

    def timed(resident, steps, warmup):
        lib.qwen_forward_state_resident(resident)
        for i in range(warmup):
            m.run(lib.forward_token_c, 1000 + i, cb)
        ts = []
        for i in range(steps):
            t0 = time.perf_counter()
            m.run(lib.forward_token_c, 2000 + i, cb)
            ts.append(time.perf_counter() - t0)
        lib.qwen_forward_state_resident(0)
        ts.sort()
        return ts[len(ts) // 2] * 1e6, sum(ts) / len(ts) * 1e6

    med_res, mean_res = timed(1, args.steps, args.warmup)
    med_sync, mean_sync = timed(0, max(5, args.steps // 5), 2)
    tb = m.token_bytes()
    cpu = None
    ref = ROOT / "oracle" / "_ref" / "libref_qwen_kernels.so"
    if not args.no_cpu and ref.exists():
        rl = ctypes.CDLL(str(ref))
        rl.init_kernels()
        fn = rl.forward_token_c
        fn.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 8
        fn.restype = ctypes.c_int
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < 10.0:
            m.run(fn, 3000 + n)
            n += 1
        el = time.perf_counter() - t0
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
        cpu = {"value": round(n / el, 3), "unit": "tokens/s", "cores": threads, "kind": "reference",
               "sample": f"{n} tokens of the reference's host-built forward_token_c (float-path GEMVs, scalar "
                         f"runtime, OpenMP) on the same synthetic model, {el:.1f} s"}
    print(json.dumps({
        "metric": "decode tokens/s (forward_token_c: 24 layers + bf16 lm_head argmax)",
        "value": round(1e6 / med_res, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "us_per_token": round(med_res, 1), "us_per_token_mean": round(mean_res, 1),
        "us_per_token_state_copies": round(med_sync, 1), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 (BFP8 int8 x int16 GEMV)", "data": "synthetic",
        "config": {"workload": "forward_token", "layers": N_LAYERS, "linear_attention_layers": 18,
                   "hidden": 1024, "vocab": 65536, "state": "device-resident",
                   "full_attention_callback": ("rmsnorm + q/k/v/o bfp8_gemv through the host ABI per full layer "
                                               "(attention step stubbed)") if args.callback == "gemv4" else None},
        "roofline": {"bound": "hbm", "achieved": round(tb / med_res / 1e3, 1), "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": round(tb / med_res / 1e3 / PEAK_HBM_GBPS, 4), "traffic": None,
                     "scope": f"whole token: {tb / 1e6:.1f} MB algorithmic per token / wall time per token"},
        "cpu_baseline": cpu}), flush=True)


if __name__ == "__main__":
    main()
