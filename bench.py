#!/usr/bin/env python3
"""Benchmark of the MTC quantized-weight matmul on one MI355X.

Headline (the `value`): packed-weight GB/s of the fp32 decode kernel at M = 1
on workload c2 (4096 x 4096 Student-t weights, PermutedQuadtreeRD (32,16,8,4)
@ 4.25 bits/weight), i.e. allocator-accounted packed bytes (alloc.total_bits/8)
per call divided by the per-call time. One step = one Y = X * W_hat call at
M = 1 on one rotating copy of the packed weight; >= 1 GiB of distinct copies
rotate so the weight is read from HBM, not the 256 MB Infinity Cache. The K
timed calls are replayed from a HIP graph (launch-bound decode loops are
graph-captured in serving too) between a synchronize on both sides.

Also reported in the same JSON line: M = 16 on c2 (fp32-VALU bound) and the
prefill kernel (bf16 MFMA) on c4 (8192 x 8192, QuadtreeRD @ 4.5, M = 4096),
and the CPU baseline (C/OpenMP port of the reference block loop) on a bounded
sample of the c2 M = 1 workload.

    python bench.py [--steps K] [--warmup W] [--no-prefill] [--no-cpu-baseline]
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400)
    ap.add_argument("--warmup", type=int, default=240)
    ap.add_argument("--rotate-gib", type=float, default=1.0)
    ap.add_argument("--prefill-steps", type=int, default=60)
    ap.add_argument("--prefill-warmup", type=int, default=100)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-m16", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--graph", type=int, default=1, help="replay the timed calls from a HIP graph")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 FETCH_SIZE/WRITE_SIZE passes")
    ap.add_argument("--pmc-child", help=argparse.SUPPRESS)
    ap.add_argument("--workload", default="c2", choices=["c2", "c3", "c5"],
                    help="c2 (default): the headline decode + c4 prefill run; c3: the 24-layer decoder "
                         "stack (168 matrices) at M=1 and M=512; c5: the adversarial leaf mix at M=1 and M=256")
    ap.add_argument("--c3-layers", type=int, default=24)
    return ap.parse_args()


COPY_BYTES = 256 << 20


def pmc_child(path):
    """Body of one counter pass: a plain device copy of known size, then the decode kernel."""
    import torch
    from tensorpack_amd.device import DeviceStream
    from tensorpack_amd.packer import PanelStream
    ps = PanelStream.load(path)
    with np.load(path.replace(".npz", "_x.npz")) as z:
        x = z["x"]
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    ds = DeviceStream(ps)
    copies = [ds] + [ds.clone() for _ in range(7)]
    X = torch.from_numpy(x).cuda()
    Y = torch.empty((X.shape[0], ps.N), dtype=torch.float32, device="cuda")
    for c in copies:
        c.workspace(X.shape[0])
    torch.cuda.synchronize()
    for _ in range(4):
        for c in copies:
            c.gemv_f32(X, out=Y)
    torch.cuda.synchronize()
    print("pmc child done", flush=True)


def traffic_passes(ps, x, kernel="k_gemv"):
    """HBM bytes per decode launch from two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE).

    Each counter is scaled by what it reads for a device copy of COPY_BYTES in the
    same pass (bytes moved / counter bytes), so unit or per-instance conventions of
    the counter cancel. Runs before this process touches the GPU; returns None
    when rocprofv3 is unavailable or a pass fails."""
    import shutil
    import subprocess
    import tempfile
    from tensorpack_amd.profiling import dispatch_values
    exe = shutil.which("rocprofv3")
    if exe is None:
        log("traffic: rocprofv3 not found")
        return None
    tmp = tempfile.mkdtemp(prefix="mtc_pmc_")
    path = os.path.join(tmp, "stream.npz")
    ps.save(path)
    np.savez(os.path.join(tmp, "stream_x.npz"), x=x)
    res = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        cmd = ["timeout", "-s", "KILL", "120", exe, "--pmc", counter, "-d", tmp, "-o", counter, "--",
               sys.executable, os.path.abspath(__file__), "--pmc-child", path]
        log("traffic pass: " + " ".join(cmd[3:]))
        r = subprocess.run(cmd, capture_output=True, text=True, env=dict(os.environ, TMPDIR="/tmp"))
        db = os.path.join(tmp, counter + "_results.db")
        if r.returncode != 0 or not os.path.exists(db):
            log(f"traffic pass {counter} failed (rc {r.returncode}): {r.stderr[-400:]}")
            return None
        kern = dispatch_values(db, counter, kernel)
        # the four COPY_BYTES device copies are the largest copy dispatches of the pass
        # (host-to-device staging copies share the kernel name but are small)
        copy = sorted(dispatch_values(db, counter, "copyBuffer"))[-4:]
        if not kern or len(copy) < 4 or min(copy) <= 0:
            log(f"traffic pass {counter}: kernel or copy dispatches missing")
            return None
        copy_kib = sum(copy) / len(copy)
        res[counter] = {"kernel_kib": sum(kern) / len(kern), "copy_kib": copy_kib,
                        "factor": COPY_BYTES / (copy_kib * 1024.0), "copy_spread": max(copy) / min(copy)}
    fetch = res["FETCH_SIZE"]["kernel_kib"] * 1024.0 * res["FETCH_SIZE"]["factor"]
    write = res["WRITE_SIZE"]["kernel_kib"] * 1024.0 * res["WRITE_SIZE"]["factor"]
    shutil.rmtree(tmp, ignore_errors=True)
    return {"bytes": fetch + write, "fetch_bytes": fetch, "write_bytes": write,
            "fetch_factor": res["FETCH_SIZE"]["factor"], "write_factor": res["WRITE_SIZE"]["factor"]}


def timed_calls(torch, launch_list, steps, warmup, use_graph):
    """Time exactly `steps` calls cycling over launch_list; returns (seconds, per-call ms)."""
    n = len(launch_list)
    stream = torch.cuda.current_stream()
    if use_graph:
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                for f in launch_list:
                    f()
        stream.wait_stream(side)
        tail = steps % n
        gt = None
        if tail:
            gt = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                with torch.cuda.graph(gt, stream=side):
                    for f in launch_list[:tail]:
                        f()
            stream.wait_stream(side)
        for _ in range(max(1, warmup // n)):
            g.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps // n):
            g.replay()
        if gt is not None:
            gt.replay()
        stop.record(stream)
        torch.cuda.synchronize()
    else:
        for i in range(warmup):
            launch_list[i % n]()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(steps):
            launch_list[i % n]()
        stop.record(stream)
        torch.cuda.synchronize()
    ms = start.elapsed_time(stop)
    return ms / 1e3, ms / steps


def graph_of(torch, fns):
    """Capture fns (in order) into one HIP graph on a side stream."""
    g = torch.cuda.CUDAGraph()
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for f in fns:
                f()
    stream.wait_stream(side)
    return g


def time_replays(torch, g, reps, warmup=2):
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / reps          # ms per replay


def run_c3(args):
    """Qwen2.5-0.5B-shaped stack: 24 layers x (q, k, v, o, gate, up, down), QT-P @ 3.125 b/w
    each; all 168 matrices back to back at M=1 (fp32 decode kernel) and at M=512 (bf16 MFMA
    prefill), each pass captured as one HIP graph. At M=1 the pass runs once with one launch
    per matrix and once with the matrices that read the same input grouped (q/k/v, gate/up:
    4 launches per layer); the grouped pass is the reported value."""
    import torch
    from tensorpack_amd import workloads
    from tensorpack_amd.kernels.gemm import MTCMatrix
    from tensorpack_amd.device import require_gpu
    mats = workloads.c3_matrices(args.c3_layers)
    t0 = time.time()
    allocs = workloads.allocate_many(mats)
    log(f"c3: {len(mats)} allocations in {time.time() - t0:.1f}s")
    dev = require_gpu()
    torch.cuda.set_device(dev)
    ms_ = [MTCMatrix.from_quadtree(a, w.W) for a, w in zip(allocs, mats)]
    packed = float(sum(m.packed_bytes for m in ms_))
    weights = sum(w.W.size for w in mats)
    xs = {}
    def x_of(K, M, dtype):
        key = (K, M, dtype)
        if key not in xs:
            xs[key] = torch.from_numpy(np.random.RandomState(3000 + K + M).randn(M, K).astype(np.float32)).to(dev).to(dtype)
        return xs[key]
    # M = 1: each pass runs every matrix once; whole copies of the stack rotate so the weights come from HBM
    streams = [m.device_stream() for m in ms_]
    ys1 = [torch.empty((1, w.W.shape[1]), dtype=torch.float32, device=dev) for w in mats]
    for s_, w, y in zip(streams, mats, ys1):
        s_.workspace(1)
        s_.gemv_f32(x_of(w.W.shape[0], 1, torch.float32), out=y)
    torch.cuda.synchronize()
    n_rot = max(1, int(np.ceil(args.rotate_gib * (1 << 30) / sum(s_.device_bytes() for s_ in streams))))
    sets = [streams] + [[s_.clone() for s_ in streams] for _ in range(n_rot - 1)]
    for ss in sets[1:]:                              # workspaces exist before capture
        for s_, w, y in zip(ss, mats, ys1):
            s_.workspace(1)
            s_.gemv_f32(x_of(w.W.shape[0], 1, torch.float32), out=y)
    torch.cuda.synchronize()
    from tensorpack_amd.device import gemv_f32_group

    def time_m1(plan):
        """Per rotating set, one graph of the pass; plan = list of index groups (one launch each)."""
        def calls(ss):
            out = []
            for grp in plan:
                if len(grp) == 1:
                    i = grp[0]
                    out.append(lambda s_=ss[i], w=mats[i], y=ys1[i]: s_.gemv_f32(x_of(w.W.shape[0], 1, torch.float32), out=y))
                else:
                    out.append(lambda g=[ss[i] for i in grp], K=mats[grp[0]].W.shape[0], ys=[ys1[i] for i in grp]:
                               gemv_f32_group(g, x_of(K, 1, torch.float32), ys))
            return out
        graphs = [graph_of(torch, calls(ss)) for ss in sets]
        for g in graphs:
            g.replay()
        torch.cuda.synchronize()
        reps = max(2, 40 // len(graphs))
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            for g in graphs:
                g.replay()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / (reps * len(graphs))

    n_per = len(workloads.QWEN_LAYER)
    # q, k, v read the layer input; gate and up read the post-attention input: one launch each
    layer_groups = [[0, 1, 2], [3], [4, 5], [6]]
    plan_grouped = [[L * n_per + i for i in grp] for L in range(args.c3_layers) for grp in layer_groups]
    ms1_single = time_m1([[i] for i in range(len(mats))])
    log(f"c3 M=1, one launch per matrix: {ms1_single * 1e3:.1f} us per pass of {len(mats)} matrices, "
        f"{packed / (ms1_single * 1e-3) / 1e9:.1f} GB/s packed")
    ms1_grouped = time_m1(plan_grouped)
    log(f"c3 M=1, grouped ({len(plan_grouped)} launches): {ms1_grouped * 1e3:.1f} us per pass, "
        f"{packed / (ms1_grouped * 1e-3) / 1e9:.1f} GB/s packed")
    # the whole pass as ONE batched launch per rotating set (each matrix its own X and Y)
    from tensorpack_amd.device import GemvBatch
    batches = [GemvBatch(ss, [x_of(w.W.shape[0], 1, torch.float32) for w in mats], ys1) for ss in sets]
    for b in batches:
        b.launch()
    torch.cuda.synchronize()
    reps = max(4, 200 // len(batches))
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        for b in batches:
            b.launch()
    stop.record()
    torch.cuda.synchronize()
    ms1 = start.elapsed_time(stop) / (reps * len(batches))
    log(f"c3 M=1, one batched launch: {ms1 * 1e3:.1f} us per pass, {packed / (ms1 * 1e-3) / 1e9:.1f} GB/s packed")
    # parity of the timed pass: every output against its own single call
    ref = [s_.gemv_f32(x_of(w.W.shape[0], 1, torch.float32)) for s_, w in zip(sets[-1], mats)]
    torch.cuda.synchronize()
    batch_bit_identical = all(torch.equal(a_, b_) for a_, b_ in zip(ref, ys1))
    log(f"c3 M=1 batched outputs bit-identical to single calls: {batch_bit_identical}")
    del sets, batches
    # M = 512: prefill of every matrix
    M = 512
    tiles = [m.device_tiles() for m in ms_]
    ysp = [torch.empty((M, w.W.shape[1]), dtype=torch.float32, device=dev) for w in mats]
    from tensorpack_amd.device import gemm_bf16_group

    def time_prefill(plan):
        fns = []
        for grp in plan:
            K = mats[grp[0]].W.shape[0]
            if len(grp) == 1:
                i = grp[0]
                fns.append(lambda t=tiles[i], K=K, y=ysp[i]: t.gemm_bf16(x_of(K, M, torch.bfloat16), out=y))
            else:
                fns.append(lambda ts=[tiles[i] for i in grp], K=K, ys=[ysp[i] for i in grp]:
                           gemm_bf16_group(ts, x_of(K, M, torch.bfloat16), ys))
        for f in fns:
            f()
        torch.cuda.synchronize()
        return time_replays(torch, graph_of(torch, fns), 5)

    flop = 2.0 * M * weights
    msp_single = time_prefill([[i] for i in range(len(mats))])
    log(f"c3 M=512, one matrix per launch: {msp_single:.3f} ms per pass, {flop / (msp_single * 1e-3) / 1e12:.1f} TFLOP/s")
    msp = time_prefill(plan_grouped)
    tf = flop / (msp * 1e-3) / 1e12
    log(f"c3 M=512, grouped: {msp:.3f} ms per pass, {tf:.1f} TFLOP/s")
    return {"metric": "packed-weight GB/s at M=1 over the 168-matrix stack (fp32 decode kernel)",
            "value": packed / (ms1 * 1e-3) / 1e9, "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
            "dtype": "f32", "data": "synthetic (seeded N(0, 0.02) weights per matrix, random-init)",
            "config": {"workload": f"c3 Qwen2.5-0.5B-shaped stack, {args.c3_layers} layers, QT-P @ 3.125",
                       "matrices": len(mats), "weights": weights, "packed_bytes": packed,
                       "rotating_sets": n_rot},
            "us_per_pass_m1": ms1 * 1e3, "launches_m1": 1, "batch_bit_identical": batch_bit_identical,
            "us_per_pass_m1_grouped": ms1_grouped * 1e3, "launches_m1_grouped": len(plan_grouped),
            "us_per_pass_m1_one_launch_per_matrix": ms1_single * 1e3,
            "roofline": {"bound": "hbm", "achieved": packed / (ms1 * 1e-3) / 1e9, "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": packed / (ms1 * 1e-3) / 1e9 / HBM_PEAK_GBS},
            "prefill_m512": {"ms_per_pass": msp, "TFLOPs": tf, "frac_bf16_peak": tf / BF16_PEAK_TFLOPS,
                             "ms_per_pass_one_matrix_per_launch": msp_single}}


def run_c5(args):
    """Adversarial leaf mix (QT @ 2.5 b/w, many 4x4 and P0 leaves): M=1 fp32 decode over
    rotating copies, and M=256 through the bf16 MFMA path (fp32 X staged to bf16)."""
    import torch
    from tensorpack_amd import workloads
    from tensorpack_amd.kernels.gemm import MTCMatrix
    from tensorpack_amd.device import require_gpu
    wl = workloads.c5()
    t0 = time.time()
    a = wl.allocate()
    log(f"c5 allocation {time.time() - t0:.1f}s, {a.bits_per_element:.4f} b/w")
    dev = require_gpu()
    torch.cuda.set_device(dev)
    m = MTCMatrix.from_quadtree(a, wl.W)
    ds = m.device_stream()
    n_copies = max(1, int(np.ceil(args.rotate_gib * (1 << 30) / ds.device_bytes())))
    copies = [ds] + [ds.clone() for _ in range(n_copies - 1)]
    X1 = torch.from_numpy(wl.activations(1)).to(dev)
    Y1 = torch.empty((1, wl.W.shape[1]), dtype=torch.float32, device=dev)
    for c in copies:
        c.workspace(1)
        c.gemv_f32(X1, out=Y1)
    torch.cuda.synchronize()
    secs, ms = timed_calls(torch, [lambda c=c: c.gemv_f32(X1, out=Y1) for c in copies], args.steps, args.warmup,
                           bool(args.graph))
    gbs = m.packed_bytes / (ms * 1e-3) / 1e9
    log(f"c5 M=1: {ms * 1e3:.2f} us/call, {gbs:.1f} GB/s packed")
    M = 256
    t = m.device_tiles()
    X = torch.from_numpy(wl.activations(M)).to(dev)
    Y = torch.empty((M, wl.W.shape[1]), dtype=torch.float32, device=dev)
    t.gemm_bf16(X, out=Y)
    torch.cuda.synchronize()
    s2, ms2 = timed_calls(torch, [lambda: t.gemm_bf16(X, out=Y)], 50, 5, bool(args.graph))
    tf = 2.0 * M * wl.W.size / (ms2 * 1e-3) / 1e12
    log(f"c5 M=256: {ms2 * 1e3:.1f} us/call, {tf:.1f} TFLOP/s")
    return {"metric": "packed-weight GB/s at M=1 (fp32 decode kernel)", "value": gbs, "unit": "GB/s",
            "n_gpus": 1, "higher_is_better": True, "dtype": "f32",
            "data": "synthetic (seeded np.random.RandomState weights/activations, random-init)",
            "config": {"workload": wl.name + " M=1", "packed_bytes": m.packed_bytes,
                       "stream_bytes": ds.device_bytes(), "rotating_copies": n_copies, "us_per_call": ms * 1e3},
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS},
            "m256": {"us_per_call": ms2 * 1e3, "TFLOPs": tf, "frac_bf16_peak": tf / BF16_PEAK_TFLOPS,
                     "x_dtype": "f32 (staged to bf16 by k_stage_x)"}}


def main():
    args = parse()
    if args.pmc_child:
        pmc_child(args.pmc_child)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if args.workload != "c2":
        print(json.dumps(run_c3(args) if args.workload == "c3" else run_c5(args)), flush=True)
        return
    import torch
    from tensorpack_amd import workloads
    from tensorpack_amd.kernels.gemm import MTCMatrix
    from tensorpack_amd.device import require_gpu

    res = {}

    # ---------------- c2 decode ----------------
    wl = workloads.c2()
    t0 = time.time()
    alloc = wl.allocate()
    log(f"c2 allocation {time.time() - t0:.1f}s, {alloc.bits_per_element:.4f} b/w")
    m = MTCMatrix.from_quadtree(alloc, wl.W)
    traffic = None
    if not args.no_traffic:
        # counter passes run in child processes before this one initialises the GPU
        traffic = traffic_passes(m.panel_stream(m.decode_chunk_rows(1)), wl.activations(1))
    dev = require_gpu()
    torch.cuda.set_device(dev)
    t0 = time.time()
    ds = m.device_stream()
    log(f"c2 packed in {time.time() - t0:.1f}s: chunk_rows={ds.host.chunk_rows} stream {ds.device_bytes()} B, "
        f"accounted {m.packed_bytes:.0f} B")
    packed = m.packed_bytes
    per_copy = ds.device_bytes()
    n_copies = max(1, int(np.ceil(args.rotate_gib * (1 << 30) / per_copy)))
    copies = [ds] + [ds.clone() for _ in range(n_copies - 1)]
    X1 = torch.from_numpy(wl.activations(1)).to(dev)
    Y1 = torch.empty((1, wl.W.shape[1]), dtype=torch.float32, device=dev)
    for c in copies:
        c.workspace(1)
        c.gemv_f32(X1, out=Y1)
    torch.cuda.synchronize()
    launches = [lambda c=c: c.gemv_f32(X1, out=Y1) for c in copies]
    secs, ms = timed_calls(torch, launches, args.steps, args.warmup, bool(args.graph))
    gbs = packed / (ms * 1e-3) / 1e9
    log(f"c2 M=1: {ms * 1e3:.2f} us/call, {gbs:.1f} GB/s packed ({n_copies} copies)")
    y_gpu = Y1.cpu().numpy().copy()

    if not args.no_m16:
        d16 = m.device_stream(None, dev, 16)
        c16 = [d16] + [d16.clone() for _ in range(max(1, int(np.ceil(args.rotate_gib * (1 << 30) / d16.device_bytes()))) - 1)]
        X16 = torch.from_numpy(wl.activations(16)).to(dev)
        Y16 = torch.empty((16, wl.W.shape[1]), dtype=torch.float32, device=dev)
        for c in c16:
            c.workspace(16)
            c.gemv_f32(X16, out=Y16)
        torch.cuda.synchronize()
        l16 = [lambda c=c: c.gemv_f32(X16, out=Y16) for c in c16]
        s16, ms16 = timed_calls(torch, l16, max(args.steps // 4, len(c16)), args.warmup // 4, bool(args.graph))
        flop16 = 2.0 * 16 * wl.W.shape[0] * wl.W.shape[1]
        res["c2_m16"] = {"us_per_call": ms16 * 1e3, "packed_GBps": packed / (ms16 * 1e-3) / 1e9,
                         "TFLOPs": flop16 / (ms16 * 1e-3) / 1e12,
                         "frac_fp32_peak": flop16 / (ms16 * 1e-3) / 1e12 / FP32_PEAK_TFLOPS,
                         "chunk_rows": d16.host.chunk_rows}
        del c16
        log(f"c2 M=16: {ms16 * 1e3:.2f} us/call, {res['c2_m16']['TFLOPs']:.2f} TFLOP/s")

    # ---------------- achievable HBM bandwidth: a plain 1 GiB device copy ----------------
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * src.numel() * 4 * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9     # read + write bytes
    del src, dst
    log(f"device copy: {copy_gbs:.0f} GB/s (read + write)")
    # the same for copies of the packed weight's size, rotated over ~1 GiB and replayed
    # from a graph like the decode: what a launch of this size achieves on the copy path
    n_el = int(packed) // 4
    n_rot = max(2, (1 << 30) // (2 * 4 * n_el))
    srcs = [torch.empty(n_el, dtype=torch.float32, device=dev) for _ in range(n_rot)]
    dsts = [torch.empty_like(s) for s in srcs]
    g = graph_of(torch, [lambda s=s, d=d: d.copy_(s) for s, d in zip(srcs, dsts)])
    copy_small_us = time_replays(torch, g, 5) * 1e3 / n_rot
    del g, srcs, dsts
    log(f"device copy of {4 * n_el} B: {copy_small_us:.2f} us per copy ({n_rot} rotating pairs)")

    # ---------------- CPU baseline (bounded sample) ----------------
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import mtc_oracle as O
        inner = alloc.inner
        la = O.LeafArena(inner.weights, inner.sizes, inner.leaf, inner.modes, inner.scales,
                         alloc.row_perm, alloc.col_perm)
        x = wl.activations(1)
        y_cpu = O.cpu_qt_gemm(x, la)
        calls, t0 = 0, time.time()
        while True:
            O.cpu_qt_gemm(x, la)
            calls += 1
            if time.time() - t0 >= args.cpu_seconds and calls >= 3:
                break
        el = time.time() - t0
        cores = int(O.cpu_lib().oracle_threads())
        cpu = {"value": packed * calls / el / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
               "sample": f"{calls} calls of c2 M=1 (full 4096x4096 matrix) in {el:.1f}s, C/OpenMP port of the "
                         f"reference block loop (gemm.py:124-210)",
               "gpu_vs_cpu_rel_frobenius": O.relative_frobenius_error(y_cpu, y_gpu)}
        log(f"cpu baseline {cpu['value']:.3f} GB/s on {cores} threads; gpu-vs-cpu rel {cpu['gpu_vs_cpu_rel_frobenius']:.2e}")
        # the reference's own inference path: X @ the cached dequantized weight (LinearMTCAdaptive.forward,
        # mtc/nn/layers.py:150-151), numpy BLAS over a dense fp32 W_hat
        w_hat = np.ascontiguousarray(alloc.dequant, dtype=np.float32)
        x @ w_hat
        n_np, t0 = 0, time.time()
        while time.time() - t0 < 2.0 or n_np < 3:
            x @ w_hat
            n_np += 1
        el_np = time.time() - t0
        cpu["numpy_dequant_matmul"] = {"ms_per_call": 1e3 * el_np / n_np,
                                       "packed_GBps": packed * n_np / el_np / 1e9,
                                       "dense_fp32_GBps": w_hat.nbytes * n_np / el_np / 1e9,
                                       "sample": f"{n_np} calls of x (1 x 4096) @ W_hat (4096 x 4096 fp32) in {el_np:.1f}s"}
        log(f"cpu numpy X @ W_hat: {1e3 * el_np / n_np:.2f} ms/call")
        del w_hat

    # ---------------- c4 prefill ----------------
    if not args.no_prefill:
        wl4 = workloads.c4()
        t0 = time.time()
        a4 = wl4.allocate()
        log(f"c4 allocation {time.time() - t0:.1f}s, {a4.bits_per_element:.4f} b/w")
        m4 = MTCMatrix.from_quadtree(a4, wl4.W)
        t0 = time.time()
        g4 = m4.device_tiles()
        log(f"c4 packed in {time.time() - t0:.1f}s")
        M4 = 4096
        X4 = torch.from_numpy(wl4.activations(M4)).to(dev).to(torch.bfloat16)
        Y4 = torch.empty((M4, wl4.W.shape[1]), dtype=torch.float32, device=dev)
        g4.gemm_bf16(X4, out=Y4)
        torch.cuda.synchronize()
        s4, ms4 = timed_calls(torch, [lambda: g4.gemm_bf16(X4, out=Y4)], args.prefill_steps, args.prefill_warmup, False)
        flop4 = 2.0 * M4 * wl4.W.shape[0] * wl4.W.shape[1]
        tf = flop4 / (ms4 * 1e-3) / 1e12
        res["c4_prefill"] = {"M": M4, "ms_per_call": ms4, "TFLOPs": tf, "frac_bf16_peak": tf / BF16_PEAK_TFLOPS,
                             "packed_bytes": m4.packed_bytes}
        log(f"c4 M=4096: {ms4:.3f} ms/call, {tf:.1f} TFLOP/s ({100 * tf / BF16_PEAK_TFLOPS:.1f}% of bf16 peak)")

    K, N = wl.W.shape
    out = {
        "metric": "packed-weight GB/s at M=1 (fp32 decode kernel)",
        "value": gbs,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded np.random.RandomState weights/activations, random-init)",
        "config": {"workload": wl.name + " M=1", "K": K, "N": N, "M": 1, "budget_bits": wl.budget,
                   "bits_per_weight": alloc.bits_per_element, "packed_bytes": packed,
                   "stream_bytes": per_copy, "rotating_copies": n_copies,
                   "chunk_rows": ds.host.chunk_rows, "graph_replay": bool(args.graph)},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None if traffic is None else traffic["bytes"],
                     "copy_GBps": copy_gbs, "frac_of_copy": gbs / copy_gbs,
                     "copy_same_bytes_us": copy_small_us, "us_per_call": ms * 1e3,
                     "kernel": "k_gemv<1>", "stream_GBps": per_copy / (ms * 1e-3) / 1e9,
                     "traffic_detail": traffic},
        "cpu_baseline": cpu,
        "extra": res,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
