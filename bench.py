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

Also reported in the same JSON line (`extra`), each with its own roofline object:
M = 16 on c2; the prefill kernel (bf16 MFMA) on c4 (8192 x 8192, QuadtreeRD @
4.5, M = 4096), its output checked on 64 sampled rows against the fp64 product;
the 168-matrix c3 stack at M = 1 (one batched launch per pass) and M = 512; the
adversarial c5 mix at M = 1 and M = 256. CPU baselines (C/OpenMP port of the
reference block loop) run on bounded samples of c2, c3 and c5. All allocations
(the c3 stack through forked worker processes) and the rocprofv3 counter passes
run before this process initialises the GPU.

    python bench.py [--steps K] [--warmup W] [--workload all|c2|c3|c5] [--no-cpu-baseline]
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


M1_LAYOUT = None              # layout of the M = 1 decode streams (None: MTCMatrix.decode_layout(1))


def m1_layout(m):
    return m.decode_layout(1) if M1_LAYOUT is None else M1_LAYOUT


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
    ap.add_argument("--pmc-child-batch", help=argparse.SUPPRESS)
    ap.add_argument("--pmc-child-tiles", help=argparse.SUPPRESS)
    ap.add_argument("--workload", default="all", choices=["all", "c2", "c3", "c5"],
                    help="all (default): the headline c2 decode plus c4 prefill, the c3 stack and c5; c2: c2 and "
                         "c4 only; c3: the 24-layer decoder stack (168 matrices) at M=1 and M=512 with per-launch "
                         "comparisons; c5: the adversarial leaf mix at M=1 and M=256")
    ap.add_argument("--m1-layout", default="auto", choices=["auto", "v1", "mx"],
                    help="payload layout of the M=1 decode streams: auto (MTCMatrix.decode_layout(1)), v1 "
                         "(chunk-contiguous, vector decode) or mx (matrix-core decode)")
    ap.add_argument("--c3-layers", type=int, default=24)
    ap.add_argument("--no-c3", action="store_true")
    ap.add_argument("--no-c5", action="store_true")
    return ap.parse_args()


COPY_BYTES = 256 << 20


def pmc_copies(torch):
    """The counter calibration: four plain device copies of COPY_BYTES."""
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()


def pmc_child(path):
    """Body of one counter pass: a plain device copy of known size, then the decode kernel."""
    import torch
    from tensorpack_amd.device import DeviceStream
    from tensorpack_amd.packer import PanelStream
    ps = PanelStream.load(path)
    with np.load(path.replace(".npz", "_x.npz")) as z:
        x = z["x"]
    pmc_copies(torch)
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


def pmc_child_batch(folder):
    """Body of one counter pass of the batched decode: the calibration copies, then four
    launches of one batch over the streams saved in `folder` (stream_NNN.npz; one input per
    K in x.npz, shared by every stream of that K)."""
    import torch
    from tensorpack_amd.device import DeviceStream, GemvBatch
    from tensorpack_amd.packer import PanelStream
    with np.load(os.path.join(folder, "x.npz")) as z:
        xs = {int(k[1:]): z[k] for k in z.files}
    n = len([f for f in os.listdir(folder) if f.startswith("stream_")])
    pss = [PanelStream.load(os.path.join(folder, f"stream_{i:03d}.npz")) for i in range(n)]
    pmc_copies(torch)
    streams = [DeviceStream(ps) for ps in pss]
    X = {K: torch.from_numpy(x).cuda() for K, x in xs.items()}
    batch = GemvBatch(streams, [X[s.K] for s in streams])
    torch.cuda.synchronize()
    for _ in range(4):
        batch.launch()
    torch.cuda.synchronize()
    print("pmc child done", flush=True)


TILE_FIELDS = ("cells", "step_off", "payload")


def save_tiles(ts, path):
    """A tile stream as plain arrays (no pickles): its fields plus the permutations, if any."""
    arrs = {f: getattr(ts, f) for f in TILE_FIELDS}
    arrs["shape"] = np.array([ts.K, ts.N, ts.n_ksteps, ts.n_col_tiles], dtype=np.int64)
    for f in ("row_perm", "col_perm"):
        if getattr(ts, f) is not None:
            arrs[f] = getattr(ts, f)
    np.savez(path, **arrs)


def load_tiles(path):
    from tensorpack_amd.tilestream import TileStream
    with np.load(path) as z:
        K, N, nk, nc = (int(v) for v in z["shape"])
        return TileStream(K, N, nk, nc, *(z[f] for f in TILE_FIELDS),
                          row_perm=z["row_perm"] if "row_perm" in z.files else None,
                          col_perm=z["col_perm"] if "col_perm" in z.files else None)


def pmc_child_tiles(folder):
    """Body of one counter pass of the prefill: the calibration copies, then four calls over the
    tile streams saved in `folder` (tiles_NNN.npz; inputs x.npz, one per K, fp32 or bf16 bits):
    one matrix runs gemm_bf16 (gemm_f32 when the folder holds a file named f32), several one
    batched prefill (GemmBatch)."""
    import torch
    from tensorpack_amd.device import DeviceTiles, GemmBatch
    n = len([f for f in os.listdir(folder) if f.startswith("tiles_")])
    tss = [load_tiles(os.path.join(folder, f"tiles_{i:03d}.npz")) for i in range(n)]
    with np.load(os.path.join(folder, "x.npz")) as z:
        xs = {int(k[1:]): z[k] for k in z.files}
    pmc_copies(torch)
    tiles = [DeviceTiles(ts) for ts in tss]

    def dev_x(x):
        if x.dtype == np.uint16:
            return torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16)
        return torch.from_numpy(x).cuda()
    X = {K: dev_x(x) for K, x in xs.items()}
    M = next(iter(X.values())).shape[0]
    Ys = [torch.empty((M, t.N), dtype=torch.float32, device="cuda") for t in tiles]
    if n == 1 and os.path.exists(os.path.join(folder, "f32")):
        launch = lambda: tiles[0].gemm_f32(X[tiles[0].K], out=Ys[0])
    elif n == 1:
        launch = lambda: tiles[0].gemm_bf16(X[tiles[0].K], out=Ys[0])
    else:
        batch = GemmBatch(tiles, [X[t.K] for t in tiles], Ys)
        launch = batch.launch
    launch()
    torch.cuda.synchronize()
    for _ in range(4):
        launch()
    torch.cuda.synchronize()
    print("pmc child done", flush=True)


# the prefill's launches: X staging, the tile kernel and its split-K reduction, or, on the
# decode-once path, the bf16 decode of W_hat and hipBLASLt's GEMM (its kernels' names start Cijk_)
PREFILL_KERNELS = ("k_stage_x", "k_gemm_tile", "k_splitk_reduce", "k_tile_dequant_bf16", "Cijk_")
F32_TILE_KERNELS = ("k_stage_x_f32", "k_gemm_f32", "k_splitk_reduce")


def traffic_passes_tiles(tss, xs, f32=False):
    """HBM bytes per prefill call over the tile streams `tss` (one: gemm_bf16, or gemm_f32 with
    `f32`; several: one batched prefill), summed over the call's launches (X staging, tiles,
    split-K reduction); `xs`: one input per K, fp32 or bf16 (as uint16 bits). See counter_passes."""
    import tempfile
    tmp = tempfile.mkdtemp(prefix="mtc_pmc_")
    for i, ts in enumerate(tss):
        save_tiles(ts, os.path.join(tmp, f"tiles_{i:03d}.npz"))
    np.savez(os.path.join(tmp, "x.npz"), **{f"k{K}": x for K, x in xs.items()})
    if f32:
        open(os.path.join(tmp, "f32"), "w").close()
    return counter_passes(tmp, ["--pmc-child-tiles", tmp], F32_TILE_KERNELS if f32 else PREFILL_KERNELS, launches=5)


def bf16_bits(x):
    """fp32 array -> bf16 bits (uint16, round to nearest even), the input of a bf16 prefill call."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def traffic_passes(ps, x, kernel="k_gemv"):
    """HBM bytes per decode launch of one stream (`ps`, input `x`); see counter_passes."""
    import tempfile
    tmp = tempfile.mkdtemp(prefix="mtc_pmc_")
    path = os.path.join(tmp, "stream.npz")
    ps.save(path)
    np.savez(os.path.join(tmp, "stream_x.npz"), x=x)
    return counter_passes(tmp, ["--pmc-child", path], kernel)


def traffic_passes_batch(pss, xs, kernel="k_gemv_batch"):
    """HBM bytes per batched decode launch over the streams `pss` (`xs`: one input per K);
    see counter_passes."""
    import tempfile
    tmp = tempfile.mkdtemp(prefix="mtc_pmc_")
    for i, ps in enumerate(pss):
        ps.save(os.path.join(tmp, f"stream_{i:03d}.npz"))
    np.savez(os.path.join(tmp, "x.npz"), **{f"k{K}": x for K, x in xs.items()})
    return counter_passes(tmp, ["--pmc-child-batch", tmp], kernel, launches=4)


def counter_passes(tmp, child_args, kernel, launches=None):
    """HBM bytes per launch of `kernel` from two rocprofv3 --pmc passes (FETCH_SIZE, then
    WRITE_SIZE) over a child run of this script (`child_args`, inputs saved in `tmp`).
    With `launches`, the child's dispatches of `kernel` are summed and divided by that
    many launches (a batched launch may dispatch once per block shape); otherwise the
    mean over dispatches is taken.

    Each counter is scaled by what it reads for a device copy of COPY_BYTES in the
    same pass (bytes moved / counter bytes), so unit or per-instance conventions of
    the counter cancel. Runs before this process touches the GPU; returns None
    when rocprofv3 is unavailable or a pass fails."""
    import shutil
    exe = shutil.which("rocprofv3")
    if exe is None:
        log("traffic: rocprofv3 not found")
        shutil.rmtree(tmp, ignore_errors=True)
        return None
    try:
        return _counter_passes(exe, tmp, child_args, kernel, launches)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def _counter_passes(exe, tmp, child_args, kernel, launches):
    import subprocess
    from tensorpack_amd.profiling import dispatch_values
    res = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        cmd = ["timeout", "-s", "KILL", "120", exe, "--pmc", counter, "-d", tmp, "-o", counter, "--",
               sys.executable, os.path.abspath(__file__)] + child_args
        log("traffic pass: " + " ".join(cmd[3:]))
        r = subprocess.run(cmd, capture_output=True, text=True, env=dict(os.environ, TMPDIR="/tmp"))
        db = os.path.join(tmp, counter + "_results.db")
        if r.returncode != 0 or not os.path.exists(db):
            log(f"traffic pass {counter} failed (rc {r.returncode}): {r.stderr[-400:]}")
            return None
        kern = kernel_values(db, counter, kernel)
        # the four COPY_BYTES device copies are the largest copy dispatches of the pass
        # (host-to-device staging copies share the kernel name but are small)
        copy = sorted(dispatch_values(db, counter, "copyBuffer"))[-4:]
        if not kern or len(copy) < 4 or min(copy) <= 0:
            log(f"traffic pass {counter}: kernel or copy dispatches missing")
            return None
        copy_kib = sum(copy) / len(copy)
        res[counter] = {"kernel_kib": sum(kern) / (launches or len(kern)), "copy_kib": copy_kib,
                        "factor": COPY_BYTES / (copy_kib * 1024.0), "copy_spread": max(copy) / min(copy)}
    fetch = res["FETCH_SIZE"]["kernel_kib"] * 1024.0 * res["FETCH_SIZE"]["factor"]
    write = res["WRITE_SIZE"]["kernel_kib"] * 1024.0 * res["WRITE_SIZE"]["factor"]
    out = {"bytes": fetch + write, "fetch_bytes": fetch, "write_bytes": write,
           "fetch_factor": res["FETCH_SIZE"]["factor"], "write_factor": res["WRITE_SIZE"]["factor"]}
    issue = _issue_pass(exe, tmp, child_args, kernel, launches)
    if issue is not None:
        out["issue"] = issue
    waves = _issue_pass(exe, tmp, child_args, kernel, launches, WAVE_COUNTERS, "WAVES")
    if waves is not None:
        out["waves"] = waves
    return out


# Instruction-issue counters of one pass (SQ block: at most 8 per pass; GRBM: 2).
ISSUE_COUNTERS = ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD", "SQ_ACTIVE_INST_VALU",
                  "SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE")
# Wave-state counters of a second pass: waves, their cycles, cycles waiting on an instruction's
# operands, cycles issuing, MFMA instructions, LDS bank conflicts, instruction fetches.
WAVE_COUNTERS = ("SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_ANY",
                 "SQ_INSTS_MFMA", "SQ_LDS_BANK_CONFLICT", "SQ_IFETCH", "GRBM_GUI_ACTIVE")


def kernel_values(db, counter, kernel):
    """Per-dispatch values of `counter` for the kernels named by `kernel` (a substring, or a tuple
    of substrings whose dispatches are pooled)."""
    from tensorpack_amd.profiling import dispatch_values
    names = (kernel,) if isinstance(kernel, str) else tuple(kernel)
    return [v for k in names for v in dispatch_values(db, counter, k)]


def _issue_pass(exe, tmp, child_args, kernel, launches, counters=ISSUE_COUNTERS, name="ISSUE"):
    """Per-launch values of `counters` for `kernel` from one rocprofv3 --pmc pass over the same
    child run. ISSUE_COUNTERS: VALU / SALU / LDS / vector-memory-read wave-instructions, the
    waves' VALU issue cycles, SQ busy cycles, MFMA busy cycles and the GPU's active cycles."""
    import subprocess
    cmd = ["timeout", "-s", "KILL", "120", exe, "--pmc", *counters, "-d", tmp, "-o", name, "--",
           sys.executable, os.path.abspath(__file__)] + child_args
    log(f"{name.lower()} pass: " + " ".join(cmd[3:]))
    r = subprocess.run(cmd, capture_output=True, text=True, env=dict(os.environ, TMPDIR="/tmp"))
    db = os.path.join(tmp, f"{name}_results.db")
    if r.returncode != 0 or not os.path.exists(db):
        log(f"{name.lower()} pass failed (rc {r.returncode}): {r.stderr[-400:]}")
        return None
    out = {}
    for c in counters:
        v = kernel_values(db, c, kernel)
        if not v:
            log(f"{name.lower()} pass: no {c} values for {kernel}")
            return None
        out[c] = sum(v) / (launches or len(v))
    return out


def issue_ratios(traffic, weights):
    """Per-weight issue figures of a decode launch from its counter pass (`traffic["issue"]`):
    VALU lane-instructions per weight (64 lanes per wave-instruction; weights = K * N summed
    over the matrices, P0 leaves included) and the fraction of the SIMDs' VALU issue slots the
    launch used (a wave-instruction occupies a 16-lane SIMD for 4 cycles; 1024 SIMDs). The
    reader sums GRBM_GUI_ACTIVE over the 8 XCD instances, so the launch's cycles are an eighth."""
    if not traffic or "issue" not in traffic:
        return None
    c = traffic["issue"]
    gpu = (c.get("GRBM_GUI_ACTIVE") or 0.0) / 8.0
    return {"valu_lane_insts_per_weight": 64.0 * c["SQ_INSTS_VALU"] / weights,
            "salu_insts_per_weight_x64": 64.0 * c["SQ_INSTS_SALU"] / weights,
            "valu_issue_fraction": (4.0 * c["SQ_INSTS_VALU"] / (1024.0 * gpu)) if gpu else None,
            "mfma_busy_fraction": (c["SQ_VALU_MFMA_BUSY_CYCLES"] / (1024.0 * gpu)) if gpu else None,
            "gpu_cycles": gpu, "weights": weights,
            "wave_wait_fraction": (traffic["waves"]["SQ_WAIT_INST_ANY"] / traffic["waves"]["SQ_WAVE_CYCLES"])
            if traffic.get("waves") and traffic["waves"]["SQ_WAVE_CYCLES"] else None,
            "wave_issue_fraction": (traffic["waves"]["SQ_ACTIVE_INST_ANY"] / traffic["waves"]["SQ_WAVE_CYCLES"])
            if traffic.get("waves") and traffic["waves"]["SQ_WAVE_CYCLES"] else None}


def timed_calls(torch, launch_list, steps, warmup, use_graph):
    """Time exactly `steps` calls cycling over launch_list; returns (seconds, per-call ms). With a
    graph, timed_calls.last_median_ms is the median per-call ms over 10 segments of the replays
    (the last segment also holds the remainder calls)."""
    timed_calls.last_median_ms = None
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
        if gt is not None:
            gt.replay()              # a graph's first replay uploads it: keep that out of the timed region
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # one event per tenth of the replays as well, for the median of 10 segments; recording
        # an event between replays adds no work to the timed stream
        reps = steps // n
        marks = sorted({(reps * j) // 10 for j in range(1, 10)} - {0, reps})
        seg = [torch.cuda.Event(enable_timing=True) for _ in marks]
        start.record(stream)
        k = 0
        for r in range(reps):
            if k < len(marks) and r == marks[k]:
                seg[k].record(stream)
                k += 1
            g.replay()
        if gt is not None:
            gt.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        if len(marks) == 9:
            ev = [start] + seg + [stop]
            cuts = [0] + marks + [reps]
            calls = [(cuts[j + 1] - cuts[j]) * n + (tail if j == 9 else 0) for j in range(10)]
            per = sorted(ev[j].elapsed_time(ev[j + 1]) / calls[j] for j in range(10) if calls[j] > 0)
            timed_calls.last_median_ms = per[len(per) // 2]
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


def rotating(stream, n_bytes_target):
    """The stream plus clones of it totalling at least n_bytes_target device bytes, so that
    timed calls cycling over them read the weight from HBM, not from the 256 MB MALL."""
    n = max(1, int(np.ceil(n_bytes_target / stream.device_bytes())))
    return [stream] + [stream.clone() for _ in range(n - 1)]


def rel_frobenius(ref, got):
    ref = np.asarray(ref, np.float64)
    d = np.linalg.norm(ref - np.asarray(got, np.float64))
    n = np.linalg.norm(ref)
    return float(d if n < 1e-12 else d / n)


def cpu_port_gbs(las, xs, packed_bytes, seconds, what):
    """C/OpenMP port of the reference block loop (gemm.py:124-210) over the listed matrices,
    timed on this host for about `seconds`: packed-weight GB/s and the sample it ran."""
    from oracle import mtc_oracle as O
    for la, x in zip(las, xs):
        O.cpu_qt_gemm(x, la)
    passes, t0 = 0, time.time()
    while True:
        for la, x in zip(las, xs):
            O.cpu_qt_gemm(x, la)
        passes += 1
        if time.time() - t0 >= seconds and passes >= 3:
            break
    el = time.time() - t0
    return {"value": packed_bytes * passes / el / 1e9, "unit": "GB/s", "cores": int(O.cpu_lib().oracle_threads()),
            "kind": "port", "sample": f"{passes} passes of {what} in {el:.1f}s, C/OpenMP port of the reference "
                                      f"block loop (gemm.py:124-210)"}


def leaf_arena(alloc, W):
    """The oracle's leaf list of an allocation (CPU baseline input)."""
    from oracle import mtc_oracle as O
    if hasattr(alloc, "inner"):
        i = alloc.inner
        return O.LeafArena(i.weights, i.sizes, i.leaf, i.modes, i.scales, alloc.row_perm, alloc.col_perm)
    return O.LeafArena(W, alloc.sizes, alloc.leaf, alloc.modes, alloc.scales)


# ----------------------------------------------------------------------------------------------
# c2: the headline decode (M = 1), and M = 16
# ----------------------------------------------------------------------------------------------
def bench_c2(args, wl, alloc, traffic, dev, traffic16=None):
    import torch
    from tensorpack_amd.kernels.gemm import MTCMatrix
    m = MTCMatrix.from_quadtree(alloc, wl.W)
    t0 = time.time()
    ds = m.device_stream(None, dev, 1, M1_LAYOUT)
    log(f"c2 packed in {time.time() - t0:.1f}s: chunk_rows={ds.host.chunk_rows} stream {ds.device_bytes()} B, "
        f"accounted {m.packed_bytes:.0f} B")
    packed = m.packed_bytes
    copies = rotating(ds, args.rotate_gib * (1 << 30))
    X1 = torch.from_numpy(wl.activations(1)).to(dev)
    Y1 = torch.empty((1, wl.W.shape[1]), dtype=torch.float32, device=dev)
    for c in copies:
        c.workspace(1)
        c.gemv_f32(X1, out=Y1)
    torch.cuda.synchronize()
    secs, ms = timed_calls(torch, [lambda c=c: c.gemv_f32(X1, out=Y1) for c in copies], args.steps, args.warmup,
                           bool(args.graph))
    ms_median = timed_calls.last_median_ms
    gbs = packed / (ms * 1e-3) / 1e9
    log(f"c2 M=1: {ms * 1e3:.2f} us/call, {gbs:.1f} GB/s packed ({len(copies)} copies)")
    res = {"m": m, "ds": ds, "packed": packed, "ms": ms, "gbs": gbs, "n_copies": len(copies), "ms_median": ms_median,
           "y": Y1.cpu().numpy().copy(), "x": wl.activations(1)}
    del copies
    if not args.no_m16:
        d16 = m.device_stream(None, dev, 16)
        c16 = rotating(d16, args.rotate_gib * (1 << 30))
        X16 = torch.from_numpy(wl.activations(16)).to(dev)
        Y16 = torch.empty((16, wl.W.shape[1]), dtype=torch.float32, device=dev)
        for c in c16:
            c.workspace(16)
            c.gemv_f32(X16, out=Y16)
        torch.cuda.synchronize()
        s16, ms16 = timed_calls(torch, [lambda c=c: c.gemv_f32(X16, out=Y16) for c in c16],
                                max(args.steps // 4, len(c16)), args.warmup // 4, bool(args.graph))
        flop16 = 2.0 * 16 * wl.W.shape[0] * wl.W.shape[1]
        tf = flop16 / (ms16 * 1e-3) / 1e12
        # the timed output against the fp64 product with the allocator's W_hat
        rel16 = rel_frobenius(wl.activations(16).astype(np.float64) @ np.asarray(alloc.dequant, np.float64),
                              Y16.cpu().numpy())
        if not rel16 < 1e-5:
            raise SystemExit(f"c2 M=16 output differs from the fp64 product: rel {rel16:.3e} >= 1e-5")
        res["m16"] = {"us_per_call": ms16 * 1e3, "packed_GBps": packed / (ms16 * 1e-3) / 1e9, "TFLOPs": tf,
                      "frac_fp32_peak": tf / FP32_PEAK_TFLOPS, "chunk_rows": d16.host.chunk_rows,
                      "rel_frobenius_vs_fp64": rel16,
                      "roofline": {"bound": "mfma", "achieved": tf, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                                   "frac": tf / FP32_PEAK_TFLOPS,
                                   "traffic": None if traffic16 is None else traffic16["bytes"],
                                   "kernel": "k_gemv<16>"}}
        if traffic16 is not None:
            res["m16"]["roofline"]["traffic_detail"] = dict(traffic16, traffic_over_packed=traffic16["bytes"] / packed,
                                                            issue_ratios=issue_ratios(traffic16, wl.W.size))
            log(f"c2 M=16 traffic {traffic16['bytes'] / 1e6:.2f} MB per launch = {traffic16['bytes'] / packed:.3f}x packed")
        log(f"c2 M=16: {ms16 * 1e3:.2f} us/call, {tf:.2f} TFLOP/s; vs fp64 rel {rel16:.2e}")
        del c16
    return res


def device_copy_rates(dev, packed):
    """A plain 1 GiB device copy (achievable HBM bandwidth) and graph-replayed copies of the
    packed weight's size (what one launch of that size reaches on the copy path)."""
    import torch
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
    copy_gbs = 2 * src.numel() * 4 * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    n_el = int(packed) // 4
    n_rot = max(2, (1 << 30) // (2 * 4 * n_el))
    srcs = [torch.empty(n_el, dtype=torch.float32, device=dev) for _ in range(n_rot)]
    dsts = [torch.empty_like(s) for s in srcs]
    g = graph_of(torch, [lambda s=s, d=d: d.copy_(s) for s, d in zip(srcs, dsts)])
    small_us = time_replays(torch, g, 5) * 1e3 / n_rot
    log(f"device copy: {copy_gbs:.0f} GB/s (read + write); copy of {4 * n_el} B: {small_us:.2f} us")
    return copy_gbs, small_us


# ----------------------------------------------------------------------------------------------
# c4: prefill (bf16 MFMA), with its own output checked against a fp64 product
# ----------------------------------------------------------------------------------------------
def p0_area_fraction(a):
    """Fraction of the matrix's weights in P0 leaves (flop counts are dense-equivalent: the
    kernels skip those leaves' work, the metric does not subtract it)."""
    q = getattr(a, "inner", a)
    area = sum(float(((q.leaf[s] & (q.modes[s] == 0))).sum()) * s * s for s in q.sizes)
    return area / float(q.shape[0] * q.shape[1])


def bench_c4(args, wl4, a4, dev, m4=None, traffic=None):
    """c4 prefill at M = 4096; `m4`: the MTCMatrix, if already built; `traffic`: counter bytes of
    one call (traffic_passes_tiles)."""
    import torch
    from tensorpack_amd.kernels.gemm import MTCMatrix
    if m4 is None:
        m4 = MTCMatrix.from_quadtree(a4, wl4.W)
    g4 = m4.device_tiles(dev)
    M4 = 4096
    X4 = torch.from_numpy(wl4.activations(M4)).to(dev).to(torch.bfloat16)
    Y4 = torch.empty((M4, wl4.W.shape[1]), dtype=torch.float32, device=dev)
    from tensorpack_amd.device import set_prefill_decode_once
    # the library's own choice at this shape: W_hat decoded once into bf16, then hipBLASLt's GEMM
    g4.gemm_bf16(X4, out=Y4)
    torch.cuda.synchronize()
    s4, ms4 = timed_calls(torch, [lambda: g4.gemm_bf16(X4, out=Y4)], args.prefill_steps, args.prefill_warmup, False)
    flop4 = 2.0 * M4 * wl4.W.shape[0] * wl4.W.shape[1]
    tf = flop4 / (ms4 * 1e-3) / 1e12
    # the fused tile kernel (k_gemm_tile) on the same call, the path switched off
    Y4t = torch.empty_like(Y4)
    prev = set_prefill_decode_once(False)
    try:
        g4.gemm_bf16(X4, out=Y4t)
        torch.cuda.synchronize()
        _, ms4t = timed_calls(torch, [lambda: g4.gemm_bf16(X4, out=Y4t)], args.prefill_steps, args.prefill_warmup, False)
    finally:
        set_prefill_decode_once(prev)
    tf_t = flop4 / (ms4t * 1e-3) / 1e12
    rel_t = rel_frobenius(Y4t.cpu().numpy().astype(np.float64), Y4.cpu().numpy())
    del Y4t
    log(f"c4 M=4096 on the fused tile kernel: {ms4t:.3f} ms/call, {tf_t:.1f} TFLOP/s "
        f"({100 * tf_t / BF16_PEAK_TFLOPS:.1f}%); decode-once vs tile kernel rel {rel_t:.2e}")
    # the timed output: 4 rows of every 256-row tile, all 8192 columns (every column tile), against
    # the fp64 product of the same bf16 X and the allocator's W_hat
    rng = np.random.RandomState(4242)
    rows = np.concatenate([rt * 256 + np.r_[0, 255, rng.choice(np.arange(1, 255), 2, replace=False)]
                           for rt in range((M4 + 255) // 256)])
    idx = torch.from_numpy(rows).to(dev)
    Xs = X4[idx].float().cpu().numpy().astype(np.float64)
    ref = Xs @ np.asarray(a4.dequant, np.float64)
    rel = rel_frobenius(ref, Y4[idx].cpu().numpy())
    log(f"c4 M=4096: {ms4:.3f} ms/call, {tf:.1f} TFLOP/s ({100 * tf / BF16_PEAK_TFLOPS:.1f}% of bf16 peak); "
        f"{rows.size} sampled rows vs fp64: rel {rel:.2e}")
    if not rel < 2e-3:
        raise SystemExit(f"c4 prefill output differs from the fp64 product: rel {rel:.3e} >= 2e-3")
    res = {"M": M4, "ms_per_call": ms4, "TFLOPs": tf, "frac_bf16_peak": tf / BF16_PEAK_TFLOPS,
           "path": "decode once (k_tile_dequant_bf16) + hipBLASLt bf16 GEMM",
           "tile_kernel": {"ms_per_call": ms4t, "TFLOPs": tf_t, "frac_bf16_peak": tf_t / BF16_PEAK_TFLOPS,
                           "rel_frobenius_vs_decode_once": rel_t},
           "packed_bytes": m4.packed_bytes, "p0_area_fraction": p0_area_fraction(a4),
           "roofline": {"bound": "mfma", "achieved": tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": tf / BF16_PEAK_TFLOPS, "traffic": None if traffic is None else traffic["bytes"],
                        "kernel": "k_tile_dequant_bf16 + hipBLASLt GEMM (whole call)"},
           "parity": {"rows": int(rows.size), "rel_frobenius_vs_fp64": rel, "tolerance": 2e-3}}
    if traffic is not None:
        res["roofline"]["traffic_detail"] = prefill_traffic_detail(traffic, M4, wl4.W.shape, m4.packed_bytes, 2)
    return res


def prefill_traffic_detail(traffic, M, shape, packed, x_bytes):
    """The counter bytes of one prefill call beside its algorithmic bytes: the packed weight,
    X read once (x_bytes per element) and fp32 Y written once."""
    K, N = shape
    alg = packed + M * K * x_bytes + 4.0 * M * N
    return dict(traffic, algorithmic_bytes=alg, traffic_over_algorithmic=traffic["bytes"] / alg)


# ----------------------------------------------------------------------------------------------
# c3: the 168-matrix Qwen2.5-0.5B-shaped stack
# ----------------------------------------------------------------------------------------------
def c3_x(K, M):
    """The c3 input of K columns and M rows (every matrix of that K shares it)."""
    return np.random.RandomState(3000 + K + M).randn(M, K).astype(np.float32)


def bench_c3(args, mats, allocs, dev, detail=False, ms_=None, traffic=None, traffic512=None):
    """M = 1: all 168 matrices (each its own X and Y) in one batched launch per pass, over rotating
    copies of the stack; M = 512: the prefill of every matrix, the q/k/v and gate/up groups sharing
    their input (12 launches per layer), one HIP graph per pass. With `detail`, also the M = 1 pass
    as one launch per matrix and as 96 grouped launches. `ms_`: the MTCMatrix of each allocation,
    if already built; `traffic`: counter bytes of one batched M = 1 launch (traffic_passes_batch)."""
    import torch
    from tensorpack_amd import workloads
    from tensorpack_amd.device import GemvBatch, gemm_bf16_group, gemv_f32_group
    from tensorpack_amd.kernels.gemm import MTCMatrix
    if ms_ is None:
        ms_ = [MTCMatrix.from_quadtree(a, w.W) for a, w in zip(allocs, mats)]
    packed = float(sum(m.packed_bytes for m in ms_))
    weights = sum(w.W.size for w in mats)
    xs = {}

    def x_of(K, M, dtype):
        key = (K, M, dtype)
        if key not in xs:
            xs[key] = torch.from_numpy(c3_x(K, M)).to(dev).to(dtype)
        return xs[key]

    streams = [m.device_stream(None, dev, 1, M1_LAYOUT) for m in ms_]
    stack_bytes = sum(s_.device_bytes() for s_ in streams)
    n_rot = max(1, int(np.ceil(args.rotate_gib * (1 << 30) / stack_bytes)))
    sets = [streams] + [[s_.clone() for s_ in streams] for _ in range(n_rot - 1)]
    ys1 = [torch.empty((1, w.W.shape[1]), dtype=torch.float32, device=dev) for w in mats]
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
    gbs = packed / (ms1 * 1e-3) / 1e9
    ref = [s_.gemv_f32(x_of(w.W.shape[0], 1, torch.float32)) for s_, w in zip(sets[-1], mats)]
    torch.cuda.synchronize()
    identical = all(torch.equal(a_, b_) for a_, b_ in zip(ref, ys1))
    log(f"c3 M=1, one batched launch per pass: {ms1 * 1e3:.1f} us, {gbs:.1f} GB/s packed "
        f"({n_rot} rotating stacks); outputs bit-identical to single calls: {identical}")
    if not identical:
        raise SystemExit("c3 batched decode differs from the single-matrix calls")
    out = {"workload": f"c3 Qwen2.5-0.5B-shaped stack, {len(mats) // 7} layers x 7 matrices, QT-P @ 3.125",
           "matrices": len(mats), "weights": weights, "packed_bytes": packed, "rotating_stacks": n_rot,
           "m1": {"us_per_pass": ms1 * 1e3, "GBps_packed": gbs, "launches": 1, "bit_identical_to_single_calls": True,
                  "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                               "frac": gbs / HBM_PEAK_GBS, "traffic": None if traffic is None else traffic["bytes"],
                               "kernel": "k_gemv_batch"}}}
    if traffic is not None:
        out["m1"]["roofline"]["traffic_detail"] = dict(traffic, traffic_over_packed=traffic["bytes"] / packed,
                                                       issue_ratios=issue_ratios(traffic, weights))
        log(f"c3 M=1 traffic {traffic['bytes'] / 1e6:.2f} MB per launch = {traffic['bytes'] / packed:.3f}x packed")
    n_per = len(workloads.QWEN_LAYER)
    layer_groups = [[0, 1, 2], [3], [4, 5], [6]]
    plan_grouped = [[L * n_per + i for i in grp] for L in range(len(mats) // n_per) for grp in layer_groups]
    if detail:
        def time_m1(plan):
            def calls(ss):
                fns = []
                for grp in plan:
                    if len(grp) == 1:
                        i = grp[0]
                        fns.append(lambda s_=ss[i], w=mats[i], y=ys1[i]: s_.gemv_f32(x_of(w.W.shape[0], 1, torch.float32), out=y))
                    else:
                        fns.append(lambda g=[ss[i] for i in grp], K=mats[grp[0]].W.shape[0], ys=[ys1[i] for i in grp]:
                                   gemv_f32_group(g, x_of(K, 1, torch.float32), ys))
                return fns
            for ss in sets:
                for s_ in ss:
                    s_.workspace(1)
            graphs = [graph_of(torch, calls(ss)) for ss in sets]
            for g in graphs:
                g.replay()
            torch.cuda.synchronize()
            r = max(2, 40 // len(graphs))
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(r):
                for g in graphs:
                    g.replay()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / (r * len(graphs))
        out["m1"]["us_per_pass_one_launch_per_matrix"] = time_m1([[i] for i in range(len(mats))]) * 1e3
        out["m1"]["us_per_pass_grouped_96_launches"] = time_m1(plan_grouped) * 1e3
        log(f"c3 M=1: one launch per matrix {out['m1']['us_per_pass_one_launch_per_matrix']:.1f} us, "
            f"96 grouped launches {out['m1']['us_per_pass_grouped_96_launches']:.1f} us")
    del sets, batches
    # M = 512 prefill
    M = 512
    tiles = [m.device_tiles(dev) for m in ms_]
    ysp = [torch.empty((M, w.W.shape[1]), dtype=torch.float32, device=dev) for w in mats]
    flop = 2.0 * M * weights
    if detail:
        fns = []
        for grp in plan_grouped:
            K = mats[grp[0]].W.shape[0]
            if len(grp) == 1:
                fns.append(lambda t=tiles[grp[0]], K=K, y=ysp[grp[0]]: t.gemm_bf16(x_of(K, M, torch.bfloat16), out=y))
            else:
                fns.append(lambda ts=[tiles[i] for i in grp], K=K, ys=[ysp[i] for i in grp]:
                           gemm_bf16_group(ts, x_of(K, M, torch.bfloat16), ys))
        for f in fns:
            f()
        torch.cuda.synchronize()
        ms_grouped = time_replays(torch, graph_of(torch, fns), 5)
        log(f"c3 M=512, {len(fns)} grouped launches per pass: {ms_grouped:.3f} ms")
    # the whole pass as one batched prefill: an X-staging, a tile and a split-K reduction launch
    from tensorpack_amd.device import GemmBatch
    pb = GemmBatch(tiles, [x_of(w.W.shape[0], M, torch.bfloat16) for w in mats], ysp)
    pb.launch()
    torch.cuda.synchronize()
    msp = time_replays(torch, graph_of(torch, [pb.launch]), 10)
    tf = flop / (msp * 1e-3) / 1e12
    # parity of the prefill pass: layer 0's matrices against the fp64 product with the allocator's W_hat
    worst = 0.0
    for i in range(n_per):
        Xb = x_of(mats[i].W.shape[0], M, torch.bfloat16).float().cpu().numpy().astype(np.float64)
        worst = max(worst, rel_frobenius(Xb @ np.asarray(allocs[i].dequant, np.float64), ysp[i].cpu().numpy()))
    log(f"c3 M=512, one batched prefill per pass: {msp:.3f} ms, {tf:.1f} TFLOP/s; layer 0 vs fp64: rel {worst:.2e}")
    if not worst < 2e-3:
        raise SystemExit(f"c3 prefill output differs from the fp64 product: rel {worst:.3e} >= 2e-3")
    out["m512"] = {"ms_per_pass": msp, "TFLOPs": tf, "launches": pb.launches, "rel_frobenius_layer0_vs_fp64": worst,
                   "roofline": {"bound": "mfma", "achieved": tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                "frac": tf / BF16_PEAK_TFLOPS,
                                "traffic": None if traffic512 is None else traffic512["bytes"],
                                "kernel": "k_gemm_tile_batch"}}
    if traffic512 is not None:
        alg = packed + sum(M * w.W.shape[0] * 2 + 4.0 * M * w.W.shape[1] for w in mats)
        out["m512"]["roofline"]["traffic_detail"] = dict(traffic512, algorithmic_bytes=alg,
                                                         traffic_over_algorithmic=traffic512["bytes"] / alg)
    if detail:
        out["m512"]["ms_per_pass_grouped_launches"] = ms_grouped
    return out


def cpu_baseline_c3(args, mats, allocs):
    """Bounded CPU sample of c3 at M=1: layer 0's seven matrices (the port's per-matrix cost scales
    with the weights; every layer has the same shapes)."""
    n_per = 7
    las = [leaf_arena(allocs[i], mats[i].W) for i in range(n_per)]
    xs = [np.random.RandomState(3000 + w.W.shape[0] + 1).randn(1, w.W.shape[0]).astype(np.float32)
          for w in mats[:n_per]]
    packed = float(sum(a.total_bits / 8.0 for a in allocs[:n_per]))
    return cpu_port_gbs(las, xs, packed, args.cpu_seconds, "layer 0 of c3 (q, k, v, o, gate, up, down) at M=1")


# ----------------------------------------------------------------------------------------------
# c5: the adversarial leaf mix
# ----------------------------------------------------------------------------------------------
def bench_c5(args, wl, a, dev, traffic=None, traffic256=None):
    """c5 at M = 1 (decode over rotating copies) and M = 256 (prefill). `traffic`: counter bytes
    of one M = 1 launch (traffic_passes), if measured."""
    import torch
    from tensorpack_amd.kernels.gemm import MTCMatrix
    m = MTCMatrix.from_quadtree(a, wl.W)
    ds = m.device_stream(None, dev, 1, M1_LAYOUT)
    copies = rotating(ds, args.rotate_gib * (1 << 30))
    X1 = torch.from_numpy(wl.activations(1)).to(dev)
    Y1 = torch.empty((1, wl.W.shape[1]), dtype=torch.float32, device=dev)
    for c in copies:
        c.workspace(1)
        c.gemv_f32(X1, out=Y1)
    torch.cuda.synchronize()
    s1, ms = timed_calls(torch, [lambda c=c: c.gemv_f32(X1, out=Y1) for c in copies], max(args.steps // 2, len(copies)),
                         args.warmup // 2, bool(args.graph))
    gbs = m.packed_bytes / (ms * 1e-3) / 1e9
    rel1 = rel_frobenius(wl.activations(1).astype(np.float64) @ np.asarray(a.dequant, np.float64), Y1.cpu().numpy())
    log(f"c5 M=1: {ms * 1e3:.2f} us/call, {gbs:.1f} GB/s packed; vs fp64 rel {rel1:.2e}")
    if not rel1 < 1e-5:
        raise SystemExit(f"c5 decode output differs from the fp64 product: rel {rel1:.3e}")
    M = 256
    t = m.device_tiles(dev)
    X = torch.from_numpy(wl.activations(M)).to(dev)
    Y = torch.empty((M, wl.W.shape[1]), dtype=torch.float32, device=dev)
    t.gemm_bf16(X, out=Y)
    torch.cuda.synchronize()
    # ten calls per graph, as a serving loop would issue them back to back: a one-call graph
    # replayed 50 times adds a graph launch (about 7 us) to every 32 us call
    s2, ms2 = timed_calls(torch, [lambda: t.gemm_bf16(X, out=Y)] * 10, 50, 5, bool(args.graph))
    tf = 2.0 * M * wl.W.size / (ms2 * 1e-3) / 1e12
    Xb = X.to(torch.bfloat16).float().cpu().numpy().astype(np.float64)
    rel2 = rel_frobenius(Xb @ np.asarray(a.dequant, np.float64), Y.cpu().numpy())
    log(f"c5 M=256: {ms2 * 1e3:.1f} us/call, {tf:.1f} TFLOP/s; vs fp64 rel {rel2:.2e}")
    if not rel2 < 2e-3:
        raise SystemExit(f"c5 prefill output differs from the fp64 product: rel {rel2:.3e}")
    m1 = {"us_per_call": ms * 1e3, "GBps_packed": gbs, "rotating_copies": len(copies), "rel_vs_fp64": rel1,
          "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": gbs / HBM_PEAK_GBS, "traffic": None if traffic is None else traffic["bytes"],
                       "kernel": "k_gemv<1>"}}
    if traffic is not None:
        m1["roofline"]["traffic_detail"] = dict(traffic, traffic_over_packed=traffic["bytes"] / m.packed_bytes,
                                                issue_ratios=issue_ratios(traffic, wl.W.size))
        log(f"c5 M=1 traffic {traffic['bytes'] / 1e6:.2f} MB per launch = {traffic['bytes'] / m.packed_bytes:.3f}x packed")
    return {"workload": wl.name, "packed_bytes": m.packed_bytes, "stream_bytes": ds.device_bytes(),
            "m1": m1,
            "m256": {"us_per_call": ms2 * 1e3, "TFLOPs": tf, "x_dtype": "f32 (rounded to bf16 by the tile kernel's consumers)",
                     "rel_vs_fp64": rel2,
                     "roofline": {"bound": "mfma", "achieved": tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                  "frac": tf / BF16_PEAK_TFLOPS,
                                  "traffic": None if traffic256 is None else traffic256["bytes"],
                                  "traffic_detail": None if traffic256 is None else
                                  prefill_traffic_detail(traffic256, M, wl.W.shape, m.packed_bytes, 4)}}}


# ----------------------------------------------------------------------------------------------
def main():
    args = parse()
    if args.pmc_child:
        pmc_child(args.pmc_child)
        return
    if args.pmc_child_batch:
        pmc_child_batch(args.pmc_child_batch)
        return
    if args.pmc_child_tiles:
        pmc_child_tiles(args.pmc_child_tiles)
        return
    global M1_LAYOUT
    if args.m1_layout != "auto":
        from tensorpack_amd.packer import LAYOUT_MX, LAYOUT_V1
        M1_LAYOUT = {"v1": LAYOUT_V1, "mx": LAYOUT_MX}[args.m1_layout]
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the library has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    from tensorpack_amd import workloads
    from tensorpack_amd.kernels.gemm import MTCMatrix
    want = {"all": ("c2", "c4", "c3", "c5"), "c2": ("c2", "c4"), "c3": ("c3",), "c5": ("c5",)}[args.workload]
    want = tuple(w for w in want if not (w == "c4" and args.no_prefill) and not (w == "c3" and args.no_c3)
                 and not (w == "c5" and args.no_c5))

    # ---- CPU phase: everything before this process initialises the GPU (the c3 pool forks) ----
    A = {}
    if "c3" in want:
        mats = workloads.c3_matrices(args.c3_layers)
        t0 = time.time()
        A["c3"] = (mats, workloads.allocate_many(mats))
        log(f"c3: {len(mats)} allocations in {time.time() - t0:.1f}s")
    for name in ("c2", "c4", "c5"):
        if name in want:
            wl = workloads.CONFIGS[name]()
            t0 = time.time()
            A[name] = (wl, wl.allocate())
            log(f"{name} allocation {time.time() - t0:.1f}s, {A[name][1].bits_per_element:.4f} b/w")
    c3_ms, c3_traffic, c3_traffic512 = None, None, None
    if "c3" in want:
        mats, allocs = A["c3"]
        c3_ms = [MTCMatrix.from_quadtree(a, w.W) for a, w in zip(allocs, mats)]
        if not args.no_traffic:
            c3_traffic = traffic_passes_batch([m.panel_stream(m.decode_chunk_rows(1), m1_layout(m)) for m in c3_ms],
                                              {w.W.shape[0]: c3_x(w.W.shape[0], 1) for w in mats})
            c3_traffic512 = traffic_passes_tiles([m.tile_stream() for m in c3_ms],
                                                 {w.W.shape[0]: bf16_bits(c3_x(w.W.shape[0], 512)) for w in mats})
    m4, traffic4 = None, None
    if "c4" in want:
        wl4, a4 = A["c4"]
        m4 = MTCMatrix.from_quadtree(a4, wl4.W)
        if not args.no_traffic:
            traffic4 = traffic_passes_tiles([m4.tile_stream()], {wl4.W.shape[0]: bf16_bits(wl4.activations(4096))})
    traffic, traffic16, traffic5 = None, None, None
    if "c2" in want and not args.no_traffic:
        wl, alloc = A["c2"]
        m = MTCMatrix.from_quadtree(alloc, wl.W)
        traffic = traffic_passes(m.panel_stream(m.decode_chunk_rows(1), m1_layout(m)), wl.activations(1))
        if not args.no_m16:
            traffic16 = traffic_passes(m.panel_stream(m.decode_chunk_rows(16), m.decode_layout(16)), wl.activations(16),
                                       kernel="k_gemv<16")
    traffic5_256 = None
    if "c5" in want and not args.no_traffic:
        wl5, a5 = A["c5"]
        m5 = MTCMatrix.from_quadtree(a5, wl5.W)
        traffic5 = traffic_passes(m5.panel_stream(m5.decode_chunk_rows(1), m1_layout(m5)), wl5.activations(1))
        traffic5_256 = traffic_passes_tiles([m5.tile_stream()], {wl5.W.shape[0]: wl5.activations(256)})

    import torch
    from tensorpack_amd.device import require_gpu
    dev = require_gpu()
    torch.cuda.set_device(dev)
    if "c2" not in want:                                  # a single detail workload
        if "c3" in want:
            r = bench_c3(args, *A["c3"], dev, detail=True, ms_=c3_ms, traffic=c3_traffic, traffic512=c3_traffic512)
            if not args.no_cpu_baseline:
                r["cpu_baseline"] = cpu_baseline_c3(args, *A["c3"])
        else:
            r = bench_c5(args, *A["c5"], dev, traffic=traffic5, traffic256=traffic5_256)
            if not args.no_cpu_baseline:
                wl, a = A["c5"]
                r["cpu_baseline"] = cpu_port_gbs([leaf_arena(a, wl.W)], [wl.activations(1)], a.total_bits / 8.0,
                                                 args.cpu_seconds, "c5 M=1 (full 4096x4096 matrix)")
        print(json.dumps(r), flush=True)
        return

    extra = {}
    wl, alloc = A["c2"]
    c2 = bench_c2(args, wl, alloc, traffic, dev, traffic16=traffic16)
    if "m16" in c2:
        extra["c2_m16"] = c2.pop("m16")
    copy_gbs, copy_small_us = device_copy_rates(dev, c2["packed"])
    if "c4" in want:
        extra["c4_prefill"] = bench_c4(args, *A["c4"], dev, m4=m4, traffic=traffic4)
    if "c3" in want:
        extra["c3"] = bench_c3(args, *A["c3"], dev, ms_=c3_ms, traffic=c3_traffic, traffic512=c3_traffic512)
    if "c5" in want:
        extra["c5"] = bench_c5(args, *A["c5"], dev, traffic=traffic5, traffic256=traffic5_256)

    # ---- CPU baselines (bounded samples on this host's cores) ----
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import mtc_oracle as O
        la = leaf_arena(alloc, wl.W)
        cpu = cpu_port_gbs([la], [c2["x"]], c2["packed"], args.cpu_seconds, "c2 M=1 (full 4096x4096 matrix)")
        cpu["gpu_vs_cpu_rel_frobenius"] = O.relative_frobenius_error(O.cpu_qt_gemm(c2["x"], la), c2["y"])
        log(f"cpu baseline c2 {cpu['value']:.3f} GB/s on {cpu['cores']} threads; gpu-vs-cpu rel "
            f"{cpu['gpu_vs_cpu_rel_frobenius']:.2e}")
        # the reference's own inference path: X @ the cached dequantized weight (LinearMTCAdaptive.forward,
        # mtc/nn/layers.py:150-151), numpy BLAS over a dense fp32 W_hat
        w_hat = np.ascontiguousarray(alloc.dequant, dtype=np.float32)
        x = c2["x"]
        x @ w_hat
        n_np, t0 = 0, time.time()
        while time.time() - t0 < 2.0 or n_np < 3:
            x @ w_hat
            n_np += 1
        el_np = time.time() - t0
        cpu["numpy_dequant_matmul"] = {"ms_per_call": 1e3 * el_np / n_np, "packed_GBps": c2["packed"] * n_np / el_np / 1e9,
                                       "dense_fp32_GBps": w_hat.nbytes * n_np / el_np / 1e9,
                                       "sample": f"{n_np} calls of x (1 x 4096) @ W_hat (4096 x 4096 fp32) in {el_np:.1f}s"}
        del w_hat
        if "c3" in extra:
            extra["c3"]["cpu_baseline"] = cpu_baseline_c3(args, *A["c3"])
            log(f"cpu baseline c3 {extra['c3']['cpu_baseline']['value']:.3f} GB/s")
        if "c5" in extra:
            wl5, a5 = A["c5"]
            extra["c5"]["cpu_baseline"] = cpu_port_gbs([leaf_arena(a5, wl5.W)], [wl5.activations(1)],
                                                       a5.total_bits / 8.0, args.cpu_seconds,
                                                       "c5 M=1 (full 4096x4096 matrix)")
            log(f"cpu baseline c5 {extra['c5']['cpu_baseline']['value']:.3f} GB/s")

    K, N = wl.W.shape
    ms, gbs, ds = c2["ms"], c2["gbs"], c2["ds"]
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
                   "bits_per_weight": alloc.bits_per_element, "packed_bytes": c2["packed"],
                   "stream_bytes": ds.device_bytes(), "rotating_copies": c2["n_copies"],
                   "algorithmic_bytes": c2["packed"] + 4.0 * (K + N),
                   "chunk_rows": ds.host.chunk_rows, "graph_replay": bool(args.graph)},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None if traffic is None else traffic["bytes"],
                     "copy_GBps": copy_gbs, "frac_of_copy": gbs / copy_gbs,
                     "copy_same_bytes_us": copy_small_us, "us_per_call": ms * 1e3,
                     "us_per_call_median_of_10": None if c2["ms_median"] is None else c2["ms_median"] * 1e3,
                     "kernel": "k_gemv<1>", "stream_GBps": ds.device_bytes() / (ms * 1e-3) / 1e9,
                     "algorithmic_GBps": (c2["packed"] + 4.0 * (K + N)) / (ms * 1e-3) / 1e9,
                     "traffic_detail": None if traffic is None else
                     dict(traffic, issue_ratios=issue_ratios(traffic, K * N))},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
