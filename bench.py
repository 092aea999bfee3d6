"""MatMulNBits 4-bit benchmark on one MI355X.

Headline workload ("c2"): the Llama-3-8B gate/up
decode projection, MatMulNBits M=1 K=4096 N=14336 bits=4 block_size=128 with
packed zero points. One step streams ROT distinct weight copies (>= 1 GiB in
total, so the 256 MB Infinity Cache cannot hold them) through one mnb_run
launch each; the launches of a step are captured once in a HIP graph and the
graph is replayed K times. value = algorithmic bytes of the timed launches /
their event-timed duration (GB/s), inputs resident in HBM.

Also reported on the same line: the prefill GEMM (configs[3], M=2048
K=N=4096 bs=128 symmetric) in TFLOP/s against the fp16 dense MFMA peak, the
other decode shapes, the c5 32-layer stack, and the CPU baseline on this
host's cores over the same c2 inputs: the C oracle's fused int4 GEMV
(``kind: port``, the value) at T threads and at 1, and the reference's own
MatMulPlan<float> (built from its sources into oracle/_ref) over the weights
dequantized to fp32, at T threads and at 1.

Algorithmic bytes per launch = N*nb*bs/2 (packed B) + 4*N*nb (scales) +
N*ceil(nb/2) (zero points) + 4*M*K (A) + 4*M*N (Y); FLOPs = 2*M*N*K.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import platform
import statistics
import subprocess
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
METRIC = "MatMulNBits 4-bit: M=1 achieved HBM GB/s; M=2048 TFLOP/s; % roofline"
ROTATION_BYTES = 1 << 30

# HBM bytes per launch of the headline kernel (GemvFragKernel on c2 M=1),
# from two rocprofv3 --pmc passes over `bench.py --only decode,gemm,sweep,copy,lm_head
# --eager --steps 3 --warmup 1 --cpu-seconds 0`: FETCH_SIZE 15584.6 KiB and
# WRITE_SIZE 56.0 KiB per dispatch, each scaled by what the same counter reads
# for the copy leg's 512 MiB device copy (FETCH_SIZE 262155.5 KiB -> x1.99992,
# WRITE_SIZE 524288.0 KiB -> x1.00000). Re-measure when the kernel changes.
GEMV_M1_C2_TRAFFIC_BYTES = round((15584.6 * (524288.0 / 262155.5) + 56.0) * 1024)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="CPU baseline sampling budget over its four modes (0 disables)")
    ap.add_argument("--only", default="",
                    help="comma list of legs: decode,ceiling,gemm,sweep,lm_head,c5,gate_up,rmsnorm,"
                         "plan,cpu,copy,gemm_shapes (default: all but copy and gemm_shapes)")
    ap.add_argument("--eager", action="store_true",
                    help="launch every step directly instead of replaying a HIP graph "
                         "(for counter collection, which serialises dispatches)")
    return ap.parse_args()


def make_device_weights(torch, p, copies, seed, dev):
    """`copies` independent random weight sets for projection p, generated on device."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    sets = []
    for _ in range(copies):
        B = torch.randint(0, 256, (p.N, p.nb, p.block_size // 2), dtype=torch.uint8,
                          device=dev, generator=g)
        S = (torch.rand((p.N, p.nb), device=dev, generator=g) * (p.scale_hi - p.scale_lo)
             + p.scale_lo).to(torch.float32)
        Z = (torch.randint(0, 256, (p.N, p.zp_row_bytes), dtype=torch.uint8, device=dev,
                           generator=g) if p.has_zero_points else None)
        sets.append((B, S, Z))
    return sets


EAGER = False
SETTLE_S = 0.2


def time_graph(torch, launches, steps, warmup, stream):
    """Captures `launches` (a callable issuing one step) into a graph, replays it
    (or, with --eager, calls it directly). Returns (ms per step from the events
    bracketing all steps on `stream`, wall seconds of the timed region, median
    and interquartile range of the per-step ms from an event before every
    step)."""
    with torch.cuda.stream(stream):
        launches()  # eager warmup outside capture; allocates any workspace
    torch.cuda.synchronize()
    if EAGER:
        def step():
            with torch.cuda.stream(stream):
                launches()
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            launches()
        step = graph.replay
    # graph.replay() launches on the current stream: keep `stream` current so
    # the events bracket the replays. Before the warmup steps, SETTLE_S of
    # untimed replays let the GPU leave its idle clocks (a timed region that
    # starts from idle measured the prefill GEMM 8% slower than steady state).
    with torch.cuda.stream(stream):
        t_settle = time.perf_counter() + SETTLE_S
        while time.perf_counter() < t_settle:
            for _ in range(4):
                step()
            torch.cuda.synchronize()
        for _ in range(warmup):
            step()
    torch.cuda.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for i in range(steps):
            marks[i].record(stream)
            step()
        marks[steps].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [marks[i].elapsed_time(marks[i + 1]) for i in range(steps)]
    q = statistics.quantiles(per, n=4) if steps >= 2 else [per[0], per[0], per[0]]
    SAMPLES.append(per)
    return marks[0].elapsed_time(marks[steps]) / steps, wall, statistics.median(per), q[2] - q[0]


# Per-step ms of every time_graph call, in call order: each leg takes the
# samples of its own timed region from here (last_samples) into its record.
SAMPLES = []


def last_samples(per_step_divisor=1.0):
    """The raw per-step samples of the last timed region, in us per launch."""
    return [round(v * 1e3 / per_step_divisor, 4) for v in SAMPLES[-1]]


def copy_leg(torch, dev, steps, warmup, stream):
    """A plain device-to-device copy of 512 MiB: the calibration that HBM
    counters (FETCH_SIZE, WRITE_SIZE) are scaled by, and a streaming ceiling."""
    n = 512 << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)

    def launches():
        dst.copy_(src)

    ms, wall, med, iqr = time_graph(torch, launches, steps, warmup, stream)
    return {"bytes_read": n, "bytes_written": n, "us_per_launch": ms * 1e3,
            "GBps": 2 * n / (ms * 1e-3) / 1e9, "wall_s": wall}


def stream_ceiling_leg(torch, pkg, dev, nbytes, steps, warmup, stream, grid=None):
    """The HBM read ceiling for one launch of nbytes: mnb_stream_read (loads
    only, 8 KiB contiguous records per wavefront) over as many rotated
    buffers as the headline leg, one launch each, graph-replayed. With grid =
    (workgroups, threads): mnb_stream_read_grid, the same reads on that grid
    (one contiguous share per wavefront)."""
    import ctypes
    rot = max(2, -(-ROTATION_BYTES // nbytes))
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(i & 0xFF) for i in range(rot)]
    words = 2048 if grid is None else grid[0] * grid[1] // 64  # one per wavefront
    out = torch.empty(words, dtype=torch.int32, device=dev)
    L = pkg.library()

    def launches():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for b in bufs:
            if grid is None:
                rc = L.mnb_stream_read(ctypes.c_void_p(b.data_ptr()), nbytes,
                                       ctypes.c_void_p(out.data_ptr()), out.numel(), st)
            else:
                rc = L.mnb_stream_read_grid(ctypes.c_void_p(b.data_ptr()), nbytes,
                                            ctypes.c_void_p(out.data_ptr()), out.numel(),
                                            grid[0], grid[1], st)
            if rc != 0:
                raise RuntimeError(f"mnb_stream_read: status {rc}")

    ms, _, med, _ = time_graph(torch, launches, steps, warmup, stream)
    us = ms * 1e3 / rot
    del bufs
    torch.cuda.empty_cache()
    kernel = ("StreamReadKernel (mnb_stream_read)" if grid is None else
              f"StreamChunkKernel (mnb_stream_read_grid, {grid[0]} x {grid[1]} threads)")
    return {"kernel": kernel, "bytes_per_launch": nbytes,
            "rotation_copies": rot, "us_per_launch": us, "us_per_launch_median": med * 1e3 / rot,
            "us_per_launch_samples": last_samples(rot), "GBps": nbytes / (us * 1e-6) / 1e9,
            "frac_of_peak": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def launch_floor_leg(torch, pkg, dev, steps, warmup, stream, launches_per_step=35):
    """The fixed cost of one graph-replayed launch: mnb_stream_read over 1 KiB
    (the ceiling kernel's grid, 2048 wavefronts, almost no loads), replayed
    back to back like the decode legs' rotated launches."""
    import ctypes
    buf = torch.zeros(1024, dtype=torch.uint8, device=dev)
    out = torch.empty(2048, dtype=torch.int32, device=dev)
    L = pkg.library()

    def launches():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for _ in range(launches_per_step):
            rc = L.mnb_stream_read(ctypes.c_void_p(buf.data_ptr()), buf.numel(),
                                   ctypes.c_void_p(out.data_ptr()), out.numel(), st)
            if rc != 0:
                raise RuntimeError(f"mnb_stream_read: status {rc}")

    ms, _, med, iqr = time_graph(torch, launches, steps, warmup, stream)
    return {"kernel": "StreamReadKernel (mnb_stream_read, 1 KiB)",
            "launches_per_step": launches_per_step,
            "us_per_launch": ms * 1e3 / launches_per_step,
            "us_per_launch_median": med * 1e3 / launches_per_step,
            "us_per_launch_samples": last_samples(launches_per_step)}


def gpu_metadata(torch, dev):
    """The device and software the run measured: gfx arch, CUs, memory, L2,
    HIP runtime and driver versions, current clocks (rocm-smi)."""
    import ctypes
    pr = torch.cuda.get_device_properties(dev)
    md = {"name": pr.name, "gcnArchName": getattr(pr, "gcnArchName", None),
          "compute_units": pr.multi_processor_count, "total_memory_bytes": pr.total_memory,
          "L2_cache_bytes": getattr(pr, "L2_cache_size", None),
          "clock_rate_khz": getattr(pr, "clock_rate", None),
          "torch": torch.__version__, "torch_hip": torch.version.hip}
    try:
        path = next(line.split()[-1] for line in open("/proc/self/maps")
                    if "libamdhip64" in line)
        hip = ctypes.CDLL(path)
        v = ctypes.c_int()
        if hip.hipRuntimeGetVersion(ctypes.byref(v)) == 0:
            md["hip_runtime_version"] = v.value
        if hip.hipDriverGetVersion(ctypes.byref(v)) == 0:
            md["hip_driver_version"] = v.value
    except (OSError, StopIteration, AttributeError) as e:
        md["hip_versions_error"] = str(e)
    # the current clock levels (the line marked *) from the driver's sysfs
    # tables, read as files (no helper process)
    clocks = {}
    for dev_dir in sorted(pathlib.Path("/sys/class/drm").glob("card*/device")):
        for table in ("pp_dpm_sclk", "pp_dpm_mclk", "pp_dpm_fclk"):
            try:
                cur = [ln.strip() for ln in (dev_dir / table).read_text().splitlines()
                       if ln.strip().endswith("*")]
            except OSError:
                continue
            if cur:
                clocks.setdefault(dev_dir.parent.name, {})[table] = cur[0]
    md["clocks_after_run"] = clocks
    return md


def fp16_gemm_reference(torch, dev, p, M, steps, warmup, stream):
    """Vendor dense fp16 GEMM on the same shape (torch.matmul -> hipBLASLt),
    fp16 A and fp16 weights already dequantized: no 4-bit decode and no fp32
    input conversion, i.e. a reference for what the fp16 matrix cores reach on
    this shape through the vendor library."""
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    A = torch.randn((M, p.K), device=dev, generator=g).to(torch.float16)
    Wt = torch.randn((p.N, p.K), device=dev, generator=g).to(torch.float16)
    Y = torch.empty((M, p.N), device=dev, dtype=torch.float16)

    def launches():
        for _ in range(CALLS_PER_STEP):
            torch.matmul(A, Wt.t(), out=Y)

    ms, _, _, _ = time_graph(torch, launches, steps, warmup, stream)
    us = ms * 1e3 / CALLS_PER_STEP
    tflops = p.flops(M) / (us * 1e-6) / 1e12
    return {"what": "torch.matmul fp16 x fp16 -> fp16 (hipBLASLt), dense weights",
            "calls_per_step": CALLS_PER_STEP,
            "us_per_launch": us, "TFLOPs": tflops, "frac_fp16_peak": tflops / FP16_PEAK_TFLOPS}


DECODE_TOL, GEMM_TOL = 1e-5, 2e-3


def reference_columns(torch, p, A, B, S, Z, cols):
    """fp64 Y[:, cols] = A * W[cols]^T with W[n, k] = (q - zp) * scale from the
    MatMulNBits definition (low nibble first, zero point 8 when absent),
    computed with torch on the device from the weights the timed launches
    read: an independent check of the timed kernels' output."""
    n = cols.numel()
    Bc = B[cols].reshape(n, -1)
    q = torch.stack([Bc & 15, Bc >> 4], dim=-1).reshape(n, p.nb, p.block_size)
    if Z is not None:
        Zc = Z[cols]
        z = torch.stack([Zc & 15, Zc >> 4], dim=-1).reshape(n, -1)[:, :p.nb]
    else:
        z = torch.full((n, p.nb), 8, dtype=torch.uint8, device=B.device)
    w = (q.to(torch.float64) - z.to(torch.float64)[..., None]) * S[cols].to(torch.float64)[..., None]
    return A.to(torch.float64) @ w.reshape(n, -1)[:, :p.K].T


def validate(torch, p, A, weights, Y, path, ncols=512, seed=0):
    """Checks a timed leg's output after timing (outside the timed region):
    Y on ncols sampled weight rows (all of A's rows) against
    reference_columns, at the path's bound: max|dy| / max|y| <= 1e-5 on the
    decode path, ||dy||_2 / ||y||_2 <= 2e-3 on the fp16 GEMM."""
    B, S, Z = weights
    g = torch.Generator(device=Y.device)
    g.manual_seed(seed)
    cols = torch.randperm(p.N, device=Y.device, generator=g)[:min(ncols, p.N)]
    ref = reference_columns(torch, p, A, B, S, Z, cols)
    got = Y[:, cols].to(torch.float64)
    if path == 2:
        err = float(torch.linalg.vector_norm(got - ref) / torch.linalg.vector_norm(ref))
        tol, metric = GEMM_TOL, "l2 relative"
    else:
        err = float((got - ref).abs().max() / ref.abs().max())
        tol, metric = DECODE_TOL, "normwise max"
    ok = bool(err <= tol) and bool(torch.isfinite(got).all())
    if not ok:
        FAILED_CHECKS.append(f"{p.name} M={A.shape[0]}: {metric} error {err:.3e} > {tol}")
    return {"checked": f"{A.shape[0]} rows x {cols.numel()} sampled columns vs fp64 torch "
                       f"reference", "metric": metric, "error": err, "tolerance": tol, "ok": ok}


FAILED_CHECKS = []


def plan_create_leg(torch, pkg, dev):
    """First-use packing time: mnb_plan_create per c5 projection (host upload of
    B, scales and zero points, the per-row scale exponents, and the re-laid
    copies for the prefill and small-M decode kernels), mnb_plan_create_device
    on weights already in HBM (the derived copies only), and the gate/up plan
    (host interleave of the two weights, then the above). Wall time per plan,
    synchronous."""
    W = pkg.workloads
    out = []
    for p in W.CONFIGS["c5"].projections:
        B, S, Z = W.make_weights(p, 5)
        dB, dS = torch.from_numpy(B).to(dev), torch.from_numpy(S).to(dev)
        dZ = torch.from_numpy(Z).to(dev) if Z is not None else None
        torch.cuda.synchronize()
        r = {"projection": p.name, "K": p.K, "N": p.N, "weight_bytes": p.weight_bytes()}
        for name, fn in (("host_ms", lambda: pkg.MatMulNBits(p.K, p.N, 4, p.block_size).prepare(B, S, Z)),
                         ("device_ms", lambda: pkg.MatMulNBits(p.K, p.N, 4, p.block_size)
                          .prepare_device(dB, dS, dZ))):
            fn().release()  # warm
            t0 = time.perf_counter()
            op = fn()
            torch.cuda.synchronize()
            r[name] = (time.perf_counter() - t0) * 1e3
            # device memory the plan owns: with host weights its own copies
            # (compact plans keep only the re-laid ones), with borrowed
            # device weights the derived copies alone
            key = "host_plan" if name == "host_ms" else "device_plan"
            r[key + "_device_bytes"] = op.device_bytes()
            r[key + "_ratio"] = r[key + "_device_bytes"] / p.weight_bytes()
            op.release()
        out.append(r)
    p = W.Projection("gate_up", 4096, 14336, 128, True)
    Bg, Sg, Zg = W.make_weights(p, 6)
    Bu, Su, Zu = W.make_weights(p, 7)
    pkg.GateUpSiLU(p.K, p.N, 4, p.block_size).prepare(Bg, Sg, Zg, Bu, Su, Zu).release()
    t0 = time.perf_counter()
    op = pkg.GateUpSiLU(p.K, p.N, 4, p.block_size).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    torch.cuda.synchronize()
    out.append({"projection": "gate_up plan (two 14336-row weights interleaved)", "K": p.K,
                "N": 2 * p.N, "weight_bytes": 2 * p.weight_bytes(),
                "host_ms": (time.perf_counter() - t0) * 1e3,
                "host_plan_device_bytes": op.device_bytes(),
                "host_plan_ratio": op.device_bytes() / (2 * p.weight_bytes())})
    op.release()
    torch.cuda.empty_cache()
    return out


def decode_leg(torch, pkg, dev, p, M, steps, warmup, seed, stream):
    """One decode shape over >= 1 GiB of rotated weight copies."""
    rot = max(2, -(-ROTATION_BYTES // p.weight_bytes()))
    sets = make_device_weights(torch, p, rot, seed, dev)
    ops = [pkg.MatMulNBits(p.K, p.N, 4, p.block_size).prepare_device(*s) for s in sets]
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 1)
    A = (torch.randn((M, p.K), device=dev, generator=g) * p.a_sigma).contiguous()
    Y = torch.empty((M, p.N), device=dev)
    path = ops[0].select_path(M)
    kernel = ops[0].kernel_name(M)

    def launches():
        for op in ops:
            op(A, out=Y, stream=torch.cuda.current_stream())

    ms, wall, med, iqr = time_graph(torch, launches, steps, warmup, stream)
    samples = last_samples(rot)
    per_launch_us = ms * 1e3 / rot
    nbytes = p.algorithmic_bytes(M)
    # the last launch of a step wrote Y with the last weight copy
    check = validate(torch, p, A, sets[-1], Y, path, seed=seed)
    for op in ops:
        op.release()
    del sets
    torch.cuda.empty_cache()
    return {
        "K": p.K, "N": p.N, "M": M, "block_size": p.block_size,
        "zero_points": p.has_zero_points, "path": path, "kernel": kernel,
        "rotation_copies": rot,
        "us_per_launch": per_launch_us, "us_per_launch_median": med * 1e3 / rot,
        "us_per_launch_iqr": iqr * 1e3 / rot, "us_per_launch_samples": samples,
        "bytes_per_launch": nbytes,
        "GBps": nbytes / (per_launch_us * 1e-6) / 1e9, "ms_per_step": ms, "wall_s": wall,
        "wall_ms_per_step": wall * 1e3 / steps,
        "launches_per_step": rot, "validation": check,
    }


# Calls per step of the prefill legs: a step replays one graph of CALLS_PER_STEP
# back-to-back calls, so the per-replay launch overhead of the graph (several
# us, measured) is spread as it is over the decode legs' rotated launches.
CALLS_PER_STEP = 8


def gemm_leg(torch, pkg, dev, p, M, steps, warmup, seed, stream):
    sets = make_device_weights(torch, p, 1, seed, dev)
    op = pkg.MatMulNBits(p.K, p.N, 4, p.block_size).prepare_device(*sets[0])
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 1)
    A = (torch.randn((M, p.K), device=dev, generator=g) * p.a_sigma).contiguous()
    Y = torch.empty((M, p.N), device=dev)

    def launches():
        for _ in range(CALLS_PER_STEP):
            op(A, out=Y, stream=torch.cuda.current_stream())

    ms, wall, med, iqr = time_graph(torch, launches, steps, warmup, stream)
    samples = last_samples(CALLS_PER_STEP)
    us = ms * 1e3 / CALLS_PER_STEP
    flops = p.flops(M)
    tflops = flops / (us * 1e-6) / 1e12
    res = {"K": p.K, "N": p.N, "M": M, "block_size": p.block_size, "path": op.select_path(M),
           "kernel": op.kernel_name(M), "calls_per_step": CALLS_PER_STEP,
           "us_per_launch": us, "us_per_launch_median": med * 1e3 / CALLS_PER_STEP,
           "us_per_launch_iqr": iqr * 1e3 / CALLS_PER_STEP, "us_per_launch_samples": samples,
           "TFLOPs": tflops, "frac_fp16_peak": tflops / FP16_PEAK_TFLOPS,
           "bytes_per_launch": p.algorithmic_bytes(M), "wall_s": wall,
           "wall_ms_per_step": wall * 1e3 / steps,
           "validation": validate(torch, p, A, sets[0], Y, op.select_path(M), seed=seed)}
    op.release()
    return res


def gemm_shapes_leg(torch, pkg, dev, Ms, steps, warmup, stream):
    """The GEMM path's kernel choice, measured (not run by default): per c5
    projection and c4 at each M, us per call of the automatic path against
    GemmKernel's own shape choice and the prefill kernel with 1, 2 and 4 K
    splits and with its own choice (mnb_run_kernel), CALLS_PER_STEP calls per
    graph replay on one weight copy; beside them hipBLASLt's dense fp16 GEMM
    of the shape (fp16_gemm_reference)."""
    W = pkg.workloads
    out = []
    projections = list(W.CONFIGS["c5"].projections) + [W.CONFIGS["c4"].projections[0]]
    for p in projections:
        B, S, Z = W.make_weights(p, 41)
        op = pkg.MatMulNBits(p.K, p.N, 4, p.block_size).prepare(B, S, Z)
        for M in Ms:
            A = torch.randn((M, p.K), device=dev)
            Y = torch.empty((M, p.N), device=dev)
            r = {"projection": p.name, "K": p.K, "N": p.N, "M": M, "auto_kernel": op.kernel_name(M)}
            variants = [("auto", lambda: op(A, out=Y, stream=torch.cuda.current_stream())),
                        ("gemm_kernel", lambda: op.run_kernel(A, pkg.KERNEL_GEMM, out=Y,
                                                              stream=torch.cuda.current_stream())),
                        ("prefill_auto_splits", lambda: op.run_kernel(
                            A, pkg.KERNEL_PREFILL, out=Y, stream=torch.cuda.current_stream()))]
            for sp in (1, 2, 4):
                variants.append((f"prefill_{sp}_splits", lambda sp=sp: op.run_kernel(
                    A, pkg.KERNEL_PREFILL, sp, out=Y, stream=torch.cuda.current_stream())))
            for name, fn in variants:
                try:
                    ms, _, _, _ = time_graph(torch, lambda fn=fn: [fn() for _ in range(CALLS_PER_STEP)],
                                             steps, warmup, stream)
                    r[name + "_us"] = ms * 1e3 / CALLS_PER_STEP
                except pkg.MatMulNBitsError:
                    r[name + "_us"] = None  # not served by this plan (compact: no original layout)
            # the vendor's dense fp16 GEMM on the shape (no 4-bit decode, no input conversion)
            r["hipblaslt_fp16_us"] = fp16_gemm_reference(torch, dev, p, M, steps, warmup,
                                                         stream)["us_per_launch"]
            r["auto_TFLOPs"] = p.flops(M) / (r["auto_us"] * 1e-6) / 1e12
            out.append(r)
            print(f"# gemm shapes {p.name} M={M}: " + " ".join(
                f"{k[:-3]}={v:.1f}" for k, v in r.items() if k.endswith("_us") and v is not None),
                file=sys.stderr, flush=True)
        op.release()
    return out


def gate_up_leg(torch, pkg, dev, Ms, steps, warmup, stream):
    """Measured fusion: the c5 gate+up projection (K=4096, two 14336-row
    weights, bs=128, zero points) as one gate/up plan writing
    silu(gate) * up, against the unfused graph -- one MatMulNBits over the
    concatenated [Wg; Wu] rows, then silu(g) * u as torch elementwise ops --
    and against that MatMulNBits alone. Decode shapes rotate 4 weight copies
    (0.47 GB per variant), prefill shapes use one."""
    import numpy as np
    import torch.nn.functional as F
    W = pkg.workloads
    K, I, bs = 4096, 14336, 128
    p = W.Projection("gate_up", K, I, bs, True, 1.0, 0.005, 0.02)
    copies = 4 if min(Ms) <= 16 else 1
    fused, plain, host = [], [], []
    for c in range(copies):
        Bg, Sg, Zg = W.make_weights(p, 1000 + 2 * c)
        Bu, Su, Zu = W.make_weights(p, 1001 + 2 * c)
        host.append(((Bg, Sg, Zg), (Bu, Su, Zu)))
        fused.append(pkg.GateUpSiLU(K, I, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, Zu))
        cat = [np.concatenate([x.reshape(I, -1), y.reshape(I, -1)])
               for x, y in ((Bg, Bu), (Sg, Su), (Zg, Zu))]
        plain.append(pkg.MatMulNBits(K, 2 * I, 4, bs).prepare(*cat))

    def check(M, A, out_t, c, what):
        # H (or [g | u]) of weight copy c on sampled columns against fp64
        rng = np.random.default_rng(M)
        cols = np.sort(rng.choice(I, 256, replace=False))
        dev_rows = lambda w: tuple(torch.from_numpy(np.ascontiguousarray(x[cols])).to(dev)
                                   for x in w)
        idx = torch.arange(cols.size, device=dev)
        q = W.Projection("gate_up", K, cols.size, bs, True)
        gr = reference_columns(torch, q, A, *dev_rows(host[c][0]), idx)
        ur = reference_columns(torch, q, A, *dev_rows(host[c][1]), idx)
        if what == "plain":
            ref = torch.cat([gr, ur], dim=1)
            got = torch.cat([out_t[:, torch.from_numpy(cols).to(dev)],
                             out_t[:, torch.from_numpy(cols + I).to(dev)]], dim=1)
        else:
            ref = gr * torch.sigmoid(gr) * ur
            got = out_t[:, torch.from_numpy(cols).to(dev)]
        got = got.to(torch.float64)
        if M > 16:
            err = float(torch.linalg.vector_norm(got - ref) / torch.linalg.vector_norm(ref))
            tol, metric = GEMM_TOL, "l2 relative"
        else:
            err = float((got - ref).abs().max() / ref.abs().max())
            # two products within 1e-5 each, composed through silu
            tol, metric = (4 * DECODE_TOL if what != "plain" else DECODE_TOL), "normwise max"
        ok = err <= tol and bool(torch.isfinite(got).all())
        if not ok:
            FAILED_CHECKS.append(f"gate_up {what} M={M}: {metric} error {err:.3e} > {tol}")
        return {"metric": metric, "error": err, "tolerance": tol, "ok": ok}

    out = []
    for M in Ms:
        n = copies if M <= 16 else 1
        reps = 1 if M <= 16 else CALLS_PER_STEP
        g = torch.Generator(device=dev)
        g.manual_seed(29 + M)
        A = torch.randn((M, K), device=dev, generator=g)
        H = torch.empty(M, I, device=dev)
        Y = torch.empty(M, 2 * I, device=dev)

        def run_fused():
            for op in fused[:n] * reps:
                op(A, out=H, stream=torch.cuda.current_stream())

        def run_plain():
            for op in plain[:n] * reps:
                op(A, out=Y, stream=torch.cuda.current_stream())

        def run_unfused():
            for op in plain[:n] * reps:
                op(A, out=Y, stream=torch.cuda.current_stream())
                torch.mul(F.silu(Y[:, :I]), Y[:, I:], out=H)

        r = {"M": M, "weight_copies": n, "calls_per_step": n * reps, "validation": {}}
        for name, fn, what, res in (("fused_us", run_fused, "fused", H),
                                    ("unfused_us", run_unfused, "unfused", H),
                                    ("matmul_only_us", run_plain, "plain", Y)):
            ms, _, _, _ = time_graph(torch, fn, steps, warmup, stream)
            r[name] = ms * 1e3 / (n * reps)
            r[name.replace("_us", "_samples_us")] = last_samples(n * reps)
            r["validation"][what] = check(M, A, res, n - 1, what)
        r["gain"] = r["unfused_us"] / r["fused_us"]
        out.append(r)
    for op in fused + plain:
        op.release()
    torch.cuda.empty_cache()
    return out


def rmsnorm_leg(torch, pkg, dev, Ms, steps, warmup, stream):
    """Measured fusion: RMSNorm into the c5 QKV projection's input (K=4096,
    N=6144, bs=128, zero points) through mnb_run_rmsnorm, against the unfused
    graph (torch's rms_norm, then the MatMulNBits node) and against the node
    alone. M = 1 and M > 16 run fused; 2 <= M <= 16 takes the library's own
    normalization pass before the decode kernel. Decode shapes rotate 8
    weight copies (0.3 GB per variant), prefill shapes use one."""
    import torch.nn.functional as F
    W = pkg.workloads
    p = W.Projection("qkv", 4096, 6144, 128, True, 1.0, 0.005, 0.02)
    copies = 8
    sets = make_device_weights(torch, p, copies, 31, dev)
    ops = [pkg.MatMulNBits(p.K, p.N, 4, p.block_size).prepare_device(*st) for st in sets]
    g = torch.Generator(device=dev)
    g.manual_seed(37)
    gamma = torch.rand(p.K, device=dev, generator=g) + 0.5
    eps = 1e-5
    out = []
    for M in Ms:
        n = copies if M <= 16 else 1
        reps = 1 if M <= 16 else CALLS_PER_STEP
        X = torch.randn((M, p.K), device=dev, generator=g) * 3.0
        Y = torch.empty(M, p.N, device=dev)

        def run_fused():
            for op in ops[:n] * reps:
                op.run_rmsnorm(X, gamma, eps, out=Y, stream=torch.cuda.current_stream())

        def run_unfused():
            for op in ops[:n] * reps:
                Xn = F.rms_norm(X, (p.K,), weight=gamma, eps=eps)
                op(Xn, out=Y, stream=torch.cuda.current_stream())

        def run_plain():
            for op in ops[:n] * reps:
                op(X, out=Y, stream=torch.cuda.current_stream())

        # fp64 RMSNorm of X, the input the fused and unfused runs multiply
        X64 = X.to(torch.float64)
        Xn64 = X64 / torch.sqrt((X64 * X64).mean(dim=1, keepdim=True) + eps) * gamma.to(torch.float64)
        path = ops[0].select_path(M)
        r = {"M": M, "weight_copies": n, "calls_per_step": n * reps, "validation": {}}
        for name, fn, inp in (("fused_us", run_fused, Xn64), ("unfused_us", run_unfused, Xn64),
                              ("matmul_only_us", run_plain, X64)):
            ms, _, _, _ = time_graph(torch, fn, steps, warmup, stream)
            r[name] = ms * 1e3 / (n * reps)
            r[name.replace("_us", "_samples_us")] = last_samples(n * reps)
            r["validation"][name[:-3]] = validate(torch, p, inp, sets[n - 1], Y, path,
                                                  ncols=256, seed=M)
        r["gain"] = r["unfused_us"] / r["fused_us"]
        out.append(r)
    for op in ops:
        op.release()
    del sets
    torch.cuda.empty_cache()
    return out


def c5_leg(torch, pkg, dev, M, steps, warmup, stream):
    """BASELINE config c5: 32 Llama-3-8B-shaped layers (QKV, O, gate+up, down;
    bs = 128, zero points; 3.74 GB of 4-bit weights) run back to back, one
    mnb_run per projection, at M tokens. Inputs are independent random
    activations (no inter-layer math), so the leg measures the 128 projections
    alone."""
    c = pkg.workloads.CONFIGS["c5"]
    ops, sets = [], []
    for layer in range(c.layers):
        for j, p in enumerate(c.projections):
            s = make_device_weights(torch, p, 1, pkg.workloads.weight_seed(c.index, layer, j), dev)
            sets.append(s)
            ops.append((p, pkg.MatMulNBits(p.K, p.N, 4, p.block_size).prepare_device(*s[0])))
    g = torch.Generator(device=dev)
    g.manual_seed(29)
    acts = {K: (torch.randn((M, K), device=dev, generator=g) * 1.0).contiguous()
            for K in sorted({p.K for p in c.projections})}
    outs = {N: torch.empty((M, N), device=dev) for N in sorted({p.N for p in c.projections})}

    def launches():
        for p, op in ops:
            op(acts[p.K], out=outs[p.N], stream=torch.cuda.current_stream())

    ms, wall, med, iqr = time_graph(torch, launches, steps, warmup, stream)
    samples = [round(v, 5) for v in SAMPLES[-1]]
    # each output buffer holds the last layer's projection of its width
    last = {}
    for (p, op), s in zip(ops, sets):
        last[p.N] = (p, op, s[0])
    checks = [validate(torch, p, acts[p.K], w, outs[N], op.select_path(M), ncols=256, seed=N)
              for N, (p, op, w) in sorted(last.items())]
    nbytes = sum(p.algorithmic_bytes(M) for p, _ in ops)
    flops = sum(p.flops(M) for p, _ in ops)
    res = {"M": M, "layers": c.layers, "launches_per_step": len(ops), "ms_per_step": ms,
           "ms_per_step_median": med, "ms_per_step_iqr": iqr, "ms_per_step_samples": samples,
           "validation": checks,
           "us_per_launch": ms * 1e3 / len(ops), "bytes_per_step": nbytes,
           "flops_per_step": flops, "GBps": nbytes / (ms * 1e-3) / 1e9,
           "TFLOPs": flops / (ms * 1e-3) / 1e12, "wall_ms_per_step": wall * 1e3 / steps}
    res["frac_hbm"] = res["GBps"] / HBM_PEAK_GBS
    res["frac_fp16_peak"] = res["TFLOPs"] / FP16_PEAK_TFLOPS
    for _, op in ops:
        op.release()
    del ops, sets
    torch.cuda.empty_cache()
    return res


def _cpu_topology():
    """lscpu's sockets x cores x threads-per-core, or None where lscpu is absent."""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    f = {}
    for line in out.splitlines():
        k, _, v = line.partition(":")
        f[k.strip()] = v.strip()
    return {"sockets": f.get("Socket(s)"), "cores_per_socket": f.get("Core(s) per socket"),
            "threads_per_core": f.get("Thread(s) per core"), "model": f.get("Model name")}


def _time_calls(fn, budget_s, max_calls=100000):
    """Median and IQR of fn() over about budget_s seconds, after 3 warmup calls, >= 7 samples."""
    for _ in range(3):
        fn()
    samples = []
    t_end = time.perf_counter() + budget_s
    while len(samples) < 7 or (time.perf_counter() < t_end and len(samples) < max_calls):
        t0 = time.perf_counter()
        fn()
        samples.append(time.perf_counter() - t0)
    med = statistics.median(samples)
    q = statistics.quantiles(samples, n=4)
    return med, q[2] - q[0], len(samples)


def cpu_leg(pkg, budget_s):
    """CPU baselines on the c2 M=1 workload, host cores of this machine.

    Four modes, about budget_s / 4 seconds each:
    - fused: the C oracle's fused unpack-scale-FMA fp32 GEMV over the packed
      4-bit weights, N-partitioned like the reference's ExecuteRanges
      (onnx_light_cpu/impl/execution.h:72-184), at T threads and at 1;
    - reference: the reference's own MatMulPlan<float> (compiled from its
      sources into oracle/_ref) over W dequantized to fp32 [N, K] once
      beforehand, i.e. the dequantize-then-fp32-MatMul order of the reference
      engine with the dequantization folded away, at T threads and at 1.
    Every rate is the workload's algorithmic bytes (4-bit weights, scales, zero
    points, A, Y) over the median call time, the unit of the GPU figure.
    """
    import numpy as np
    import __graft_entry__
    orc = __graft_entry__.load_oracle()
    c = pkg.workloads.CONFIGS["c2"]
    p = c.projections[0]
    B, S, Z = pkg.workloads.make_weights(p, pkg.workloads.weight_seed(c.index))
    A = pkg.workloads.make_activations(1, p.K, p.a_sigma, pkg.workloads.activation_seed(c.index, 1))
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    T = max(1, min(orc.default_threads(), avail))
    nbytes = p.algorithmic_bytes(1)
    per = budget_s / 4.0
    modes = []

    def add(name, threads, fn):
        med, iqr, n = _time_calls(fn, per)
        modes.append({"mode": name, "threads": threads, "GBps": nbytes / med / 1e9,
                      "median_ms": med * 1e3, "iqr_ms": iqr * 1e3, "calls": n})
        print(f"# cpu {name} threads={threads}: {med * 1e3:.2f} ms/call, "
              f"{nbytes / med / 1e9:.2f} GB/s ({n} calls)", file=sys.stderr, flush=True)

    for t in (T, 1):
        add("fused int4 GEMV (C oracle)", t,
            lambda t=t: orc.matmul_nbits_fused_f32(A, B, S, Z, p.K, p.N, p.block_size, t))
    if orc.ref_available():
        # [K, N]: the orientation an ONNX MatMul's B input has after the
        # dequantization is folded into a constant.
        W = np.ascontiguousarray(orc.dequantize(B, S, Z, p.K, p.N, p.block_size).T,
                                 dtype=np.float32)
        for t in (T, 1):
            add("reference MatMulPlan<float> on dequantized W [K,N] (oracle/_ref)", t,
                lambda t=t: orc.ref_matmul_f32(A, W, t, trans_b=False))
        del W
    head = modes[0]
    sample = (f"c2 M=1 K=4096 N=14336 bs=128 zp, full matrix per call; value = fused int4 GEMV "
              f"of the C oracle on {T} threads, {head['calls']} calls (median "
              f"{head['median_ms']:.2f} ms, IQR {head['iqr_ms']:.2f} ms); 1-thread and "
              f"reference-MatMul figures under modes (the reference plan picks kSkinnyM at "
              f"M=1, whose column-panel split gave no parallel speedup on this host); "
              f"onnx-light CpuExecutor: not available "
              f"(onnx-light absent); equivalent participants = {T}")
    return {"value": head["GBps"], "unit": "GB/s", "cores": T, "kind": "port", "sample": sample,
            "modes": modes, "host": platform.processor() or platform.machine(),
            "nproc": os.cpu_count(), "affinity": avail, "topology": _cpu_topology()}


def main():
    global EAGER
    args = parse_args()
    EAGER = args.eager
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not "
              "supported (the decode GEMV would shard column-parallel over N, one shard "
              "of weight rows per GPU)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)
    legs = (set(args.only.split(",")) if args.only
            else {"decode", "ceiling", "gemm", "sweep", "lm_head", "c5", "gate_up", "rmsnorm",
                  "plan", "cpu"})
    W = pkg.workloads

    t_start = time.perf_counter()
    out = {}
    head = None
    if "decode" in legs:
        p = W.CONFIGS["c2"].projections[0]
        head = decode_leg(torch, pkg, dev, p, 1, args.steps, args.warmup, 11, stream)
        print(f"# decode c2 M=1: {head['us_per_launch']:.2f} us/launch, "
              f"{head['GBps']:.0f} GB/s", file=sys.stderr, flush=True)
    gemm = None
    if "gemm" in legs:
        p = W.CONFIGS["c4"].projections[0]
        gemm = gemm_leg(torch, pkg, dev, p, 2048, args.steps, args.warmup, 13, stream)
        print(f"# gemm c4 M=2048: {gemm['us_per_launch']:.1f} us, {gemm['TFLOPs']:.1f} TFLOP/s",
              file=sys.stderr, flush=True)
        gemm["reference_fp16_gemm"] = fp16_gemm_reference(torch, dev, p, 2048, args.steps,
                                                          args.warmup, stream)
        print(f"# reference: dense fp16 torch.matmul c4 shape: "
              f"{gemm['reference_fp16_gemm']['us_per_launch']:.1f} us, "
              f"{gemm['reference_fp16_gemm']['TFLOPs']:.1f} TFLOP/s", file=sys.stderr, flush=True)
        # the small-M end of the GEMM path (17 <= M <= 64: the weight-streaming
        # kernel) on the c4 and c2 weights, over >= 1 GiB of rotated copies
        gemm["small_m"] = []
        for cname, M in (("c4", 32), ("c4", 64), ("c2", 32)):
            q = W.CONFIGS[cname].projections[0]
            r = decode_leg(torch, pkg, dev, q, M, max(3, args.steps // 4), 2, 19 + M, stream)
            gemm["small_m"].append({"config": cname, "M": M, "kernel": r["kernel"],
                                    "us_per_launch": r["us_per_launch"],
                                    "us_per_launch_median": r["us_per_launch_median"],
                                    "us_per_launch_iqr": r["us_per_launch_iqr"], "GBps": r["GBps"],
                                    "TFLOPs": q.flops(M) / (r["us_per_launch"] * 1e-6) / 1e12})
            print(f"# small-M gemm {cname} M={M}: {r['us_per_launch']:.2f} us, {r['GBps']:.0f} GB/s",
                  file=sys.stderr, flush=True)
    sweep = []
    if "sweep" in legs:
        # the configs, then one GPU's shard of c2 and c3 under 8-way tensor
        # parallelism (c2 column-parallel: N / 8 weight rows; c3 row-parallel:
        # K / 8 of each row), then rows too long for one workgroup per row
        # group: Llama-70B's down projection (K = 28672, N = 8192), served at
        # M <= 2 by the fragment-ordered GEMV with K segments; Qwen2.5-72B's
        # (K = 29568: not a whole number of 256-k units), Gemma-7B's at 4
        # rows (K = 24576, N = 3072: K segments on narrow weights) and a
        # wide projection whose row groups (288) leave a second round on a
        # few CUs (K = 7168, N = 18432: K segments to balance them), and a
        # Qwen2.5-14B-shaped gate+up projection at 8 rows (K = 5120 = 20 units:
        # one run of four units per wavefront in the small-M decode)
        tp8 = {"c2/tp8": W.Projection("c2/tp8", 4096, 14336 // 8, 128, True),
               "c3/tp8": W.Projection("c3/tp8", 14336 // 8, 4096, 32, True, 0.5, 0.002, 0.01),
               "70b_down": W.Projection("70b_down", 28672, 8192, 128, True),
               "qwen72b_down": W.Projection("qwen72b_down", 29568, 8192, 128, True),
               "gemma7b_down": W.Projection("gemma7b_down", 24576, 3072, 128, True),
               "wide_7168": W.Projection("wide_7168", 7168, 18432, 128, True),
               "gate_up_5120": W.Projection("gate_up_5120", 5120, 27648, 128, True)}
        for cname, Ms in (("c1", (1,)), ("c2", (4, 16)), ("c3", (1, 2, 8, 16)),
                          ("c2/tp8", (1, 16)), ("c3/tp8", (1, 16)), ("70b_down", (1, 2)),
                          ("qwen72b_down", (1, 16)), ("gemma7b_down", (4,)), ("wide_7168", (1,)),
                          ("gate_up_5120", (8,))):
            p = tp8[cname] if cname in tp8 else W.CONFIGS[cname].projections[0]
            for M in Ms:
                r = decode_leg(torch, pkg, dev, p, M, max(3, args.steps // 4), 2, 17 + M, stream)
                r["config"] = cname
                sweep.append({k: r[k] for k in ("config", "M", "us_per_launch", "us_per_launch_median",
                                                 "us_per_launch_iqr", "GBps", "path", "kernel")})
                print(f"# decode {cname} M={M}: {r['us_per_launch']:.2f} us, {r['GBps']:.0f} GB/s",
                      file=sys.stderr, flush=True)
    gemm_shapes = None
    if "gemm_shapes" in legs:
        gemm_shapes = gemm_shapes_leg(torch, pkg, dev, (128, 256, 512, 1024, 2048),
                                      max(3, args.steps // 4),
                                      2, stream)
    lm_head = None
    if "lm_head" in legs:
        # Llama-3-8B's LM head at decode: the one decode launch large enough
        # (281 MB) for the kernel's streaming rate to dominate its fixed cost
        p = W.Projection("lm_head", 4096, 128256, 128, True)
        lm_head = decode_leg(torch, pkg, dev, p, 1, max(3, args.steps // 4), 2, 23, stream)
        lm_head["frac_hbm"] = lm_head["GBps"] / HBM_PEAK_GBS
        print(f"# decode LM head M=1: {lm_head['us_per_launch']:.2f} us, "
              f"{lm_head['GBps']:.0f} GB/s", file=sys.stderr, flush=True)
    c5 = []
    if "c5" in legs:
        for M in (1, 512):
            r = c5_leg(torch, pkg, dev, M, max(3, args.steps // 4), 2, stream)
            c5.append(r)
            print(f"# c5 32 layers M={M}: {r['ms_per_step']:.3f} ms/step, {r['GBps']:.0f} GB/s, "
                  f"{r['TFLOPs']:.1f} TFLOP/s", file=sys.stderr, flush=True)
    gate_up = []
    if "gate_up" in legs:
        gate_up = gate_up_leg(torch, pkg, dev, (1, 16, 512, 2048), max(3, args.steps // 4), 2,
                              stream)
        for r in gate_up:
            print(f"# gate/up + SiLU M={r['M']}: fused {r['fused_us']:.1f} us, unfused "
                  f"{r['unfused_us']:.1f} us ({r['gain']:.2f}x), matmul alone "
                  f"{r['matmul_only_us']:.1f} us", file=sys.stderr, flush=True)
    rms = []
    if "rmsnorm" in legs:
        rms = rmsnorm_leg(torch, pkg, dev, (1, 16, 512), max(3, args.steps // 4), 2, stream)
        for r in rms:
            print(f"# RMSNorm + qkv M={r['M']}: fused {r['fused_us']:.1f} us, unfused "
                  f"{r['unfused_us']:.1f} us ({r['gain']:.2f}x), matmul alone "
                  f"{r['matmul_only_us']:.1f} us", file=sys.stderr, flush=True)
    ceiling, ceilings, floor = None, [], None
    if "ceiling" in legs:
        # plain-read ceilings of one launch at the decode shapes' byte counts,
        # and the fixed cost of a launch
        sizes = [("c2 M=1", W.CONFIGS["c2"].projections[0].algorithmic_bytes(1)),
                 ("c1 M=1", W.CONFIGS["c1"].projections[0].algorithmic_bytes(1)),
                 ("c3 M=1", W.CONFIGS["c3"].projections[0].algorithmic_bytes(1)),
                 ("LM head M=1", W.Projection("lm_head", 4096, 128256, 128, True)
                  .algorithmic_bytes(1))]
        # and c2's bytes read on GemvFragKernel's own grid: one workgroup of 8
        # wavefronts per 64-row group, 224 workgroups (the CUs it can use)
        c2 = W.CONFIGS["c2"].projections[0]
        sizes.append(("c2 M=1 on GemvFragKernel's grid", c2.algorithmic_bytes(1),
                      ((c2.N + 63) // 64, 64 * min(16, c2.K // 512))))
        for name, nbytes, *grid in sizes:
            r = stream_ceiling_leg(torch, pkg, dev, nbytes, args.steps, args.warmup, stream,
                                   grid[0] if grid else None)
            r["for"] = name
            ceilings.append(r)
            print(f"# read ceiling {name}, {nbytes} B per launch: {r['us_per_launch']:.2f} us, "
                  f"{r['GBps']:.0f} GB/s", file=sys.stderr, flush=True)
        ceiling = ceilings[0]
        floor = launch_floor_leg(torch, pkg, dev, args.steps, args.warmup, stream)
        print(f"# launch floor: {floor['us_per_launch']:.2f} us", file=sys.stderr, flush=True)
    plans = []
    if "plan" in legs:
        plans = plan_create_leg(torch, pkg, dev)
        for r in plans:
            print(f"# plan create {r['projection']}: host {r['host_ms']:.1f} ms "
                  f"({r['host_plan_ratio']:.2f}x the weights in device memory)"
                  + (f", device {r['device_ms']:.1f} ms" if "device_ms" in r else ""),
                  file=sys.stderr, flush=True)
    copy = None
    if "copy" in legs:
        copy = copy_leg(torch, dev, args.steps, args.warmup, stream)
        print(f"# copy 512 MiB: {copy['us_per_launch']:.1f} us, {copy['GBps']:.0f} GB/s",
              file=sys.stderr, flush=True)
    cpu = None
    if "cpu" in legs and args.cpu_seconds > 0:
        cpu = cpu_leg(pkg, args.cpu_seconds)
        print(f"# cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads",
              file=sys.stderr, flush=True)

    if head is not None:
        value = head["GBps"]
        ms_per_step = head["ms_per_step"]
        roof = {"bound": "hbm", "achieved": head["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": head["GBps"] / HBM_PEAK_GBS, "traffic": GEMV_M1_C2_TRAFFIC_BYTES,
                "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                "copy-calibrated)",
                "kernel": f"{head['kernel']} (c2 M=1)", "us_per_launch": head["us_per_launch"],
                "us_per_launch_median": head["us_per_launch_median"],
                "us_per_launch_iqr": head["us_per_launch_iqr"],
                "bytes_per_launch": head["bytes_per_launch"]}
        roof["validation"] = head["validation"]
        if ceiling is not None:
            roof["ceiling"] = ceiling["frac_of_peak"]
            roof["ceiling_GBps"] = ceiling["GBps"]
            roof["frac_of_ceiling"] = head["GBps"] / ceiling["GBps"]
            grid_ceiling = ceilings[-1]
            roof["grid_ceiling_GBps"] = grid_ceiling["GBps"]
            roof["frac_of_grid_ceiling"] = head["GBps"] / grid_ceiling["GBps"]
        workload = ("c2: MatMulNBits M=1 K=4096 N=14336 bits=4 block_size=128 zero_points; "
                    f"{head['rotation_copies']} rotated weight copies per step")
    else:
        value, ms_per_step, roof, workload = None, None, None, "none"
    out = {
        "metric": METRIC, "value": value, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u4xf32 (fp16 MFMA on 3-term fp16 activations and nibble subnormals, fp32 sums)",
        "data": "synthetic (seeded uniform nibbles, uniform scales, N(0,1) activations)",
        "config": {"workload": workload, "M": 1, "K": 4096, "N": 14336, "block_size": 128,
                   "zero_points": True},
        "roofline": roof,
        "cpu_baseline": cpu,
        "prefill_gemm": gemm,
        "decode_sweep": sweep,
        "c5_layer_stack": c5,
        "gate_up_fusion": gate_up,
        "read_ceiling": ceiling,
        "read_ceilings": ceilings,
        "launch_floor": floor,
        "lm_head_decode": lm_head,
        "gemm_shapes": gemm_shapes,
        "headline_samples_us_per_launch": head["us_per_launch_samples"] if head else None,
        "plan_create": plans,
        "rmsnorm_fusion": rms,
        "copy_calibration": copy,
        "timing": "eager launches" if EAGER else "HIP graph replay",
        "gpu": gpu_metadata(torch, dev),
        "validation_failures": FAILED_CHECKS,
        "bench_wall_s": time.perf_counter() - t_start,
    }
    print(json.dumps(out), flush=True)
    if FAILED_CHECKS:
        print("bench.py: outputs of timed legs failed validation: " + "; ".join(FAILED_CHECKS),
              file=sys.stderr, flush=True)
        sys.exit(1)


if __name__ == "__main__":
    main()
