"""Benchmark: RPL's GEMM hot path on one MI355X at 8192^3.

Metric: INT8 GEMM TOPS and FP32 GEMM TFLOPS at 8192^3 on one
MI355X, as a fraction of peak.  A step is one 8192^3 INT8 GEMM through
gemm_int8's layout (A [M,K], B [K,N] int8, N(0,1) data quantized per tensor,
int32 output); the FP32 8192^3 GEMM (tensor_gemm semantics, NN) is timed the
same way and reported beside it.  Inputs are generated from fixed seeds,
uploaded and quantized before the timed region (resident in HBM).

`value` is the INT8 throughput in TOP/s.  `roofline` covers the dominant
kernel (the i8-MFMA GEMM kernel, timed alone with HIP events on its stream);
`cpu_baseline` times the C oracle (a bit-identical restatement of the
reference's CPU path) on a 64-row slab of the same INT8 GEMM on the host's
cores.  Prints ONE JSON line.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

import rpl_amd  # noqa: E402
from rpl_amd import DeviceBuffer, check  # noqa: E402

METRIC = "INT8 GEMM TOPS & FP32 GEMM TFLOPS at 8192³ on 1 MI355X, % of peak"
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_FP32_TFLOPS = 157.3  # MI355X fp32 matrix
PEAK_HBM_GBS = 8000.0
SEED_BASE = 0x52504C00


def seed(cfg, stream):
    return SEED_BASE + 16 * cfg + stream


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """HIP events on one stream: average ms per call over `steps` calls."""

    def __init__(self, lib, stream):
        self.lib, self.stream = lib, stream
        self.e0, self.e1 = C.c_void_p(), C.c_void_p()
        check(lib.rplhip_event_create(C.byref(self.e0)))
        check(lib.rplhip_event_create(C.byref(self.e1)))

    def time(self, fn, steps, warmup):
        for _ in range(warmup):
            fn()
        check(self.lib.rplhip_synchronize())
        t0 = time.perf_counter()
        check(self.lib.rplhip_event_record(self.e0, self.stream))
        for _ in range(steps):
            fn()
        check(self.lib.rplhip_event_record(self.e1, self.stream))
        check(self.lib.rplhip_event_synchronize(self.e1))
        check(self.lib.rplhip_synchronize())
        wall = time.perf_counter() - t0
        ms = C.c_float()
        check(self.lib.rplhip_event_elapsed_ms(C.byref(ms), self.e0, self.e1))
        return ms.value / steps, wall


def cpu_baseline_int8(n, rows, qa, qb):
    """The oracle (reference CPU path restated, same flags) on a row slab."""
    from oracle import Oracle

    orc = Oracle()
    t0 = time.perf_counter()
    orc.gemm_int8(qa[:rows], qb, rows, n, n, rows=None)
    dt = time.perf_counter() - t0
    return 2.0 * rows * n * n / dt / 1e12, dt


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--n", type=int, default=8192)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--cpu-rows", type=int, default=512)
    ap.add_argument("--only", choices=["int8", "int8-kernel", "fp32", "skinny"],
                    help="run one leg only (for profiling); the JSON line then has nulls for the rest")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    lib = rpl_amd.lib()
    check(lib.rplhip_init(), "init")
    arch = C.create_string_buffer(64)
    cus, clk = C.c_int(), C.c_int()
    check(lib.rplhip_device_info(arch, 64, C.byref(cus), C.byref(clk)))
    stream = C.c_void_p()
    check(lib.rplhip_stream_create(C.byref(stream)))
    timer = Timer(lib, stream)
    n = args.n

    # ---- INT8: N(0,1) -> per-tensor symmetric quantization on the device (untimed)
    log(f"bench: generating inputs n={n}")
    A = rpl_amd.fill_normal(n * n, seed(4, 0))
    B = rpl_amd.fill_normal(n * n, seed(4, 1))
    dA, dB = DeviceBuffer.from_array(A), DeviceBuffer.from_array(B)
    qA, qB = DeviceBuffer(n * n), DeviceBuffer(n * n)
    sA, sB = DeviceBuffer(4), DeviceBuffer(4)
    check(lib.rplhip_quantize_symmetric(dA.ptr, n * n, qA.ptr, sA.ptr, stream))
    check(lib.rplhip_quantize_symmetric(dB.ptr, n * n, qB.ptr, sB.ptr, stream))
    check(lib.rplhip_stream_synchronize(stream))
    scales = np.concatenate([sA.to_array(np.float32, (1,)), sB.to_array(np.float32, (1,))])
    dC = DeviceBuffer(n * n * 4)
    ops = 2.0 * n * n * n

    def int8_step():
        check(lib.rplhip_gemm_int8(qA.ptr, qB.ptr, dC.ptr, n, n, n, float(scales[0]), float(scales[1]), 1.0, 0, 0,
                                   stream))

    want = lambda leg: args.only in (None, leg)  # noqa: E731
    ms_i8 = wall_i8 = tops = ms_k = kern_tops = ms_f32 = wall_f32 = tflops = float("nan")
    if want("int8"):
        log("bench: int8 gemm_int8 8192^3")
        ms_i8, wall_i8 = timer.time(int8_step, args.steps, args.warmup)
        tops = ops / (ms_i8 * 1e-3) / 1e12

    # Dominant kernel alone: the i8-MFMA GEMM on B already in [N,K] (what
    # gemm_int8 runs after its transpose pass).
    kern = lambda: check(lib.rplhip_linear_int8(qA.ptr, qB.ptr, None, dC.ptr, n, n, n, stream))  # noqa: E731
    if want("int8-kernel") or args.only is None:
        log("bench: int8 GEMM kernel alone")
        ms_k, _ = timer.time(kern, args.steps, args.warmup)
        kern_tops = ops / (ms_k * 1e-3) / 1e12

    # ---- FP32 8192^3 NN (tensor_gemm semantics, alpha=1, beta=0)
    dCf = DeviceBuffer(n * n * 4)
    check(lib.rplhip_memset(dCf.ptr, 0, n * n * 4, stream))

    def fp32_step():
        check(lib.rplhip_sgemm(0, 0, n, n, n, 1.0, dA.ptr, n, dB.ptr, n, 0.0, dCf.ptr, n, stream))

    if want("fp32"):
        log("bench: fp32 sgemm 8192^3")
        ms_f32, wall_f32 = timer.time(fp32_step, max(args.steps // 2, 3), 2)
        tflops = ops / (ms_f32 * 1e-3) / 1e12

    # ---- skinny INT8 (M in {1,4,16}, K=N=8192, per-channel W): HBM-bound.
    # Rotate 6 distinct 64 MiB weight copies (> 256 MB MALL) across calls.
    skinny = {}
    if n == 8192 and want("skinny"):
        K = N = n
        nw = 6
        Ws = [DeviceBuffer(N * K) for _ in range(nw)]
        for w in Ws:
            check(lib.rplhip_memcpy_dtod(w.ptr, qB.ptr, N * K, stream))
        sw = DeviceBuffer.from_array(np.full(N, scales[1], np.float32))
        sx = DeviceBuffer.from_array(np.float32([scales[0]]))
        Y = DeviceBuffer(16 * N * 4)
        for M in (1, 4, 16):
            it = [0]

            def sk():
                w = Ws[it[0] % nw]
                it[0] += 1
                check(lib.rplhip_linear_int8_dequant(qA.ptr, sx.ptr, 0, w.ptr, sw.ptr, 1, Y.ptr, M, K, N, stream))

            ms_s, _ = timer.time(sk, 60, 12)
            byts = N * K + M * K + M * N * 4 + N * 4 + 4
            skinny[f"M{M}"] = {"us": round(ms_s * 1e3, 2), "GB/s": round(byts / (ms_s * 1e-3) / 1e9, 1),
                               "frac_hbm": round(byts / (ms_s * 1e-3) / 1e9 / PEAK_HBM_GBS, 3)}
        del Ws

    cpu = None
    if not args.no_cpu and args.only is None:
        log(f"bench: cpu baseline (oracle, {args.cpu_rows}-row slab)")
        qa = qA.to_array(np.int8, (n, n))
        qb = qB.to_array(np.int8, (n, n))
        cpu_tops, cpu_s = cpu_baseline_int8(n, args.cpu_rows, qa, qb)
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        cpu = {"value": round(cpu_tops, 6), "unit": "TOP/s", "cores": threads, "kind": "port",
               "sample": f"oracle gemm_int8 (reference ops_extended.c:83-123 restated, -O3 -fopenmp) on a "
                         f"{args.cpu_rows}x{n}x{n} row slab of the same quantized inputs, {cpu_s:.1f} s"}

    traffic = None
    tpath = os.path.join(REPO, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("gemm_i8_nt_8192", {}).get("bytes_per_launch")

    out = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_i8, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"gemm_int8 {n}x{n}x{n} per-tensor (BASELINE configs[4]), A [M,K] B [K,N] int8 "
                               f"-> int32 requant; plus sgemm {n}^3 NN fp32",
                   "M": n, "N": n, "K": n},
        "pct_peak_int8": round(100 * tops / PEAK_INT8_TOPS, 2),
        "fp32": {"value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(ms_f32, 4),
                 "pct_peak": round(100 * tflops / PEAK_FP32_TFLOPS, 2), "dtype": "f32"},
        "roofline": {"bound": "mfma", "achieved": round(kern_tops, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TFLOP/s", "frac": round(kern_tops / PEAK_INT8_TOPS, 4), "traffic": traffic,
                     "kernel": "k_gemm_i8_nt (int8 ops/s)", "ms_per_launch": round(ms_k, 4)},
        "roofline_fp32": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP32_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP32_TFLOPS, 4), "kernel": "k_sgemm"},
        "skinny_int8": skinny,
        "cpu_baseline": cpu,
        "device": {"arch": arch.value.decode(), "cus": cus.value, "clock_mhz": clk.value // 1000},
        "wall_s": {"int8": round(wall_i8, 3), "fp32": round(wall_f32, 3)},
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
