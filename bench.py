"""Benchmark: RPL's GEMM hot path on one MI355X at 8192^3.

Metric: INT8 GEMM TOPS and FP32 GEMM TFLOPS at 8192^3 on one
MI355X, as a fraction of peak.  A step is one 8192^3 INT8 GEMM through
gemm_int8's layout (A [M,K], B [K,N] int8, N(0,1) data quantized per tensor,
int32 output); the FP32 8192^3 GEMM (tensor_gemm semantics, NN) is timed the
same way and reported beside it.  Inputs are generated from fixed seeds,
uploaded and quantized before the timed region (resident in HBM).

`value` is the INT8 throughput in TOP/s.  `roofline` covers the dominant
kernel: at 8192^3 gemm_int8 is exactly one launch of the i8-MFMA GEMM
kernel that reads B [K,N] in place, so the headline leg's HIP-event time on
its stream is that kernel's average launch duration (`nt_kernel` times the
same kernel on B already [N,K], linear_int8's layout); `power` samples the
socket power and shader clock (sysfs hwmon) while the INT8 and FP32 GEMMs
run back to back, untimed;
`cpu_baseline` times the reference's own CPU gemm_int8 (built from its
sources into oracle/_ref/libref.so; the C oracle, a bit-identical
restatement, when that build is absent) on a 512-row slab of the same INT8
GEMM on the host's cores.  Prints ONE JSON line.
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


def _hwmon_dirs():
    import glob
    return sorted(glob.glob("/sys/class/drm/card*/device/hwmon/hwmon*"))


def _read(path):
    try:
        with open(path) as f:
            return f.read()
    except OSError:
        return None


def _sample_power_clock():
    """(socket W, shader clock MHz) of the first GPU that reports both, from
    hwmon power1_input (uW) and the active level of pp_dpm_sclk."""
    for d in _hwmon_dirs():
        pw = _read(os.path.join(d, "power1_input")) or _read(os.path.join(d, "power1_average"))
        sclk = _read(os.path.join(os.path.dirname(os.path.dirname(d)), "pp_dpm_sclk"))
        if pw is None or sclk is None:
            continue
        mhz = None
        for line in sclk.splitlines():
            if line.strip().endswith("*"):
                mhz = float(line.split(":")[1].strip().rstrip("*").strip().lower().replace("mhz", ""))
        return int(pw) / 1e6, mhz
    return None, None


def power_while(lib, stream, fn, seconds):
    """Run fn back to back on `stream` for `seconds` (untimed) while a thread
    samples socket power and shader clock every 50 ms; medians over the
    second half.  The GPU never idles: each batch is queued before the host
    waits for the previous one, and the last batch is still running when
    this returns, so a timed leg queued next starts with no idle gap (an idle
    gap of a few ms on a power-capped MI355X is followed by a clock dip that
    lasts ~20 launches of the 8192^3 INT8 GEMM)."""
    import threading

    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            samples.append(_sample_power_clock())
            stop.wait(0.05)

    ev = [C.c_void_p(), C.c_void_p()]
    for e in ev:
        check(lib.rplhip_event_create(C.byref(e)))
    _KEEP.extend(ev)  # destroyed never: the last one may still be pending on return
    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        check(lib.rplhip_event_record(ev[i % 2], stream))
        if i:
            check(lib.rplhip_event_synchronize(ev[(i - 1) % 2]))
        i += 1
    for _ in range(16):  # keep the GPU busy through the bookkeeping below and the caller's next launches
        fn()
    stop.set()  # the sampler ends by itself; no join while the GPU must stay busy
    got = list(samples)
    tail = [s for s in got[len(got) // 2:] if s[0] is not None]
    if not tail:
        return None
    med = lambda v: float(np.median([x for x in v if x is not None])) if any(x is not None for x in v) else None  # noqa
    return {"socket_W": round(med([s[0] for s in tail]), 1), "sclk_MHz": med([s[1] for s in tail]),
            "samples": len(tail), "seconds": seconds,
            "source": "hwmon power1_input and the active pp_dpm_sclk level, median of the second half"}


_KEEP = []


def host_cpu():
    """Host CPU model and the cores this process may run on."""
    model = None
    for line in (_read("/proc/cpuinfo") or "").splitlines():
        if line.startswith("model name"):
            model = line.split(":", 1)[1].strip()
            break
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return model, affinity


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


REF_LIB = os.path.join(REPO, "oracle", "_ref", "libref.so")


def cpu_baseline_int8(n, rows, qa, qb):
    """The reference's own CPU gemm_int8 (src/ops_extended.c:124-129 ->
    gemm_int8_fallback :83-122, OpenMP over output elements), compiled from
    the reference sources into oracle/_ref/libref.so by oracle/Makefile, on a
    row slab of the same inputs; the oracle's restatement (same loop, same
    flags) when that build is absent.  Returns (TOP/s, seconds, kind)."""
    a = np.ascontiguousarray(qa[:rows])
    b = np.ascontiguousarray(qb)
    out = np.empty((rows, n), np.int32)
    if os.path.exists(REF_LIB):
        f = C.CDLL(REF_LIB).gemm_int8
        f.restype = None
        f.argtypes = [C.c_void_p] * 3 + [C.c_uint32] * 3 + [C.c_float] * 3 + [C.c_int32] * 2
        t0 = time.perf_counter()
        f(a.ctypes.data, b.ctypes.data, out.ctypes.data, rows, n, n, 1.0, 1.0, 1.0, 0, 0)
        kind = "reference"
    else:
        from oracle import Oracle

        orc = Oracle()
        t0 = time.perf_counter()
        orc.gemm_int8(a, b, rows, n, n)
        kind = "port"
    dt = time.perf_counter() - t0
    return 2.0 * rows * n * n / dt / 1e12, dt, kind


def _tensor(lib, arr, requires_grad=False):
    arr = np.ascontiguousarray(arr, np.float32)
    shape = (C.c_uint32 * arr.ndim)(*arr.shape)
    t = lib.tensor_create(arr.ndim, shape, requires_grad)
    C.memmove(t.contents.data, arr.ctypes.data, arr.nbytes)
    return t


def _cpu_ms(fn, reps=1):
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) * 1e3 / reps


def bench_configs(lib, stream, timer, steps, with_cpu):
    """BASELINE configs 0-3 on the device (inputs resident, HIP events on one
    stream), each with the oracle (the reference's CPU path restated, same
    flags, all host cores) timed on the same inputs or a stated row sample."""
    from oracle import Oracle

    orc = Oracle() if with_cpu else None
    out = {}
    sync = lambda: check(lib.rplhip_stream_synchronize(stream))  # noqa: E731

    # cfg 0: FP32 512^3 NN, U[-1,1]
    n = 512
    A = rpl_amd.fill_uniform(n * n, seed(0, 0)).reshape(n, n)
    B = rpl_amd.fill_uniform(n * n, seed(0, 1)).reshape(n, n)
    dA, dB, dC = DeviceBuffer.from_array(A), DeviceBuffer.from_array(B), DeviceBuffer(n * n * 4)
    f = lambda: check(lib.rplhip_sgemm(0, 0, n, n, n, 1.0, dA.ptr, n, dB.ptr, n, 0.0, dC.ptr, n, stream))  # noqa
    ms, _ = timer.time(f, steps * 5, 5)
    e = {"us": round(ms * 1e3, 2), "TFLOP/s": round(2 * n ** 3 / (ms * 1e-3) / 1e12, 2)}
    if orc:
        c = _cpu_ms(lambda: orc.sgemm(A, B, np.zeros((n, n), np.float32), n, n, n))
        e["cpu_ms"] = round(c, 2)
    out["cfg0_fp32_512"] = e

    # cfg 1: INT8 512^3: N(0,1) -> per-tensor symmetric quantize (both) ->
    # i8 GEMM with the fused fp32 dequant (scale_A * scale_B); a step is the
    # two quantizations and the GEMM.
    A = rpl_amd.fill_normal(n * n, seed(1, 0))
    B = rpl_amd.fill_normal(n * n, seed(1, 1))
    dA, dB = DeviceBuffer.from_array(A), DeviceBuffer.from_array(B)
    qA, qB, sA, sB = DeviceBuffer(n * n), DeviceBuffer(n * n), DeviceBuffer(4), DeviceBuffer(4)
    dY = DeviceBuffer(n * n * 4)

    def cfg1():
        check(lib.rplhip_quantize_symmetric(dA.ptr, n * n, qA.ptr, sA.ptr, stream))
        check(lib.rplhip_quantize_symmetric(dB.ptr, n * n, qB.ptr, sB.ptr, stream))
        check(lib.rplhip_gemm_int8_dequant(qA.ptr, sA.ptr, 0, qB.ptr, sB.ptr, 0, dY.ptr, n, n, n, stream))

    ms, _ = timer.time(cfg1, steps * 5, 5)
    e = {"us": round(ms * 1e3, 2), "TOP/s_incl_quantize": round(2 * n ** 3 / (ms * 1e-3) / 1e12, 2)}
    if orc:
        def cpu1():
            qa, sa = orc.quantize_symmetric(A)
            qb, sb = orc.quantize_symmetric(B)
            orc.gemm_int8(qa.reshape(n, n), qb.reshape(n, n), n, n, n)
        e["cpu_ms"] = round(_cpu_ms(cpu1), 2)
    out["cfg1_int8_512"] = e

    # cfg 2: MLP 784 -> 128 (ReLU) -> 10 training step at batch 4096 through
    # include/rpl.h (linear_forward, tensor_relu, tensor_mse_loss,
    # tensor_backward), every tensor GPU-resident; a step also zeroes the
    # parameter gradients and frees the step's tensors.
    Bt, IN, H, O = 4096, 784, 128, 10
    X = rpl_amd.fill_uniform(Bt * IN, seed(2, 0), 0.0, 1.0).reshape(Bt, IN)
    _, Y = rpl_amd.fill_labels(Bt, seed(2, 1), O)
    W1 = rpl_amd.fill_uniform(H * IN, seed(2, 2), -np.sqrt(6 / IN), np.sqrt(6 / IN)).reshape(H, IN)
    W2 = rpl_amd.fill_uniform(O * H, seed(2, 3), -np.sqrt(6 / H), np.sqrt(6 / H)).reshape(O, H)
    l1, l2 = lib.linear_create(IN, H), lib.linear_create(H, O)
    for layer, W in ((l1, W1), (l2, W2)):
        C.memmove(layer.contents.weight.contents.data, W.ctypes.data, W.nbytes)
        lib.tensor_fill(layer.contents.bias, 0.0)
        lib.tensor_to_gpu(layer.contents.weight)
        lib.tensor_to_gpu(layer.contents.bias)
    tX, tY = _tensor(lib, X), _tensor(lib, Y)
    lib.tensor_to_gpu(tX)
    lib.tensor_to_gpu(tY)
    params = (l1.contents.weight, l1.contents.bias, l2.contents.weight, l2.contents.bias)

    def cfg2():
        for t in params:
            lib.tensor_zero_grad(t)
        h = lib.linear_forward(l1, tX)
        a = lib.tensor_relu(h)
        o = lib.linear_forward(l2, a)
        loss = lib.tensor_mse_loss(o, tY)
        lib.tensor_backward(loss)
        for t in (loss, o, a, h):
            lib.tensor_free(t)

    for _ in range(3):
        cfg2()
    lib.rpl_gpu_synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        cfg2()
    lib.rpl_gpu_synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    err = lib.rpl_last_error()
    flop = 1_675_624_448
    e = {"us": round(ms * 1e3, 1), "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 3), "timing": "host clock, synced",
         "error": err.decode() if err else None}
    if orc:
        b = np.zeros(H, np.float32), np.zeros(O, np.float32)
        e["cpu_ms"] = round(_cpu_ms(lambda: orc.mlp_step(X, Y, W1, b[0], W2, b[1])), 1)
    out["cfg2_mlp_step_b4096"] = e

    # The same step followed by optimizer_sgd_step (momentum 0.9) on the
    # device: a whole training iteration with no host round trip.
    arr = (C.POINTER(rpl_amd.Tensor) * 4)(*params)
    opt = lib.optimizer_sgd_create(arr, 4, 0.05, 0.9, 0.0, 0.0, False)

    def cfg2_sgd():
        cfg2()
        lib.optimizer_sgd_step(opt)

    for _ in range(3):
        cfg2_sgd()
    lib.rpl_gpu_synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        cfg2_sgd()
    lib.rpl_gpu_synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    err = lib.rpl_last_error()
    out["cfg2_mlp_step_sgd_b4096"] = {"us": round(ms * 1e3, 1), "timing": "host clock, synced",
                                      "error": err.decode() if err else None}
    for layer in (l1, l2):
        lib.linear_free(layer)
    lib.tensor_free(tX)
    lib.tensor_free(tY)

    # cfg 3: INT8 linear layers, M=2048 tokens, K=4096, N in {4096, 11008}:
    # X N(0,1) quantized per token on the device each step, W N(0,0.02)
    # quantized per output channel once (weights), fused fp32 dequant.
    M, K = 2048, 4096
    X = rpl_amd.fill_normal(M * K, seed(3, 0)).reshape(M, K)
    dX, qX, sX = DeviceBuffer.from_array(X), DeviceBuffer(M * K), DeviceBuffer(M * 4)
    for N in (4096, 11008):
        W = rpl_amd.fill_normal(N * K, seed(3, 1), 0.0, 0.02).reshape(N, K)
        dW, qW, sW = DeviceBuffer.from_array(W), DeviceBuffer(N * K), DeviceBuffer(N * 4)
        check(lib.rplhip_quantize_per_channel(dW.ptr, N, K, qW.ptr, sW.ptr, stream))
        dY = DeviceBuffer(M * N * 4)
        gemm = lambda: check(lib.rplhip_linear_int8_dequant(qX.ptr, sX.ptr, 1, qW.ptr, sW.ptr, 1, dY.ptr, M, K, N,  # noqa
                                                            stream))
        check(lib.rplhip_quantize_per_channel(dX.ptr, M, K, qX.ptr, sX.ptr, stream))
        ms_g, _ = timer.time(gemm, steps * 2, 3)

        def step():
            check(lib.rplhip_quantize_per_channel(dX.ptr, M, K, qX.ptr, sX.ptr, stream))
            gemm()

        ms_s, _ = timer.time(step, steps * 2, 3)
        ops = 2.0 * M * N * K
        e = {"gemm_us": round(ms_g * 1e3, 2), "gemm_TOP/s": round(ops / (ms_g * 1e-3) / 1e12, 1),
             "step_us_incl_x_quantize": round(ms_s * 1e3, 2)}
        if orc:
            rows = 128
            sync()
            qx = qX.to_array(np.int8, (M, K))[:rows]
            qw = qW.to_array(np.int8, (N, K))
            c = _cpu_ms(lambda: orc.linear_int8(qx, qw, None, rows, K, N))
            e["cpu_TOP/s"] = round(2.0 * rows * N * K / (c * 1e-3) / 1e12, 4)
            e["cpu_sample"] = f"linear_int8 oracle on {rows} of {M} rows"
        out[f"cfg3_linear_int8_N{N}"] = e
        del dW, qW, sW, dY
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--n", type=int, default=8192)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--cpu-rows", type=int, default=512)
    ap.add_argument("--settle-ms", type=float, default=1000.0,
                    help="untimed gemm_int8 work before the first timed leg (power and clock are sampled during "
                         "it): the first ~100 ms of load on an idle MI355X run at boost clock and then through a "
                         "power-management dip")
    ap.add_argument("--only", choices=["int8", "int8-nt", "fp32", "skinny", "configs"],
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
    # Let the power state settle (measured: the first ~25 back-to-back calls
    # after idle run 496 -> 644 -> 515 us) so every leg sees steady state;
    # the socket power and shader clock are sampled meanwhile.
    power = {"int8": power_while(lib, stream, int8_step, args.settle_ms * 1e-3)}
    ms_i8 = wall_i8 = tops = ms_f32 = wall_f32 = tflops = float("nan")
    if want("int8"):
        # At 8192^3 gemm_int8 is exactly one kernel launch
        # (k_gemm_i8_pairs<kRequantUnit, BKN>, B [K,N] read in place), so
        # these HIP events on its stream time that kernel alone.
        log("bench: int8 gemm_int8 8192^3")
        ms_i8, wall_i8 = timer.time(int8_step, args.steps, args.warmup)
        tops = ops / (ms_i8 * 1e-3) / 1e12
    # The same kernel on B already [N,K] (linear_int8's layout, raw int32).
    nt = None
    if want("int8-nt") or args.only is None:
        log("bench: int8 NT kernel (linear_int8)")
        ms_nt, _ = timer.time(lambda: check(lib.rplhip_linear_int8(qA.ptr, qB.ptr, None, dC.ptr, n, n, n, stream)),
                              args.steps, args.warmup)
        nt = {"kernel": "k_gemm_i8_pairs<0, false>", "ms_per_launch": round(ms_nt, 4),
              "achieved": round(ops / (ms_nt * 1e-3) / 1e12, 2), "unit": "TOP/s"}

    # ---- FP32 8192^3 NN (tensor_gemm semantics, alpha=1, beta=0)
    dCf = DeviceBuffer(n * n * 4)
    check(lib.rplhip_memset(dCf.ptr, 0, n * n * 4, stream))

    def fp32_step():
        check(lib.rplhip_sgemm(0, 0, n, n, n, 1.0, dA.ptr, n, dB.ptr, n, 0.0, dCf.ptr, n, stream))

    if want("fp32"):
        log("bench: fp32 sgemm 8192^3")
        ms_f32, wall_f32 = timer.time(fp32_step, max(args.steps // 2, 3), 2)
        tflops = ops / (ms_f32 * 1e-3) / 1e12
        if args.only is None:
            power["fp32"] = power_while(lib, stream, fp32_step, 0.5)
            check(lib.rplhip_synchronize())

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
        # Measured device-to-device copy rate on the same rotation of
        # buffers (bytes read + written), the practical HBM ceiling.
        cp = [0]

        def copy():
            src, dst = Ws[cp[0] % nw], Ws[(cp[0] + 1) % nw]
            cp[0] += 1
            check(lib.rplhip_memcpy_dtod(dst.ptr, src.ptr, N * K, stream))

        ms_c, _ = timer.time(copy, 30, 5)
        copy_gbs = 2 * N * K / (ms_c * 1e-3) / 1e9
        skinny["copy"] = {"GB/s": round(copy_gbs, 1), "frac_hbm": round(copy_gbs / PEAK_HBM_GBS, 3),
                          "what": "hipMemcpyAsync device-to-device, 64 MiB, read + written bytes"}
        orc = None
        if not args.no_cpu:
            from oracle import Oracle
            orc = Oracle()
            qw_host = qB.to_array(np.int8, (N, K))
            qa_host = qA.to_array(np.int8, (16, K))
        for M in (1, 4, 16):
            it = [0]

            def sk():
                w = Ws[it[0] % nw]
                it[0] += 1
                check(lib.rplhip_linear_int8_dequant(qA.ptr, sx.ptr, 0, w.ptr, sw.ptr, 1, Y.ptr, M, K, N, stream))

            ms_s, _ = timer.time(sk, 60, 12)
            byts = N * K + M * K + M * N * 4 + N * 4 + 4
            gbs = byts / (ms_s * 1e-3) / 1e9
            skinny[f"M{M}"] = {"us": round(ms_s * 1e3, 2), "GB/s": round(gbs, 1),
                               "frac_hbm": round(gbs / PEAK_HBM_GBS, 3), "frac_copy": round(gbs / copy_gbs, 3)}
            if orc is not None:
                # The reference's CPU path on the same shape: linear_int8
                # (rpl_quantization.c:314-353) then the dequant.
                swh = np.full(N, scales[1], np.float32)

                def cpu_sk():
                    acc = orc.linear_int8(np.ascontiguousarray(qa_host[:M]), qw_host, None, M, K, N)
                    orc.dequant_acc(acc, np.float32([scales[0]]), False, swh, True)

                skinny[f"M{M}"]["cpu_ms"] = round(_cpu_ms(cpu_sk), 2)
        del Ws

    configs = None
    if n == 8192 and want("configs"):
        log("bench: configs 0-3")
        configs = bench_configs(lib, stream, timer, max(args.steps // 2, 5), not args.no_cpu)

    cpu = None
    if not args.no_cpu and args.only is None:
        log(f"bench: cpu baseline ({args.cpu_rows}-row slab)")
        qa = qA.to_array(np.int8, (n, n))
        qb = qB.to_array(np.int8, (n, n))
        cpu_tops, cpu_s, kind = cpu_baseline_int8(n, args.cpu_rows, qa, qb)
        model, affinity = host_cpu()
        threads = int(os.environ.get("OMP_NUM_THREADS") or affinity or 1)
        what = ("the reference's gemm_int8 (src/ops_extended.c:83-129, built from its sources with -O3 -fopenmp "
                "into oracle/_ref/libref.so)" if kind == "reference" else
                "oracle gemm_int8 (reference src/ops_extended.c:83-129 restated, -O3 -fopenmp)")
        cpu = {"value": round(cpu_tops, 6), "unit": "TOP/s", "cores": threads, "kind": kind,
               "sample": f"{what} on a {args.cpu_rows}x{n}x{n} row slab of the same quantized inputs, {cpu_s:.1f} s",
               "cpu_model": model, "affinity_cores": affinity,
               "threads": "OpenMP, OMP_NUM_THREADS (else every core in the affinity mask)"}

    # HBM/MALL bytes per launch of the roofline kernel, from the committed
    # FETCH_SIZE / WRITE_SIZE passes (scaled by a copy kernel of known size).
    traffic, traffic_kernel = None, "k_gemm_i8_pairs<4, true>"
    tpath = os.path.join(REPO, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            rec = json.load(f).get("gemm_int8_8192", {})
        traffic, traffic_kernel = rec.get("bytes_per_launch"), rec.get("kernel", traffic_kernel)

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
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TOP/s", "frac": round(tops / PEAK_INT8_TOPS, 4), "traffic": traffic,
                     "kernel": traffic_kernel, "ms_per_launch": round(ms_i8, 4)},
        "nt_kernel": nt,
        "roofline_fp32": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP32_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP32_TFLOPS, 4), "kernel": "k_sgemm_dma<false, false>"},
        "skinny_int8": skinny,
        "configs": configs,
        "cpu_baseline": cpu,
        "device": {"arch": arch.value.decode(), "cus": cus.value, "clock_mhz_max": clk.value // 1000},
        "power": power,
        "wall_s": {"int8": round(wall_i8, 3), "fp32": round(wall_f32, 3)},
        "settle_ms": args.settle_ms,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
