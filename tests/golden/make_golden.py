"""Generate tests/golden/golden.npz from the reference's own compiled sources.

Runs only where /root/reference is mounted: `make -C oracle ref` compiles the
reference's hot-path files (src/rpl_core.c, ops_extended.c,
rpl_quantization.c, rpl_nn.c, gemm_optimized.c, rpl_training.c) into
oracle/_ref/libref.so,
and this script calls them through ctypes on seeded inputs, recording inputs
and outputs.  The committed .npz is pure data (numpy arrays, no pickles);
tests/test_oracle.py checks the C restatement in oracle/ against it
bit-for-bit, and the GPU tests check the device path against the same data.

Inputs come from rpl_amd's counter-based generator (host-only C code), so
large cases are stored as a seed plus the SHA-256 of the reference output.

    python tests/golden/make_golden.py
"""
import ctypes as C
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import rpl_amd  # noqa: E402  (host-side generator + struct layouts only)
from rpl_amd import (FakeQuantize, HalfTensor, Linear, Optimizer, PerChannelQuantizedTensor,  # noqa: E402
                     QuantizationCalibrator, QuantizedTensor, SGDState, Tensor)
from oracle import REF_PATH  # noqa: E402

SEED_BASE = 0x52504C00  # seed(config, stream) = SEED_BASE + 16*config + stream


def seed(cfg, stream):
    return SEED_BASE + 16 * cfg + stream


def load_ref():
    if not os.path.exists(REF_PATH):
        sys.exit(f"{REF_PATH} missing: run `make -C oracle ref` where /root/reference is mounted")
    lib = C.CDLL(REF_PATH)
    PT, PQ = C.POINTER(Tensor), C.POINTER(QuantizedTensor)
    u32, i32, f32, b = C.c_uint32, C.c_int32, C.c_float, C.c_bool
    protos = {
        "tensor_create": (PT, [u32, C.POINTER(u32), b]),
        "tensor_free": (None, [PT]),
        "tensor_gemm": (None, [PT, PT, PT, f32, f32, b, b]),
        "tensor_matmul": (PT, [PT, PT]),
        "gemm_int8": (None, [C.c_void_p, C.c_void_p, C.c_void_p, u32, u32, u32, f32, f32, f32, i32, i32]),
        "tensor_quantize_int8": (PQ, [PT, f32, i32]),
        "tensor_quantize_int8_symmetric": (PQ, [PT]),
        "tensor_quantize_int8_asymmetric": (PQ, [PT]),
        "tensor_quantize_per_channel": (C.POINTER(PerChannelQuantizedTensor), [PT, u32]),
        "tensor_dequantize_int8": (PT, [PQ]),
        "tensor_get_min_max": (None, [PT, C.POINTER(f32), C.POINTER(f32)]),
        "quantized_tensor_free": (None, [PQ]),
        "linear_int8": (None, [PQ, PQ, PQ, C.c_void_p, u32, u32, u32]),
        "calibrator_create": (C.POINTER(QuantizationCalibrator), []),
        "calibrator_update": (None, [C.POINTER(QuantizationCalibrator), PT]),
        "calibrator_compute_params": (None, [C.POINTER(QuantizationCalibrator), b]),
        "linear_create": (C.POINTER(Linear), [u32, u32]),
        "linear_forward": (PT, [C.POINTER(Linear), PT]),
        "tensor_relu": (PT, [PT]),
        "tensor_mse_loss": (PT, [PT, PT]),
        "tensor_backward": (None, [PT]),
        "parallel_gemm_optimized": (None, [C.c_void_p, C.c_void_p, C.c_void_p, u32, u32, u32]),
        "optimizer_sgd_create": (C.POINTER(Optimizer), [C.POINTER(PT), u32, f32, f32, f32, f32, b]),
        "optimizer_sgd_step": (None, [C.POINTER(Optimizer)]),
        "tensor_sigmoid": (PT, [PT]),
        "tensor_tanh_inplace": (None, [PT]),
        "tensor_gelu_inplace": (None, [PT]),
        "scaled_dot_product_attention": (PT, [PT, PT, PT, PT, f32, b]),
        "tensor_to_half": (C.POINTER(HalfTensor), [PT]),
        "tensor_from_half": (PT, [C.POINTER(HalfTensor)]),
        "fake_quantize_create": (C.POINTER(FakeQuantize), []),
        "fake_quantize_forward": (PT, [C.POINTER(FakeQuantize), PT]),
    }
    for n, (r, a) in protos.items():
        f = getattr(lib, n)
        f.restype, f.argtypes = r, a
    return lib


class Ref:
    def __init__(self):
        self.lib = load_ref()

    def tensor(self, arr, requires_grad=False):
        arr = np.ascontiguousarray(arr, np.float32)
        shape = (C.c_uint32 * max(arr.ndim, 1))(*(arr.shape or (1,)))
        t = self.lib.tensor_create(max(arr.ndim, 1), shape, requires_grad)
        if arr.size:
            C.memmove(t.contents.data, arr.ctypes.data, arr.nbytes)
        return t

    @staticmethod
    def data(t):
        n = t.contents.size
        return np.ctypeslib.as_array(t.contents.data, shape=(n,)).copy()

    @staticmethod
    def grad(t):
        n = t.contents.size
        return np.ctypeslib.as_array(t.contents.grad, shape=(n,)).copy()

    @staticmethod
    def qdata(q):
        return np.ctypeslib.as_array(q.contents.data, shape=(q.contents.size,)).copy()


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    ref = Ref()
    L = ref.lib
    g = {}

    # ---- tensor_gemm, all transposes, alpha/beta (rpl_core.c:199-217)
    M, N, K = 37, 29, 53
    for name, ta, tb in (("nn", 0, 0), ("nt", 0, 1), ("tn", 1, 0), ("tt", 1, 1)):
        A = rpl_amd.fill_uniform(M * K, seed(90, 0)).reshape((K, M) if ta else (M, K))
        B = rpl_amd.fill_uniform(K * N, seed(90, 1)).reshape((N, K) if tb else (K, N))
        C0 = rpl_amd.fill_uniform(M * N, seed(90, 2)).reshape(M, N)
        tA, tB, tC = ref.tensor(A), ref.tensor(B), ref.tensor(C0)
        L.tensor_gemm(tC, tA, tB, 0.75, -0.5, bool(ta), bool(tb))
        g[f"sgemm_{name}_A"], g[f"sgemm_{name}_B"], g[f"sgemm_{name}_C0"] = A, B, C0
        g[f"sgemm_{name}_C"] = ref.data(tC).reshape(M, N)
        for t in (tA, tB, tC):
            L.tensor_free(t)
    # beta = 0 still reads C: a NaN in C propagates (rpl_core.c:214)
    A = np.arange(16, dtype=np.float32).reshape(4, 4) / 7
    C0 = np.zeros((4, 4), np.float32)
    C0[1, 2] = np.nan
    tA, tB, tC = ref.tensor(A), ref.tensor(A), ref.tensor(C0)
    L.tensor_gemm(tC, tA, tB, 1.0, 0.0, False, False)
    g["sgemm_nan_A"], g["sgemm_nan_C0"], g["sgemm_nan_C"] = A, C0, ref.data(tC).reshape(4, 4)
    for t in (tA, tB, tC):
        L.tensor_free(t)

    # ---- tensor_gemm on multi_head_attention_forward's 3-D projections
    # (rpl_attention.c:175-177,232): C [b,s,d] zero-filled, A [b,s,d],
    # W [d,d], trans_b, alpha 1, beta 0.  tensor_gemm reads shape[0..1] only,
    # so M = b, K = s, N = d: it multiplies the first b*s values of A, taken
    # as a [b,s] matrix, by the first d*s values of W, taken as [d,s], into
    # the first b*d values of C; every read stays in bounds when s <= d.
    for name, (bb, ss, dd) in (("mha_s5_d8", (2, 5, 8)), ("mha_s8_d8", (3, 8, 8)), ("mha_s3_d16", (4, 3, 16))):
        X3 = rpl_amd.fill_uniform(bb * ss * dd, seed(90, 3)).reshape(bb, ss, dd)
        W = rpl_amd.fill_uniform(dd * dd, seed(90, 4)).reshape(dd, dd)
        tX, tW = ref.tensor(X3), ref.tensor(W)
        tC = ref.tensor(np.zeros((bb, ss, dd), np.float32))
        L.tensor_gemm(tC, tX, tW, 1.0, 0.0, False, True)
        g[f"sgemm3d_{name}_A"], g[f"sgemm3d_{name}_W"] = X3, W
        g[f"sgemm3d_{name}_C"] = ref.data(tC).reshape(bb, ss, dd)
        for t in (tX, tW, tC):
            L.tensor_free(t)

    # ---- parallel_gemm_optimized at N == 4, where the reference kernel is
    # correct (C += A*B); pins the entry point's intended semantics.
    M, N, K = 8, 4, 16
    A = rpl_amd.fill_uniform(M * K, seed(91, 0)).reshape(M, K)
    B = rpl_amd.fill_uniform(K * N, seed(91, 1)).reshape(K, N)
    C0 = rpl_amd.fill_uniform(M * N, seed(91, 2)).reshape(M, N)
    Cg = C0.copy()
    L.parallel_gemm_optimized(A.ctypes.data, B.ctypes.data, Cg.ctypes.data, M, N, K)
    g["gemmopt_A"], g["gemmopt_B"], g["gemmopt_C0"], g["gemmopt_C"] = A, B, C0, Cg

    # ---- gemm_int8 (ops_extended.c:83-129)
    rng = np.random.default_rng(seed(92, 0))
    cases = []
    M, N, K = 33, 47, 129
    A8 = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B8 = rng.integers(-128, 128, (K, N), dtype=np.int8)
    cases.append(("zp", A8, B8, 0.01, 0.02, 0.5, 3, -5))
    cases.append(("unit", A8, B8, 1.0, 1.0, 1.0, 0, 0))
    full = np.full((2, 1041), 127, np.int8)
    cases.append(("k1041", full, np.ascontiguousarray(full.T), 1.0, 1.0, 1.0, 0, 0))  # 16790289 -> 16790288
    cases.append(("overflow", A8, B8, 1e20, 1e20, 1.0, 0, 0))  # +-inf -> INT_MIN
    cases.append(("sc0", A8, B8, 1.0, 1.0, 0.0, 0, 0))  # x/0 -> inf or NaN -> INT_MIN
    cases.append(("tiny", A8[:1, :7], B8[:7, :3], 0.3, 0.7, 0.11, 0, 0))
    for name, a, b, sa, sb, sc, za, zb in cases:
        a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
        m, k = a.shape
        n = b.shape[1]
        out = np.zeros((m, n), np.int32)
        L.gemm_int8(a.ctypes.data, b.ctypes.data, out.ctypes.data, m, n, k, sa, sb, sc, za, zb)
        g[f"i8_{name}_A"], g[f"i8_{name}_B"], g[f"i8_{name}_C"] = a, b, out
        g[f"i8_{name}_params"] = np.array([sa, sb, sc], np.float32)
        g[f"i8_{name}_zp"] = np.array([za, zb], np.int32)

    # ---- tensor_quantize_int8 (rpl_core.c:511-530): ties, casts, clamps
    special = np.array([0.5, 1.5, 2.5, -0.5, -2.5, 1e10, -1e10, np.nan, np.inf, -np.inf, 127.4, 127.5,
                        -128.5, -127.5, 0.0, -0.0, 3.49999976, 1e-30, 2.5e9, -2.2e9], np.float32)
    for i, (scale, zp) in enumerate(((1.0, 0), (0.3, 3), (1.0, -7), (0.0, 0), (2.0, 300))):
        t = ref.tensor(special)
        q = L.tensor_quantize_int8(t, scale, zp)
        g[f"q_special_{i}"] = ref.qdata(q)
        g[f"q_special_{i}_params"] = np.array([scale, zp], np.float64)
        L.quantized_tensor_free(q)
        L.tensor_free(t)
    g["q_special_x"] = special

    # ---- symmetric / asymmetric (rpl_quantization.c:77-107)
    xs = {
        "normal": rpl_amd.fill_normal(4099, seed(93, 0)),
        "uniform": rpl_amd.fill_uniform(1000, seed(93, 1), -1.0, 3.0),
        "zeros": np.zeros(64, np.float32),
        "ties": np.array([127.0, 63.5, -63.5, 0.5, -0.5, 1.5, 31.75], np.float32),
    }
    for name, x in xs.items():
        t = ref.tensor(x)
        q = L.tensor_quantize_int8_symmetric(t)
        g[f"sym_{name}_x"], g[f"sym_{name}_q"] = x, ref.qdata(q)
        g[f"sym_{name}_scale"] = np.array([q.contents.scale], np.float32)
        L.quantized_tensor_free(q)
        q = L.tensor_quantize_int8_asymmetric(t)
        g[f"asym_{name}_q"] = ref.qdata(q)
        g[f"asym_{name}_scale"] = np.array([q.contents.scale], np.float32)
        g[f"asym_{name}_zp"] = np.array([q.contents.zero_point], np.int32)
        L.quantized_tensor_free(q)
        L.tensor_free(t)

    # ---- per-channel (rpl_quantization.c:120-160), incl. the axis quirk
    pcs = {
        "known": (np.array([[1, -2, 4], [0.5, 0.25, -1]], np.float32), 0),
        "rows": (rpl_amd.fill_normal(16 * 100, seed(94, 0)).reshape(16, 100), 0),
        "axis1": (rpl_amd.fill_normal(6 * 10, seed(94, 1)).reshape(6, 10), 1),
        "zero_row": (np.vstack([np.zeros(8, np.float32), np.linspace(-1, 1, 8, dtype=np.float32)]), 0),
    }
    for name, (x, axis) in pcs.items():
        t = ref.tensor(x)
        p = L.tensor_quantize_per_channel(t, axis)
        nc = p.contents.num_channels
        g[f"pc_{name}_x"] = x
        g[f"pc_{name}_axis"] = np.array([axis], np.int32)
        g[f"pc_{name}_q"] = np.ctypeslib.as_array(p.contents.data, shape=(x.size,)).copy()
        g[f"pc_{name}_scales"] = np.ctypeslib.as_array(p.contents.scales, shape=(nc,)).copy()
        L.tensor_free(t)  # per-channel struct leaks in this short-lived script

    # ---- dequantize (ops_extended.c:64-73)
    q = np.random.default_rng(seed(95, 0)).integers(-128, 128, 333, dtype=np.int8)
    for i, (scale, zp) in enumerate(((0.05, 0), (0.0123, 7), (3.0, -128))):
        t = ref.tensor(np.zeros(333, np.float32))
        qt = L.tensor_quantize_int8(t, 1.0, 0)
        C.memmove(qt.contents.data, q.ctypes.data, 333)
        qt.contents.scale, qt.contents.zero_point = scale, zp
        y = L.tensor_dequantize_int8(qt)
        g[f"dq_{i}_y"] = ref.data(y)
        g[f"dq_{i}_params"] = np.array([scale, zp], np.float64)
        L.tensor_free(y)
        L.quantized_tensor_free(qt)
        L.tensor_free(t)
    g["dq_q"] = q

    # ---- tensor_get_min_max (ops_extended.c:52-61)
    mms = {
        "normal": rpl_amd.fill_normal(777, seed(96, 0)),
        "nan_first": np.array([np.nan, 1.0, -2.0, 3.0], np.float32),
        "nan_later": np.array([1.0, np.nan, -2.0, 3.0, np.nan], np.float32),
        "zeros": np.array([0.0, -0.0, 0.0, -0.0], np.float32),
        "negzero_first": np.array([-0.0, 0.0, 1.0, 0.0], np.float32),
        "inf": np.array([np.inf, np.inf], np.float32),
    }
    for name, x in mms.items():
        t = ref.tensor(x)
        mn, mx = C.c_float(0), C.c_float(0)
        L.tensor_get_min_max(t, C.byref(mn), C.byref(mx))
        g[f"mm_{name}_x"] = x
        g[f"mm_{name}_out"] = np.array([mn.value, mx.value], np.float32)
        L.tensor_free(t)

    # ---- linear_int8 (rpl_quantization.c:314-353)
    rng = np.random.default_rng(seed(97, 0))
    for name, (m, k, n, with_bias) in {"bias": (5, 67, 9, True), "nobias": (17, 64, 33, False),
                                         "m1": (1, 200, 40, True)}.items():
        x = rng.integers(-128, 128, (m, k), dtype=np.int8)
        w = rng.integers(-128, 128, (n, k), dtype=np.int8)
        bias = rng.integers(-128, 128, n, dtype=np.int8)
        qs = []
        for arr in (x, w, bias):
            t = ref.tensor(np.zeros(arr.size, np.float32))
            qt = L.tensor_quantize_int8(t, 1.0, 0)
            C.memmove(qt.contents.data, arr.ctypes.data, arr.size)
            qs.append(qt)
            L.tensor_free(t)
        out = np.zeros((m, n), np.int32)
        L.linear_int8(qs[0], qs[1], qs[2] if with_bias else None, out.ctypes.data, m, k, n)
        g[f"lin8_{name}_x"], g[f"lin8_{name}_w"], g[f"lin8_{name}_out"] = x, w, out
        if with_bias:
            g[f"lin8_{name}_bias"] = bias
        for qt in qs:
            L.quantized_tensor_free(qt)

    # ---- calibrator (rpl_quantization.c:26-67)
    c1 = rpl_amd.fill_normal(300, seed(98, 0))
    c2 = rpl_amd.fill_uniform(200, seed(98, 1), -4.0, 0.5)
    for sym in (True, False):
        cal = L.calibrator_create()
        for x in (c1, c2):
            t = ref.tensor(x)
            L.calibrator_update(cal, t)
            L.tensor_free(t)
        L.calibrator_compute_params(cal, sym)
        c = cal.contents
        g[f"cal_{int(sym)}"] = np.array([c.min_val, c.max_val, c.scale], np.float32)
        g[f"cal_{int(sym)}_zp"] = np.array([c.zero_point, c.num_samples], np.int32)
    g["cal_x1"], g["cal_x2"] = c1, c2

    # ---- MLP training step through the reference's Linear + autograd
    B, IN, H, O = 64, 20, 16, 10
    X = rpl_amd.fill_uniform(B * IN, seed(2, 0), 0.0, 1.0).reshape(B, IN)
    labels, Y = rpl_amd.fill_labels(B, seed(2, 1), O)
    W1 = rpl_amd.fill_uniform(H * IN, seed(2, 2), -np.sqrt(6 / IN), np.sqrt(6 / IN)).reshape(H, IN)
    W2 = rpl_amd.fill_uniform(O * H, seed(2, 3), -np.sqrt(6 / H), np.sqrt(6 / H)).reshape(O, H)
    b1 = rpl_amd.fill_uniform(H, seed(2, 4), -0.1, 0.1)
    b2 = rpl_amd.fill_uniform(O, seed(2, 5), -0.1, 0.1)
    l1, l2 = L.linear_create(IN, H), L.linear_create(H, O)
    for layer, W, bb in ((l1, W1, b1), (l2, W2, b2)):
        C.memmove(layer.contents.weight.contents.data, W.ctypes.data, W.nbytes)
        C.memmove(layer.contents.bias.contents.data, bb.ctypes.data, bb.nbytes)
    tX, tY = ref.tensor(X), ref.tensor(Y)
    h = L.linear_forward(l1, tX)
    a = L.tensor_relu(h)
    o = L.linear_forward(l2, a)
    loss = L.tensor_mse_loss(o, tY)
    L.tensor_backward(loss)
    g.update(mlp_X=X, mlp_Y=Y, mlp_W1=W1, mlp_W2=W2, mlp_b1=b1, mlp_b2=b2)
    g["mlp_loss"] = ref.data(loss)
    g["mlp_o"] = ref.data(o).reshape(B, O)
    g["mlp_dW1"] = ref.grad(l1.contents.weight).reshape(H, IN)
    g["mlp_db1"] = ref.grad(l1.contents.bias)
    g["mlp_dW2"] = ref.grad(l2.contents.weight).reshape(O, H)
    g["mlp_db2"] = ref.grad(l2.contents.bias)

    # ---- backward_matmul's layout guess on a square, non-transposed B
    A = np.array([[1, 2], [3, 4]], np.float32)
    Bm = np.array([[5, 6], [7, 8]], np.float32)
    tA, tB = ref.tensor(A, True), ref.tensor(Bm, True)
    out = L.tensor_matmul(tA, tB)
    L.tensor_backward(out)
    g["bmm_A"], g["bmm_B"] = A, Bm
    g["bmm_out"] = ref.data(out).reshape(2, 2)
    g["bmm_dA"], g["bmm_dB"] = ref.grad(tA).reshape(2, 2), ref.grad(tB).reshape(2, 2)

    # ---- optimizer_sgd_step (rpl_training.c:70-114): two parameter tensors,
    # two steps each; grad is modified in place (weight decay, Nesterov).
    rng = np.random.default_rng(seed(5, 0))
    shapes = [(37, 53), (53,)]
    cases = {"plain": (0.1, 0.0, 0.0, 0.0, False), "wd": (0.05, 0.0, 0.0, 1e-2, False),
             "mom": (0.03, 0.9, 0.0, 0.0, False), "nest": (0.02, 0.9, 0.1, 5e-4, True)}
    for name, (lr, mom, damp, wd, nest) in cases.items():
        ps = [ref.tensor(rng.uniform(-1, 1, s).astype(np.float32), requires_grad=True) for s in shapes]
        arr = (C.POINTER(Tensor) * len(ps))(*ps)
        opt = L.optimizer_sgd_create(arr, len(ps), lr, mom, damp, wd, nest)
        for k, t in enumerate(ps):
            g[f"sgd_{name}_p{k}_init"] = ref.data(t)
        for step in range(2):
            for k, t in enumerate(ps):
                gr = (rng.standard_normal(t.contents.size) * 0.1).astype(np.float32)
                C.memmove(t.contents.grad, gr.ctypes.data, gr.nbytes)
                g[f"sgd_{name}_s{step}_g{k}_in"] = gr
            L.optimizer_sgd_step(opt)
            st = C.cast(opt.contents.state, C.POINTER(SGDState)).contents
            for k, t in enumerate(ps):
                g[f"sgd_{name}_s{step}_p{k}"] = ref.data(t)
                g[f"sgd_{name}_s{step}_g{k}"] = ref.grad(t)
                if mom:
                    g[f"sgd_{name}_s{step}_v{k}"] = ref.data(st.velocity[k])
        g[f"sgd_{name}_hyper"] = np.array([lr, mom, damp, wd, float(nest)], np.float32)

    # ---- activations of the device seam, CPU formulas (rpl_core.c:302-304,
    # 490-497): uniform inputs plus specials (signed zeros, subnormals, the
    # exp overflow edges, +-inf, NaN, huge values).
    rng = np.random.default_rng(seed(6, 0))
    specials = np.array([0.0, -0.0, 1e-40, -1e-40, 1e-8, -1e-8, 88.7, -88.7, 88.8, -88.8, 100.0, -100.0,
                         np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 0.5, -0.5, 3.0, -3.0], np.float32)
    xa = np.concatenate([rng.uniform(-12, 12, 4096).astype(np.float32), specials])
    g["act_x"] = xa
    t = ref.tensor(xa)
    g["act_sigmoid"] = ref.data(L.tensor_sigmoid(t))
    for kind in ("tanh", "gelu"):
        t = ref.tensor(xa)
        getattr(L, f"tensor_{kind}_inplace")(t)
        g[f"act_{kind}"] = ref.data(t)

    # ---- scaled_dot_product_attention (rpl_attention.c:16-111), with and
    # without a mask (a 0/1 pattern plus one fully masked row).
    rng = np.random.default_rng(seed(7, 0))
    for name, (B, Sq, Sk, dk, dv) in {"small": (2, 5, 7, 8, 6), "mid": (3, 33, 65, 64, 32)}.items():
        Q = rng.standard_normal((B, Sq, dk)).astype(np.float32)
        Kt = rng.standard_normal((B, Sk, dk)).astype(np.float32)
        V = rng.standard_normal((B, Sk, dv)).astype(np.float32)
        mask = (rng.random((B, Sq, Sk)) < 0.7).astype(np.float32)
        mask[0, Sq - 1, :] = 0.0
        g.update({f"att_{name}_Q": Q, f"att_{name}_K": Kt, f"att_{name}_V": V, f"att_{name}_mask": mask})
        for masked in (False, True):
            o = L.scaled_dot_product_attention(ref.tensor(Q), ref.tensor(Kt), ref.tensor(V),
                                               ref.tensor(mask) if masked else None, 0.0, False)
            g[f"att_{name}_out{'_m' if masked else ''}"] = ref.data(o).reshape(B, Sq, dv)

    # ---- FP16 codec (rpl_half.c:10-107): every half value, and floats over
    # every exponent with mantissas at the truncation boundaries, both signs,
    # NaN payloads, plus random bit patterns.
    hh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ht = HalfTensor()
    ht.data = hh.ctypes.data_as(C.POINTER(C.c_uint16))
    ht.dims, ht.size, ht.device = 1, hh.size, 0
    ht.shape[0] = hh.size
    g["half_all_f32"] = ref.data(L.tensor_from_half(C.byref(ht)))
    mant = np.array([0, 1, 0x0FFF, 0x1000, 0x1FFF, 0x2000, 0x2001, 0x3FFF, 0x400000, 0x7FE000, 0x7FFFFF], np.uint32)
    bits = ((np.arange(256, dtype=np.uint32)[:, None] << 23) | mant[None, :]).ravel()
    bits = np.concatenate([bits, bits | 0x80000000, rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32)])
    fx = bits.view(np.float32)
    th = L.tensor_to_half(ref.tensor(fx))
    g["half_from_f32_x"] = fx
    g["half_from_f32_h"] = np.ctypeslib.as_array(th.contents.data, shape=(fx.size,)).copy()

    # ---- fake_quantize_forward (rpl_quantization.c:195-237): two training
    # steps (scale / zero-point moving averages) and one eval step.
    fq = L.fake_quantize_create()
    steps = [((rng.standard_normal(1000) * 3).astype(np.float32), True),
             ((rng.standard_normal(1000) * 2 + 1).astype(np.float32), True),
             ((rng.standard_normal(1000) * 4).astype(np.float32), False)]
    for step, (x, train) in enumerate(steps):
        fq.contents.training = train
        y = L.fake_quantize_forward(fq, ref.tensor(x))
        g[f"fq_{step}_x"] = x
        g[f"fq_{step}_y"] = ref.data(y)
        g[f"fq_{step}_state"] = np.float32([fq.contents.scale.contents.data[0],
                                            fq.contents.zero_point.contents.data[0], float(train)])

    # ---- configs 0 and 1 at 512^3: hashes of the reference outputs
    n = 512
    A = rpl_amd.fill_uniform(n * n, seed(0, 0)).reshape(n, n)
    Bm = rpl_amd.fill_uniform(n * n, seed(0, 1)).reshape(n, n)
    tA, tB = ref.tensor(A), ref.tensor(Bm)
    tC = L.tensor_matmul(tA, tB)
    Cc = ref.data(tC)
    g["cfg0_sha"] = np.frombuffer(sha(Cc).encode(), np.uint8)
    g["cfg0_sample"] = Cc[:4096]
    A = rpl_amd.fill_normal(n * n, seed(1, 0)).reshape(n, n)
    Bm = rpl_amd.fill_normal(n * n, seed(1, 1)).reshape(n, n)
    tA, tB = ref.tensor(A), ref.tensor(Bm)
    qa, qb = L.tensor_quantize_int8_symmetric(tA), L.tensor_quantize_int8_symmetric(tB)
    qA, qB = ref.qdata(qa), ref.qdata(qb)
    acc = np.zeros((n, n), np.int32)
    L.gemm_int8(qA.ctypes.data, qB.ctypes.data, acc.ctypes.data, n, n, n, 1.0, 1.0, 1.0, 0, 0)
    g["cfg1_scales"] = np.array([qa.contents.scale, qb.contents.scale], np.float32)
    g["cfg1_qA_sha"] = np.frombuffer(sha(qA).encode(), np.uint8)
    g["cfg1_qB_sha"] = np.frombuffer(sha(qB).encode(), np.uint8)
    g["cfg1_acc_sha"] = np.frombuffer(sha(acc).encode(), np.uint8)
    g["cfg1_acc_sample"] = acc[:8].copy()

    out = os.path.join(HERE, "golden.npz")
    np.savez_compressed(out, **g)
    print(f"wrote {out}: {len(g)} arrays, {os.path.getsize(out)} bytes")


if __name__ == "__main__":
    main()
