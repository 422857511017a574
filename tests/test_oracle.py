"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Three kinds of pins, chosen so that a plausible slip in the restatement (a
dropped term, a wrong index or transpose, a different rounding) fails one:
  1. golden vectors produced by the reference's own compiled sources
     (tests/golden/make_golden.py), compared bit-for-bit;
  2. the compiled reference itself (oracle/_ref, where it was built) on
     fresh seeded inputs, bit-for-bit;
  3. mathematics: closed forms, exact integer brute force, float64 bounds,
     the reference's own known answers (tests/full_system_check.py:33-37:
     eye @ ones == ones; examples/gpu_test.c:106-128: ones @ I == 1).
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import bits_equal, gemm_err_ratio, seed

import oracle as oracle_mod


# --------------------------------------------------------------- golden

@pytest.mark.parametrize("name,ta,tb", [("nn", 0, 0), ("nt", 0, 1), ("tn", 1, 0), ("tt", 1, 1)])
def test_sgemm_golden(orc, golden, name, ta, tb):
    A, B, C0 = golden[f"sgemm_{name}_A"], golden[f"sgemm_{name}_B"], golden[f"sgemm_{name}_C0"]
    M, N = C0.shape
    K = A.shape[0] if ta else A.shape[1]
    out = orc.sgemm(A, B, C0, M, N, K, 0.75, -0.5, bool(ta), bool(tb))
    assert bits_equal(out, golden[f"sgemm_{name}_C"])


def test_sgemm_nan_in_c_propagates(orc, golden):
    A, C0 = golden["sgemm_nan_A"], golden["sgemm_nan_C0"]
    out = orc.sgemm(A, A, C0, 4, 4, 4, 1.0, 0.0)
    assert bits_equal(out, golden["sgemm_nan_C"])
    assert np.isnan(out[1, 2]) and np.isfinite(out[0, 0])


MHA_CASES = ["mha_s5_d8", "mha_s8_d8", "mha_s3_d16"]


@pytest.mark.parametrize("name", MHA_CASES)
def test_sgemm_3d_projection_golden(orc, golden, name):
    # tensor_gemm on multi_head_attention_forward's [b,s,d] tensors
    # (rpl_attention.c:175-177): M = b, K = s, N = d from shape[0..1], the
    # first b*s values of A against the first d*s of W, into the first b*d
    # values of C; the rest of C keeps its zeros.
    A, W, want = golden[f"sgemm3d_{name}_A"], golden[f"sgemm3d_{name}_W"], golden[f"sgemm3d_{name}_C"]
    b, s, d = A.shape
    out = orc.sgemm(A.reshape(-1)[:b * s], W.reshape(-1)[:d * s], np.zeros((b, d), np.float32), b, d, s, tb=True)
    assert bits_equal(out.reshape(-1), want.reshape(-1)[:b * d])
    assert not want.reshape(-1)[b * d:].any()
    # The same product in float64 (closed form of the dense reading).
    ref = A.reshape(-1)[:b * s].astype(np.float64).reshape(b, s) @ W.reshape(-1)[:d * s].astype(np.float64).reshape(d, s).T
    assert np.max(np.abs(out - ref)) <= 1e-6 * s


def test_gemm_optimized_intended_semantics(orc, golden):
    # parallel_gemm_optimized is C += A*B: tensor_gemm with alpha = beta = 1.
    A, B, C0 = golden["gemmopt_A"], golden["gemmopt_B"], golden["gemmopt_C0"]
    out = orc.sgemm(A, B, C0, 8, 4, 16, 1.0, 1.0)
    assert gemm_err_ratio(out, A, B, golden["gemmopt_C"]) < 1e-6


@pytest.mark.parametrize("case", ["zp", "unit", "k1041", "overflow", "sc0", "tiny"])
def test_gemm_int8_golden(orc, golden, case):
    A, B = golden[f"i8_{case}_A"], golden[f"i8_{case}_B"]
    sa, sb, sc = (float(v) for v in golden[f"i8_{case}_params"])
    za, zb = (int(v) for v in golden[f"i8_{case}_zp"])
    M, K = A.shape
    N = B.shape[1]
    assert bits_equal(orc.gemm_int8(A, B, M, N, K, sa, sb, sc, za, zb), golden[f"i8_{case}_C"])


def test_quantize_special_golden(orc, golden):
    x = golden["q_special_x"]
    for i in range(5):
        scale, zp = golden[f"q_special_{i}_params"]
        assert bits_equal(orc.quantize_int8(x, float(scale), int(zp)), golden[f"q_special_{i}"]), i


@pytest.mark.parametrize("name", ["normal", "uniform", "zeros", "ties"])
def test_quantize_sym_asym_golden(orc, golden, name):
    x = golden[f"sym_{name}_x"]
    q, s = orc.quantize_symmetric(x)
    assert bits_equal(q, golden[f"sym_{name}_q"]) and bits_equal(np.float32([s]), golden[f"sym_{name}_scale"])
    q, s, z = orc.quantize_asymmetric(x)
    assert bits_equal(q, golden[f"asym_{name}_q"])
    assert bits_equal(np.float32([s]), golden[f"asym_{name}_scale"])
    assert z == int(golden[f"asym_{name}_zp"][0])


@pytest.mark.parametrize("name", ["known", "rows", "axis1", "zero_row"])
def test_per_channel_golden(orc, golden, name):
    x = golden[f"pc_{name}_x"]
    axis = int(golden[f"pc_{name}_axis"][0])
    q, s = orc.quantize_per_channel(x, x.shape[axis])
    assert bits_equal(q.reshape(-1), golden[f"pc_{name}_q"])
    assert bits_equal(s, golden[f"pc_{name}_scales"])


def test_dequantize_golden(orc, golden):
    for i in range(3):
        scale, zp = golden[f"dq_{i}_params"]
        assert bits_equal(orc.dequantize_int8(golden["dq_q"], float(scale), int(zp)), golden[f"dq_{i}_y"])


@pytest.mark.parametrize("name", ["normal", "nan_first", "nan_later", "zeros", "negzero_first", "inf"])
def test_get_min_max_golden(orc, golden, name):
    mn, mx = orc.get_min_max(golden[f"mm_{name}_x"])
    assert bits_equal(np.float32([mn, mx]), golden[f"mm_{name}_out"])


@pytest.mark.parametrize("name", ["bias", "nobias", "m1"])
def test_linear_int8_golden(orc, golden, name):
    x, w = golden[f"lin8_{name}_x"], golden[f"lin8_{name}_w"]
    bias = golden.get(f"lin8_{name}_bias")
    M, K = x.shape
    N = w.shape[0]
    assert bits_equal(orc.linear_int8(x, w, bias, M, K, N), golden[f"lin8_{name}_out"])


def test_calibrator_golden(orc, golden):
    for sym in (1, 0):
        mn, mx, s, z = orc.calibrate([golden["cal_x1"], golden["cal_x2"]], bool(sym))
        assert bits_equal(np.float32([mn, mx, s]), golden[f"cal_{sym}"])
        assert z == int(golden[f"cal_{sym}_zp"][0])


def test_mlp_step_golden(orc, golden):
    r = orc.mlp_step(golden["mlp_X"], golden["mlp_Y"], golden["mlp_W1"], golden["mlp_b1"], golden["mlp_W2"],
                     golden["mlp_b2"])
    assert bits_equal(np.float32([r["loss"]]), golden["mlp_loss"])
    for k in ("o", "dW1", "db1", "dW2", "db2"):
        assert bits_equal(r[k], golden[f"mlp_{k}"]), k


def test_backward_matmul_layout_guess_golden(orc, golden):
    A, B = golden["bmm_A"], golden["bmm_B"]
    dt = np.ones((2, 2), np.float32)
    da, db = orc.matmul_backward(dt, A, B, 2, 2, 2, B.shape, da=np.zeros((2, 2)), db=np.zeros((2, 2)))
    assert bits_equal(da, golden["bmm_dA"]) and bits_equal(db, golden["bmm_dB"])
    np.testing.assert_array_equal(da, [[12, 14], [12, 14]])  # not the true [[11, 15], [11, 15]]


def test_config0_config1_hashes(orc, golden, rpl):
    import hashlib

    import rpl_amd

    n = 512
    A = rpl_amd.fill_uniform(n * n, seed(0, 0)).reshape(n, n)
    B = rpl_amd.fill_uniform(n * n, seed(0, 1)).reshape(n, n)
    out = orc.sgemm(A, B, np.zeros((n, n), np.float32), n, n, n)
    assert hashlib.sha256(out.tobytes()).hexdigest().encode() == golden["cfg0_sha"].tobytes()
    A = rpl_amd.fill_normal(n * n, seed(1, 0))
    B = rpl_amd.fill_normal(n * n, seed(1, 1))
    qa, sa = orc.quantize_symmetric(A)
    qb, sb = orc.quantize_symmetric(B)
    assert bits_equal(np.float32([sa, sb]), golden["cfg1_scales"])
    assert hashlib.sha256(qa.tobytes()).hexdigest().encode() == golden["cfg1_qA_sha"].tobytes()
    assert hashlib.sha256(qb.tobytes()).hexdigest().encode() == golden["cfg1_qB_sha"].tobytes()
    acc = orc.gemm_int8(qa.reshape(n, n), qb.reshape(n, n), n, n, n)
    assert hashlib.sha256(acc.tobytes()).hexdigest().encode() == golden["cfg1_acc_sha"].tobytes()


# ------------------------------------------------- the compiled reference

@pytest.fixture(scope="module")
def reflib():
    if not oracle_mod.ref_available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    lib = C.CDLL(oracle_mod.REF_PATH)
    lib.gemm_int8.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p] + [C.c_uint32] * 3 + [C.c_float] * 3 + [C.c_int32] * 2
    lib.gemm_int8.restype = None
    return lib


def test_gemm_int8_vs_reference_build(orc, reflib):
    rng = np.random.default_rng(7)
    for (M, N, K, za, zb) in [(19, 23, 301, 0, 0), (64, 3, 77, -2, 9), (2, 130, 1024, 128, -128)]:
        A = rng.integers(-128, 128, (M, K), dtype=np.int8)
        B = rng.integers(-128, 128, (K, N), dtype=np.int8)
        out = np.zeros((M, N), np.int32)
        reflib.gemm_int8(A.ctypes.data, B.ctypes.data, out.ctypes.data, M, N, K, 0.013, 0.7, 0.29, za, zb)
        assert bits_equal(orc.gemm_int8(A, B, M, N, K, 0.013, 0.7, 0.29, za, zb), out)


# ------------------------------------------------------------ mathematics

def test_sgemm_known_answers(orc):
    # tests/full_system_check.py:33-37 and examples/gpu_test.c:106-128
    eye = np.eye(128, dtype=np.float32)
    ones = np.ones((128, 128), np.float32)
    assert bits_equal(orc.sgemm(eye, ones, np.zeros_like(ones), 128, 128, 128), ones)
    o32 = np.ones((32, 32), np.float32)
    assert bits_equal(orc.sgemm(o32, np.eye(32, dtype=np.float32), np.zeros_like(o32), 32, 32, 32), o32)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_float64_bound(orc, ta, tb):
    rng = np.random.default_rng(11 + 2 * ta + tb)
    M, N, K = 45, 38, 300
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    Ag = np.ascontiguousarray(A.T) if ta else A
    Bg = np.ascontiguousarray(B.T) if tb else B
    out = orc.sgemm(Ag, Bg, C0, M, N, K, 1.5, 0.25, bool(ta), bool(tb))
    ref = 1.5 * (A.astype(np.float64) @ B.astype(np.float64)) + 0.25 * C0
    denom = 1.5 * (np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64))) + 0.25 * np.abs(C0)
    assert np.max(np.abs(out - ref) / denom) < K * 6e-8
    # A transposed operand read with the wrong index would fail this.
    assert np.max(np.abs(out - ref)) < 1e-3


def test_gemm_int8_integer_brute_force(orc):
    rng = np.random.default_rng(5)
    M, N, K, za, zb = 13, 17, 515, 4, -3
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    exact = (A.astype(np.int64) - za) @ (B.astype(np.int64) - zb)
    assert np.all(np.abs(exact) < 2 ** 24)  # exactly representable through the float requant
    assert np.array_equal(orc.gemm_int8(A, B, M, N, K, 1.0, 1.0, 1.0, za, zb), exact)
    # Requant: roundf ties away from zero of ((acc*sa)*sb)/sc in float32.
    sa, sb, sc = np.float32(0.01), np.float32(0.02), np.float32(0.5)
    r = ((exact.astype(np.float32) * sa) * sb) / sc  # float32, left to right
    r64 = r.astype(np.float64)  # exact; |r| + 0.5 is exact in float64
    want = (np.sign(r64) * np.floor(np.abs(r64) + 0.5)).astype(np.int64)
    got = orc.gemm_int8(A, B, M, N, K, float(sa), float(sb), float(sc), za, zb)
    assert np.array_equal(got, want)


def test_quantize_closed_forms(orc):
    ties = np.array([0.5, 1.5, 2.5, -0.5, -2.5], np.float32)
    np.testing.assert_array_equal(orc.quantize_int8(ties, 1.0), [1, 2, 3, -1, -3])  # away from zero
    np.testing.assert_array_equal(orc.quantize_int8(np.zeros(5, np.float32), 0.0), [-128] * 5)  # 0/0 -> INT_MIN
    np.testing.assert_array_equal(orc.quantize_int8(np.float32([1e10, -1e10]), 1.0), [-128, -128])
    x = np.random.default_rng(3).standard_normal(1000).astype(np.float32)
    q, s = orc.quantize_symmetric(x)
    assert s == np.float32(np.max(np.abs(x))) / np.float32(127)
    r = x / s
    np.testing.assert_array_equal(q, np.clip(np.sign(r) * np.floor(np.abs(r) + 0.5), -128, 127))
    W = np.array([[1, -2, 4], [0.5, 0.25, -1]], np.float32)
    q, s = orc.quantize_per_channel(W, 2)
    np.testing.assert_array_equal(s, np.float32([4, 1]) / np.float32(127))
    np.testing.assert_array_equal(q.reshape(-1), [32, -64, 127, 64, 32, -127])


def test_dequant_and_linear_int8_closed_forms(orc):
    rng = np.random.default_rng(9)
    q = rng.integers(-128, 128, 257, dtype=np.int8)
    np.testing.assert_array_equal(orc.dequantize_int8(q, 0.37, 5), (q.astype(np.int32) - 5).astype(np.float32) * np.float32(0.37))
    x = rng.integers(-128, 128, (7, 300), dtype=np.int8)
    w = rng.integers(-128, 128, (11, 300), dtype=np.int8)
    b = rng.integers(-128, 128, 11, dtype=np.int8)
    np.testing.assert_array_equal(orc.linear_int8(x, w, b, 7, 300, 11), x.astype(np.int64) @ w.T.astype(np.int64) + b)
    acc = x.astype(np.int32) @ w.T.astype(np.int32)
    sx = rng.random(7).astype(np.float32)
    sw = rng.random(11).astype(np.float32)
    y = orc.dequant_acc(acc, sx, True, sw, True)
    np.testing.assert_array_equal(y, (acc.astype(np.float32) * sx[:, None]) * sw[None, :])
    y = orc.dequant_acc(acc, sx[:1], False, sw[:1], False)
    np.testing.assert_array_equal(y, (acc.astype(np.float32) * sx[0]) * sw[0])


def test_autograd_pieces_closed_forms(orc):
    rng = np.random.default_rng(12)
    M, N, K = 33, 7, 19
    dt = rng.standard_normal((M, N)).astype(np.float32)
    a = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((N, K)).astype(np.float32)  # Linear layout: b_trans
    da, db = orc.matmul_backward(dt, a, w, M, N, K, w.shape, da=np.zeros((M, K)), db=np.zeros((N, K)))
    np.testing.assert_allclose(da, dt.astype(np.float64) @ w, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(db, dt.T.astype(np.float64) @ a, rtol=1e-5, atol=1e-5)
    b = rng.standard_normal((K, N)).astype(np.float32)  # [K,N]: not b_trans when K != N
    da, db = orc.matmul_backward(dt, a, b, M, N, K, b.shape, da=np.zeros((M, K)), db=np.zeros((K, N)))
    np.testing.assert_allclose(da, dt.astype(np.float64) @ b.T, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(db, a.T.astype(np.float64) @ dt, rtol=1e-5, atol=1e-5)
    dy = rng.standard_normal(M * N).astype(np.float32)
    _, dbias = orc.add_backward(dy, None, np.zeros(N, np.float32))
    np.testing.assert_allclose(dbias, dy.reshape(M, N).astype(np.float64).sum(0), rtol=1e-5, atol=1e-5)
    x = rng.standard_normal(100).astype(np.float32)
    g = rng.standard_normal(100).astype(np.float32)
    np.testing.assert_array_equal(orc.relu(x), np.maximum(x, 0))
    np.testing.assert_array_equal(orc.relu_backward(x, g, np.zeros(100)), np.where(x > 0, g, 0))
    t = rng.standard_normal(100).astype(np.float32)
    assert abs(orc.mse_loss(x, t) - np.mean((x.astype(np.float64) - t) ** 2)) < 1e-5
    np.testing.assert_allclose(orc.mse_backward(x, t, 1.0, np.zeros(100)), 2.0 / 100 * (x - t), rtol=1e-6, atol=1e-7)


def test_mlp_step_finite_differences(orc):
    rng = np.random.default_rng(21)
    B, IN, H, O = 6, 5, 4, 3
    X = rng.random((B, IN)).astype(np.float32)
    Y = np.eye(O, dtype=np.float32)[rng.integers(0, O, B)]
    W1 = rng.standard_normal((H, IN)).astype(np.float32)
    b1 = rng.standard_normal(H).astype(np.float32) * 0.1
    W2 = rng.standard_normal((O, H)).astype(np.float32)
    b2 = rng.standard_normal(O).astype(np.float32) * 0.1
    r = orc.mlp_step(X, Y, W1, b1, W2, b2)

    def loss64(W1, b1, W2, b2):
        h = X.astype(np.float64) @ W1.T + b1
        o = np.maximum(h, 0) @ W2.T + b2
        return np.mean((o - Y) ** 2)

    assert abs(r["loss"] - loss64(W1, b1, W2, b2)) < 1e-5
    eps = 1e-3
    for name, P, dP in (("W1", W1, r["dW1"]), ("b1", b1, r["db1"]), ("W2", W2, r["dW2"]), ("b2", b2, r["db2"])):
        P64 = P.astype(np.float64)
        it = np.nditer(P64, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            args = {"W1": W1.astype(np.float64), "b1": b1.astype(np.float64), "W2": W2.astype(np.float64),
                    "b2": b2.astype(np.float64)}
            args[name] = P64.copy()
            args[name][idx] += eps
            lp = loss64(**args)
            args[name][idx] -= 2 * eps
            lm = loss64(**args)
            assert abs((lp - lm) / (2 * eps) - dP[idx]) < 1e-3, (name, idx)


@pytest.mark.parametrize("name", ["plain", "wd", "mom", "nest"])
def test_sgd_step_golden(orc, golden, name):
    # optimizer_sgd_step (rpl_training.c:70-114) replayed on the reference
    # build's inputs: parameters, in-place gradients and velocities after
    # each of two steps, bit for bit.
    lr, mom, damp, wd, nest = (float(x) for x in golden[f"sgd_{name}_hyper"])
    for k in range(2):
        p = golden[f"sgd_{name}_p{k}_init"].copy()
        v = np.zeros_like(p)
        for step in range(2):
            g = golden[f"sgd_{name}_s{step}_g{k}_in"].copy()
            orc.sgd_step(p, g, v if mom else None, lr, mom, damp, wd, bool(nest))
            assert bits_equal(p, golden[f"sgd_{name}_s{step}_p{k}"]), (name, k, step)
            assert bits_equal(g, golden[f"sgd_{name}_s{step}_g{k}"]), (name, k, step)
            if mom:
                assert bits_equal(v, golden[f"sgd_{name}_s{step}_v{k}"]), (name, k, step)


def test_sgd_step_closed_forms(orc):
    # Mathematics, not the formula again: plain SGD is p - lr*g rounded once
    # (within one float32 ulp of the float64 value); from v = 0 with no
    # dampening, one momentum step leaves v == g exactly and moves p exactly
    # like plain SGD; weight decay with g = 0 makes g == wd*p (one rounding).
    rng = np.random.default_rng(5)
    p0 = rng.uniform(-1, 1, 4096).astype(np.float32)
    g0 = (rng.standard_normal(4096) * 0.1).astype(np.float32)
    p, g = p0.copy(), g0.copy()
    orc.sgd_step(p, g, None, 0.03, 0.0, 0.0, 0.0, False)
    exact = p0.astype(np.float64) - np.float64(np.float32(0.03)) * g0.astype(np.float64)
    assert np.max(np.abs(p - exact) / np.spacing(np.abs(exact).astype(np.float32))) <= 1.0
    pm, gm, v = p0.copy(), g0.copy(), np.zeros_like(p0)
    orc.sgd_step(pm, gm, v, 0.03, 0.9, 0.0, 0.0, False)
    assert bits_equal(v, g0) and bits_equal(pm, p)
    pw, gw = p0.copy(), np.zeros_like(p0)
    orc.sgd_step(pw, gw, None, 0.0, 0.0, 0.0, 0.25, False)
    assert bits_equal(gw, (np.float32(0.25) * p0).astype(np.float32)) and bits_equal(pw, p0)


@pytest.mark.parametrize("kind", ["sigmoid", "tanh", "gelu"])
def test_activations_golden(orc, golden, kind):
    # tensor_sigmoid / tensor_tanh_inplace / tensor_gelu_inplace
    # (rpl_core.c:302-304, 490-497) on the reference build's inputs.
    assert bits_equal(orc.activation(kind, golden["act_x"]), golden[f"act_{kind}"])


def test_activations_float64(orc):
    # The mathematics in float64 (numpy's exp/tanh, an independent
    # implementation): each float32 result within a few ulp, plus exact
    # special values.
    x = np.linspace(-9, 9, 20001).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = {"sigmoid": 1 / (1 + np.exp(-x64)), "tanh": np.tanh(x64),
           "gelu": 0.5 * x64 * (1 + np.tanh(np.sqrt(2 / np.pi) * (x64 + 0.044715 * x64 ** 3)))}
    for kind, r in ref.items():
        y = orc.activation(kind, x).astype(np.float64)
        tol = 4 * np.spacing(np.abs(r).astype(np.float32)).astype(np.float64) + (2.0 ** -22) * np.abs(x64) * (
            kind == "gelu")
        assert np.all(np.abs(y - r) <= tol), kind
    z = np.float32([0.0])
    assert orc.activation("sigmoid", z)[0] == 0.5 and orc.activation("tanh", z)[0] == 0.0
    assert orc.activation("gelu", z)[0] == 0.0


@pytest.mark.parametrize("name", ["small", "mid"])
@pytest.mark.parametrize("masked", [False, True])
def test_sdpa_golden(orc, golden, name, masked):
    # scaled_dot_product_attention (rpl_attention.c:16-111) on the reference
    # build's inputs, bit for bit.
    Q, K, V = golden[f"att_{name}_Q"], golden[f"att_{name}_K"], golden[f"att_{name}_V"]
    out = orc.sdpa(Q, K, V, golden[f"att_{name}_mask"] if masked else None)
    assert bits_equal(out, golden[f"att_{name}_out{'_m' if masked else ''}"])


def test_sdpa_mathematics(orc):
    rng = np.random.default_rng(7)
    B, Sq, Sk, dk, dv = 2, 9, 13, 16, 5
    Q = rng.standard_normal((B, Sq, dk)).astype(np.float32)
    K = rng.standard_normal((B, Sk, dk)).astype(np.float32)
    # Every key carries the same value row: the weights sum to 1, so the
    # output is that row (within a few ulp).
    V = np.broadcast_to(rng.standard_normal(dv).astype(np.float32), (B, Sk, dv)).copy()
    assert np.allclose(orc.sdpa(Q, K, V), V[:, :1, :], rtol=1e-6, atol=1e-6)
    # Q = 0: equal scores, uniform weights: the mean of V over the keys.
    V = rng.standard_normal((B, Sk, dv)).astype(np.float32)
    mean = V.astype(np.float64).mean(1, keepdims=True)
    assert np.allclose(orc.sdpa(np.zeros_like(Q), K, V), mean, rtol=1e-5, atol=1e-6)
    # Masked keys (-1e9 before the softmax) get weight exactly 0: changing
    # their values leaves the output bit-identical.
    mask = np.ones((B, Sq, Sk), np.float32)
    mask[:, :, 3] = 0.0
    V2 = V.copy()
    V2[:, 3, :] = 1e3
    assert bits_equal(orc.sdpa(Q, K, V, mask), orc.sdpa(Q, K, V2, mask))


def test_half_codec_golden(orc, golden):
    # rpl_half.c:10-75: every half, and the float sweep, bit for bit.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert bits_equal(orc.half_to_float(h), golden["half_all_f32"])
    assert np.array_equal(orc.float_to_half(golden["half_from_f32_x"]), golden["half_from_f32_h"])


def test_half_codec_closed_forms(orc):
    # Normal halves survive the round trip exactly; floats are truncated
    # (1 + 2^-11 -> 1, 65519.99 -> 65504), >= 65536 overflows to inf,
    # subnormal results flush to signed zero.
    h = np.array([0x3C00, 0x7BFF, 0x0400, 0xC2AA, 0x8401], np.uint16)
    assert np.array_equal(orc.float_to_half(orc.half_to_float(h)), h)
    x = np.float32([1 + 2 ** -11, 65519.99, 65536.0, -1e10, 2 ** -15, -2 ** -20, np.inf])
    assert np.array_equal(orc.float_to_half(x), np.array([0x3C00, 0x7BFF, 0x7C00, 0xFC00, 0x0000, 0x8000, 0x7C00],
                                                         np.uint16))


def test_fake_quant_golden(orc, golden):
    # fake_quantize_forward (rpl_quantization.c:195-237): outputs and the
    # moving-average state after two training steps and one eval step.
    s, z = np.float32(1.0), np.float32(0.0)
    for step in range(3):
        y, s, z = orc.fake_quant(golden[f"fq_{step}_x"], s, z, bool(golden[f"fq_{step}_state"][2]))
        assert bits_equal(y, golden[f"fq_{step}_y"])
        assert bits_equal(np.float32([s, z]), golden[f"fq_{step}_state"][:2])


def test_fake_quant_closed_form(orc):
    # scale 1, zero point 0, eval: y = clamp(roundf(x), -128, 127), ties away.
    x = np.float32([0.5, -0.5, 1.5, 2.5, -2.5, 126.6, 300.0, -300.0, 0.49999997])
    y, s, z = orc.fake_quant(x, 1.0, 0.0, False)
    assert np.array_equal(y, np.float32([1, -1, 2, 3, -3, 127, 127, -128, 0])) and (s, z) == (1.0, 0.0)
