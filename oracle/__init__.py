"""CPU oracle loader -- TEST INFRASTRUCTURE ONLY.

Loads oracle/liboracle.so (the C restatement of the reference algorithms,
oracle/oracle.c) and, where it was built, oracle/_ref/libref.so (the
reference's own hot-path sources compiled by oracle/Makefile).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use this module, as
the checker; the product library never links or calls it.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.environ.get("RPL_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

_vp, _u32, _i32, _f32, _b = C.c_void_p, C.c_uint32, C.c_int32, C.c_float, C.c_bool

PROTOTYPES = {
    "orc_sgemm": (None, [_vp, _vp, _vp, _u32, _u32, _u32, _f32, _f32, _b, _b]),
    "orc_sgemm_rows": (None, [_vp, _vp, _vp, _u32, _u32, _u32, _f32, _f32, _b, _b, _u32, _u32]),
    "orc_gemm_int8": (None, [_vp, _vp, _vp, _u32, _u32, _u32, _f32, _f32, _f32, _i32, _i32]),
    "orc_gemm_int8_rows": (None, [_vp, _vp, _vp, _u32, _u32, _u32, _f32, _f32, _f32, _i32, _i32, _u32, _u32]),
    "orc_quantize_int8": (None, [_vp, _u32, _f32, _i32, _vp]),
    "orc_quantize_symmetric": (_f32, [_vp, _u32, _vp]),
    "orc_quantize_asymmetric": (None, [_vp, _u32, _vp, _vp, _vp]),
    "orc_quantize_per_channel": (None, [_vp, _u32, _u32, _vp, _vp, _vp]),
    "orc_dequantize_int8": (None, [_vp, _u32, _f32, _i32, _vp]),
    "orc_get_min_max": (None, [_vp, _u32, _vp, _vp]),
    "orc_calibrator_update": (None, [_vp, _u32, _vp, _vp]),
    "orc_calibrator_params": (None, [_f32, _f32, _b, _vp, _vp]),
    "orc_linear_int8": (None, [_vp, _vp, _vp, _vp, _u32, _u32, _u32]),
    "orc_dequant_acc": (None, [_vp, _u32, _u32, _vp, _b, _vp, _b, _vp]),
    "orc_add_broadcast": (None, [_vp, _vp, _vp, _u32, _u32]),
    "orc_relu": (None, [_vp, _vp, _u32]),
    "orc_relu_backward": (None, [_vp, _vp, _vp, _u32]),
    "orc_add_backward": (None, [_vp, _u32, _vp, _vp, _u32]),
    "orc_matmul_backward": (None, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp, _vp]),
    "orc_mse_loss": (_f32, [_vp, _vp, _u32]),
    "orc_mse_backward": (None, [_vp, _vp, _u32, _f32, _vp]),
    "orc_mlp_step": (_f32, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32] + [_vp] * 7),
    "orc_sgd_step": (None, [_vp, _vp, _vp, _u32, _f32, _f32, _f32, _f32, _b]),
    "orc_sigmoid": (None, [_vp, _vp, _u32]),
    "orc_tanh": (None, [_vp, _vp, _u32]),
    "orc_gelu": (None, [_vp, _vp, _u32]),
    "orc_sdpa": (None, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32]),
    "orc_float_to_half": (None, [_vp, _vp, _u32]),
    "orc_half_to_float": (None, [_vp, _vp, _u32]),
    "orc_fake_quant": (None, [_vp, _vp, _u32, _vp, _vp, _b]),
}


def _p(a):
    if a is None:
        return None
    assert isinstance(a, np.ndarray) and a.flags["C_CONTIGUOUS"], type(a)
    return a.ctypes.data_as(C.c_void_p)


class Oracle:
    """numpy-friendly wrappers around liboracle.so (argument order follows
    the reference functions each one restates)."""

    def __init__(self, path=ORACLE_PATH):
        if not os.path.exists(path):
            raise ImportError(f"{path} is not built (make -C oracle)")
        self.lib = C.CDLL(path)
        for n, (r, a) in PROTOTYPES.items():
            f = getattr(self.lib, n)
            f.restype, f.argtypes = r, a

    def sgemm(self, A, B, C_in, M, N, K, alpha=1.0, beta=0.0, ta=False, tb=False, rows=None):
        Cout = np.array(C_in, dtype=np.float32, copy=True).reshape(M, N)
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        if rows is None:
            self.lib.orc_sgemm(_p(A), _p(B), _p(Cout), M, N, K, alpha, beta, ta, tb)
        else:
            self.lib.orc_sgemm_rows(_p(A), _p(B), _p(Cout), M, N, K, alpha, beta, ta, tb, rows[0], rows[1])
        return Cout

    def gemm_int8(self, A, B, M, N, K, sa=1.0, sb=1.0, sc=1.0, za=0, zb=0, rows=None):
        Cout = np.zeros((M, N), np.int32)
        A = np.ascontiguousarray(A, np.int8)
        B = np.ascontiguousarray(B, np.int8)
        if rows is None:
            self.lib.orc_gemm_int8(_p(A), _p(B), _p(Cout), M, N, K, sa, sb, sc, za, zb)
        else:
            self.lib.orc_gemm_int8_rows(_p(A), _p(B), _p(Cout), M, N, K, sa, sb, sc, za, zb, rows[0], rows[1])
        return Cout

    def quantize_int8(self, x, scale, zp=0):
        x = np.ascontiguousarray(x, np.float32)
        q = np.empty(x.shape, np.int8)
        self.lib.orc_quantize_int8(_p(x), x.size, scale, zp, _p(q))
        return q

    def quantize_symmetric(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.empty(x.shape, np.int8)
        s = self.lib.orc_quantize_symmetric(_p(x), x.size, _p(q))
        return q, np.float32(s)

    def quantize_asymmetric(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.empty(x.shape, np.int8)
        s = np.zeros(1, np.float32)
        z = np.zeros(1, np.int32)
        self.lib.orc_quantize_asymmetric(_p(x), x.size, _p(q), _p(s), _p(z))
        return q, s[0], int(z[0])

    def quantize_per_channel(self, x, num_channels):
        x = np.ascontiguousarray(x, np.float32)
        cs = x.size // num_channels
        q = np.empty(x.shape, np.int8)
        s = np.empty(num_channels, np.float32)
        zp = np.empty(num_channels, np.int32)
        self.lib.orc_quantize_per_channel(_p(x), num_channels, cs, _p(q), _p(s), _p(zp))
        return q, s

    def dequantize_int8(self, q, scale, zp=0):
        q = np.ascontiguousarray(q, np.int8)
        y = np.empty(q.shape, np.float32)
        self.lib.orc_dequantize_int8(_p(q), q.size, scale, zp, _p(y))
        return y

    def get_min_max(self, x, init=(0.0, 0.0)):
        x = np.ascontiguousarray(x, np.float32)
        mn = np.array([init[0]], np.float32)
        mx = np.array([init[1]], np.float32)
        self.lib.orc_get_min_max(_p(x), x.size, _p(mn), _p(mx))
        return mn[0], mx[0]

    def calibrate(self, xs, symmetric):
        mn = np.array([np.finfo(np.float32).max], np.float32)
        mx = np.array([-np.finfo(np.float32).max], np.float32)
        for x in xs:
            x = np.ascontiguousarray(x, np.float32)
            self.lib.orc_calibrator_update(_p(x), x.size, _p(mn), _p(mx))
        s = np.zeros(1, np.float32)
        z = np.zeros(1, np.int32)
        self.lib.orc_calibrator_params(mn[0], mx[0], symmetric, _p(s), _p(z))
        return mn[0], mx[0], s[0], int(z[0])

    def linear_int8(self, x, w, bias, M, K, N):
        out = np.zeros((M, N), np.int32)
        x = np.ascontiguousarray(x, np.int8)
        w = np.ascontiguousarray(w, np.int8)
        b = None if bias is None else np.ascontiguousarray(bias, np.int8)
        self.lib.orc_linear_int8(_p(x), _p(w), _p(b), _p(out), M, K, N)
        return out

    def dequant_acc(self, acc, sx, sx_per_row, sw, sw_per_col):
        acc = np.ascontiguousarray(acc, np.int32)
        M, N = acc.shape
        y = np.empty((M, N), np.float32)
        sx = np.ascontiguousarray(sx, np.float32).reshape(-1)
        sw = np.ascontiguousarray(sw, np.float32).reshape(-1)
        self.lib.orc_dequant_acc(_p(acc), M, N, _p(sx), sx_per_row, _p(sw), sw_per_col, _p(y))
        return y

    def add_broadcast(self, a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        out = np.empty(a.shape, np.float32)
        self.lib.orc_add_broadcast(_p(a), _p(b), _p(out), a.size, b.size)
        return out

    def relu(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(x.shape, np.float32)
        self.lib.orc_relu(_p(x), _p(y), x.size)
        return y

    def relu_backward(self, x, dy, dx):
        dx = np.array(dx, np.float32, copy=True)
        self.lib.orc_relu_backward(_p(np.ascontiguousarray(x, np.float32)), _p(np.ascontiguousarray(dy, np.float32)),
                                   _p(dx), dx.size)
        return dx

    def add_backward(self, dy, da, db):
        dy = np.ascontiguousarray(dy, np.float32)
        da = None if da is None else np.array(da, np.float32, copy=True)
        db = None if db is None else np.array(db, np.float32, copy=True)
        self.lib.orc_add_backward(_p(dy), dy.size, _p(da), _p(db), 0 if db is None else db.size)
        return da, db

    def matmul_backward(self, dt, a, b, M, N, K, b_shape, da=None, db=None):
        da = None if da is None else np.array(da, np.float32, copy=True)
        db = None if db is None else np.array(db, np.float32, copy=True)
        self.lib.orc_matmul_backward(_p(np.ascontiguousarray(dt, np.float32)), _p(np.ascontiguousarray(a, np.float32)),
                                     _p(np.ascontiguousarray(b, np.float32)), M, N, K, b_shape[0], b_shape[1], _p(da),
                                     _p(db))
        return da, db

    def mse_loss(self, p, t):
        p = np.ascontiguousarray(p, np.float32)
        return np.float32(self.lib.orc_mse_loss(_p(p), _p(np.ascontiguousarray(t, np.float32)), p.size))

    def mse_backward(self, p, t, g0, dp):
        dp = np.array(dp, np.float32, copy=True)
        self.lib.orc_mse_backward(_p(np.ascontiguousarray(p, np.float32)), _p(np.ascontiguousarray(t, np.float32)),
                                  dp.size, g0, _p(dp))
        return dp

    def sgd_step(self, p, g, v, lr, momentum, dampening, weight_decay, nesterov):
        """One optimizer_sgd_step on one parameter tensor, in place on p, g, v
        (float32 arrays); v may be None when momentum == 0."""
        v = v if v is not None else np.zeros(1, np.float32)
        self.lib.orc_sgd_step(_p(p), _p(g), _p(v), p.size, lr, momentum, dampening, weight_decay, bool(nesterov))

    def activation(self, kind, x):
        """kind in {"sigmoid", "tanh", "gelu"}: the reference's CPU formula."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        getattr(self.lib, f"orc_{kind}")(_p(x), _p(y), x.size)
        return y

    def sdpa(self, Q, K, V, mask=None):
        """scaled_dot_product_attention: Q [B,Sq,dk], K [B,Sk,dk], V [B,Sk,dv]."""
        Q, K, V = (np.ascontiguousarray(a, np.float32) for a in (Q, K, V))
        B, Sq, dk = Q.shape
        Sk, dv = K.shape[1], V.shape[2]
        m = None if mask is None else np.ascontiguousarray(mask, np.float32)
        out = np.empty((B, Sq, dv), np.float32)
        self.lib.orc_sdpa(_p(Q), _p(K), _p(V), None if m is None else _p(m), _p(out), B, Sq, Sk, dk, dv)
        return out

    def float_to_half(self, x):
        x = np.ascontiguousarray(x, np.float32)
        h = np.empty(x.shape, np.uint16)
        self.lib.orc_float_to_half(_p(x), _p(h), x.size)
        return h

    def half_to_float(self, h):
        h = np.ascontiguousarray(h, np.uint16)
        x = np.empty(h.shape, np.float32)
        self.lib.orc_half_to_float(_p(h), _p(x), h.size)
        return x

    def fake_quant(self, x, scale, zp, training):
        """Returns (y, scale, zp) after one fake_quantize_forward."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        s, z = np.float32([scale]), np.float32([zp])
        self.lib.orc_fake_quant(_p(x), _p(y), x.size, _p(s), _p(z), bool(training))
        return y, s[0], z[0]

    def mlp_step(self, X, Y, W1, b1, W2, b2):
        X, Y, W1, b1, W2, b2 = (np.ascontiguousarray(v, np.float32) for v in (X, Y, W1, b1, W2, b2))
        B, IN = X.shape
        H, O = W1.shape[0], W2.shape[0]
        h = np.empty((B, H), np.float32)
        a = np.empty((B, H), np.float32)
        o = np.empty((B, O), np.float32)
        dW1, db1 = np.zeros_like(W1), np.zeros_like(b1)
        dW2, db2 = np.zeros_like(W2), np.zeros_like(b2)
        loss = self.lib.orc_mlp_step(_p(X), _p(Y), _p(W1), _p(b1), _p(W2), _p(b2), B, IN, H, O, _p(h), _p(a), _p(o),
                                     _p(dW1), _p(db1), _p(dW2), _p(db2))
        return dict(loss=np.float32(loss), h=h, a=a, o=o, dW1=dW1, db1=db1, dW2=dW2, db2=db2)


def ref_available():
    return os.path.exists(REF_PATH)
