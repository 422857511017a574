"""scaled_dot_product_attention (src/rpl_attention.c:16-111) on the device:
QK^T and PV on the FP32 GEMMs, a masked softmax kernel between them.

fp32 bar, written here: with S = QK^T/sqrt(dk) and P its row softmax (both
float64), each output element within
    (2e-5 sqrt(dk) max_j(sum_k |q_k k_jk|)/sqrt(dk) + 1e-5 sqrt(Sk) + 4e-6) * sum_j P_ij |V_jk|
of the reference: the GEMM bound on the scores moves each weight by at most
twice the largest score error (relative), the PV GEMM adds its own bound, and
exp / divide a few ulp.  Masked keys get weight exactly 0, so changing their
values changes no output bit."""
import ctypes as C

import numpy as np
import pytest

import rpl_amd
from conftest import bits_equal
from gpu_util import down, empty, say, up
from test_gpu_linear import host, tensor_from

pytestmark = pytest.mark.gpu


def device_sdpa(lib, Q, K, V, mask=None):
    B, Sq, dk = Q.shape
    Sk, dv = K.shape[1], V.shape[2]
    dq, dk_, dv_ = up(Q), up(K), up(V)
    dm = up(mask) if mask is not None else None
    out = empty((B, Sq, dv), np.float32)
    rpl_amd.check(lib.rplhip_attention(dq.ptr, dk_.ptr, dv_.ptr, dm.ptr if dm else None, out.ptr, B, Sq, Sk, dk,
                                       dv, None))
    return down(out, np.float32, (B, Sq, dv))


def check_close(got, Q, K, V, mask, ref):
    Q64, K64, V64 = (a.astype(np.float64) for a in (Q, K, V))
    dk, Sk = Q.shape[2], K.shape[1]
    scale = 1.0 / np.sqrt(dk)
    S = np.einsum("bik,bjk->bij", Q64, K64) * scale
    A = np.einsum("bik,bjk->bij", np.abs(Q64), np.abs(K64)) * scale
    if mask is not None:
        S = np.where(mask == 0, -1e9, S)
    P = np.exp(S - S.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    T = np.einsum("bij,bjk->bik", P, np.abs(V64))
    tol = (2e-5 * np.sqrt(dk) * A.max(-1, keepdims=True) + 1e-5 * np.sqrt(Sk) + 4e-6) * T + 1e-30
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= tol), float(np.max(err / tol))


@pytest.mark.parametrize("name", ["small", "mid"])
@pytest.mark.parametrize("masked", [False, True])
def test_attention_vs_reference(gpu, golden, name, masked):
    Q, K, V = golden[f"att_{name}_Q"], golden[f"att_{name}_K"], golden[f"att_{name}_V"]
    mask = golden[f"att_{name}_mask"] if masked else None
    say("attention", name, masked)
    got = device_sdpa(gpu, Q, K, V, mask)
    check_close(got, Q, K, V, mask, golden[f"att_{name}_out{'_m' if masked else ''}"])


def test_attention_larger_vs_oracle_and_mask_invariance(gpu, orc):
    rng = np.random.default_rng(21)
    B, Sq, Sk, dk, dv = 8, 256, 320, 64, 64
    Q = rng.standard_normal((B, Sq, dk)).astype(np.float32)
    K = rng.standard_normal((B, Sk, dk)).astype(np.float32)
    V = rng.standard_normal((B, Sk, dv)).astype(np.float32)
    mask = np.tril(np.ones((Sq, Sk), np.float32), k=Sk - Sq)[None].repeat(B, 0)  # causal
    say("attention larger", B, Sq, Sk, dk, dv)
    got = device_sdpa(gpu, Q, K, V, mask)
    check_close(got, Q, K, V, mask, orc.sdpa(Q, K, V, mask))
    # Mask key 5 for every query, change its values, compare bit for bit.
    mask2 = mask.copy()
    mask2[:, :, 5] = 0.0
    V2 = V.copy()
    V2[:, 5, :] = 1e3
    assert bits_equal(device_sdpa(gpu, Q, K, V, mask2), device_sdpa(gpu, Q, K, V2, mask2))


@pytest.mark.parametrize("resident", [False, True])
def test_attention_rpl_api(gpu, golden, resident):
    lib = gpu
    Q, K, V = golden["att_mid_Q"], golden["att_mid_K"], golden["att_mid_V"]
    mask = golden["att_mid_mask"]
    tq, tk, tv, tm = (tensor_from(lib, a) for a in (Q, K, V, mask))
    if resident:
        for t in (tq, tk, tv, tm):
            lib.tensor_to_gpu(t)
    say("attention rpl.h", "resident" if resident else "host")
    out = lib.scaled_dot_product_attention(tq, tk, tv, tm, 0.1, True)  # dropout: a no-op, as in the reference
    err = lib.rpl_last_error()
    assert not err, err
    assert (out.contents.device == rpl_amd.DEVICE_GPU) == resident
    if resident:
        lib.tensor_from_gpu(out)
    got = host(out, (Q.shape[0], Q.shape[1], V.shape[2]))
    check_close(got, Q, K, V, mask, golden["att_mid_out_m"])
    # A mask of the wrong size is refused (the reference would overrun it).
    bad = tensor_from(lib, np.ones(7, np.float32))
    assert not lib.scaled_dot_product_attention(tq, tk, tv, bad, 0.0, False)
    assert b"mask has 7 elements" in lib.rpl_last_error()
    for t in (tq, tk, tv, tm, out, bad):
        lib.tensor_free(t)
