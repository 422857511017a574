"""The device seam's activations (tensor_sigmoid_gpu / tensor_tanh_gpu /
tensor_gelu_gpu, src/rpl_gpu.c:437-522) and tensor_relu_gpu.

The reference computes these with glibc (CPU formulas, src/rpl_core.c:
302-304, 490-497); the device's exp / tanh / pow are different correctly
approximating implementations, so the bar is numeric, written here:
|device - reference| <= 4 ulp(reference), plus 2^-22 |x| for GELU (its
1 + tanh(u) cancels for negative x, turning one ulp of tanh into an absolute
error of |x| 2^-24); NaN where the reference gives NaN, identical infinities
and signed zeros."""
import ctypes as C

import numpy as np
import pytest

import rpl_amd
from gpu_util import down, empty, say, up
from test_gpu_linear import host, tensor_from

pytestmark = pytest.mark.gpu


def close(got, ref, x, kind):
    got, ref, x = (np.asarray(v, np.float64) for v in (got, ref, x))
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    inf = np.isinf(ref)
    assert np.array_equal(got[inf], ref[inf])
    fin = ~nan & ~inf
    tol = 4 * np.spacing(np.abs(ref[fin]).astype(np.float32)).astype(np.float64)
    if kind == "gelu":
        tol = tol + 2.0 ** -22 * np.abs(x[fin])
    err = np.abs(got[fin] - ref[fin])
    assert np.all(err <= tol), (kind, float(np.max(err - tol)))


@pytest.mark.parametrize("kind", ["sigmoid", "tanh", "gelu"])
def test_activation_device_vs_reference(gpu, golden, kind):
    lib = gpu
    x = golden["act_x"]
    dx, dy = up(x), empty(x.shape, np.float32)
    say("activation", kind, x.size)
    rpl_amd.check(getattr(lib, f"rplhip_{kind}")(dx.ptr, dy.ptr, x.size, None))
    close(down(dy, np.float32, x.shape), golden[f"act_{kind}"], x, kind)


@pytest.mark.parametrize("kind", ["relu", "sigmoid", "tanh", "gelu"])
def test_seam_functions_rpl_api(gpu, orc, golden, kind):
    # `in` on the host moves to the device; an output not yet resident takes
    # in's shape and becomes resident (src/rpl_gpu.c:443-450).
    lib = gpu
    x = golden["act_x"][:4096].reshape(64, 64)
    tin = tensor_from(lib, x)
    tout = tensor_from(lib, np.zeros(64 * 64, np.float32))  # 1-D, same size
    say("seam", kind)
    getattr(lib, f"tensor_{kind}_gpu")(tout, tin)
    err = lib.rpl_last_error()
    assert not err, err
    assert tin.contents.device == rpl_amd.DEVICE_GPU and tout.contents.device == rpl_amd.DEVICE_GPU
    assert tout.contents.dims == 2 and tuple(tout.contents.shape[:2]) == (64, 64)
    lib.tensor_from_gpu(tout)
    got = host(tout, (64, 64))
    if kind == "relu":
        assert np.array_equal(got, np.maximum(x, 0))
    else:
        close(got.ravel(), golden[f"act_{kind}"][:4096], x.ravel(), kind)
    # A resident output of another size is refused, not overrun.
    small = tensor_from(lib, np.zeros(100, np.float32))
    lib.tensor_to_gpu(small)
    getattr(lib, f"tensor_{kind}_gpu")(small, tin)
    assert b"output has 100 elements" in lib.rpl_last_error()
    for t in (tin, tout, small):
        lib.tensor_free(t)


def test_add_gpu_elementwise_and_broadcast(gpu):
    lib = gpu
    rng = np.random.default_rng(9)
    a = rng.standard_normal((32, 48)).astype(np.float32)
    b = rng.standard_normal(48).astype(np.float32)
    ta, tb = tensor_from(lib, a), tensor_from(lib, b)
    tout = tensor_from(lib, np.zeros((32, 48), np.float32))
    say("tensor_add_gpu")
    lib.tensor_add_gpu(tout, ta, tb)
    assert not lib.rpl_last_error()
    lib.tensor_from_gpu(tout)
    assert np.array_equal(host(tout, (32, 48)), a + b[None, :])
    for t in (ta, tb, tout):
        lib.tensor_free(t)
