"""FP16 codec (src/rpl_half.c) and QAT fake quantization
(src/rpl_quantization.c:170-260) on the device, bit-exact with the
reference build's golden vectors."""
import ctypes as C

import numpy as np
import pytest

import rpl_amd
from conftest import bits_equal
from gpu_util import down, empty, say, up
from test_gpu_linear import host, tensor_from

pytestmark = pytest.mark.gpu


def test_half_codec_device(gpu, golden, orc):
    lib = gpu
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dh, dx = up(h), empty(h.shape, np.float32)
    say("half -> float, all 65536")
    rpl_amd.check(lib.rplhip_half_to_float(dh.ptr, dx.ptr, h.size, None))
    assert bits_equal(down(dx, np.float32, h.shape), golden["half_all_f32"])
    x = golden["half_from_f32_x"]
    rng = np.random.default_rng(3)
    x = np.concatenate([x, rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    dx2, dh2 = up(x), empty(x.shape, np.uint16)
    say("float -> half", x.size)
    rpl_amd.check(lib.rplhip_float_to_half(dx2.ptr, dh2.ptr, x.size, None))
    got = down(dh2, np.uint16, x.shape)
    n0 = golden["half_from_f32_h"].size
    assert np.array_equal(got[:n0], golden["half_from_f32_h"])
    assert np.array_equal(got, orc.float_to_half(x))


def test_half_codec_rpl_api(gpu, golden):
    lib = gpu
    x = golden["half_from_f32_x"][:4096].reshape(64, 64)
    t = tensor_from(lib, x)
    lib.tensor_to_gpu(t)
    say("tensor_to_half / tensor_from_half")
    ht = lib.tensor_to_half(t)
    assert ht.contents.device == rpl_amd.DEVICE_CPU and ht.contents.size == 4096
    got = np.ctypeslib.as_array(ht.contents.data, shape=(4096,)).copy()
    assert np.array_equal(got, golden["half_from_f32_h"][:4096])
    back = lib.tensor_from_half(ht)
    assert not lib.rpl_last_error()
    assert bits_equal(host(back, (4096,)), golden["half_all_f32"][got.astype(np.int64)])
    lib.half_tensor_free(ht)
    for tt in (t, back):
        lib.tensor_free(tt)


@pytest.mark.parametrize("resident", [False, True])
def test_fake_quant_rpl_api(gpu, golden, resident):
    lib = gpu
    fq = lib.fake_quantize_create()
    for step in range(3):
        x = golden[f"fq_{step}_x"]
        fq.contents.training = bool(golden[f"fq_{step}_state"][2])
        t = tensor_from(lib, x, requires_grad=True)
        if resident:
            lib.tensor_to_gpu(t)
        say("fake quant", step, "resident" if resident else "host")
        y = lib.fake_quantize_forward(fq, t)
        err = lib.rpl_last_error()
        assert not err, err
        if resident:
            assert y.contents.device == rpl_amd.DEVICE_GPU
            lib.tensor_from_gpu(y)
        assert bits_equal(host(y, (x.size,)), golden[f"fq_{step}_y"])
        st = np.float32([fq.contents.scale.contents.data[0], fq.contents.zero_point.contents.data[0]])
        assert bits_equal(st, golden[f"fq_{step}_state"][:2])
        # Straight-through estimator: the input gradient gains the output's.
        g = np.random.default_rng(step).standard_normal(x.size).astype(np.float32)
        C.memmove(y.contents.grad, g.ctypes.data, g.nbytes)
        if resident:
            rpl_amd.check(lib.rplhip_memcpy_htod(lib.rpl_tensor_device_grad(y), g.ctypes.data, g.nbytes))
        lib.tensor_zero_grad(t)
        lib.backward_fake_quant(y)
        if resident:
            lib.tensor_from_gpu(t)
        assert bits_equal(host(t, (x.size,), grad=True), g)
        for tt in (t, y):
            lib.tensor_free(tt)
    lib.fake_quantize_free(fq)
