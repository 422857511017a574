"""Quantize / dequantize / min-max kernels vs the reference golden vectors and
the oracle.  Bar: bit-exact (int8 values, scales, zero points, fp32 outputs)."""
import ctypes as C

import numpy as np
import pytest

import rpl_amd
from conftest import bits_equal, seed
from gpu_util import down, empty, say, up

pytestmark = pytest.mark.gpu


def dev_quantize(lib, x, scale, zp):
    dx, dq = up(x), empty(x.size, np.int8)
    rpl_amd.check(lib.rplhip_quantize_int8(dx.ptr, x.size, scale, zp, dq.ptr, None))
    return down(dq, np.int8, x.shape)


def dev_symmetric(lib, x):
    dx, dq, ds = up(x), empty(x.size, np.int8), empty(1, np.float32)
    rpl_amd.check(lib.rplhip_quantize_symmetric(dx.ptr, x.size, dq.ptr, ds.ptr, None))
    return down(dq, np.int8, x.shape), down(ds, np.float32, (1,))


def dev_asymmetric(lib, x):
    dx, dq, ds, dz = up(x), empty(x.size, np.int8), empty(1, np.float32), empty(1, np.int32)
    rpl_amd.check(lib.rplhip_quantize_asymmetric(dx.ptr, x.size, dq.ptr, ds.ptr, dz.ptr, None))
    return down(dq, np.int8, x.shape), down(ds, np.float32, (1,)), down(dz, np.int32, (1,))


def dev_per_channel(lib, x, nc):
    cs = x.size // nc
    dx, dq, ds = up(x), empty(x.size, np.int8), empty(nc, np.float32)
    rpl_amd.check(lib.rplhip_quantize_per_channel(dx.ptr, nc, cs, dq.ptr, ds.ptr, None))
    return down(dq, np.int8, (x.size,)), down(ds, np.float32, (nc,))


def test_quantize_special_golden(gpu, golden):
    x = golden["q_special_x"]
    for i in range(5):
        scale, zp = golden[f"q_special_{i}_params"]
        say("quantize special", i)
        assert bits_equal(dev_quantize(gpu, x, float(scale), int(zp)), golden[f"q_special_{i}"]), i


@pytest.mark.parametrize("name", ["normal", "uniform", "zeros", "ties"])
def test_sym_asym_golden(gpu, golden, name):
    x = golden[f"sym_{name}_x"]
    say("symmetric/asymmetric", name)
    q, s = dev_symmetric(gpu, x)
    assert bits_equal(q, golden[f"sym_{name}_q"]) and bits_equal(s, golden[f"sym_{name}_scale"])
    q, s, z = dev_asymmetric(gpu, x)
    assert bits_equal(q, golden[f"asym_{name}_q"]) and bits_equal(s, golden[f"asym_{name}_scale"])
    assert bits_equal(z, golden[f"asym_{name}_zp"])


@pytest.mark.parametrize("name", ["known", "rows", "axis1", "zero_row"])
def test_per_channel_golden(gpu, golden, name):
    x = golden[f"pc_{name}_x"]
    axis = int(golden[f"pc_{name}_axis"][0])
    say("per-channel", name)
    q, s = dev_per_channel(gpu, x, x.shape[axis])
    assert bits_equal(q, golden[f"pc_{name}_q"]) and bits_equal(s, golden[f"pc_{name}_scales"])


def test_dequantize_golden(gpu, golden):
    q = golden["dq_q"]
    for i in range(3):
        scale, zp = golden[f"dq_{i}_params"]
        dq, dy = up(q), empty(q.size, np.float32)
        say("dequantize", i)
        rpl_amd.check(gpu.rplhip_dequantize_int8(dq.ptr, q.size, float(scale), int(zp), dy.ptr, None))
        assert bits_equal(down(dy, np.float32, q.shape), golden[f"dq_{i}_y"])


@pytest.mark.parametrize("name", ["normal", "nan_first", "nan_later", "zeros", "negzero_first", "inf"])
def test_get_min_max_golden(gpu, golden, name):
    x = golden[f"mm_{name}_x"]
    dx, d2 = up(x), empty(2, np.float32)
    say("get_min_max", name)
    rpl_amd.check(gpu.rplhip_get_min_max(dx.ptr, x.size, d2.ptr, None))
    assert bits_equal(down(d2, np.float32, (2,)), golden[f"mm_{name}_out"])


def test_calibrator_rpl_api(gpu, golden):
    from rpl_amd import Tensor  # noqa: F401

    lib = gpu
    for sym in (1, 0):
        cal = lib.calibrator_create()
        for key in ("cal_x1", "cal_x2"):
            x = golden[key]
            t = lib.tensor_create(1, (C.c_uint32 * 1)(x.size), False)
            C.memmove(t.contents.data, x.ctypes.data, x.nbytes)
            say("calibrator", sym, key)
            lib.calibrator_update(cal, t)
            lib.tensor_free(t)
        lib.calibrator_compute_params(cal, bool(sym))
        c = cal.contents
        assert bits_equal(np.float32([c.min_val, c.max_val, c.scale]), golden[f"cal_{sym}"])
        assert [c.zero_point, c.num_samples] == list(golden[f"cal_{sym}_zp"])
        lib.calibrator_free(cal)


def test_rpl_api_quantizers(gpu, golden):
    """include/rpl.h quantizers on host tensors return the reference's structs."""
    lib = gpu
    x = golden["sym_normal_x"]
    t = lib.tensor_create(1, (C.c_uint32 * 1)(x.size), False)
    C.memmove(t.contents.data, x.ctypes.data, x.nbytes)
    say("rpl.h symmetric")
    q = lib.tensor_quantize_int8_symmetric(t)
    got = np.ctypeslib.as_array(q.contents.data, shape=(x.size,)).copy()
    assert bits_equal(got, golden["sym_normal_q"]) and q.contents.zero_point == 0
    assert np.float32(q.contents.scale) == golden["sym_normal_scale"][0]
    say("rpl.h dequantize")
    y = lib.tensor_dequantize_int8(q)
    yv = np.ctypeslib.as_array(y.contents.data, shape=(x.size,)).copy()
    assert bits_equal(yv, got.astype(np.float32) * np.float32(q.contents.scale))
    lib.tensor_free(y)
    lib.quantized_tensor_free(q)
    mn, mx = C.c_float(0), C.c_float(0)
    lib.tensor_get_min_max(t, C.byref(mn), C.byref(mx))
    assert (mn.value, mx.value) == (float(x.min()), float(x.max()))
    lib.tensor_free(t)


@pytest.mark.parametrize("n", [0, 1, 3, 5, 4097, 1 << 20])
def test_quantize_sizes_vs_oracle(gpu, orc, n):
    x = rpl_amd.fill_normal(n, seed(93, 5)) * np.float32(3)
    say("quantize sizes", n)
    if n == 0:
        dq = empty(1, np.int8)
        rpl_amd.check(gpu.rplhip_quantize_int8(None, 0, 1.0, 0, dq.ptr, None))
        return
    assert bits_equal(dev_quantize(gpu, x, 0.037, 2), orc.quantize_int8(x, 0.037, 2))
    q, s = dev_symmetric(gpu, x)
    oq, os_ = orc.quantize_symmetric(x)
    assert bits_equal(q, oq) and bits_equal(s, np.float32([os_]))
    q, s, z = dev_asymmetric(gpu, x)
    oq, os_, oz = orc.quantize_asymmetric(x)
    assert bits_equal(q, oq) and bits_equal(s, np.float32([os_])) and int(z[0]) == oz


def test_quantize_unaligned_pointers(gpu, orc):
    # Offsets that break 16-byte alignment take the scalar paths.
    x = rpl_amd.fill_normal(1001, seed(93, 6))
    big = up(np.concatenate([np.zeros(1, np.float32), x]))
    dq = empty(1008, np.int8)
    src = C.c_void_p(big.ptr.value + 4)
    dst = C.c_void_p(dq.ptr.value + 1)
    say("quantize unaligned")
    rpl_amd.check(gpu.rplhip_quantize_int8(src, 1001, 0.05, 0, dst, None))
    got = down(dq, np.int8, (1008,))[1:1002]
    assert bits_equal(got, orc.quantize_int8(x, 0.05, 0))


# Rows of up to 8192 floats with cols % 4 == 0 and aligned rows are held in
# registers (k_quantize_rows_wave<NV, WPR>): rows of 1024 floats or more by 4
# waves each (NV = 1, 2, 4, 8 float4 per lane for up to 1024, 2048, 4096,
# 8192 floats; ragged ends re-read the last float4), shorter rows by one wave
# each (NV = 1, 2, 4 up to 256, 512, 1020; row counts that are not a multiple
# of the block's 4 rows); others are read twice, one block per row
# (k_quantize_rows: 33 x 1001, 3 x 9000, odd row starts).
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (8192, 8192), (33, 1001), (3, 9000), (1, 64), (2048, 4096),
                                       (7, 4112), (5, 16), (9, 1004), (6, 8192), (13, 2060), (3, 4),
                                       (11, 260), (6, 512), (10, 1024), (5, 1500), (3, 2048), (2, 3000),
                                       (17, 252), (5, 1020), (3, 1028), (5, 4100), (4, 7000), (2, 5120)])
def test_per_channel_vs_oracle(gpu, orc, rows, cols):
    x = rpl_amd.fill_normal(rows * cols, seed(94, 7)).reshape(rows, cols)
    say("per-channel", rows, cols)
    q, s = dev_per_channel(gpu, x, rows)
    oq, os_ = orc.quantize_per_channel(x, rows)
    assert bits_equal(q, oq.reshape(-1)) and bits_equal(s, os_)


@pytest.mark.parametrize("cols", [48, 1024, 2052, 4096, 6164])
def test_per_channel_special_rows(gpu, orc, cols):
    """Rows that are all zero (scale 0: 0/0 -> -128), hold NaN (never the
    min or max; NaN / scale -> -128), +-inf (scale inf), signed zeros, exact
    .5 ties and the largest finite floats."""
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((8, cols)).astype(np.float32)
    x[0] = 0.0
    x[1, 5] = np.nan
    x[2, 3] = np.inf
    x[3, :] = -0.0
    x[3, 7] = 0.0
    x[4, :4] = [127.0, 63.5, -63.5, 0.5]
    x[5, 1] = np.finfo(np.float32).max
    x[5, 2] = -np.finfo(np.float32).max
    x[6, :] = np.nan
    x[7, 9] = -np.inf
    say("per-channel special rows", cols)
    q, s = dev_per_channel(gpu, x, 8)
    oq, os_ = orc.quantize_per_channel(x, 8)
    assert bits_equal(q, oq.reshape(-1)) and bits_equal(s, os_)


def test_per_channel_empty_slices(gpu, orc):
    """channel_size 0: no element is read; min/max keep their FLT_MAX /
    -FLT_MAX starting values, so every scale is FLT_MAX/127."""
    say("per-channel, 5 empty slices")
    dx, dq, ds = empty(4, np.float32), empty(16, np.int8), empty(5, np.float32)
    rpl_amd.check(gpu.rplhip_quantize_per_channel(dx.ptr, 5, 0, dq.ptr, ds.ptr, None))
    s = down(ds, np.float32, (5,))
    _, os_ = orc.quantize_per_channel(np.zeros((5, 0), np.float32), 5)
    assert bits_equal(s, os_) and s[0] == np.float32(np.finfo(np.float32).max) / np.float32(127)


def test_symmetric_8192_squared_vs_oracle(gpu, orc):
    n = 8192 * 8192
    x = rpl_amd.fill_normal(n, seed(4, 0))
    say("symmetric 8192^2")
    q, s = dev_symmetric(gpu, x)
    oq, os_ = orc.quantize_symmetric(x)
    assert bits_equal(s, np.float32([os_])) and bits_equal(q, oq)
