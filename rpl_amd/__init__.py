"""ctypes binding of rpl_amd/librpl.so: RPL's GEMM hot path on MI355X (gfx950).

The library exports two C interfaces (see include/):
  * rpl.h    -- the reference's own entry points (tensor_gemm, gemm_int8,
                linear_int8, the quantizers, Linear + autograd) with the
                reference's struct layouts;
  * rplhip.h -- the device C ABI (device pointers, status codes, streams).

This module only declares prototypes and offers small helpers (device
buffers, status checking).  There is no Python or CPU compute path: if the
library is not built, importing `lib` raises; if no gfx950 device is
present, every compute call returns RPLHIP_ERR_NO_DEVICE and `check` raises
RplError with the reason.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
# RPL_LIB selects another build of the same library (the host sanitizer
# build, rpl_amd/librpl_san.so, in tests/test_host_sanitizers.py).
LIB_PATH = os.environ.get("RPL_LIB") or os.path.join(HERE, "librpl.so")
INCLUDE_DIR = os.path.join(REPO, "include")

MAX_DIMS = 8
DEVICE_CPU, DEVICE_GPU = 0, 1
OK, ERR_INVALID, ERR_NO_DEVICE, ERR_HIP, ERR_NOMEM, ERR_UNSUPPORTED = range(6)


class RplError(RuntimeError):
    """A non-OK rplhip_status, with rplhip_last_error() as the message."""

    def __init__(self, status, msg):
        super().__init__(f"status {status}: {msg}")
        self.status = status


class Tensor(C.Structure):
    """include/rpl.h `Tensor` (reference include/rpl.h:57-78), C field order."""


Tensor._fields_ = [
    ("data", C.POINTER(C.c_float)),
    ("grad", C.POINTER(C.c_float)),
    ("dims", C.c_uint32),
    ("shape", C.c_uint32 * MAX_DIMS),
    ("strides", C.c_uint32 * MAX_DIMS),
    ("size", C.c_uint32),
    ("requires_grad", C.c_bool),
    ("_allocation", C.c_void_p),
    ("_alloc_size", C.c_size_t),
    ("device", C.c_int),
    ("gpu_buffer", C.c_uint32),
    ("is_leaf", C.c_bool),
    ("parent1", C.POINTER(Tensor)),
    ("parent2", C.POINTER(Tensor)),
    ("backward_fn", C.c_void_p),
]


class QuantizedTensor(C.Structure):
    """include/rpl.h `QuantizedTensor` (reference include/rpl.h:167-174)."""

    _fields_ = [
        ("data", C.POINTER(C.c_int8)),
        ("scale", C.c_float),
        ("zero_point", C.c_int32),
        ("size", C.c_uint32),
        ("dims", C.c_uint32),
        ("shape", C.c_uint32 * MAX_DIMS),
    ]


class PerChannelQuantizedTensor(C.Structure):
    """Reference src/rpl_quantization.c:110-118."""

    _fields_ = [
        ("data", C.POINTER(C.c_int8)),
        ("scales", C.POINTER(C.c_float)),
        ("zero_points", C.POINTER(C.c_int32)),
        ("num_channels", C.c_uint32),
        ("channel_size", C.c_uint32),
        ("dims", C.c_uint32),
        ("shape", C.c_uint32 * MAX_DIMS),
    ]


class QuantizationCalibrator(C.Structure):
    """Reference src/rpl_quantization.c:18-24."""

    _fields_ = [
        ("min_val", C.c_float),
        ("max_val", C.c_float),
        ("scale", C.c_float),
        ("zero_point", C.c_int32),
        ("num_samples", C.c_uint32),
    ]


class Linear(C.Structure):
    """Reference src/rpl_nn.c:16-21."""

    _fields_ = [
        ("weight", C.POINTER(Tensor)),
        ("bias", C.POINTER(Tensor)),
        ("in_features", C.c_uint32),
        ("out_features", C.c_uint32),
    ]


class HalfTensor(C.Structure):
    """Reference include/rpl.h:82-92."""

    _fields_ = [
        ("data", C.POINTER(C.c_uint16)),
        ("dims", C.c_uint32),
        ("shape", C.c_uint32 * 8),
        ("strides", C.c_uint32 * 8),
        ("size", C.c_uint32),
        ("_allocation", C.c_void_p),
        ("device", C.c_int),
        ("gpu_buffer", C.c_uint32),
    ]


class FakeQuantize(C.Structure):
    """Reference src/rpl_quantization.c:174-179 (file-local there)."""

    _fields_ = [
        ("scale", C.POINTER(Tensor)),
        ("zero_point", C.POINTER(Tensor)),
        ("training", C.c_bool),
        ("num_batches_tracked", C.c_uint32),
    ]


class Optimizer(C.Structure):
    """Reference src/rpl_training.c:20-28 (opaque in include/rpl.h)."""

    _fields_ = [
        ("type", C.c_int),
        ("learning_rate", C.c_float),
        ("weight_decay", C.c_float),
        ("num_params", C.c_uint32),
        ("parameters", C.POINTER(C.POINTER(Tensor))),
        ("state", C.c_void_p),
    ]


class SGDState(C.Structure):
    """Reference src/rpl_training.c:34-39."""

    _fields_ = [
        ("momentum", C.c_float),
        ("dampening", C.c_float),
        ("nesterov", C.c_bool),
        ("velocity", C.POINTER(C.POINTER(Tensor))),
    ]


_vp, _u32, _u64, _i32, _f32, _int, _sz = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32, C.c_float, C.c_int, C.c_size_t
_PT, _PQ = C.POINTER(Tensor), C.POINTER(QuantizedTensor)
_fp, _i8p, _i32p = C.POINTER(C.c_float), C.POINTER(C.c_int8), C.POINTER(C.c_int32)

# name -> (restype, argtypes)
PROTOTYPES = {
    # ---- rplhip.h
    "rplhip_init": (_int, []),
    "rplhip_last_error": (C.c_char_p, []),
    "rplhip_device_info": (_int, [C.c_char_p, _sz, C.POINTER(_int), C.POINTER(_int)]),
    "rplhip_malloc": (_int, [C.POINTER(_vp), _sz]),
    "rplhip_free": (_int, [_vp]),
    "rplhip_memcpy_htod": (_int, [_vp, _vp, _sz]),
    "rplhip_memcpy_dtoh": (_int, [_vp, _vp, _sz]),
    "rplhip_memcpy_dtod": (_int, [_vp, _vp, _sz, _vp]),
    "rplhip_memset": (_int, [_vp, _int, _sz, _vp]),
    "rplhip_synchronize": (_int, []),
    "rplhip_stream_create": (_int, [C.POINTER(_vp)]),
    "rplhip_stream_destroy": (_int, [_vp]),
    "rplhip_stream_synchronize": (_int, [_vp]),
    "rplhip_event_create": (_int, [C.POINTER(_vp)]),
    "rplhip_event_destroy": (_int, [_vp]),
    "rplhip_event_record": (_int, [_vp, _vp]),
    "rplhip_event_synchronize": (_int, [_vp]),
    "rplhip_event_elapsed_ms": (_int, [C.POINTER(_f32), _vp, _vp]),
    "rplhip_sgemm": (_int, [_int, _int, _u32, _u32, _u32, _f32, _vp, _u32, _vp, _u32, _f32, _vp, _u32, _vp]),
    "rplhip_sgemm_batched": (_int, [_int, _int, _u32, _u32, _u32, _f32, _vp, _u32, _u64, _vp, _u32, _u64, _f32, _vp,
                                    _u32, _u64, _u32, _int, _vp]),
    "rplhip_gemm_int8": (_int, [_vp, _vp, _vp, _u32, _u32, _u32, _f32, _f32, _f32, _i32, _i32, _vp]),
    "rplhip_gemm_int8_noalloc": (_int, [_vp, _vp, _vp, _u32, _u32, _u32, _f32, _f32, _f32, _i32, _i32, _vp]),
    "rplhip_linear_int8": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "rplhip_linear_int8_dequant": (_int, [_vp, _vp, _int, _vp, _vp, _int, _vp, _u32, _u32, _u32, _vp]),
    "rplhip_gemm_int8_dequant": (_int, [_vp, _vp, _int, _vp, _vp, _int, _vp, _u32, _u32, _u32, _vp]),
    "rplhip_quantize_int8": (_int, [_vp, _u64, _f32, _i32, _vp, _vp]),
    "rplhip_quantize_symmetric": (_int, [_vp, _u64, _vp, _vp, _vp]),
    "rplhip_quantize_asymmetric": (_int, [_vp, _u64, _vp, _vp, _vp, _vp]),
    "rplhip_quantize_per_channel": (_int, [_vp, _u32, _u32, _vp, _vp, _vp]),
    "rplhip_dequantize_int8": (_int, [_vp, _u64, _f32, _i32, _vp, _vp]),
    "rplhip_min_max": (_int, [_vp, _u64, _vp, _vp]),
    "rplhip_get_min_max": (_int, [_vp, _u64, _vp, _vp]),
    "rplhip_add_broadcast": (_int, [_vp, _vp, _vp, _u64, _u64, _vp]),
    "rplhip_relu": (_int, [_vp, _vp, _u64, _vp]),
    "rplhip_bias_add_relu": (_int, [_vp, _vp, _vp, _vp, _u64, _u64, _vp]),
    "rplhip_relu_backward": (_int, [_vp, _vp, _vp, _u64, _vp]),
    "rplhip_accumulate": (_int, [_vp, _vp, _u64, _vp]),
    "rplhip_bias_grad": (_int, [_vp, _u64, _vp, _u64, _vp]),
    "rplhip_mse_loss": (_int, [_vp, _vp, _u64, _vp, _vp]),
    "rplhip_mse_backward": (_int, [_vp, _vp, _u64, _vp, _vp, _vp]),
    "rplhip_sgd_step": (_int, [_vp, _vp, _vp, _u64, _f32, _f32, _f32, _f32, _int, _vp]),
    "rplhip_sigmoid": (_int, [_vp, _vp, _u64, _vp]),
    "rplhip_tanh": (_int, [_vp, _vp, _u64, _vp]),
    "rplhip_gelu": (_int, [_vp, _vp, _u64, _vp]),
    "rplhip_attention": (_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp]),
    "rplhip_fake_quant": (_int, [_vp, _vp, _u64, _f32, _f32, _vp]),
    "rplhip_float_to_half": (_int, [_vp, _vp, _u64, _vp]),
    "rplhip_half_to_float": (_int, [_vp, _vp, _u64, _vp]),
    "rplhip_fill": (_int, [_vp, _u64, _f32, _vp]),
    # ---- rpl.h
    "tensor_create": (_PT, [_u32, C.POINTER(_u32), C.c_bool]),
    "tensor_free": (None, [_PT]),
    "rpitorch_aligned_alloc": (_vp, [_sz, _sz]),
    "rpitorch_aligned_free": (None, [_vp]),
    "tensor_fill": (None, [_PT, _f32]),
    "rpl_gpu_init": (C.c_bool, []),
    "rpl_gpu_shutdown": (None, []),
    "tensor_to_gpu": (None, [_PT]),
    "tensor_from_gpu": (None, [_PT]),
    "tensor_sigmoid_gpu": (None, [_PT, _PT]),
    "tensor_tanh_gpu": (None, [_PT, _PT]),
    "tensor_gelu_gpu": (None, [_PT, _PT]),
    "tensor_add_gpu": (None, [_PT, _PT, _PT]),
    "tensor_matmul_gpu": (None, [_PT, _PT, _PT]),
    "tensor_relu_gpu": (None, [_PT, _PT]),
    "tensor_gemm": (None, [_PT, _PT, _PT, _f32, _f32, C.c_bool, C.c_bool]),
    "tensor_matmul": (_PT, [_PT, _PT]),
    "gemm_optimized_cortex_a72": (None, [_fp, _fp, _fp, _int, _int, _int, _int, _int, _int]),
    "parallel_gemm_optimized": (None, [_fp, _fp, _fp, _u32, _u32, _u32]),
    "gemm_init_buffers": (None, []),
    "gemm_free_buffers": (None, []),
    "tensor_quantize_int8": (_PQ, [_PT, _f32, _i32]),
    "tensor_quantize_int8_symmetric": (_PQ, [_PT]),
    "tensor_quantize_int8_asymmetric": (_PQ, [_PT]),
    "tensor_quantize_per_channel": (C.POINTER(PerChannelQuantizedTensor), [_PT, _u32]),
    "per_channel_quantized_tensor_free": (None, [C.POINTER(PerChannelQuantizedTensor)]),
    "quantized_tensor_free": (None, [_PQ]),
    "tensor_get_min_max": (None, [_PT, _fp, _fp]),
    "tensor_dequantize_int8": (_PT, [_PQ]),
    "gemm_int8": (None, [_i8p, _i8p, _i32p, _u32, _u32, _u32, _f32, _f32, _f32, _i32, _i32]),
    "linear_int8": (None, [_PQ, _PQ, _PQ, _i32p, _u32, _u32, _u32]),
    "calibrator_create": (C.POINTER(QuantizationCalibrator), []),
    "calibrator_update": (None, [C.POINTER(QuantizationCalibrator), _PT]),
    "calibrator_compute_params": (None, [C.POINTER(QuantizationCalibrator), C.c_bool]),
    "calibrator_free": (None, [C.POINTER(QuantizationCalibrator)]),
    "tensor_add": (_PT, [_PT, _PT]),
    "tensor_add_out": (None, [_PT, _PT, _PT]),
    "tensor_relu": (_PT, [_PT]),
    "tensor_mse_loss": (_PT, [_PT, _PT]),
    "tensor_backward": (None, [_PT]),
    "tensor_zero_grad": (None, [_PT]),
    "backward_add": (None, [_PT]),
    "backward_matmul": (None, [_PT]),
    "backward_relu": (None, [_PT]),
    "backward_mse": (None, [_PT]),
    "linear_create": (C.POINTER(Linear), [_u32, _u32]),
    "linear_forward": (_PT, [C.POINTER(Linear), _PT]),
    "linear_free": (None, [C.POINTER(Linear)]),
    "optimizer_sgd_create": (C.POINTER(Optimizer), [C.POINTER(_PT), _u32, _f32, _f32, _f32, _f32, C.c_bool]),
    "optimizer_sgd_step": (None, [C.POINTER(Optimizer)]),
    "scaled_dot_product_attention": (_PT, [_PT, _PT, _PT, _PT, _f32, C.c_bool]),
    "tensor_to_half": (C.POINTER(HalfTensor), [_PT]),
    "tensor_from_half": (_PT, [C.POINTER(HalfTensor)]),
    "half_tensor_free": (None, [C.POINTER(HalfTensor)]),
    "fake_quantize_create": (C.POINTER(FakeQuantize), []),
    "fake_quantize_forward": (_PT, [C.POINTER(FakeQuantize), _PT]),
    "backward_fake_quant": (None, [_PT]),
    "fake_quantize_free": (None, [C.POINTER(FakeQuantize)]),
    "rpl_last_error": (C.c_char_p, []),
    "rpl_clear_last_error": (None, []),
    "rpl_gpu_synchronize": (None, []),
    "rpl_gpu_stream": (_vp, []),
    "rpl_tensor_device_data": (_fp, [_PT]),
    "rpl_tensor_device_grad": (_fp, [_PT]),
    "rpl_fill_uniform": (None, [_fp, _u64, _u64, _f32, _f32]),
    "rpl_fill_normal": (None, [_fp, _u64, _u64, _f32, _f32]),
    "rpl_fill_labels": (None, [C.POINTER(_u32), _fp, _u64, _u64, _u32]),
}


def load(path=LIB_PATH):
    """Load librpl.so and declare every prototype; raises if not built."""
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = C.CDLL(path)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def check(status, what=""):
    """Raise RplError for a non-OK rplhip status."""
    if status != OK:
        msg = lib().rplhip_last_error().decode(errors="replace")
        raise RplError(status, f"{what}: {msg}" if what else msg)


def ptr(a):
    """Host pointer of a contiguous numpy array."""
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


class DeviceBuffer:
    """A device allocation from rplhip_malloc (freed on close / GC)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().rplhip_malloc(C.byref(p), self.nbytes), "rplhip_malloc")
        self.ptr = p

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            check(lib().rplhip_memcpy_htod(b.ptr, ptr(a), a.nbytes), "htod")
        b.dtype, b.shape = a.dtype, a.shape
        return b

    def to_array(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        if out.nbytes:
            check(lib().rplhip_memcpy_dtoh(ptr(out), self.ptr, out.nbytes), "dtoh")
        return out

    def close(self):
        if self.ptr is not None and _LIB is not None:
            _LIB.rplhip_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def fill_uniform(n, seed, lo=-1.0, hi=1.0):
    out = np.empty(int(n), dtype=np.float32)
    lib().rpl_fill_uniform(out.ctypes.data_as(_fp), out.size, seed, lo, hi)
    return out


def fill_normal(n, seed, mean=0.0, std=1.0):
    out = np.empty(int(n), dtype=np.float32)
    lib().rpl_fill_normal(out.ctypes.data_as(_fp), out.size, seed, mean, std)
    return out


def fill_labels(n, seed, classes):
    labels = np.empty(int(n), dtype=np.uint32)
    one_hot = np.empty((int(n), classes), dtype=np.float32)
    lib().rpl_fill_labels(labels.ctypes.data_as(C.POINTER(_u32)), one_hot.ctypes.data_as(_fp), labels.size, seed,
                          classes)
    return labels, one_hot
