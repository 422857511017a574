"""CPU-side checks of the C ABI: the library loads, exports every function
include/*.h declares, refuses to compute without a gfx950 device (no CPU
fallback), and its seeded input generator is pinned."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import rpl_amd

DECL = re.compile(r"^\s*(?:[A-Za-z_][\w\s\*]*?[\s\*])([A-Za-z_]\w*)\s*\(", re.M)


def declared_functions(header):
    text = open(os.path.join(rpl_amd.INCLUDE_DIR, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = set()
    for stmt in text.split(";"):
        stmt = stmt.strip()
        if "(" not in stmt or stmt.startswith("#") or "typedef" in stmt or "{" in stmt:
            continue
        m = DECL.search(stmt)
        if m:
            names.add(m.group(1))
    return names


@pytest.mark.parametrize("header", ["rpl.h", "rplhip.h"])
def test_every_declared_symbol_is_exported(header):
    lib = rpl_amd.lib()
    names = declared_functions(header)
    assert len(names) > 15, names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    undeclared = [n for n in sorted(names) if n not in rpl_amd.PROTOTYPES]
    assert not undeclared, undeclared


def test_struct_layouts_match_reference():
    # Offsets of the reference's include/rpl.h:57-78 as gcc lays it out on
    # x86-64 (device/gpu_buffer sit between _alloc_size and is_leaf).
    T = rpl_amd.Tensor
    assert (T.device.offset, T.gpu_buffer.offset, T.is_leaf.offset, T.backward_fn.offset) == (112, 116, 120, 144)
    assert C.sizeof(T) == 152
    assert C.sizeof(rpl_amd.QuantizedTensor) == 56
    assert C.sizeof(rpl_amd.PerChannelQuantizedTensor) == 72
    # src/rpl_training.c:20-39 (the SGD golden vectors read the reference's
    # momentum buffers through these layouts).
    O, S = rpl_amd.Optimizer, rpl_amd.SGDState
    assert (O.learning_rate.offset, O.weight_decay.offset, O.num_params.offset, O.parameters.offset,
            O.state.offset, C.sizeof(O)) == (4, 8, 12, 16, 24, 32)
    assert (S.dampening.offset, S.nesterov.offset, S.velocity.offset, C.sizeof(S)) == (4, 8, 16, 24)
    # include/rpl.h:82-92 and src/rpl_quantization.c:174-179.
    H, F = rpl_amd.HalfTensor, rpl_amd.FakeQuantize
    assert (H.dims.offset, H.size.offset, H._allocation.offset, H.device.offset, C.sizeof(H)) == (8, 76, 80, 88, 96)
    assert (F.training.offset, F.num_batches_tracked.offset, C.sizeof(F)) == (16, 20, 24)


def test_no_device_fails_loudly(rpl):
    st = rpl.rplhip_init()
    if st == rpl_amd.OK:
        pytest.skip("a gfx950 device is present")
    assert st == rpl_amd.ERR_NO_DEVICE
    assert rpl.rplhip_last_error()
    # A compute call returns the status instead of computing on the CPU ...
    p = C.c_void_p()
    assert rpl.rplhip_malloc(C.byref(p), 16) == rpl_amd.ERR_NO_DEVICE
    x = np.ones(8, np.float32)
    assert rpl.rplhip_quantize_int8(rpl_amd.ptr(x), 8, 1.0, 0, rpl_amd.ptr(np.zeros(8, np.int8)), None) == rpl_amd.ERR_NO_DEVICE
    # ... and the reference API leaves outputs untouched and says why.
    Cout = np.full((2, 2), 7, np.int32)
    A = np.ones((2, 2), np.int8)
    rpl.gemm_int8(A.ctypes.data_as(C.POINTER(C.c_int8)), A.ctypes.data_as(C.POINTER(C.c_int8)),
                  Cout.ctypes.data_as(C.POINTER(C.c_int32)), 2, 2, 2, 1.0, 1.0, 1.0, 0, 0)
    assert np.all(Cout == 7)
    assert b"gfx950" in rpl.rpl_last_error() or b"device" in rpl.rpl_last_error()


def splitmix64(seed, i):
    m = (1 << 64) - 1
    z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def test_generator_pinned_and_split_independent():
    u = rpl_amd.fill_uniform(300000, 1234, -1.0, 1.0)
    for i in (0, 1, 2, 99999, 299999):
        want = np.float32(-1.0 + 2.0 * (splitmix64(1234, i) >> 40) / 16777216.0)
        assert u[i] == want
    # Element i does not depend on n (thread partition).
    assert np.array_equal(rpl_amd.fill_uniform(1000, 1234, -1.0, 1.0), u[:1000])
    z = rpl_amd.fill_normal(200000, 99)
    assert np.array_equal(rpl_amd.fill_normal(77, 99), z[:77])
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    labels, one_hot = rpl_amd.fill_labels(5000, 7, 10)
    assert labels.max() == 9 and np.array_equal(one_hot.argmax(1), labels) and np.all(one_hot.sum(1) == 1)


def test_add_out_rejects_sizes_that_do_not_broadcast(rpl):
    # The reference overruns its buffers here; the size check comes before
    # any device work, so it is visible without a GPU.
    def mk(n):
        shape = (C.c_uint32 * 1)(n)
        return rpl.tensor_create(1, shape, False)
    out, a, b = mk(12), mk(10), mk(4)
    rpl.tensor_add_out(out, a, b)
    assert b"do not broadcast" in rpl.rpl_last_error()
    for t in (out, a, b):
        rpl.tensor_free(t)
