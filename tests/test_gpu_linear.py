"""Linear forward/backward and the MLP training step on the device, through
the reference's own API (linear_create / linear_forward / tensor_relu /
tensor_mse_loss / tensor_backward) with GPU-resident tensors.

fp32 bar (as BASELINE.json's north star states it): each GEMM-shaped output
within max |err| / sum|terms| <= 1e-5 * sqrt(K), K its reduction length,
checked op by op on the inputs the device itself used; elementwise outputs
bit-exact or within one ulp; the MSE loss within a bound derived from its
reduction tree."""
import ctypes as C

import numpy as np
import pytest

import rpl_amd
from conftest import bits_equal, seed
from gpu_util import down, empty, say, up

pytestmark = pytest.mark.gpu


def tensor_from(lib, arr, requires_grad=False):
    arr = np.ascontiguousarray(arr, np.float32)
    shape = (C.c_uint32 * arr.ndim)(*arr.shape)
    t = lib.tensor_create(arr.ndim, shape, requires_grad)
    C.memmove(t.contents.data, arr.ctypes.data, arr.nbytes)
    return t


def host(t, shape, grad=False):
    p = t.contents.grad if grad else t.contents.data
    return np.ctypeslib.as_array(p, shape=(t.contents.size,)).copy().reshape(shape)


def run_mlp(lib, X, Y, W1, b1, W2, b2):
    """One training step through include/rpl.h with everything GPU-resident.
    Returns the device's outputs and the intermediates every later op read
    (h, a = relu(h), o and their gradients), so that each op can be checked
    against the oracle on exactly the inputs the device used."""
    B, IN = X.shape
    H, O = W1.shape[0], W2.shape[0]
    l1, l2 = lib.linear_create(IN, H), lib.linear_create(H, O)
    for layer, W, bb in ((l1, W1, b1), (l2, W2, b2)):
        C.memmove(layer.contents.weight.contents.data, W.ctypes.data, W.nbytes)
        C.memmove(layer.contents.bias.contents.data, bb.ctypes.data, bb.nbytes)
        lib.tensor_to_gpu(layer.contents.weight)
        lib.tensor_to_gpu(layer.contents.bias)
    tX, tY = tensor_from(lib, X), tensor_from(lib, Y)
    lib.tensor_to_gpu(tX)
    lib.tensor_to_gpu(tY)
    h = lib.linear_forward(l1, tX)
    a = lib.tensor_relu(h)
    o = lib.linear_forward(l2, a)
    loss = lib.tensor_mse_loss(o, tY)
    assert all(t.contents.device == rpl_amd.DEVICE_GPU for t in (h, a, o, loss))
    lib.tensor_backward(loss)
    for t in (loss, o, a, h, l1.contents.weight, l1.contents.bias, l2.contents.weight, l2.contents.bias):
        lib.tensor_from_gpu(t)
    r = dict(loss=host(loss, (1,))[0], o=host(o, (B, O)), a=host(a, (B, H)), h=host(h, (B, H)),
             dO=host(o, (B, O), True), dA=host(a, (B, H), True), dH=host(h, (B, H), True),
             dW1=host(l1.contents.weight, (H, IN), True), db1=host(l1.contents.bias, (H,), True),
             dW2=host(l2.contents.weight, (O, H), True), db2=host(l2.contents.bias, (O,), True))
    err = lib.rpl_last_error()
    assert not err, err
    return r


def _rel(got, want, scale):
    """max |got - want| / scale (float64), scale = sum of |terms| per output."""
    return float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64)) / (scale + 1e-30)))


def mse_depth(n):
    """Longest chain of dependent adds in the device's MSE reduction
    (linear.hip).  n <= 2^18, k_sqerr_single: a strided sum per thread over
    1024 threads (4 consecutive elements per step), a 64-lane butterfly (6
    adds), the 16 wave sums in order.
    Larger n, k_sqerr_partial / k_sqerr_finish: a grid-stride sum per thread
    over at most 1024 x 256 threads, a 64-lane butterfly, 4 wave partials,
    then the same for <= 1024 block partials in one block."""
    if n <= 1 << 18:
        # 128-bit loop: 4 adds per 4096 elements; then at most one remainder add
        return 4 * -(-n // 4096) + 1 + 6 + 16
    g = min(1024, max(1, (n + 255) // 256))
    per_thread = -(-n // (g * 256))
    return per_thread + 6 + 4 + -(-g // 256) + 6 + 4


def check_mlp(orc, r, X, Y, W1, b1, W2, b2):
    """Every op of the step against the oracle on the device's own inputs.

    GEMM-shaped outputs (h, o, dA, dW1, dW2, db1, db2) at the north-star
    bound max |err| / sum|terms| <= 1e-5 * sqrt(K), K the op's reduction
    length; ReLU, its backward and the bias add are elementwise with one
    rounding and must match bit for bit (bias add, ReLU) or within one ulp
    (dO, whose FMA contraction could differ); the loss, a sum of n squares,
    within (depth + 4) * 2^-24 relative of its float64 value, depth being
    the longest chain of adds in the device's reduction."""
    B, IN = X.shape
    H, O = W1.shape[0], W2.shape[0]
    tol = lambda K: 1e-5 * np.sqrt(K)  # noqa: E731
    X64, W164, W264 = (v.astype(np.float64) for v in (X, W1, W2))
    # Forward: h = X W1^T + b1, a = relu(h), o = a W2^T + b2.
    h_ref = orc.add_broadcast(orc.sgemm(X, W1, np.zeros((B, H), np.float32), B, H, IN, tb=True), b1)
    assert _rel(r["h"], h_ref, np.abs(X64) @ np.abs(W164.T) + np.abs(b1)) <= tol(IN)
    assert bits_equal(r["a"], orc.relu(r["h"]))
    o_ref = orc.add_broadcast(orc.sgemm(r["a"], W2, np.zeros((B, O), np.float32), B, O, H, tb=True), b2)
    assert _rel(r["o"], o_ref, np.abs(r["a"].astype(np.float64)) @ np.abs(W264.T) + np.abs(b2)) <= tol(H)
    # Loss on the device's o.
    d64 = r["o"].astype(np.float64) - Y
    exact = float(np.mean(d64 * d64))
    assert abs(float(r["loss"]) - exact) <= (mse_depth(r["o"].size) + 4) * 2.0 ** -24 * exact
    # Backward, op by op on the device's upstream gradients.
    dO_ref = orc.mse_backward(r["o"], Y, 1.0, np.zeros((B, O), np.float32))
    assert np.all(np.abs(r["dO"].astype(np.float64) - dO_ref) <= 2.0 ** -23 * np.abs(dO_ref.astype(np.float64)))
    dA_ref, dW2_ref = orc.matmul_backward(r["dO"], r["a"], W2, B, O, H, (O, H), da=np.zeros((B, H), np.float32),
                                          db=np.zeros((O, H), np.float32))
    dO64, a64 = np.abs(r["dO"].astype(np.float64)), np.abs(r["a"].astype(np.float64))
    assert _rel(r["dA"], dA_ref, dO64 @ np.abs(W264)) <= tol(O)
    assert _rel(r["dW2"], dW2_ref, dO64.T @ a64) <= tol(B)
    _, db2_ref = orc.add_backward(r["dO"], None, np.zeros(O, np.float32))
    assert _rel(r["db2"], db2_ref, dO64.sum(0)) <= tol(B)
    assert bits_equal(r["dH"], orc.relu_backward(r["h"], r["dA"], np.zeros((B, H), np.float32)))
    _, dW1_ref = orc.matmul_backward(r["dH"], X, W1, B, H, IN, (H, IN), db=np.zeros((H, IN), np.float32))
    dH64 = np.abs(r["dH"].astype(np.float64))
    assert _rel(r["dW1"], dW1_ref, dH64.T @ np.abs(X64)) <= tol(B)
    _, db1_ref = orc.add_backward(r["dH"], None, np.zeros(H, np.float32))
    assert _rel(r["db1"], db1_ref, dH64.sum(0)) <= tol(B)
    # The step computes dO and dH inside the bias-gradient passes of the
    # adds that produced o and h; they must be the bits of the device's own
    # MSE and ReLU backward kernels on the same tensors.
    lib = rpl_amd.lib()
    # (both accumulate: into zeros, the bits of the step's overwrite)
    do_, dh_ = up(np.zeros(r["o"].size, np.float32)), up(np.zeros(r["h"].size, np.float32))
    dev_o, dev_y, dev_g0 = up(r["o"]), up(Y), up(np.float32([1.0]))  # held: a freed buffer could be reused
    rpl_amd.check(lib.rplhip_mse_backward(dev_o.ptr, dev_y.ptr, r["o"].size, dev_g0.ptr, do_.ptr, None))
    dev_h, dev_da = up(r["h"]), up(r["dA"])
    rpl_amd.check(lib.rplhip_relu_backward(dev_h.ptr, dev_da.ptr, dh_.ptr, r["h"].size, None))
    assert bits_equal(r["dO"], down(do_, np.float32, r["o"].shape))
    assert bits_equal(r["dH"], down(dh_, np.float32, r["h"].shape))


def _two_consumer_graph(lib, X, Y, W1, b1, W2, b2, resident):
    """h = X W1^T + b1 feeds two ReLUs, each through layer 2; their sum goes
    into the MSE loss.  Returns every tensor's values and gradients."""
    B, IN = X.shape
    H, O = W1.shape[0], W2.shape[0]
    l1, l2 = lib.linear_create(IN, H), lib.linear_create(H, O)
    for layer, W, bb in ((l1, W1, b1), (l2, W2, b2)):
        C.memmove(layer.contents.weight.contents.data, W.ctypes.data, W.nbytes)
        C.memmove(layer.contents.bias.contents.data, bb.ctypes.data, bb.nbytes)
    params = [l1.contents.weight, l1.contents.bias, l2.contents.weight, l2.contents.bias]
    tX, tY = tensor_from(lib, X), tensor_from(lib, Y)
    if resident:
        for t in params + [tX, tY]:
            lib.tensor_to_gpu(t)
    for t in params:
        lib.tensor_zero_grad(t)
    h = lib.linear_forward(l1, tX)
    a1, a2 = lib.tensor_relu(h), lib.tensor_relu(h)
    o1, o2 = lib.linear_forward(l2, a1), lib.linear_forward(l2, a2)
    ssum = lib.tensor_add(o1, o2)
    loss = lib.tensor_mse_loss(ssum, tY)
    lib.tensor_backward(loss)
    err = lib.rpl_last_error()
    assert not err, err
    named = dict(loss=(loss, (1,)), s=(ssum, (B, O)), o1=(o1, (B, O)), o2=(o2, (B, O)), a1=(a1, (B, H)),
                 a2=(a2, (B, H)), h=(h, (B, H)), W1=(params[0], (H, IN)), b1=(params[1], (H,)),
                 W2=(params[2], (O, H)), b2=(params[3], (O,)))
    out = {}
    for k, (t, shape) in named.items():
        if t.contents.device == rpl_amd.DEVICE_GPU:
            lib.tensor_from_gpu(t)
        assert (t.contents.device == rpl_amd.DEVICE_GPU) == resident, k
        out[k] = host(t, shape)
        out["d" + k] = host(t, shape, True)
    for t in (loss, ssum, o2, o1, a2, a1, h, tX, tY):
        lib.tensor_free(t)
    lib.linear_free(l1)
    lib.linear_free(l2)
    return out


def test_fused_backward_matches_staged(gpu):
    # All tensors GPU-resident, the backward folds the MSE and both ReLU
    # backwards into the add-backward passes that follow them (h's pass runs
    # once per ReLU, each time on h's gradient so far, as the reference's
    # recursion does); with the tensors in host memory every op is staged
    # and runs the standalone kernels.  Same kernels otherwise, so every
    # value and gradient must agree bit for bit.
    lib = gpu
    B, IN, H, O = 256, 96, 64, 10
    rng = np.random.default_rng(33)
    X = rng.uniform(0, 1, (B, IN)).astype(np.float32)
    Y = rng.uniform(0, 1, (B, O)).astype(np.float32)
    W1 = rng.uniform(-0.2, 0.2, (H, IN)).astype(np.float32)
    W2 = rng.uniform(-0.3, 0.3, (O, H)).astype(np.float32)
    b1 = rng.uniform(-0.1, 0.1, H).astype(np.float32)
    b2 = rng.uniform(-0.1, 0.1, O).astype(np.float32)
    say("fused backward vs staged, resident")
    dev = _two_consumer_graph(lib, X, Y, W1, b1, W2, b2, True)
    say("fused backward vs staged, host")
    hst = _two_consumer_graph(lib, X, Y, W1, b1, W2, b2, False)
    for k in dev:
        assert bits_equal(dev[k], hst[k]), k
    assert np.any(dev["dh"] != 0) and np.any(dev["db1"] != 0)


def test_mlp_step_golden(gpu, golden, orc):
    X, Y = golden["mlp_X"], golden["mlp_Y"]
    W1, b1, W2, b2 = golden["mlp_W1"], golden["mlp_b1"], golden["mlp_W2"], golden["mlp_b2"]
    say("mlp golden step")
    r = run_mlp(gpu, X, Y, W1, b1, W2, b2)
    ref = orc.mlp_step(X, Y, W1, b1, W2, b2)
    for k in ("o", "dW1", "db1", "dW2", "db2"):  # the oracle reproduces the reference golden bit-exactly
        assert np.array_equal(ref[k], golden[f"mlp_{k}"])
    check_mlp(orc, r, X, Y, W1, b1, W2, b2)


def test_config2_mlp_step(gpu, orc):
    """Config 2: MLP 784 -> 128 (ReLU) -> 10, batch 4096, MSE."""
    B, IN, H, O = 4096, 784, 128, 10
    X = rpl_amd.fill_uniform(B * IN, seed(2, 0), 0.0, 1.0).reshape(B, IN)
    _, Y = rpl_amd.fill_labels(B, seed(2, 1), O)
    W1 = rpl_amd.fill_uniform(H * IN, seed(2, 2), -np.sqrt(6 / IN), np.sqrt(6 / IN)).reshape(H, IN)
    W2 = rpl_amd.fill_uniform(O * H, seed(2, 3), -np.sqrt(6 / H), np.sqrt(6 / H)).reshape(O, H)
    b1, b2 = np.zeros(H, np.float32), np.zeros(O, np.float32)
    say("config 2: mlp step")
    r = run_mlp(gpu, X, Y, W1, b1, W2, b2)
    check_mlp(orc, r, X, Y, W1, b1, W2, b2)


def test_gradient_accumulation_and_zero_grad(gpu):
    """Device gradients are zeroed lazily (marked, then overwritten by the
    first accumulation).  Two backward passes without tensor_zero_grad add
    up -- exactly twice the first pass's gradients, since both passes compute
    the same values and doubling is exact -- and after tensor_zero_grad both
    tensor_from_gpu and rpl_tensor_device_grad see zeros, and a further pass
    equals the first bit for bit."""
    lib = gpu
    B, IN, H, O = 256, 96, 64, 10
    rng = np.random.default_rng(21)
    X = rng.uniform(0, 1, (B, IN)).astype(np.float32)
    Y = np.eye(O, dtype=np.float32)[rng.integers(0, O, B)]
    l1, l2 = lib.linear_create(IN, H), lib.linear_create(H, O)
    for layer in (l1, l2):
        lib.tensor_to_gpu(layer.contents.weight)
        lib.tensor_to_gpu(layer.contents.bias)
    tX, tY = tensor_from(lib, X), tensor_from(lib, Y)
    lib.tensor_to_gpu(tX)
    lib.tensor_to_gpu(tY)
    params = (l1.contents.weight, l1.contents.bias, l2.contents.weight, l2.contents.bias)
    shapes = ((H, IN), (H,), (O, H), (O,))

    def step():
        h = lib.linear_forward(l1, tX)
        a = lib.tensor_relu(h)
        o = lib.linear_forward(l2, a)
        loss = lib.tensor_mse_loss(o, tY)
        lib.tensor_backward(loss)
        for t in (loss, o, a, h):
            lib.tensor_free(t)

    def grads():
        out = []
        for t, shp in zip(params, shapes):
            lib.tensor_from_gpu(t)
            out.append(host(t, shp, grad=True))
        return out

    say("gradient accumulation: zero_grad, one pass")
    for t in params:
        lib.tensor_zero_grad(t)
    step()
    g1 = grads()
    say("gradient accumulation: second pass without zero_grad")
    step()
    g2 = grads()
    for a, b in zip(g1, g2):
        assert bits_equal(b, a * np.float32(2))
    say("gradient accumulation: zero_grad, reads")
    for t in params:
        lib.tensor_zero_grad(t)
    for t, shp in zip(params, shapes):
        t.contents.grad[0] = 7.0  # stale host value must be replaced by the device's zeros
        lib.tensor_from_gpu(t)
        assert not host(t, shp, grad=True).any()
        dg = lib.rpl_tensor_device_grad(t)
        buf = np.full(int(np.prod(shp)), 5.0, np.float32)
        rpl_amd.check(lib.rplhip_memcpy_dtoh(buf.ctypes.data, dg, buf.nbytes))
        assert not buf.any()
    say("gradient accumulation: pass after zero_grad")
    step()
    for a, b in zip(g1, grads()):
        assert bits_equal(b, a)
    assert not lib.rpl_last_error()
    lib.tensor_free(tX)
    lib.tensor_free(tY)
    lib.linear_free(l1)
    lib.linear_free(l2)


def test_backward_matmul_layout_guess(gpu, golden):
    lib = gpu
    tA, tB = tensor_from(lib, golden["bmm_A"], True), tensor_from(lib, golden["bmm_B"], True)
    lib.tensor_to_gpu(tA)
    lib.tensor_to_gpu(tB)
    say("backward_matmul layout guess")
    out = lib.tensor_matmul(tA, tB)
    lib.tensor_backward(out)
    for t in (out, tA, tB):
        lib.tensor_from_gpu(t)
    assert np.array_equal(host(out, (2, 2)), golden["bmm_out"])
    assert np.array_equal(host(tA, (2, 2), True), golden["bmm_dA"])
    assert np.array_equal(host(tB, (2, 2), True), golden["bmm_dB"])


@pytest.mark.parametrize("n,nb", [(4096 * 128, 128), (4096 * 10, 10), (1000, 7), (1003, 7), (64, 64), (5, 1)])
def test_bias_pieces_vs_oracle(gpu, orc, n, nb):
    lib = gpu
    rng = np.random.default_rng(n + nb)
    mm = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(nb).astype(np.float32)
    dmm, db_, dout, dact = up(mm), up(b), empty(n, np.float32), empty(n, np.float32)
    say("bias_add_relu", n, nb)
    rpl_amd.check(lib.rplhip_bias_add_relu(dmm.ptr, db_.ptr, dout.ptr, dact.ptr, n, nb, None))
    out = orc.add_broadcast(mm, b)
    assert np.array_equal(down(dout, np.float32, (n,)), out)
    assert np.array_equal(down(dact, np.float32, (n,)), orc.relu(out))
    g0 = rng.standard_normal(nb).astype(np.float32)
    dg = up(g0)
    say("bias_grad", n, nb)
    rpl_amd.check(lib.rplhip_bias_grad(dmm.ptr, n, dg.ptr, nb, None))
    _, ref = orc.add_backward(mm, None, g0)
    scale = np.zeros(nb)
    np.add.at(scale, np.arange(n) % nb, np.abs(mm))
    assert np.max(np.abs(down(dg, np.float32, (nb,)) - ref) / (scale + np.abs(g0))) <= 1e-5 * np.sqrt(n / nb + 1)
    dy = rng.standard_normal(n).astype(np.float32)
    dx0 = rng.standard_normal(n).astype(np.float32)
    ddy, ddx = up(dy), up(dx0)
    say("relu_backward", n)
    rpl_amd.check(lib.rplhip_relu_backward(dmm.ptr, ddy.ptr, ddx.ptr, n, None))
    assert np.array_equal(down(ddx, np.float32, (n,)), orc.relu_backward(mm, dy, dx0))


@pytest.mark.parametrize("n,off", [(1, 0), (3, 0), (5, 1), (4097, 0), (4099, 1), (1 << 18, 0), (1 << 18, 1),
                                   ((1 << 18) + 1, 0), (1 << 20, 0)])
def test_mse_loss_sizes(gpu, n, off):
    # One block up to 2^18 elements (128-bit loads when both inputs are
    # 16-byte aligned, `off` = 1 float misaligns them), partials beyond.
    lib = gpu
    rng = np.random.default_rng(n + off)
    p = rng.standard_normal(n + off).astype(np.float32)
    t = rng.standard_normal(n + off).astype(np.float32)
    dp, dt, dl = up(p), up(t), empty(1, np.float32)
    say("mse sizes", n, off)
    rpl_amd.check(lib.rplhip_mse_loss(C.c_void_p(dp.ptr.value + 4 * off), C.c_void_p(dt.ptr.value + 4 * off), n,
                                      dl.ptr, None))
    loss = down(dl, np.float32, (1,))[0]
    d64 = p[off:].astype(np.float64) - t[off:]
    exact = float(np.mean(d64 * d64))
    assert abs(float(loss) - exact) <= (mse_depth(n) + 4) * 2.0 ** -24 * exact


def test_mse_vs_oracle(gpu, orc):
    lib = gpu
    n = 40960
    rng = np.random.default_rng(2)
    p = rng.standard_normal(n).astype(np.float32)
    t = rng.standard_normal(n).astype(np.float32)
    dp, dt, dl = up(p), up(t), empty(1, np.float32)
    say("mse")
    rpl_amd.check(lib.rplhip_mse_loss(dp.ptr, dt.ptr, n, dl.ptr, None))
    loss = down(dl, np.float32, (1,))[0]
    d64 = p.astype(np.float64) - t
    exact = float(np.mean(d64 * d64))
    # Both the device's tree and the reference's sequential sum are within
    # their depth * 2^-24 of the exact value (a sum of non-negative terms).
    assert abs(float(loss) - exact) <= (mse_depth(n) + 4) * 2.0 ** -24 * exact
    assert abs(float(orc.mse_loss(p, t)) - exact) <= (n + 4) * 2.0 ** -24 * exact
    g0 = up(np.float32([1.0]))
    d0 = rng.standard_normal(n).astype(np.float32)
    dd = up(d0)
    rpl_amd.check(lib.rplhip_mse_backward(dp.ptr, dt.ptr, n, g0.ptr, dd.ptr, None))
    np.testing.assert_allclose(down(dd, np.float32, (n,)), orc.mse_backward(p, t, 1.0, d0), rtol=1e-6, atol=1e-7)
