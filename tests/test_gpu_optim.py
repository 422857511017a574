"""optimizer_sgd_step (src/rpl_training.c:70-114) on the device.

Bit-exact against the reference build's golden vectors (parameters,
in-place gradients and momentum buffers after each of two steps), through
the device ABI and through include/rpl.h with host-resident and
GPU-resident parameters; then a short MLP training loop on the device
against the oracle (fp32 GEMM bound, as for the training step)."""
import ctypes as C

import numpy as np
import pytest

import rpl_amd
from conftest import bits_equal, seed
from gpu_util import down, say, up
from test_gpu_linear import host, tensor_from

pytestmark = pytest.mark.gpu

CASES = ["plain", "wd", "mom", "nest"]


def hyper(golden, name):
    lr, mom, damp, wd, nest = (float(x) for x in golden[f"sgd_{name}_hyper"])
    return lr, mom, damp, wd, bool(nest)


@pytest.mark.parametrize("name", CASES)
def test_sgd_step_device_golden(gpu, golden, name):
    lib = gpu
    lr, mom, damp, wd, nest = hyper(golden, name)
    for k in range(2):
        p0 = golden[f"sgd_{name}_p{k}_init"]
        dp, dv = up(p0), up(np.zeros_like(p0))
        for step in range(2):
            dg = up(golden[f"sgd_{name}_s{step}_g{k}_in"])
            say("sgd device", name, k, step)
            rpl_amd.check(lib.rplhip_sgd_step(dp.ptr, dg.ptr, dv.ptr if mom else None, p0.size, lr, mom, damp, wd,
                                              int(nest), None))
            assert bits_equal(down(dp, np.float32, p0.shape), golden[f"sgd_{name}_s{step}_p{k}"])
            assert bits_equal(down(dg, np.float32, p0.shape), golden[f"sgd_{name}_s{step}_g{k}"])
            if mom:
                assert bits_equal(down(dv, np.float32, p0.shape), golden[f"sgd_{name}_s{step}_v{k}"])


@pytest.mark.parametrize("resident", [False, True])
@pytest.mark.parametrize("name", CASES)
def test_optimizer_sgd_rpl_api(gpu, golden, name, resident):
    lib = gpu
    lr, mom, damp, wd, nest = hyper(golden, name)
    shapes = [(37, 53), (53,)]
    ps = [tensor_from(lib, golden[f"sgd_{name}_p{k}_init"].reshape(s), requires_grad=True)
          for k, s in enumerate(shapes)]
    if resident:
        for t in ps:
            lib.tensor_to_gpu(t)
    arr = (C.POINTER(rpl_amd.Tensor) * 2)(*ps)
    opt = lib.optimizer_sgd_create(arr, 2, lr, mom, damp, wd, nest)
    for step in range(2):
        for k, t in enumerate(ps):
            gr = golden[f"sgd_{name}_s{step}_g{k}_in"]
            C.memmove(t.contents.grad, gr.ctypes.data, gr.nbytes)
            if resident:
                rpl_amd.check(lib.rplhip_memcpy_htod(lib.rpl_tensor_device_grad(t), gr.ctypes.data, gr.nbytes))
        say("sgd rpl.h", name, "resident" if resident else "host", step)
        lib.optimizer_sgd_step(opt)
        err = lib.rpl_last_error()
        assert not err, err
        st = C.cast(opt.contents.state, C.POINTER(rpl_amd.SGDState)).contents
        for k, t in enumerate(ps):
            if resident:
                assert t.contents.device == rpl_amd.DEVICE_GPU
                lib.tensor_from_gpu(t)
            n = t.contents.size
            assert bits_equal(host(t, (n,)), golden[f"sgd_{name}_s{step}_p{k}"])
            assert bits_equal(host(t, (n,), grad=True), golden[f"sgd_{name}_s{step}_g{k}"])
            if mom:
                v = st.velocity[k]
                # The momentum buffer of a resident parameter lives on the device.
                assert (v.contents.device == rpl_amd.DEVICE_GPU) == resident
                if resident:
                    lib.tensor_from_gpu(v)
                assert bits_equal(host(v, (n,)), golden[f"sgd_{name}_s{step}_v{k}"])
    for t in ps:
        lib.tensor_free(t)


@pytest.mark.parametrize("mom,damp,wd,nest", [(0.0, 0.0, 0.0, False), (0.9, 0.1, 1e-2, True), (0.5, 0.0, 0.0, False)])
def test_optimizer_sgd_many_params(gpu, orc, mom, damp, wd, nest):
    # More parameters than one launch takes (eight device tensors per launch),
    # of ragged sizes, with host-resident ones in between: every parameter
    # bit for bit as the oracle's per-tensor update, over two steps.
    lib = gpu
    lr = 0.05
    sizes = [1, 7, 256, 257, 1000, 65537, 3, 9, 1_200_000, 64, 5, 4097]
    on_host = {3, 9}
    ps, ref, vel = [], [], []
    for k, n in enumerate(sizes):
        a = rpl_amd.fill_uniform(n, seed(7, k), -1.0, 1.0)
        t = tensor_from(lib, a, requires_grad=True)
        if k not in on_host:
            lib.tensor_to_gpu(t)
        ps.append(t)
        ref.append(a.copy())
        vel.append(np.zeros(n, np.float32))
    arr = (C.POINTER(rpl_amd.Tensor) * len(ps))(*ps)
    opt = lib.optimizer_sgd_create(arr, len(ps), lr, mom, damp, wd, nest)
    for step in range(2):
        grads = []
        for k, t in enumerate(ps):
            gr = rpl_amd.fill_uniform(sizes[k], seed(8, 100 * step + k), -2.0, 2.0)
            grads.append(gr)
            C.memmove(t.contents.grad, gr.ctypes.data, gr.nbytes)
            if k not in on_host:
                rpl_amd.check(lib.rplhip_memcpy_htod(lib.rpl_tensor_device_grad(t), gr.ctypes.data, gr.nbytes))
        say("sgd many params", mom, damp, wd, nest, "step", step)
        lib.optimizer_sgd_step(opt)
        err = lib.rpl_last_error()
        assert not err, err
        for k, t in enumerate(ps):
            g = grads[k].copy()
            orc.sgd_step(ref[k], g, vel[k] if mom else None, lr, mom, damp, wd, nest)
            if k not in on_host:
                lib.tensor_from_gpu(t)
            assert bits_equal(host(t, (sizes[k],)), ref[k]), (step, k)
            assert bits_equal(host(t, (sizes[k],), grad=True), g), (step, k)
    for t in ps:
        lib.tensor_free(t)


def test_mlp_training_loop_on_device(gpu, orc):
    # Five steps of zero_grad / forward / backward / SGD with momentum, every
    # tensor GPU-resident, against the oracle's step + SGD on the same data.
    lib = gpu
    Bt, IN, H, O = 512, 784, 128, 10
    X = rpl_amd.fill_uniform(Bt * IN, seed(2, 0), 0.0, 1.0).reshape(Bt, IN)
    _, Y = rpl_amd.fill_labels(Bt, seed(2, 1), O)
    W1 = rpl_amd.fill_uniform(H * IN, seed(2, 2), -np.sqrt(6 / IN), np.sqrt(6 / IN)).reshape(H, IN)
    W2 = rpl_amd.fill_uniform(O * H, seed(2, 3), -np.sqrt(6 / H), np.sqrt(6 / H)).reshape(O, H)
    b1, b2 = np.zeros(H, np.float32), np.zeros(O, np.float32)
    lr, mom = 0.5, 0.9
    l1, l2 = lib.linear_create(IN, H), lib.linear_create(H, O)
    for layer, W, bb in ((l1, W1, b1), (l2, W2, b2)):
        C.memmove(layer.contents.weight.contents.data, W.ctypes.data, W.nbytes)
        C.memmove(layer.contents.bias.contents.data, bb.ctypes.data, bb.nbytes)
        lib.tensor_to_gpu(layer.contents.weight)
        lib.tensor_to_gpu(layer.contents.bias)
    tX, tY = tensor_from(lib, X), tensor_from(lib, Y)
    lib.tensor_to_gpu(tX)
    lib.tensor_to_gpu(tY)
    params = [l1.contents.weight, l1.contents.bias, l2.contents.weight, l2.contents.bias]
    arr = (C.POINTER(rpl_amd.Tensor) * 4)(*params)
    opt = lib.optimizer_sgd_create(arr, 4, lr, mom, 0.0, 0.0, False)
    ref = [W1.copy(), b1.copy(), W2.copy(), b2.copy()]
    vel = [np.zeros_like(r) for r in ref]
    for step in range(5):
        say("mlp training loop step", step)
        for t in params:
            lib.tensor_zero_grad(t)
        h = lib.linear_forward(l1, tX)
        a = lib.tensor_relu(h)
        o = lib.linear_forward(l2, a)
        loss = lib.tensor_mse_loss(o, tY)
        lib.tensor_backward(loss)
        lib.optimizer_sgd_step(opt)
        for t in (loss, o, a, h):
            lib.tensor_free(t)
        r = orc.mlp_step(X, Y, *ref)
        for k, gk in enumerate(("dW1", "db1", "dW2", "db2")):
            g = r[gk].copy()
            orc.sgd_step(ref[k], g, vel[k], lr, mom, 0.0, 0.0, False)
    err = lib.rpl_last_error()
    assert not err, err
    for k, (t, shape) in enumerate(zip(params, [(H, IN), (H,), (O, H), (O,)])):
        lib.tensor_from_gpu(t)
        got = host(t, shape)
        # Gradients agree to the fp32 GEMM bound each step; five steps of
        # lr 0.5 with momentum keep the drift well under 1e-4.
        assert np.max(np.abs(got - ref[k])) <= 1e-4 * (1 + np.max(np.abs(ref[k]))), k
        assert not np.array_equal(got, [W1, b1, W2, b2][k])  # the weights moved
    lib.tensor_free(tX)
    lib.tensor_free(tY)
    lib.linear_free(l1)
    lib.linear_free(l2)
