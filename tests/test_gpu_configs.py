"""BASELINE configurations at full size on the GPU, checked against the oracle.

Configs 0-2 are compared element by element over the whole output.  The
oracle restatement runs the reference's loops in a few seconds at these
sizes.  The MLP (config 4) runs through torch_rs autograd at full size.
Its gradients are first checked bit for bit against the same step composed
explicitly from device ops.  That composition is then checked stage by stage
against the oracle over every element: elementwise stages bit for bit, GEMM
stages within 1e-5*sqrt(K)*(|A||B|) against the reference-order product
(the oracle's row-blocked loop split over threads), and the loss within the
summation bounds.  The timed MLP step (fused activation, split-K GEMMs) is
checked bit for bit against the eager step.  exp is checked exhaustively,
over all 2^32 inputs, against glibc.
"""
import numpy as np
import pytest

import gpu_util as U
import oracle as O
import torch_rs
from helpers import assert_bitwise_equal, ulp_of
from trs_backend.configs import generate

pytestmark = pytest.mark.gpu


def dev(a, requires_grad=False):
    return torch_rs.tensor(a, device="cuda", requires_grad=requires_grad)


def test_config0_relu_bias_full_bit_exact():
    x = generate("relu_bias", "x").reshape(4096, 4096)
    b = generate("relu_bias", "b")
    want = O.unary_contig(O.RELU, O.row_broadcast(O.ADD, x.ravel(), b, 4096, 4096))
    X, B = dev(x), dev(b)
    eager = (X + B).relu()
    assert eager.shape == (4096, 4096) and eager.stride() == (4096, 1)
    assert_bitwise_equal(eager.numpy().ravel(), want)
    fused = torch_rs.fuse(lambda x, b: (x + b).relu())(X, B)
    assert_bitwise_equal(fused.numpy().ravel(), want)


def test_config1_fused_chain_full_within_exp_bound():
    n = 1 << 28
    x, y, z = (generate("fused_chain", k) for k in ("x", "y", "z"))
    t = O.binary_contig(O.ADD, O.binary_contig(O.MUL, x, y), z)
    want = O.unary_contig(O.RELU, O.scalar_contig(O.S_SUB, O.unary_contig(O.EXP, t), 1.0))
    lim = 2 * ulp_of(O.unary_contig(O.EXP, t))
    del x, y, z
    xs = [dev(generate("fused_chain", k)) for k in ("x", "y", "z")]
    chain = lambda a, b, c: ((a * b + c).exp() - 1.0).relu()
    got = torch_rs.fuse(chain)(*xs).numpy()
    assert got.size == n
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= lim), (int(np.argmax(err - lim)), err.max())
    # the unfused eager chain: identical except through exp
    got_eager = chain(*xs).numpy()
    assert np.all(np.abs(got_eager.astype(np.float64) - want) <= lim)


def test_config2_broadcast_strided_full_bit_exact():
    a = generate("broadcast_strided", "a").reshape(64, 1, 1024)
    b = generate("broadcast_strided", "b").reshape(1, 512, 1024)
    c = generate("broadcast_strided", "c").reshape(64, 1024, 512)
    oshape = (64, 512, 1024)
    ocs = O.contiguous_strides(oshape)
    s = O.binary(O.ADD, a.ravel(), a.shape, O.contiguous_strides(a.shape), 0,
                 b.ravel(), b.shape, O.contiguous_strides(b.shape), 0, oshape, ocs)
    want = O.binary(O.MUL, s, oshape, ocs, 0, c.ravel(), oshape, (1024 * 512, 1, 512), 0, oshape, ocs)
    A, B, C = dev(a), dev(b), dev(c)
    eager = (A + B) * C.mT
    assert eager.shape == oshape and eager.stride() == tuple(ocs)
    assert_bitwise_equal(eager.numpy().ravel(), want)
    fused = torch_rs.fuse(lambda a, b, c: (a + b) * c)(A, B, C.mT)
    assert_bitwise_equal(fused.numpy().ravel(), want)


def test_exp_exhaustive_over_all_bit_patterns():
    chunk = 1 << 28
    worst = 0
    for k in range(16):
        first = k * chunk
        x = np.arange(first, first + chunk, dtype=np.uint64).astype(np.uint32).view(np.float32)
        got = U.unary(O.EXP, x, (chunk,), (1,), 0, (1,))
        del x
        w, idx = O.exp_max_ulp(got, first, threads=16)
        assert w <= 2, (hex(first + idx), w)
        worst = max(worst, w)
    assert worst <= 2


def test_relu_neg_relu_vjp_and_scalar_ops_exhaustive_over_all_bit_patterns():
    """relu (src/tensor.rs:4392-4400), neg (:4388-4390) and relu's VJP
    (:4422-4432) on the device at every one of the 2^32 float bit patterns,
    bit for bit against the oracle (NaN payloads included: all three only
    pass bits through, flip the sign or return +0.0).  The configs' scalar
    ops, x - 1.0 (sub_scalar) and x * f32(1/0.9), and dropout-apply
    (h * f32(mask)) * f32(1/0.9) with each mask value, too:
    one IEEE rounding each, so subnormal inputs and results pin the
    device's denormal mode (NaNs compared as NaN)."""
    import ctypes
    from trs_backend import abi
    from trs_backend.abi import check, layout_of
    chunk = 1 << 28
    lay = layout_of((chunk,))
    up = np.full(chunk, 1.25, np.float32)
    dup = U.dev(up)
    out = U.out_buffer(chunk)
    want_vjp_pass = np.float32(1.25)
    scale = float(np.float32(1.0 / 0.9))
    m0 = (np.arange(chunk) & 1).astype(np.uint8)
    m1 = (1 - m0).astype(np.uint8)
    dmask0, dmask1 = (U.dev(m0), m0), (U.dev(m1), m1)
    for k in range(16):
        first = k * chunk
        x = np.arange(first, first + chunk, dtype=np.uint64).astype(np.uint32).view(np.float32)
        dx = U.dev(x)
        for op in (O.RELU, O.NEG):
            check(abi.lib.trs_unary_f32(op, dx.ptr, ctypes.byref(lay), out.ptr, ctypes.byref(lay)))
            assert_bitwise_equal(out.to_numpy(count=chunk), O.unary_contig(op, x), nan_equal=False)
        # dropout-apply (h * f32(m)) * s with complementary masks, so both mask
        # values meet every h
        for mask in (dmask0, dmask1):
            check(abi.lib.trs_mask_apply_f32(dx.ptr, ctypes.byref(lay), mask[0].ptr, ctypes.byref(lay),
                                             ctypes.c_float(scale), out.ptr, ctypes.byref(lay)))
            assert_bitwise_equal(out.to_numpy(count=chunk), O.mask_apply(x, mask[1], scale))
        for op, s in ((O.S_SUB, 1.0), (O.S_MUL, float(np.float32(1.0 / 0.9)))):
            check(abi.lib.trs_binary_scalar_f32(op, dx.ptr, ctypes.byref(lay), ctypes.c_float(s), out.ptr,
                                                ctypes.byref(lay)))
            assert_bitwise_equal(out.to_numpy(count=chunk), O.scalar_contig(op, x, s))
        check(abi.lib.trs_relu_backward_f32(dx.ptr, ctypes.byref(lay), dup.ptr, out.ptr))
        got = out.to_numpy(count=chunk)
        want = O.relu_backward(x, (chunk,), (1,), 0, up)
        assert_bitwise_equal(got, want, nan_equal=False)
        assert set(np.unique(got.view(np.uint32)).tolist()) <= {0, int(want_vjp_pass.view(np.uint32))}
        del x, dx


def _threads():
    import os
    return max(1, min(16, len(os.sched_getaffinity(0))))


def _check_gemm(name, got, a, b):
    """Every element of got = a @ b against the reference-order oracle,
    within 1e-5*sqrt(K)*(|a||b|) (the bound in float64)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    k = a.shape[1]
    want = O.matmul_threads(a, b, threads=_threads())
    bound = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    lim = 1e-5 * np.sqrt(k) * bound
    ok = err <= lim
    assert ok.all(), (name, int((~ok).sum()), float(err.max()))


def _relu_backward_on_device(z1, up):
    """relu'(z1) * up on the device: autograd through relu of a fresh leaf,
    whose upstream is up itself (1 * up is exact)."""
    leaf = z1.detach().requires_grad_()
    (leaf.relu() * up).sum().backward()
    return leaf.grad


def test_config4_mlp_full_size_autograd_and_stagewise_parity():
    F = torch_rs.nn.functional
    mask_apply = torch_rs._C.mask_apply
    x = generate("mlp", "X").reshape(8192, 4096)
    w1 = generate("mlp", "W1").reshape(4096, 4096)
    w2 = generate("mlp", "W2").reshape(4096, 1024)
    mask = generate("mlp", "mask").reshape(8192, 4096)
    scale = np.float32(1 / 0.9)
    X, W1, W2 = dev(x, True), dev(w1, True), dev(w2, True)
    b1, b2 = torch_rs.zeros(4096, device="cuda"), torch_rs.zeros(1024, device="cuda")
    mdev = F.keep_mask(mask)
    out = F.dropout((X @ W1 + b1).relu(), 0.1, mask=mdev) @ W2 + b2
    loss = out.sum()
    loss.backward()
    gW1, gW2, gX = W1.grad.numpy(), W2.grad.numpy(), X.grad.numpy()

    # 1. the same step composed explicitly from device ops, outside autograd
    with torch_rs.no_grad():
        Xd, W1d, W2d = X.detach(), W1.detach(), W2.detach()
        z1 = Xd @ W1d + b1
        h = z1.relu()
        d = F.dropout(h, 0.1, mask=mdev)
        o = d @ W2d + b2
        dout = torch_rs.ones(8192, 1024, device="cuda")
        dd = dout @ W2d.mT
        dw2 = d.mT @ dout
        dh = mask_apply(dd * scale, mdev, np.float32(1.0))
    dz1 = _relu_backward_on_device(z1, dh)
    with torch_rs.no_grad():
        dw1 = Xd.mT @ dz1
        dx = dz1 @ W1d.mT
    assert_bitwise_equal(o.numpy().ravel(), out.numpy().ravel())
    assert_bitwise_equal(dw2.numpy().ravel(), gW2.ravel())
    assert_bitwise_equal(dw1.numpy().ravel(), gW1.ravel())
    assert_bitwise_equal(dx.numpy().ravel(), gX.ravel())

    # 2. each stage of the composition against the oracle, every element
    z1h, hh, dhh, ddh, dh_h, dz1h = (t.numpy() for t in (z1, h, d, dd, dh, dz1))
    oh = o.numpy()
    _check_gemm("Z1", z1h, x, w1)  # + b1 (zeros) is exact
    assert_bitwise_equal(hh.ravel(), O.unary_contig(O.RELU, z1h.ravel()))
    assert_bitwise_equal(dhh.ravel(), O.mask_apply(hh.ravel(), mask.ravel(), scale))
    _check_gemm("out", oh, dhh, w2)
    ones = np.ones((8192, 1024), np.float32)
    _check_gemm("dD", ddh, ones, w2.T)
    assert_bitwise_equal(dh_h.ravel(), O.mask_apply(O.scalar_contig(O.S_MUL, ddh.ravel(), scale), mask.ravel(),
                                                     np.float32(1.0)))
    assert_bitwise_equal(dz1h.ravel(), O.relu_backward(z1h.ravel(), (8192, 4096), (4096, 1), 0, dh_h.ravel()))
    _check_gemm("dW1", gW1, x.T, dz1h)
    _check_gemm("dX", gX, dz1h, w1.T)
    _check_gemm("dW2", gW2, dhh.T, ones)

    # 3. the loss (a sum over the 2^23 outputs) against the reference's
    # sequential fold and the exact sum: the device tree's own bound
    # gamma_d * sum|out| with d = ceil(8192/256) + 20 = 52, the fold's
    # gamma_(n-1) * sum|out|, and their sum between the two.
    import math
    n = oh.size
    loss_dev = float(np.float32(loss.item()))
    fold = float(O.sum_f32(oh.ravel(), (n,)))
    exact = math.fsum(oh.ravel().astype(np.float64))
    abs_sum = O.sum_abs(oh.ravel())

    def gamma(k):
        return k * 2.0 ** -24 / (1 - k * 2.0 ** -24)

    assert abs(loss_dev - exact) <= gamma(52) * abs_sum, (loss_dev, exact)
    assert abs(fold - exact) <= gamma(n - 1) * abs_sum
    assert abs(loss_dev - fold) <= (gamma(52) + gamma(n - 1)) * abs_sum


def test_config4_timed_mlp_step_equals_eager_bitwise():
    """The step bench.py times (mlp_bench.build(): bias add, relu and
    dropout-apply fused into one autograd node, split-K GEMMs) against the
    eager step at full size: loss and the three gradients bit for bit."""
    from trs_backend import mlp_bench
    fused = mlp_bench.build(fused=True)
    eager = mlp_bench.build(fused=False)
    lf, xf, w1f, w2f = fused()
    le, xe, w1e, w2e = eager()
    assert_bitwise_equal(lf.numpy().ravel(), le.numpy().ravel())
    for a, b in ((xf, xe), (w1f, w1e), (w2f, w2e)):
        assert_bitwise_equal(a.grad.numpy().ravel(), b.grad.numpy().ravel())
    # a second fused step (cached blocks and kernels) repeats the first exactly
    lf2, xf2, w1f2, w2f2 = fused()
    assert_bitwise_equal(lf2.numpy().ravel(), lf.numpy().ravel())
    assert_bitwise_equal(w1f2.grad.numpy().ravel(), w1f.grad.numpy().ravel())
