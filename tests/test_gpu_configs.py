"""BASELINE configurations at full size on the GPU, checked against the oracle.

Configs 0-2 are compared element by element over the whole output.  The
oracle restatement runs the reference's loops in a few seconds at these
sizes.  The MLP (config 4) runs through torch_rs autograd at full size.
Its gradients are first checked bit for bit against the same step composed
explicitly from device ops.  That composition is then checked stage by stage
against the oracle: elementwise stages over every element, GEMM stages on
sampled rows within 1e-5*sqrt(K)*(|A||B|).  exp is checked exhaustively,
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


def _mm_rows(a, b, rows):
    """Oracle rows (reference order) and |A||B| bound rows for C = a @ b."""
    m, k = a.shape
    _, n = b.shape
    return O.matmul_rows(np.ascontiguousarray(a).ravel(), (m, k), (k, 1), np.ascontiguousarray(b).ravel(),
                         (k, n), (n, 1), rows)


def _within(got_rows, want_rows, bound_rows, k):
    err = np.abs(got_rows.astype(np.float64) - want_rows)
    return np.all(err <= 1e-5 * np.sqrt(k) * bound_rows + 1e-30), err.max()


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
    out.sum().backward()
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

    # 2. each stage of the composition against the oracle
    rows = np.array([0, 1, 777, 4095, 4096, 8191])
    cols = np.array([0, 5, 2047, 4095])
    z1h, hh, dhh, ddh, dh_h, dz1h = (t.numpy() for t in (z1, h, d, dd, dh, dz1))
    want, bound = _mm_rows(x, w1, rows)
    ok, e = _within(z1h[rows], want, bound, 4096)  # + b1 (zeros) is exact
    assert ok, ("Z1", e)
    assert_bitwise_equal(hh.ravel(), O.unary_contig(O.RELU, z1h.ravel()))
    assert_bitwise_equal(dhh.ravel(), O.mask_apply(hh.ravel(), mask.ravel(), scale))
    want, bound = _mm_rows(dhh, w2, rows)
    ok, e = _within(o.numpy()[rows], want, bound, 4096)
    assert ok, ("out", e)
    want, bound = _mm_rows(np.ones((8192, 1024), np.float32), np.ascontiguousarray(w2.T), rows)
    ok, e = _within(ddh[rows], want, bound, 1024)
    assert ok, ("dD", e)
    assert_bitwise_equal(dh_h.ravel(), O.mask_apply(O.scalar_contig(O.S_MUL, ddh.ravel(), scale), mask.ravel(),
                                                     np.float32(1.0)))
    assert_bitwise_equal(dz1h.ravel(), O.relu_backward(z1h.ravel(), (8192, 4096), (4096, 1), 0, dh_h.ravel()))
    want, bound = _mm_rows(np.ascontiguousarray(x.T), dz1h, cols)  # rows of dW1 = X^T dZ1
    ok, e = _within(gW1[cols], want, bound, 8192)
    assert ok, ("dW1", e)
    want, bound = _mm_rows(dz1h, np.ascontiguousarray(w1.T), rows)
    ok, e = _within(gX[rows], want, bound, 4096)
    assert ok, ("dX", e)
    want, bound = _mm_rows(np.ascontiguousarray(dhh.T), np.ones((8192, 1024), np.float32), cols)
    ok, e = _within(gW2[cols], want, bound, 8192)
    assert ok, ("dW2", e)
