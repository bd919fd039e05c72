"""GPU parity of the torch_rs host engine (C++ over libtrs_hip.so).

Known-answer autograd vectors come from the reference's tests/autograd.rs
(tests/golden/reference_vectors.json); random strided/broadcast cases are
checked against the CPU oracle bit for bit, output strides included; the
VJPs this backend adds (matmul, tensor add/sub, exp) are checked against
closed forms on exactly representable inputs and against oracle compositions.
"""
import threading

import numpy as np
import pytest

import oracle as O
import torch_rs
from helpers import assert_bitwise_equal, check_bits, f32_from_bits, golden, ulp_of

pytestmark = pytest.mark.gpu
G = golden()
F = torch_rs.nn.functional


def cuda(a, requires_grad=False):
    return torch_rs.tensor(np.asarray(a, np.float32), device="cuda", requires_grad=requires_grad)


def vals(t):
    return t.numpy().ravel()


# ---- reference autograd known answers (tests/autograd.rs) ------------------------

def test_square_sum_accumulates_across_backward_calls():
    g = G["autograd_square_sum"]
    x = cuda(g["x"], requires_grad=True)
    (x * x).sum().backward()
    assert vals(x.grad).tolist() == g["grad_once"]
    (x * x).sum().backward()
    assert vals(x.grad).tolist() == g["grad_twice"]


def test_mul_unbroadcast_gradients():
    g = G["autograd_mul_unbroadcast"]
    l = cuda(np.array(g["left"]).reshape(g["left_shape"]), requires_grad=True)
    r = cuda(np.array(g["right"]).reshape(g["right_shape"]), requires_grad=True)
    (l * r).sum().backward()
    assert vals(l.grad).tolist() == g["left_grad"]
    assert vals(r.grad).tolist() == g["right_grad"]
    assert l.grad.shape == tuple(g["left_shape"])


@pytest.mark.parametrize("scalar_on_left", [True, False])
def test_rank_zero_multiply_through_index_and_transpose_views(scalar_on_left):
    g = G["autograd_rank_zero_view"]
    source = cuda(np.array(g["storage"]).reshape(2, 2, 3), requires_grad=True)
    view = source[1].transpose(0, 1)
    scalar = cuda(np.float32(g["scalar"]), requires_grad=True)
    out = scalar * view if scalar_on_left else view * scalar
    assert out.shape == (3, 2) and out.stride() == (1, 3)
    out.sum().backward()
    assert vals(scalar.grad).tolist() == [g["scalar_grad"]]
    assert vals(source.grad).tolist() == g["source_grad"]


def test_relu_vjp_bits_including_nan_inf_and_signed_zero():
    g = G["autograd_relu_vjp"]
    x = torch_rs.tensor(f32_from_bits(g["input_bits"]), device="cuda", requires_grad=True)
    w = torch_rs.tensor(f32_from_bits(g["weight_bits"]), device="cuda")
    (x.relu() * w).sum().backward()
    check_bits(vals(x.grad), g["expected_gradient_bits"])
    assert x.relu().grad_fn.name() == "ReluBackward0"


def test_transform_chain_gradients():
    leaf = cuda(np.arange(1, 7, dtype=np.float32).reshape(1, 2, 3), requires_grad=True)
    packed = leaf.permute(2, 0, 1).contiguous()
    assert packed.requires_grad
    squeezed = packed.view(3, 2)  # squeeze_dim(1): the same identity mapping
    cloned = squeezed[1].reshape(2, 1).clone()
    assert cloned.requires_grad
    (cloned * cloned).sum().backward()
    assert vals(leaf.grad).tolist() == [0.0, 4.0, 0.0, 0.0, 10.0, 0.0]

    g = G["autograd_transform"]
    rl = cuda(np.array(g["leaf"]).reshape(g["leaf_shape"]), requires_grad=True)
    rc = rl.transpose(0, 1).reshape(6)
    (rc * cuda(g["weights"])).sum().backward()
    assert vals(rl.grad).tolist() == g["leaf_grad"]


def test_first_negative_zero_contribution_is_kept_only_without_broadcast():
    g = G["autograd_negative_zero"]
    left = cuda(g["no_broadcast"]["left"], requires_grad=True)
    right = torch_rs.tensor(f32_from_bits(g["no_broadcast"]["right_bits"]), device="cuda")
    (left * right).sum().backward()
    check_bits(vals(left.grad), g["no_broadcast"]["left_grad_bits"])
    bl = cuda(np.float32(g["broadcast"]["left"]), requires_grad=True)
    br = torch_rs.tensor(f32_from_bits(g["broadcast"]["right_bits"]), device="cuda")
    (bl * br).sum().backward()
    check_bits(vals(bl.grad), g["broadcast"]["left_grad_bits"])


def test_second_backward_through_saved_values_fails_and_metadata_graphs_repeat():
    x = cuda([1.0, 2.0], requires_grad=True)
    loss = (x * x).sum()
    loss.backward()
    with pytest.raises(RuntimeError, match="Trying to backward through the graph a second time"):
        loss.backward()
    y = cuda([1.0, 2.0, 3.0], requires_grad=True)
    s = (y + 1.0).sum()  # add_scalar + sum save no values
    s.backward()
    s.backward()
    assert vals(y.grad).tolist() == [2.0, 2.0, 2.0]


def test_concurrent_backward_on_shared_graph_commits_one_traversal():
    leaf = cuda(np.float32(3.0), requires_grad=True)
    fwd, rev = leaf * 1.0, leaf * 1.0
    for _ in range(200):
        fwd, rev = fwd * 1.0, rev * 1.0
    roots = [(fwd * rev).sum(), (rev * fwd).sum()]
    results = [None, None]
    barrier = threading.Barrier(3)

    def run(i):
        barrier.wait()
        try:
            roots[i].backward()
            results[i] = "ok"
        except RuntimeError as e:
            results[i] = str(e)

    ts = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    barrier.wait()
    for t in ts:
        t.join()
    assert results.count("ok") == 1
    assert sum("backward through the graph a second time" in r for r in results if r != "ok") == 1
    assert vals(leaf.grad).tolist() == [6.0]


def test_deep_graph_backward_and_teardown():
    x = cuda([1.0], requires_grad=True)
    y = x
    for _ in range(20000):
        y = y + 1.0
    y.sum().backward()
    assert vals(x.grad).tolist() == [1.0]
    del y  # iterative teardown of the 20k-node chain


# ---- random strided / broadcast ops against the oracle ---------------------------------

def _view_case(rng, storage_len=4096):
    """A random strided view of a device storage: (tensor, storage, shape, strides, offset)."""
    rank = int(rng.integers(1, 4))
    base_shape = [int(rng.integers(1, 6)) for _ in range(rank + 1)]
    base = rng.standard_normal(int(np.prod(base_shape))).astype(np.float32)
    t = cuda(base.reshape(base_shape))
    kind = rng.integers(0, 4)
    if kind == 0:
        v = t[int(rng.integers(0, base_shape[0]))]
    elif kind == 1:
        v = t.permute(*rng.permutation(rank + 1).tolist())
    elif kind == 2:
        v = t.transpose(0, rank)
    else:
        v = t
    return v, base


def test_random_views_binary_ops_match_oracle_values_and_strides():
    rng = np.random.default_rng(11)
    ops = [(O.ADD, lambda a, b: a + b), (O.SUB, lambda a, b: a - b), (O.MUL, lambda a, b: a * b),
           (O.DIV, lambda a, b: a / b)]
    for case in range(60):
        a, abase = _view_case(rng)
        # right operand: same shape (permuted differently) or a broadcastable suffix
        shape = a.shape
        if rng.random() < 0.5:
            rshape = tuple(1 if rng.random() < 0.3 else d for d in shape[len(shape) - int(rng.integers(0, len(shape) + 1)):])
        else:
            rshape = shape
        rbase = rng.standard_normal(max(int(np.prod(rshape)), 1)).astype(np.float32)
        b = cuda(rbase[:int(np.prod(rshape))].reshape(rshape))
        if len(rshape) >= 2 and rng.random() < 0.5:
            b = cuda(rbase[:int(np.prod(rshape))].reshape(rshape[:-2] + (rshape[-1], rshape[-2]))).mT
        for code, fn in ops:
            out = fn(a, b)
            want_shape, want_strides = O.binary_output_layout(a.shape, a.stride(), b.shape, b.stride())
            assert out.shape == want_shape and out.stride() == want_strides, (case, a.shape, a.stride(), b.shape, b.stride())
            bst = b.numpy().ravel() if b.is_contiguous() else None
            # oracle on logical values (contiguous copies of both operands)
            ref = O.binary(code, a.numpy().ravel(), a.shape, O.contiguous_strides(a.shape), 0,
                           b.numpy().ravel(), b.shape, O.contiguous_strides(b.shape), 0,
                           want_shape, O.contiguous_strides(want_shape))
            assert_bitwise_equal(out.numpy().ravel(), ref)
            del bst


def test_random_views_unary_and_scalar_ops_match_oracle():
    rng = np.random.default_rng(12)
    for case in range(40):
        v, _ = _view_case(rng)
        x = v.numpy().ravel()
        cs = O.contiguous_strides(v.shape)
        for code, t in ((O.RELU, v.relu()), (O.NEG, -v)):
            assert t.stride() == O.unary_output_strides(v.shape, v.stride())
            assert_bitwise_equal(t.numpy().ravel(), O.unary(code, x, v.shape, cs, 0, cs))
        e = v.exp()
        want = O.unary(O.EXP, x, v.shape, cs, 0, cs)
        got = e.numpy().ravel()
        assert np.all(np.abs(got.astype(np.float64) - want) <= 2 * ulp_of(want))
        for code, t in ((O.S_ADD, v + 0.25), (O.S_SUB, v - 1.0), (O.S_MUL, v * 1.5), (O.S_DIV, v / 3.0),
                        (O.S_RSUB, 2.0 - v), (O.S_RDIV, 3.0 / v)):
            s = {O.S_ADD: 0.25, O.S_SUB: 1.0, O.S_MUL: 1.5, O.S_DIV: 3.0, O.S_RSUB: 2.0, O.S_RDIV: 3.0}[code]
            if code != O.S_RDIV:
                assert t.stride() == O.scalar_output_strides(v.shape, v.stride())
            assert_bitwise_equal(t.numpy().ravel(), O.scalar(code, x, v.shape, cs, 0, s, cs))


# ---- VJPs this backend adds -------------------------------------------------------------------

def test_matmul_vjp_exact_on_small_integers():
    rng = np.random.default_rng(3)
    for m, k, n in [(5, 7, 3), (64, 96, 80), (130, 33, 17)]:
        a = rng.integers(-3, 4, (m, k)).astype(np.float32)
        b = rng.integers(-3, 4, (k, n)).astype(np.float32)
        w = rng.integers(-2, 3, (m, n)).astype(np.float32)
        A, B = cuda(a, True), cuda(b, True)
        out = A @ B
        assert out.grad_fn.name() == "MmBackward0"
        (out * cuda(w)).sum().backward()
        assert np.array_equal(A.grad.numpy(), (w.astype(np.int64) @ b.T.astype(np.int64)).astype(np.float32))
        assert np.array_equal(B.grad.numpy(), (a.T.astype(np.int64) @ w.astype(np.int64)).astype(np.float32))


def test_small_batch_linear_layer_forward_and_backward_exact():
    """x @ W.mT with 1 or 3 rows of x and W [4096, 4096] (the layout of a
    linear layer's weight): the forward is a matrix-vector product, dX = up @ W
    a skinny product with K split, and dW = up^T @ x an outer product of depth
    1 or 3.  Small integers make every order exact."""
    rng = np.random.default_rng(6)
    for m in (1, 3):
        x = rng.integers(-3, 4, (m, 4096)).astype(np.float32)
        wt = rng.integers(-3, 4, (4096, 4096)).astype(np.float32)
        up = rng.integers(-2, 3, (m, 4096)).astype(np.float32)
        X, W = cuda(x, True), cuda(wt, True)
        out = X @ W.mT
        assert np.array_equal(out.numpy(), (x.astype(np.float64) @ wt.T.astype(np.float64)).astype(np.float32))
        (out * cuda(up)).sum().backward()
        assert np.array_equal(X.grad.numpy(), (up.astype(np.float64) @ wt.astype(np.float64)).astype(np.float32))
        assert np.array_equal(W.grad.numpy(), (up.T.astype(np.float64) @ x.astype(np.float64)).astype(np.float32))


def test_batched_matmul_vjp_exact_on_small_integers():
    rng = np.random.default_rng(4)
    a = rng.integers(-3, 4, (4, 20, 12)).astype(np.float32)
    b = rng.integers(-3, 4, (4, 12, 9)).astype(np.float32)
    A, B = cuda(a, True), cuda(b, True)
    out = A @ B
    assert out.grad_fn.name() == "BmmBackward0"
    out.sum().backward()
    ones = np.ones((4, 20, 9), np.int64)
    assert np.array_equal(A.grad.numpy(), (ones @ b.transpose(0, 2, 1).astype(np.int64)).astype(np.float32))
    assert np.array_equal(B.grad.numpy(), (a.transpose(0, 2, 1).astype(np.int64) @ ones).astype(np.float32))


def test_matmul_vjp_with_transposed_operands_within_tolerance():
    rng = np.random.default_rng(5)
    m, k, n = 96, 200, 72
    a = rng.standard_normal((k, m)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    A, B = cuda(a, True), cuda(b, True)
    out = A.mT @ B.mT  # both operands are .mT views
    w = rng.standard_normal((m, n)).astype(np.float32)
    (out * cuda(w)).sum().backward()
    # dA^T = W @ B  ->  A.grad = (W @ B)^T
    want = O.matmul(w.ravel(), (m, n), (n, 1), 0, b.ravel(), (n, k), (k, 1), 0).reshape(m, k).T
    bound = 1e-5 * np.sqrt(n) * (np.abs(w).astype(np.float64) @ np.abs(b).astype(np.float64)).T
    assert np.all(np.abs(A.grad.numpy() - want) <= bound + 1e-30)


def test_broadcast_add_and_sub_vjps_reduce_in_reference_order():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((37, 64)).astype(np.float32)
    bvec = rng.standard_normal(64).astype(np.float32)
    w = rng.standard_normal((37, 64)).astype(np.float32)
    X, Bv = cuda(x, True), cuda(bvec, True)
    out = X + Bv
    assert out.grad_fn.name() == "AddBackward0"
    (out * cuda(w)).sum().backward()
    assert_bitwise_equal(vals(Bv.grad), O.reduce_to_shape(w.ravel(), (37, 64), (64,)))
    assert_bitwise_equal(X.grad.numpy().ravel(), w.ravel())
    X2, B2 = cuda(x, True), cuda(bvec.reshape(1, 64), True)
    ((X2 - B2) * cuda(w)).sum().backward()
    assert_bitwise_equal(vals(B2.grad), -O.reduce_to_shape(w.ravel(), (37, 64), (1, 64)))


def test_exp_vjp_is_upstream_times_output():
    rng = np.random.default_rng(7)
    x = rng.uniform(-5, 5, 1000).astype(np.float32)
    w = rng.standard_normal(1000).astype(np.float32)
    X = cuda(x, True)
    e = X.exp()
    assert e.grad_fn.name() == "ExpBackward0"
    (e * cuda(w)).sum().backward()
    assert_bitwise_equal(vals(X.grad), w * e.numpy())  # one rounding of up * exp(x)


# ---- config 5: 2-layer MLP forward + backward ------------------------------------------------

def _mlp_reference(x, w1, w2, mask, scale):
    """The reference composition on the oracle (matmul in its sequential order)."""
    mm = lambda a, b: O.matmul(a.ravel(), a.shape, O.contiguous_strides(a.shape), 0,
                               b.ravel(), b.shape, O.contiguous_strides(b.shape), 0).reshape(a.shape[0], b.shape[1])
    z1 = O.row_broadcast(O.ADD, mm(x, w1).ravel(), np.zeros(w1.shape[1], np.float32), x.shape[0],
                         w1.shape[1]).reshape(x.shape[0], w1.shape[1])  # + b1 (zeros)
    h = O.unary_contig(O.RELU, z1.ravel()).reshape(z1.shape)
    d = O.mask_apply(h.ravel(), mask.ravel(), scale).reshape(h.shape)
    out = O.row_broadcast(O.ADD, mm(d, w2).ravel(), np.zeros(w2.shape[1], np.float32), d.shape[0],
                          w2.shape[1]).reshape(d.shape[0], w2.shape[1])  # + b2 (zeros)
    up = np.ones_like(out)
    dd = mm(up, np.ascontiguousarray(w2.T))
    dw2 = mm(np.ascontiguousarray(d.T), up)
    dh = O.mask_apply(O.scalar_contig(O.S_MUL, dd.ravel(), scale), mask.ravel(), np.float32(1.0)).reshape(dd.shape)
    dz1 = O.relu_backward(z1.ravel(), z1.shape, O.contiguous_strides(z1.shape), 0, dh.ravel()).reshape(dh.shape)
    dw1 = mm(np.ascontiguousarray(x.T), dz1)
    dx = mm(dz1, np.ascontiguousarray(w1.T))
    return out, dw1, dw2, dx


def _mlp_device(x, w1, w2, mask, p):
    X, W1, W2 = cuda(x, True), cuda(w1, True), cuda(w2, True)
    b1, b2 = torch_rs.zeros(w1.shape[1], device="cuda"), torch_rs.zeros(w2.shape[1], device="cuda")
    h = (X @ W1 + b1).relu()
    d = F.dropout(h, p, training=True, mask=mask)
    out = d @ W2 + b2
    out.sum().backward()
    return out.numpy(), W1.grad.numpy(), W2.grad.numpy(), X.grad.numpy()


def test_mlp_forward_backward_bit_exact_on_dyadic_inputs():
    rng = np.random.default_rng(8)
    x = rng.integers(-2, 3, (64, 128)).astype(np.float32)
    w1 = (rng.integers(-4, 5, (128, 96)) / 8).astype(np.float32)
    w2 = (rng.integers(-4, 5, (96, 32)) / 8).astype(np.float32)
    mask = (rng.random((64, 96)) < 0.5).astype(np.uint8)
    got = _mlp_device(x, w1, w2, mask, 0.5)
    want = _mlp_reference(x, w1, w2, mask, np.float32(2.0))
    for g, w in zip(got, want):
        assert_bitwise_equal(g.ravel(), w.ravel())


def test_mlp_config5_distribution_within_matmul_tolerance():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((256, 512)).astype(np.float32)
    w1 = rng.uniform(-1 / 64, 1 / 64, (512, 512)).astype(np.float32)
    w2 = rng.uniform(-1 / 64, 1 / 64, (512, 128)).astype(np.float32)
    mask = (rng.random((256, 512)) < 0.9).astype(np.uint8)
    got = _mlp_device(x, w1, w2, mask, 0.1)
    want = _mlp_reference(x, w1, w2, mask, np.float32(1 / 0.9))
    names = ["out", "dW1", "dW2", "dX"]
    for name, g, w in zip(names, got, want):
        scale = np.abs(w).max()
        err = np.abs(g.astype(np.float64) - w)
        # sqrt(K) * 1e-5 relative per GEMM, two GEMMs deep, against the tensor's scale
        assert err.max() <= 4e-5 * np.sqrt(512) * scale, (name, err.max(), scale)


# ---- fusion -------------------------------------------------------------------------------

def test_fused_chain_matches_eager_within_two_ulp_of_exp():
    rng = np.random.default_rng(10)
    xs = [cuda(rng.uniform(-4, 4, 100003)) for _ in range(3)]
    chain = lambda x, y, z: ((x * y + z).exp() - 1.0).relu()
    fused = torch_rs.fuse(chain)(*xs)
    eager = chain(*xs)
    t = O.binary_contig(O.ADD, O.binary_contig(O.MUL, xs[0].numpy(), xs[1].numpy()), xs[2].numpy())
    lim = 2 * ulp_of(np.exp(t.astype(np.float64)).astype(np.float32))
    assert np.all(np.abs(fused.numpy().astype(np.float64) - eager.numpy()) <= lim)
    assert fused.stride() == eager.stride()


def test_fused_broadcast_strided_chain_is_bit_exact_with_eager():
    rng = np.random.default_rng(13)
    a = cuda(rng.standard_normal((8, 1, 96)))
    b = cuda(rng.standard_normal((1, 40, 96)))
    c = cuda(rng.standard_normal((8, 96, 40))).mT
    f = torch_rs.fuse(lambda a, b, c: (a + b) * c - 0.5 / c)
    got, want = f(a, b, c), (a + b) * c - 0.5 / c
    assert got.shape == want.shape and got.stride() == want.stride()
    assert_bitwise_equal(got.numpy().ravel(), want.numpy().ravel())


def test_fused_call_with_grad_inputs_records_and_backpropagates():
    x = cuda([1.0, -2.0, 3.0], True)
    y = torch_rs.fuse(lambda x: (x * 2.0).relu())(x)
    assert y.grad_fn is not None
    y.sum().backward()
    assert vals(x.grad).tolist() == [2.0, 0.0, 2.0]


# ---- allocator and transfers ------------------------------------------------------------

def test_block_cache_reuses_freed_storage():
    from trs_backend import abi
    import ctypes
    t = torch_rs.zeros(1 << 20, device="cuda")
    del t
    live, cached = ctypes.c_size_t(), ctypes.c_size_t()
    abi.check(abi.lib.trs_memory_stats(ctypes.byref(live), ctypes.byref(cached)))
    assert cached.value >= 4 << 20
    u = torch_rs.full((1 << 20,), 3.0, device="cuda")
    abi.check(abi.lib.trs_memory_stats(ctypes.byref(live), ctypes.byref(cached)))
    assert live.value >= 4 << 20
    assert vals(u)[:4].tolist() == [3.0] * 4


def test_host_device_round_trip_preserves_bits_and_views():
    rng = np.random.default_rng(14)
    a = rng.standard_normal((6, 5)).astype(np.float32)
    t = cuda(a)
    assert t.device == torch_rs.device("cuda", 0) and str(t.device) == "cuda:0" and t.is_cuda
    assert_bitwise_equal(t.mT.cpu().numpy().ravel(), a.T.ravel())
    back = t.mT.cpu().cuda()
    assert back.is_contiguous() and back.shape == (5, 6)


def test_device_objects_select_the_gpu_and_accelerator_reports_it():
    dev = torch_rs.device("cuda")
    assert torch_rs.cuda.current_device() == 0
    t = torch_rs.tensor([1.5, -2.0], device=dev)
    assert t.device == torch_rs.device("cuda", 0) and t.get_device() == 0 and not t.is_cpu
    u = torch_rs.zeros(3, device=torch_rs.device("cuda", 0))
    assert u.device == t.device
    h = t.to(torch_rs.device("cpu"))
    assert h.device == torch_rs.device("cpu") and h.get_device() == -1
    for back in (h.to(dev), h.to(device="cuda:0"), h.cuda(), h.cuda(0), h.cuda(torch_rs.device("cuda", 0))):
        assert back.device == torch_rs.device("cuda", 0)
        assert vals(back).tolist() == [1.5, -2.0]
    with pytest.raises(RuntimeError, match="must be cuda device"):
        h.cuda("cpu")
    acc = torch_rs.accelerator
    assert acc.is_available() and acc.device_count() >= 1
    assert acc.current_accelerator(check_available=True) == torch_rs.device("cuda")


def test_backward_through_a_host_to_device_transfer_raises_before_consuming():
    x = torch_rs.tensor([1.0, 2.0], requires_grad=True)  # a host leaf
    y = x.to("cuda")
    assert y.requires_grad and not y.is_leaf
    loss = (y * y).sum()
    with pytest.raises(RuntimeError, match="backward through a device transfer is not supported"):
        loss.backward()
    assert x.grad is None


def test_pass_through_gradients_accumulate_without_aliasing():
    # x feeds two identity edges and one add: every contribution must land once.
    x = cuda([1.0, 2.0, 3.0], requires_grad=True)
    y = x.view(3) + 1.0          # identity edges (view, add_scalar)
    z = x.reshape(1, 3).view(3)  # identity edges
    w = y + z                    # add: upstream handed to one side, copied to the other
    (w * 2.0).sum().backward()
    assert vals(x.grad).tolist() == [4.0, 4.0, 4.0]
    b = cuda([[1.0, 2.0], [3.0, 4.0]], requires_grad=True)
    c = cuda([10.0, 20.0], requires_grad=True)
    ((b + c) * cuda([[1.0, 2.0], [3.0, 4.0]])).sum().backward()
    assert vals(b.grad).tolist() == [1.0, 2.0, 3.0, 4.0]
    assert vals(c.grad).tolist() == [4.0, 6.0]


def test_dropout_backward_is_scale_then_mask_in_one_pass():
    rng = np.random.default_rng(15)
    h = cuda(rng.standard_normal(5000), True)
    mask = (rng.random(5000) < 0.9).astype(np.uint8)
    mask[:3] = [0, 1, 3]  # a non-0/1 byte keeps the two-rounding order observable
    up = rng.standard_normal(5000).astype(np.float32)
    up[0] = -np.inf
    with np.errstate(invalid="ignore"):
        want = (np.float32(1 / 0.9) * up) * mask.astype(np.float32)
    (F.dropout(h, 0.1, mask=mask) * cuda(up)).sum().backward()
    assert_bitwise_equal(vals(h.grad), want)


def test_unbatched_dropout1d_identity_view_passes_gradients_through():
    # unsqueeze(0) then squeeze(0) (src/python_nn_functional.rs:168-178): a new
    # view whose SqueezeBackward1 and UnsqueezeBackward0 edges reach the leaf.
    x = cuda(np.arange(6, dtype=np.float32).reshape(2, 3), requires_grad=True)
    y = F.dropout1d(x, p=0.5, training=False)
    assert y is not x and y.grad_fn.name() == "SqueezeBackward1"
    w = cuda(np.float32([[1, -2, 3], [-4, 5, -6]]))
    (y * w).sum().backward()
    assert x.grad.numpy().tolist() == [[1, -2, 3], [-4, 5, -6]]
    z = cuda(np.ones((1, 1, 1, 1, 2), np.float32))
    assert F.dropout3d(z, p=1.0, training=True).numpy().reshape(-1).tolist() == [0.0, 0.0]


def test_scalar_operands_convert_to_f32_as_the_reference_does():
    # into_arithmetic_f32 (src/python.rs:10258-10277): Python and NumPy numbers
    # are rounded to f32 once, then the op rounds once.
    x = cuda([1.0, -3.0])
    assert (x + 2 ** 63).numpy().tolist() == [np.float32(2.0 ** 63) + np.float32(1), np.float32(2.0 ** 63) - 3]
    assert (x * np.float64(0.1)).numpy().tolist() == (np.float32([1.0, -3.0]) * np.float32(0.1)).tolist()
    assert (x - np.bool_(True)).numpy().tolist() == [0.0, -4.0]
    assert (np.float32(2) / x).numpy().tolist() == (np.float32(2) / np.float32([1.0, -3.0])).tolist()
    assert (x + np.int64(-7)).numpy().tolist() == [-6.0, -10.0]


def test_mul_method_spellings_match_the_operator():
    """tests/test_mul.py's cases on device tensors: Tensor.mul(other) and
    mul(other=) equal `*` in values, strides and offset, for tensors and
    every scalar kind, strided empties and special bit patterns; autograd
    through the method equals the operator's."""
    def same(a, b):
        assert a.shape == b.shape and a.stride() == b.stride() and a.storage_offset() == b.storage_offset()
        assert a.requires_grad == b.requires_grad
        assert_bitwise_equal(vals(a), vals(b))

    left = cuda(np.array([[[1.0, 4.0], [2.0, 5.0], [3.0, 6.0]]], np.float32)).transpose(0, 2)
    right = cuda(np.array([[2.0], [3.0], [4.0]], np.float32))
    same(left.mul(right), left * right)
    same(left.mul(other=right), left * right)
    view = left[1]
    for s in (True, -2, 2.5, np.bool_(False), np.int64(3), np.float32(-0.0)):
        same(view.mul(s), view * s)
        same(view.mul(other=s), view * s)
    empty = torch_rs.zeros((2, 0, 3), device="cuda").transpose(0, 2)
    ones = torch_rs.ones((1, 1, 2), device="cuda")
    same(empty.mul(other=ones), empty * ones)
    special = cuda(np.array([0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC12345], np.uint32).view(np.float32))
    got, want = special.mul(-0.0), special * -0.0
    assert got.shape == want.shape
    assert_bitwise_equal(vals(got), vals(want))

    ml = cuda(np.array([[2.0, 3.0]], np.float32), True)
    mr = cuda(np.array([[5.0], [7.0], [11.0]], np.float32), True)
    ol = cuda(np.array([[2.0, 3.0]], np.float32), True)
    orr = cuda(np.array([[5.0], [7.0], [11.0]], np.float32), True)
    mo = ml.transpose(0, 1).mul(other=mr.transpose(0, 1))
    oo = ol.transpose(0, 1) * orr.transpose(0, 1)
    same(mo, oo)
    mo.sum().backward()
    oo.sum().backward()
    same(ml.grad, ol.grad)
    same(mr.grad, orr.grad)
    shared_m = cuda(np.array([2.0, -3.0], np.float32), True)
    shared_o = cuda(np.array([2.0, -3.0], np.float32), True)
    shared_m.mul(shared_m).sum().backward()
    (shared_o * shared_o).sum().backward()
    same(shared_m.grad, shared_o.grad)
    assert vals(shared_m.grad).tolist() == [4.0, -6.0]
    em = torch_rs.zeros((2, 0, 3), device="cuda", requires_grad=True)
    eo = torch_rs.zeros((2, 0, 3), device="cuda", requires_grad=True)
    em.mul(other=torch_rs.ones((1, 1, 3), device="cuda")).sum().backward()
    (eo * torch_rs.ones((1, 1, 3), device="cuda")).sum().backward()
    same(em.grad, eo.grad)
    a = cuda(np.array([[1.0, 2.0]], np.float32), True)
    b = cuda(np.array([[3.0], [4.0]], np.float32), True)
    with torch_rs.no_grad():
        assert not a.transpose(0, 1).mul(b.transpose(0, 1)).requires_grad
        assert not a.mul(other=2.0).requires_grad
    assert a.mul(b.transpose(0, 1)).requires_grad


def test_leaf_grad_is_one_live_object_that_sees_accumulation():
    """tests/test_autograd.py's leaf contract: `.grad` is None before backward,
    then the same object on every read, and a retained `.grad` shows the
    next backward's accumulation (in place in the leaf's storage)."""
    x = cuda(np.array([-2.0, 0.5, 3.0], np.float32), True)
    assert x.grad is None
    (x * x).sum().backward()
    g = x.grad
    assert g is x.grad and not g.requires_grad and g.is_leaf
    assert vals(g).tolist() == [-4.0, 1.0, 6.0]
    (x * x).sum().backward()
    assert g is x.grad
    assert vals(g).tolist() == [-8.0, 2.0, 12.0]
    # a non-leaf has no .grad; a fresh leaf of the same values starts empty
    y = x * 2.0
    assert y.grad is None
    z = x.detach().with_requires_grad(True)
    assert z.grad is None
    # repeated backward through a graph with no saved values accumulates
    w = cuda(np.array([2.0, 3.0], np.float32), True)
    loss = (w + 1.0).sum()
    loss.backward()
    kept = w.grad
    loss.backward()
    assert kept is w.grad and vals(kept).tolist() == [2.0, 2.0]


def test_saved_values_of_a_live_gradient_are_frozen_at_forward():
    """tests/test_autograd.py: a product saved with a live `.grad` operand
    keeps the values of forward time although the gradient accumulates in
    place afterwards (SavedTensor::try_from_tensor snapshots shared-gradient
    storage, src/tensor.rs:2809-2825)."""
    source = cuda([4.0, 5.0], True)
    source.sum().backward()
    live = source.grad
    weights = cuda([2.0, 3.0], True)
    saved_loss = (weights * live).sum()
    source.sum().backward()
    assert vals(live).tolist() == [2.0, 2.0]
    saved_loss.backward()
    assert vals(weights.grad).tolist() == [1.0, 1.0]
