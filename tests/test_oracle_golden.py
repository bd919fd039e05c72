"""Pin the CPU oracle against the reference's own known-answer tests.

Every vector comes from tests/golden/reference_vectors.json, transcribed from
the reference's Rust tests (each entry cites file:line).  These run on any
host: they check the checker before it is trusted for GPU parity.
"""
import numpy as np
import pytest

import oracle as O
from helpers import check_bits, f32_from_bits, golden

G = golden()


def test_relu_bits_offset_and_transposed_views():
    g = G["relu_bits"]
    storage = np.concatenate([np.full(12, 1.0, np.float32), f32_from_bits(g["input_bits"])])
    v = g["offset_view"]
    assert O.unary_output_strides(v["shape"], v["strides"]) == tuple(v["out_strides"])
    out = O.unary(O.RELU, storage, v["shape"], v["strides"], v["offset"], v["out_strides"])
    check_bits(out, g["expected_bits"])
    t = g["transposed_view"]
    assert O.unary_output_strides(t["shape"], t["strides"]) == tuple(t["out_strides"])
    out = O.unary(O.RELU, storage, t["shape"], t["strides"], t["offset"], t["out_strides"])
    # logical order of a [4,3] output with strides [1,4]
    logical = np.array([out[i * 1 + j * 4] for i in range(4) for j in range(3)], dtype=np.float32)
    check_bits(logical, g["transposed_expected_bits"])


def test_exp_values_within_reference_tolerance():
    g = G["exp_values"]
    x = np.array(g["inputs"], dtype=np.float32)
    out = O.unary_contig(O.EXP, x)
    ref = np.array(g["pytorch_reference"], dtype=np.float32)
    atol = f32_from_bits([g["atol_bits"]])[0]
    assert np.all(np.abs(out - ref) <= atol + g["rtol"] * np.abs(ref))


def test_exp_special_cases():
    g = G["exp_special"]
    out = O.unary_contig(O.EXP, f32_from_bits(g["input_bits"]))
    for v, chk in zip(out, g["checks"]):
        if chk.startswith("bits:"):
            assert int(np.float32(v).view(np.uint32)) == int(chk[5:], 16)
        elif chk == "subnormal":
            assert 0 < abs(v) < np.finfo(np.float32).tiny
        elif chk == "finite":
            assert np.isfinite(v)
        elif chk == "nan":
            assert np.isnan(v)


def test_exp_indexed_view():
    g = G["exp_indexed_view"]
    s = np.array(g["storage"], dtype=np.float32)
    out = O.unary(O.EXP, s, g["shape"], g["strides"], g["offset"], (1,))
    exp = np.array(g["expected"], dtype=np.float32)
    assert np.all(np.abs(out - exp) <= g["rtol"] * exp)


@pytest.mark.parametrize("op,key", [(O.ADD, "add"), (O.SUB, "sub"), (O.MUL, "mul"), (O.DIV, "div")])
def test_broadcast_mixed_ranks(op, key):
    g = G["broadcast_mixed_ranks"]
    ls, rs = g["left_shape"], g["right_shape"]
    oshape, ostrides = O.binary_output_layout(ls, O.contiguous_strides(ls), rs, O.contiguous_strides(rs))
    assert oshape == tuple(g["out_shape"])
    out = O.binary(op, np.array(g["left"], np.float32), ls, O.contiguous_strides(ls), 0,
                   np.array(g["right"], np.float32), rs, O.contiguous_strides(rs), 0, oshape, ostrides)
    assert out.tolist() == g[key]


def test_rank_zero_broadcast():
    g = G["rank_zero_broadcast"]
    m = np.array(g["matrix"], np.float32)
    s = np.array([g["scalar"]], np.float32)
    out = O.binary(O.ADD, m, (2, 2), (2, 1), 0, s, (), (), 0, (2, 2), (2, 1))
    assert out.tolist() == g["matrix_add_scalar"]
    out = O.binary(O.SUB, s, (), (), 0, m, (2, 2), (2, 1), 0, (2, 2), (2, 1))
    assert out.tolist() == g["scalar_sub_matrix"]


@pytest.mark.parametrize("op,s,key", [
    (O.S_ADD, 2.0, "add_scalar_2"), (O.S_SUB, 2.0, "sub_scalar_2"), (O.S_RSUB, 2.0, "scalar_sub_2"),
    (O.S_MUL, 2.0, "mul_scalar_2"), (O.S_DIV, -0.0, "div_scalar_neg0"), (O.S_RDIV, -0.0, "scalar_div_neg0")])
def test_scalar_ops_signed_zero(op, s, key):
    g = G["scalar_signed_zero"]
    check_bits(O.scalar_contig(op, np.array(g["input"], np.float32), s), g[key])


def test_scalar_div_uses_reciprocal_multiplication():
    g = G["scalar_div_reciprocal"]
    d = f32_from_bits([g["denominator_bits"]])
    s = f32_from_bits([g["scalar_bits"]])[0]
    check_bits(O.scalar_contig(O.S_RDIV, d, s), [g["expected_bits"]])
    tiny = np.array([1.0e-39], np.float32)
    assert np.isinf(O.scalar_contig(O.S_RDIV, tiny, 1.0e-38)[0])
    assert np.isnan(O.scalar_contig(O.S_RDIV, tiny, 0.0)[0])


@pytest.mark.parametrize("key,op", [("sub_nonfinite", O.SUB), ("div_nonfinite", O.DIV)])
def test_nonfinite_and_signed_zero(key, op):
    g = G[key]
    out = O.binary_contig(op, f32_from_bits(g["left"]), f32_from_bits(g["right"]))
    check_bits(out, g["expected"])


def test_sum_known_answer_and_transposed_view():
    g = G["sum_small"]
    assert O.sum_f32(np.array(g["input"], np.float32), (3,)) == g["expected"]
    s = G["stride_aware_broadcast"]
    storage = np.arange(24, dtype=np.float32)
    total = O.sum_f32(storage, s["shape"], s["strides"])
    assert int(np.float32(total).view(np.uint32)) == int(s["sum_bits"], 16)


def test_transposed_logical_values_and_broadcast_row():
    g = G["transpose_logical_values"]
    storage = np.arange(g["storage_len"], dtype=np.float32)
    out = O.unary(O.COPY, storage, g["shape"], g["strides"], 0, O.contiguous_strides(g["shape"]))
    assert out.tolist() == g["expected"]
    s = G["stride_aware_broadcast"]
    row = np.array(s["row"], np.float32)
    oshape, ostr = O.binary_output_layout(s["shape"], s["strides"], (2,), (1,))
    assert ostr == tuple(s["strides"])
    out = O.binary(O.ADD, storage, s["shape"], s["strides"], 0, row, (2,), (1,), 0, oshape, ostr)
    logical = O.unary(O.COPY, out, oshape, ostr, 0, O.contiguous_strides(oshape))
    assert logical[:6].tolist() == s["first_six_logical"]


@pytest.mark.parametrize("key", ["matmul_known", "matmul_transposed", "matmul_indexed_transposed"])
def test_matmul_known_answers(key):
    g = G[key]
    if key == "matmul_known":
        a = np.array(g["left"], np.float32)
        b = np.array(g["right"], np.float32)
        la = (g["left_shape"], O.contiguous_strides(g["left_shape"]), 0)
        lb = (g["right_shape"], O.contiguous_strides(g["right_shape"]), 0)
    else:
        a = np.arange(g["left_storage_len"], dtype=np.float32)
        b = np.arange(g["right_storage_len"], dtype=np.float32)
        la = (g["left_shape"], g["left_strides"], g["left_offset"])
        lb = (g["right_shape"], g["right_strides"], g["right_offset"])
    out = O.matmul(a, *la, b, *lb)
    assert out.tolist() == g["expected"]


def _stride_case_error(case):
    return {"stride_overflow": -3, "shape_mismatch": -4}[case["error"]]


@pytest.mark.parametrize("case", G["output_strides"]["unary"], ids=lambda c: c["src"])
def test_unary_output_strides(case):
    if "error" in case:
        with pytest.raises(O.OracleError) as e:
            O.unary_output_strides(case["shape"], case["strides"])
        assert e.value.args[0] == _stride_case_error(case)
    else:
        assert O.unary_output_strides(case["shape"], case["strides"]) == tuple(case["expected"])


@pytest.mark.parametrize("case", G["output_strides"]["scalar"], ids=lambda c: c["src"])
def test_scalar_output_strides(case):
    assert O.scalar_output_strides(case["shape"], case["strides"]) == tuple(case["expected"])


@pytest.mark.parametrize("case", G["output_strides"]["binary"], ids=lambda c: c["src"])
def test_binary_output_layout(case):
    args = (case["left_shape"], case["left_strides"], case["right_shape"], case["right_strides"])
    if "error" in case:
        with pytest.raises(O.OracleError) as e:
            O.binary_output_layout(*args)
        assert e.value.args[0] == _stride_case_error(case)
    else:
        shape, strides = O.binary_output_layout(*args)
        assert shape == tuple(case["out_shape"])
        assert strides == tuple(case["expected"])


def test_mul_vjp_square_sum():
    g = G["autograd_square_sum"]
    x = np.array(g["x"], np.float32)
    up = np.ones(3, np.float32)  # Sum VJP fill of 1.0
    # x*x: both operands are x; the two contributions are merged by add_gradient.
    left = O.mul_backward(up, (3,), x, (3,), (1,), 0, (3,))
    right = O.mul_backward(up, (3,), x, (3,), (1,), 0, (3,))
    total = left + right
    assert total.tolist() == g["grad_once"]
    assert (total + total).tolist() == g["grad_twice"]


def test_mul_vjp_unbroadcast():
    g = G["autograd_mul_unbroadcast"]
    l = np.array(g["left"], np.float32)
    r = np.array(g["right"], np.float32)
    up = np.ones(6, np.float32)
    lg = O.mul_backward(up, (2, 3), r, g["right_shape"], (3, 1), 0, g["left_shape"])
    rg = O.mul_backward(up, (2, 3), l, g["left_shape"], (1, 1), 0, g["right_shape"])
    assert lg.tolist() == g["left_grad"]
    assert rg.tolist() == g["right_grad"]


def test_mul_vjp_rank_zero_and_view():
    g = G["autograd_rank_zero_view"]
    storage = np.array(g["storage"], np.float32)
    s = np.array([g["scalar"]], np.float32)
    up = np.ones(6, np.float32)
    sg = O.mul_backward(up, (3, 2), storage, g["view_shape"], g["view_strides"], g["view_offset"], ())
    assert sg.tolist() == [g["scalar_grad"]]
    vg = O.mul_backward(up, (3, 2), s, (), (), 0, g["view_shape"])  # grad in the view's logical order
    # The view's gradient lands back in source storage through the index/transpose views.
    src = np.zeros(12, np.float32)
    for i in range(3):
        for j in range(2):
            src[g["view_offset"] + i * g["view_strides"][0] + j * g["view_strides"][1]] = vg[i * 2 + j]
    assert src.tolist() == g["source_grad"]


def test_mul_vjp_negative_zero_first_contribution():
    g = G["autograd_negative_zero"]
    nb = g["no_broadcast"]
    out = O.mul_backward(np.ones(1, np.float32), (1,), f32_from_bits(nb["right_bits"]), (1,), (1,), 0, (1,))
    check_bits(out, nb["left_grad_bits"])
    b = g["broadcast"]
    out = O.mul_backward(np.ones(2, np.float32), (2,), f32_from_bits(b["right_bits"]), (2,), (1,), 0, ())
    check_bits(out, b["left_grad_bits"])


def test_relu_vjp_bits():
    g = G["autograd_relu_vjp"]
    x = f32_from_bits(g["input_bits"])
    w = f32_from_bits(g["weight_bits"])
    n = x.size
    # loss = sum(relu(x) * w): d relu(x) = 1 * w (no broadcast, stored as is).
    up_relu = O.mul_backward(np.ones(n, np.float32), (n,), w, (n,), (1,), 0, (n,))
    grad = O.relu_backward(x, (n,), (1,), 0, up_relu)
    check_bits(grad, g["expected_gradient_bits"])


def test_permute_vjp_transform():
    g = G["autograd_transform"]
    w = np.array(g["weights"], np.float32)
    # reshape-copy of the transposed [3,2] view: gradient (= weights) maps back through permute [1,0].
    grad = O.permute_backward(w, (3, 2), (1, 0), (2, 3))
    assert grad.tolist() == g["leaf_grad"]


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).ravel()


def test_matmul_paths_agree_on_special_values():
    """src/tensor.rs:4711-4886: every matmul path gives the same bits (NaN
    payloads included) on inf/NaN/huge-cancellation inputs, with the pinned
    elements: the oracle's general strided loop and the reference's 4-row
    blocked loop agree, and element 0 is 1e20 + (-1e20) + 1 = 1.0."""
    g = G["matmul_contiguous_specials"]
    a = f32_from_bits(g["left_bits"]).reshape(g["left_shape"])
    b = f32_from_bits(g["right_bits"]).reshape(g["right_shape"])
    plain = O.matmul(a.ravel(), (2, 3), (3, 1), 0, b.ravel(), (3, 3), (3, 1), 0)
    assert int(_bits(plain)[0]) == g["expected_first_bits"]
    assert np.array_equal(_bits(plain), _bits(O.matmul_row_blocked(a, b)))

    g = G["matmul_blocked_pattern"]
    rows, inner, cols, fb = g["rows"], g["inner"], g["columns"], g["finite_bits"]
    left = f32_from_bits([fb[(i * 5 + i // inner) % 8] for i in range(rows * inner)]).reshape(rows, inner)

    def rbits(d, c):
        if c % 8 == 3 and d == 7:
            return 0x7F800000
        if c % 8 == 4 and d == 11:
            return 0xFF800000
        if c % 8 == 5 and d == 13:
            return 0x7FC12345
        return fb[(d * 3 + c) % 8]

    right = f32_from_bits([rbits(d, c) for d in range(inner) for c in range(cols)]).reshape(inner, cols)
    plain = O.matmul(left.ravel(), (rows, inner), (inner, 1), 0, right.ravel(), (inner, cols), (cols, 1), 0)
    blocked = O.matmul_row_blocked(left, right)
    assert np.array_equal(_bits(plain), _bits(blocked))
    assert np.isnan(blocked[:, 5]).all() and np.isnan(blocked).sum() >= rows

    g = G["matmul_strided_specials"]
    lay = g["layout"]
    ls = np.concatenate([np.zeros(9, np.float32), f32_from_bits(g["left_bits"])])
    rs = np.concatenate([np.zeros(9, np.float32), f32_from_bits(g["right_bits"])])
    strided = O.matmul(ls, tuple(lay["shape"]), tuple(lay["strides"]), lay["offset"],
                       rs, tuple(lay["shape"]), tuple(lay["strides"]), lay["offset"])
    assert int(_bits(strided)[3]) == g["expected_index3_bits"]
    lc = f32_from_bits(g["left_bits"]).reshape(3, 3).T
    rc = f32_from_bits(g["right_bits"]).reshape(3, 3).T
    assert np.array_equal(_bits(strided), _bits(O.matmul_row_blocked(lc, rc)))


def test_matmul_empty_dimensions():
    """src/tensor.rs:4817-4839: empty outputs stay empty; K = 0 gives +0.0."""
    for case in G["matmul_empty_dims"]["cases"]:
        (m, k), (_, n) = case["left"], case["right"]
        out = O.matmul(np.zeros(max(m * k, 1), np.float32), (m, k), (max(k, 1), 1), 0,
                       np.zeros(max(k * n, 1), np.float32), (k, n), (max(n, 1), 1), 0)
        assert out.size == m * n
        if "all_bits" in case:
            assert (_bits(out) == case["all_bits"]).all()
