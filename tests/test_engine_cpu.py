"""Host-side checks of the C++ engine behind torch_rs (no GPU needed).

The engine's output-layout planner is product code restated from
src/tensor.rs; here it is pinned against the reference's golden stride
fixtures and against the independent oracle restatement on random layouts.
View metadata, graph recording on views, error messages and the fusion
tracer are host logic and are checked on CPU tensors.
"""
import itertools
import random

import numpy as np
import pytest

import oracle as O
import torch_rs
from helpers import golden

L = torch_rs._C.layout
G = golden()


# ---- golden output-stride fixtures (tests/tensor_baseline.rs) -------------------

@pytest.mark.parametrize("case", G["output_strides"]["unary"], ids=lambda c: c["src"])
def test_engine_unary_output_strides_golden(case):
    n = int(np.prod(case["shape"], dtype=object)) if case["shape"] else 1
    if "error" in case:
        with pytest.raises(RuntimeError, match="Stride calculation overflowed"):
            L.unary_output_strides(case["shape"], case["strides"], n)
    else:
        assert tuple(L.unary_output_strides(case["shape"], case["strides"], n)) == tuple(case["expected"])


@pytest.mark.parametrize("case", G["output_strides"]["scalar"], ids=lambda c: c["src"])
def test_engine_scalar_output_strides_golden(case):
    assert tuple(L.scalar_output_strides(case["shape"], case["strides"])) == tuple(case["expected"])


@pytest.mark.parametrize("case", G["output_strides"]["binary"], ids=lambda c: c["src"])
def test_engine_binary_output_layout_golden(case):
    args = (case["left_shape"], case["left_strides"], case["right_shape"], case["right_strides"])
    if "error" in case:
        msg = {"stride_overflow": "Stride calculation overflowed",
               "shape_mismatch": "must match the size of tensor b"}[case["error"]]
        with pytest.raises(RuntimeError, match=msg):
            L.binary_output_layout(*args)
    else:
        shape, strides = L.binary_output_layout(*args)
        assert shape == tuple(case["out_shape"])
        assert strides == tuple(case["expected"])


def test_shape_mismatch_message_matches_reference():
    g = G["shape_mismatch_message"]
    a = torch_rs.zeros(*g["left_shape"])
    b = torch_rs.zeros(*g["right_shape"])
    with pytest.raises(RuntimeError) as e:
        a + b
    assert str(e.value) == g["message"]


# ---- engine planner == oracle planner on random layouts ---------------------------

def _random_layout(rng, rank):
    shape = [rng.choice([0, 1, 1, 2, 3, 4]) if rng.random() < 0.15 else rng.choice([1, 2, 3, 4, 5])
             for _ in range(rank)]
    kind = rng.random()
    cs = list(O.contiguous_strides(shape))
    if kind < 0.3:
        strides = cs
    elif kind < 0.6:  # permuted dense
        perm = list(range(rank))
        rng.shuffle(perm)
        pshape = [shape[p] for p in perm]
        pcs = O.contiguous_strides(pshape)
        strides = [0] * rank
        for i, p in enumerate(perm):
            strides[p] = pcs[i]
    elif kind < 0.8:  # sliced / strided
        strides = [s * rng.choice([1, 2, 3]) for s in cs]
    else:  # arbitrary, incl. zero strides
        strides = [rng.choice([0, 1, 2, 3, 5, 7, 12]) for _ in range(rank)]
    return shape, strides


def _broadcast_partner(rng, shape):
    rank = rng.randint(0, len(shape))
    out = list(shape[len(shape) - rank:])
    for i in range(len(out)):
        if rng.random() < 0.3:
            out[i] = 1
    return out


def test_engine_planner_matches_oracle_on_random_layouts():
    rng = random.Random(0xC0FFEE)
    checked = 0
    for _ in range(3000):
        rank = rng.randint(0, 5)
        shape, strides = _random_layout(rng, rank)
        n = int(np.prod(shape)) if shape else 1
        assert L.is_contiguous(shape, strides, n) == O.is_contiguous(shape, strides)
        assert L.is_non_overlapping_and_dense(shape, strides, n) == O.is_non_overlapping_and_dense(shape, strides)
        assert tuple(L.unary_output_strides(shape, strides, n)) == O.unary_output_strides(shape, strides)
        assert tuple(L.scalar_output_strides(shape, strides)) == O.scalar_output_strides(shape, strides)
        rshape = _broadcast_partner(rng, shape) if rng.random() < 0.5 else list(shape)
        _, rstrides = _random_layout(rng, len(rshape))
        rstrides = rstrides if rshape == shape or rng.random() < 0.5 else list(O.contiguous_strides(rshape))
        if rng.random() < 0.5:
            shape, strides, rshape, rstrides = rshape, rstrides, shape, strides
        want = O.binary_output_layout(shape, strides, rshape, rstrides)
        got = L.binary_output_layout(shape, strides, rshape, rstrides)
        assert got == want, (shape, strides, rshape, rstrides)
        checked += 1
    assert checked == 3000


# ---- reshape / view strides ----------------------------------------------------------

def _offsets(shape, strides):
    return [sum(i * s for i, s in zip(idx, strides)) for idx in itertools.product(*[range(d) for d in shape])]


def test_reshape_view_strides_are_sound_on_random_layouts():
    rng = random.Random(7)
    views = 0
    for _ in range(2000):
        rank = rng.randint(1, 4)
        shape = [rng.choice([1, 2, 3, 4]) for _ in range(rank)]
        _, strides = _random_layout(rng, rank)
        n = int(np.prod(shape))
        # a random factorisation of n as the new shape
        new, rem = [], n
        while rem > 1 and len(new) < 4:
            f = rng.choice([d for d in range(1, rem + 1) if rem % d == 0])
            new.append(f)
            rem //= f
        new.append(rem)
        got = L.reshape_view_strides(shape, strides, new, n)
        if got is not None:
            views += 1
            assert _offsets(new, got) == _offsets(shape, strides)
    assert views > 500


def test_view_of_transposed_matrix_is_rejected_and_reshape_copies_on_device_only():
    x = torch_rs.zeros(2, 3)
    with pytest.raises(RuntimeError, match="view size is not compatible"):
        x.mT.view(6)
    assert x.view(3, 2).stride() == (2, 1)
    assert x.view(-1).shape == (6,)
    with pytest.raises(RuntimeError, match="only one dimension can be inferred"):
        x.view(-1, -1)
    with pytest.raises(RuntimeError, match=r"shape '\[4, -1\]' is invalid for input of size 6"):
        x.view(4, -1)


# ---- view metadata and graph recording on host tensors ------------------------------

def test_view_metadata_matches_reference_rules():
    x = torch_rs.zeros(2, 3, 4)
    p = x.permute(2, 0, 1)
    assert p.shape == (4, 2, 3) and p.stride() == (1, 12, 4)
    t = x.transpose(0, 2)
    assert t.shape == (4, 3, 2) and t.stride() == (1, 4, 12)
    assert x.mT.shape == (2, 4, 3) and x.mT.stride() == (12, 1, 4)
    assert x.T.shape == (4, 3, 2)
    s = x[1]
    assert s.shape == (3, 4) and s.storage_offset() == 12
    assert x[-1].storage_offset() == 12
    with pytest.raises(IndexError, match="index 2 is out of bounds for dimension 0 with size 2"):
        x[2]
    with pytest.raises(RuntimeError, match="duplicate dims"):
        x.permute(0, 0, 1)
    with pytest.raises(IndexError, match=r"Dimension out of range \(expected to be in range of \[-3, 2\], but got 3\)"):
        x.transpose(0, 3)
    with pytest.raises(RuntimeError, match="tensor.mT is only supported on matrices"):
        torch_rs.zeros(3).mT


def test_squeeze_and_swapdims_views_follow_reference_rules():
    # squeeze / squeeze_dim / squeeze_dims (src/tensor.rs:1305-1390): size-1
    # dims dropped, other strides and the offset kept; swapdims/swapaxes are
    # transpose (src/python.rs:3634-3672).
    x = torch_rs.zeros(2, 1, 3, 1, requires_grad=True)
    s = x.squeeze()
    assert s.shape == (2, 3) and s.stride() == (3, 1) and s.grad_fn.name() == "SqueezeBackward0"
    s1 = x.squeeze(1)
    assert s1.shape == (2, 3, 1) and s1.stride() == (3, 1, 1) and s1.grad_fn.name() == "SqueezeBackward1"
    assert x.squeeze(0).shape == (2, 1, 3, 1)  # size 2: unchanged metadata
    assert x.squeeze(-1).shape == (2, 1, 3)
    s2 = x.squeeze((1, -1))
    assert s2.shape == (2, 3) and s2.grad_fn.name() == "SqueezeBackward2"
    assert x.squeeze(()).shape == (2, 1, 3, 1)
    with pytest.raises(RuntimeError, match="dim 1 appears multiple times in the list of dims"):
        x.squeeze((1, -3))
    with pytest.raises(IndexError, match=r"Dimension out of range \(expected to be in range of \[-4, 3\]"):
        x.squeeze(4)
    o = torch_rs.zeros(2, 3, 4)[1].squeeze()
    assert o.storage_offset() == 12 and o.stride() == (4, 1)
    sc = torch_rs.zeros(())
    assert sc.squeeze().shape == () and sc.squeeze(0).shape == () and sc.squeeze(-1).shape == ()
    w = torch_rs.zeros(2, 3, 4, requires_grad=True).swapdims(0, -1)
    assert w.shape == (4, 3, 2) and w.stride() == (1, 4, 12) and w.grad_fn.name() == "TransposeBackward0"
    assert torch_rs.zeros(2, 3).swapaxes(1, 0).stride() == (1, 3)
    assert sc.swapdims(0, -1).shape == ()


def test_repr_matches_reference_known_answers():
    # Tensor.__repr__ prints every logical value with Rust's f32 `{:?}` and the
    # shape (src/python.rs:3933-3942).  Known answers: tests/test_tensor_t.py:216-219
    # and tests/test_squeeze.py:81 (a (3, 2) view with strides (4, 12), offset 1).
    source = torch_rs.tensor(np.arange(24, dtype=np.float32).reshape(2, 3, 4))
    assert repr(source.T) == (
        "tensor([0.0, 12.0, 4.0, 16.0, 8.0, 20.0, 1.0, 13.0, 5.0, 17.0, 9.0, 21.0, 2.0, 14.0, 6.0, 18.0, "
        "10.0, 22.0, 3.0, 15.0, 7.0, 19.0, 11.0, 23.0], shape=[4, 3, 2])")
    view = source.T[1]
    assert view.stride() == (4, 12) and view.storage_offset() == 1
    assert repr(view) == "tensor([1.0, 13.0, 5.0, 17.0, 9.0, 21.0], shape=[3, 2])"
    assert repr(torch_rs.tensor(2.5)) == "tensor([2.5], shape=[])"
    assert repr(torch_rs.zeros(2, 0, 3)) == "tensor([], shape=[2, 0, 3])"


@pytest.mark.parametrize("value,text", [
    (0.1, "0.1"), (1.0, "1.0"), (-0.0, "-0.0"), (100.0, "100.0"), (123456789.0, "123456790.0"),
    (1e15, "1000000000000000.0"), (1e16, "1e16"), (1.5e16, "1.5e16"), (1e-4, "0.0001"), (9.99e-5, "9.99e-5"),
    (1e-5, "1e-5"), (3.4028235e38, "3.4028235e38"), (1.1754944e-38, "1.1754944e-38"), (1e-45, "1e-45"),
    (float("nan"), "NaN"), (float("inf"), "inf"), (float("-inf"), "-inf"),
])
def test_f32_debug_format_follows_rust(value, text):
    # Rust's Debug for f32: shortest round-trip digits; exponent form when
    # 0 < |v| < 1e-4 or |v| >= 1e16, else positional with a fractional digit.
    assert torch_rs._rust_f32_debug(np.float32(value)) == text


def test_views_record_transform_nodes_and_leafness():
    x = torch_rs.zeros(2, 3, requires_grad=True)
    assert x.is_leaf and x.requires_grad and x.grad_fn is None and x.grad is None
    assert x.permute(1, 0).grad_fn.name() == "PermuteBackward0"
    assert x.transpose(0, 1).grad_fn.name() == "TransposeBackward0"
    assert x.t().grad_fn.name() == "TBackward0"
    assert x.view(6).grad_fn.name() == "ViewBackward0"
    assert x[0].grad_fn.name() == "SelectBackward0"
    v = x.view(3, 2)
    assert v.requires_grad and not v.is_leaf
    with torch_rs.no_grad():
        w = x.view(6)
        assert w.requires_grad and w.grad_fn is None  # view_requires_grad without an edge
        assert not torch_rs.is_grad_enabled()
    assert torch_rs.is_grad_enabled()
    d = x.detach()
    assert not d.requires_grad and d.is_leaf


def test_autograd_backward_option_checks_follow_the_reference():
    # python/torch_rs/autograd/__init__.py:22-127
    A = torch_rs.autograd
    x = torch_rs.zeros(2, requires_grad=True)
    with pytest.raises(TypeError, match="only supports an exact native Tensor"):
        A.backward([x, x])
    with pytest.raises(TypeError, match="only supports an exact native Tensor"):
        A.backward(None)
    for kwargs, msg in (({"grad_tensors": x}, "does not support explicit gradients"),
                        ({"retain_graph": True}, "does not support retain_graph=True"),
                        ({"create_graph": 1}, "does not support create_graph=True"),
                        ({"grad_variables": [x]}, "does not support grad_variables"),
                        ({"inputs": [x]}, "does not support inputs")):
        with pytest.raises(NotImplementedError, match=msg):
            A.backward((x,), **kwargs)
    with pytest.raises(TypeError):
        A.backward(x, create_graph=None)  # operator.index(None)
    with pytest.raises(RuntimeError, match="grad can be implicitly created only for scalar outputs"):
        A.backward([x], retain_graph=False)
    assert A.no_grad is torch_rs.no_grad


def test_backward_errors_match_reference_messages():
    x = torch_rs.zeros(2)
    with pytest.raises(RuntimeError, match="element 0 of tensors does not require grad"):
        x.backward()
    y = torch_rs.zeros(2, requires_grad=True)
    with pytest.raises(RuntimeError, match="grad can be implicitly created only for scalar outputs"):
        y.backward()


def test_host_tensors_do_not_compute():
    x = torch_rs.tensor([1.0, 2.0])
    with pytest.raises(RuntimeError, match="device tensors only"):
        x * 2.0
    with pytest.raises(RuntimeError, match="device tensors only"):
        x.exp()
    assert x.tolist() == [1.0, 2.0]
    assert np.asarray(x).dtype == np.float32


def test_scalar_operands_are_parsed_as_the_reference_does():
    # parse_arithmetic_scalar (src/python.rs:10070-10184) and binary_operation
    # (:4067-4133).  Host tensors stop at the device check once parsing passed.
    x = torch_rs.zeros(2)
    with pytest.raises(RuntimeError, match="^Subtraction, the `-` operator, with a bool tensor is not supported"):
        x - True
    with pytest.raises(RuntimeError, match="device tensors only"):
        x - np.bool_(True)  # a NumPy bool is a number, not a bool operand
    for big in (2 ** 70, -(2 ** 64)):
        with pytest.raises(OverflowError, match="^Python integer is outside the supported scalar range$"):
            x + big
    with pytest.raises(RuntimeError, match="device tensors only"):
        x + 2 ** 63  # fits u64
    with pytest.raises(RuntimeError, match="device tensors only"):
        np.float32(2) / x  # __array_priority__: NumPy defers to Tensor.__rtruediv__
    wide = np.uint64(2 ** 63 + 5)
    r = wide / x  # numpy_reflected_divide: NumPy divides by the tensor's values
    assert isinstance(r, np.ndarray) and np.isinf(r).all()
    with pytest.raises(TypeError, match="unsupported operand"):
        x + "a"


def test_array_protocol_copies_and_refuses_views():
    x = torch_rs.tensor(np.arange(6, dtype=np.float32).reshape(2, 3))
    a = np.asarray(x)
    assert a.dtype == np.float32 and a.shape == (2, 3) and a.tolist() == [[0, 1, 2], [3, 4, 5]]
    assert np.asarray(x, dtype=np.float64).dtype == np.float64
    with pytest.raises(ValueError, match="^cannot create a non-copying NumPy view of tensor storage$"):
        np.array(x, copy=False)


def test_truth_value_follows_the_reference():
    # src/python.rs:4015-4029: one element -> value != 0; otherwise an error.
    assert bool(torch_rs.tensor(2.0)) and not bool(torch_rs.tensor(0.0)) and not bool(torch_rs.tensor(-0.0))
    assert bool(torch_rs.tensor([[3.0]])) and bool(torch_rs.tensor(float("nan")))
    with pytest.raises(RuntimeError, match="^Boolean value of Tensor with more than one value is ambiguous$"):
        bool(torch_rs.zeros(2))
    with pytest.raises(RuntimeError, match="^Boolean value of Tensor with no values is ambiguous$"):
        bool(torch_rs.zeros(0))
    with pytest.raises(TypeError, match="len\\(\\) of a 0-d tensor"):
        len(torch_rs.tensor(1.0))


def test_tensor_constructor_and_scalar_conversion():
    t = torch_rs.tensor([[1, 2], [3, 4.5]])
    assert t.shape == (2, 2) and t.numpy().tolist() == [[1.0, 2.0], [3.0, 4.5]]
    assert torch_rs.tensor(0.1).numpy() == np.float32(0.1)
    assert torch_rs.tensor(np.arange(6, dtype=np.float64).reshape(2, 3)).stride() == (3, 1)
    # 0-d arrays and numpy scalars stay scalars; transposed arrays are copied row-major.
    assert torch_rs.tensor(np.array(0.5, np.float32)).shape == ()
    assert torch_rs.tensor(np.float32(0.5)).shape == ()
    assert torch_rs.tensor(np.arange(6, dtype=np.float32).reshape(2, 3).T).numpy().tolist() == [[0, 3], [1, 4], [2, 5]]
    assert torch_rs.tensor(np.zeros((2, 0, 3), np.float32)).shape == (2, 0, 3)
    with pytest.raises(TypeError, match="invalid data type 'bytes'"):
        torch_rs.tensor(b"ab")
    with pytest.raises(ValueError):
        torch_rs.tensor([[1.0], [2.0, 3.0]])
    assert torch_rs.get_float32_matmul_precision() == "highest"


def test_top_level_unary_guards_follow_the_reference():
    # apply_top_level_unary_out (src/python.rs:2673-2694, 1784-1820): `out` is
    # rejected first; torch.exp refuses to record on a grad-requiring input
    # (tests/test_top_level_exp.py:108-137).  Host tensors keep that refusal.
    x = torch_rs.tensor([[-2.0, 0.0, 1.0], [2.0, 4.0, 6.0]], requires_grad=True).transpose(0, 1)[1]
    with pytest.raises(RuntimeError, match=r"^exp\(\): autograd recording is not supported$"):
        torch_rs.exp(x)
    for fn, name in ((torch_rs.exp, "exp"), (torch_rs.neg, "neg"), (torch_rs.negative, "negative")):
        with pytest.raises(RuntimeError, match=f"^{name}\\(\\): the 'out' argument is not supported$"):
            fn(x, out=torch_rs.zeros(2))
    with torch_rs.no_grad():
        with pytest.raises(RuntimeError, match="device tensors only"):
            torch_rs.exp(x)  # past the guard; host tensors do not compute


def test_matmul_shape_and_rank_errors_come_before_the_device_check():
    # tests/test_matmul.py:326-361 and 492-539: every spelling reports the
    # reference's shape message (src/tensor_error.rs:243); other ranks report
    # src/tensor_error.rs:120.  Host tensors are never computed on, but they
    # fail with the same message as the reference first.
    for ls, rs in (((2, 3), (4, 2)), ((0, 3), (4, 0))):
        l, r = torch_rs.zeros(ls), torch_rs.zeros(rs)
        msg = f"^mat1 and mat2 shapes cannot be multiplied \\({ls[0]}x{ls[1]} and {rs[0]}x{rs[1]}\\)$"
        for call in (lambda: l.matmul(r), lambda: l @ r, lambda: l.matmul(other=r), lambda: l.matmul(x2=r),
                     lambda: torch_rs.matmul(l, r), lambda: torch_rs.matmul(input=l, other=r),
                     lambda: torch_rs.matmul(x1=l, x2=r)):
            with pytest.raises(RuntimeError, match=msg):
                call()
    for l, r in ((torch_rs.tensor(1.0), torch_rs.ones((1, 1))), (torch_rs.ones((2,)), torch_rs.ones((2, 2))),
                 (torch_rs.ones((1, 2, 2)), torch_rs.ones((2, 2))), (torch_rs.ones((2, 2, 2)), torch_rs.ones((2, 2, 2)))):
        with pytest.raises(RuntimeError) as a:
            l.matmul(r)
        with pytest.raises(RuntimeError) as b:
            l @ r
        assert str(a.value) == str(b.value) and "requires two rank-2 tensors" in str(a.value)
    with pytest.raises(TypeError, match="^matmul\\(\\) got an unexpected keyword argument 'out'$"):
        torch_rs.matmul(torch_rs.ones((1, 1)), torch_rs.ones((1, 1)), out=torch_rs.zeros((1, 1)))
    with pytest.raises(RuntimeError, match="device tensors only"):
        torch_rs.ones((2, 3)) @ torch_rs.ones((3, 2))


def test_dropout_argument_checks_follow_the_reference_order_and_messages():
    # python/torch_rs/nn/functional.py:14-31 (range check, ValueError, before
    # anything else) and src/python_nn_functional.rs:103-200 (type checks, then
    # a RuntimeError with `.6g` formatting for what passes the Python check);
    # cases after tests/test_nn_functional_dropout.py:335-560.
    F = torch_rs.nn.functional
    src = torch_rs.tensor([1.0, 2.0])
    for p, shown in ((-0.1, "-0.1"), (1.1, "1.1"), (float("inf"), "inf"), (2, "2")):
        with pytest.raises(ValueError) as e:
            F.dropout(None, p=p, training="invalid", inplace=True)
        assert str(e.value) == f"dropout probability has to be between 0 and 1, but got {shown}"
    for p in (float("nan"), np.float32(np.nan)):
        with pytest.raises(RuntimeError, match="^dropout probability has to be between 0 and 1, but got nan$"):
            F.dropout(src, p=p, training=False)
    with pytest.raises(RuntimeError, match="^dropout probability has to be between 0 and 1, but got -nan$"):
        F.dropout(src, p=-float("nan"), training=False)

    class Sneaky(float):  # defeats the Python-level comparisons
        def __lt__(self, other):
            return False

        def __gt__(self, other):
            return False

    for value, shown in ((2, "2"), (1.0000000000001, "1"), (1.23456789, "1.23457"), (999999.9, "1e+06"),
                         (-1.23456789e-7, "-1.23457e-07"), (-5e-324, "-4.94066e-324")):
        with pytest.raises(RuntimeError) as e:
            F.dropout(src, p=Sneaky(value), training=False)
        assert str(e.value) == f"dropout probability has to be between 0 and 1, but got {shown}"
    # scalar-tensor probabilities: 0-d shows the value, others the tensor with its autograd state
    for value in (-0.1, 1.1, float("inf")):
        prob = torch_rs.tensor(value)
        with pytest.raises(ValueError) as e:
            F.dropout(None, p=prob, training=False)
        assert str(e.value) == f"dropout probability has to be between 0 and 1, but got {prob.item()}"
    leaf = torch_rs.tensor([2.0], requires_grad=True)
    for prob, shown in ((torch_rs.tensor([2.0]), "tensor([2.])"), (leaf, "tensor([2.], requires_grad=True)"),
                        (leaf.reshape(1, 1), "tensor([[2.]], grad_fn=<ViewBackward0>)")):
        with pytest.raises(ValueError) as e:
            F.dropout(src, p=prob)
        assert str(e.value) == f"dropout probability has to be between 0 and 1, but got {shown}"
    with pytest.raises(RuntimeError, match="Boolean value of Tensor with more than one value is ambiguous"):
        F.dropout(src, p=torch_rs.tensor([0.1, 0.2]))
    with pytest.raises(TypeError, match=r"^dropout\(\): argument 'input' \(position 1\) must be Tensor, not NoneType$"):
        F.dropout(None, p=0)
    with pytest.raises(TypeError, match=r"^dropout_\(\): argument 'input' \(position 1\) must be Tensor, not NoneType$"):
        F.dropout(None, p=0, inplace=True)
    with pytest.raises(TypeError, match="'<' not supported between instances of 'NoneType' and 'float'"):
        F.dropout(src, p=None, training=False)
    with pytest.raises(TypeError, match=r"^dropout\(\): argument 'train' \(position 3\) must be bool, not int$"):
        F.dropout(src, p=0, training=1)
    with pytest.raises(TypeError, match=r"^dropout\(\): argument 'train' \(position 3\) must be bool, not numpy.bool$"):
        F.dropout(src, p=0, training=np.bool_(False))
    assert F.dropout(src, p=torch_rs.tensor(0.0)) is src
    assert F.dropout(torch_rs.zeros(0), p=0.5) is not None


def test_dropout_family_deterministic_cases_follow_the_reference():
    # src/python_nn_functional.rs:13-62 (kinds) and :117-200 (bridge);
    # messages after tests/test_nn_functional_dropout1d.py:297-580 and the
    # dropout2d/alpha tests.
    import warnings as _w
    F = torch_rs.nn.functional
    x3 = torch_rs.zeros((1, 2, 3), requires_grad=True)
    x2 = torch_rs.zeros((2, 3), requires_grad=True)
    # identities return the input itself, except unbatched dropout1d
    for fn, x in ((F.dropout1d, x3), (F.dropout3d, torch_rs.zeros((1, 1, 1, 1, 2)))):
        assert fn(x, p=0.75, training=False) is x
    y = F.dropout1d(x2, p=0.75, training=False)
    assert y is not x2 and y.shape == (2, 3) and y.stride() == x2.stride()
    assert y.grad_fn.name() == "SqueezeBackward1"
    assert F.alpha_dropout(x3, p=0.5) is x3  # training defaults to False
    assert F.feature_alpha_dropout(x3, p=0.5) is x3
    with pytest.raises(AttributeError, match="^'NoneType' object has no attribute 'dim'$"):
        F.dropout1d(None, p=0)
    with pytest.raises(NotImplementedError, match="^torch_rs.nn.functional.dropout1d does not support inplace=True "
                                                  "for rank-2 inputs$"):
        F.dropout1d(x2, p=0.5, inplace=True)
    with pytest.raises(NotImplementedError, match="^torch_rs.nn.functional.dropout1d only supports rank-2 or "
                                                  "rank-3 inputs$"):
        F.dropout1d(torch_rs.zeros(4), p=0.5)
    with pytest.raises(NotImplementedError, match="^torch_rs.nn.functional.dropout2d only supports rank-3 or "
                                                  "rank-4 inputs$"):
        F.dropout2d(x2, p=0.5, training=False)
    with pytest.raises(NotImplementedError, match="^torch_rs.nn.functional.dropout3d only supports rank-5 inputs$"):
        F.dropout3d(x3, p=0.5, training=False)
    with _w.catch_warnings(record=True) as caught:
        _w.simplefilter("always")
        assert F.dropout2d(x3, p=0.5, training=False) is x3
    assert any("Received a 3D input to dropout2d" in str(w.message) for w in caught)
    for fn in (F.dropout1d, F.dropout2d, F.feature_alpha_dropout, F.alpha_dropout):
        with pytest.raises(NotImplementedError, match=f"^torch_rs.nn.functional.{fn.__name__} does not support "
                                                      "sampling$"):
            fn(x3, p=0.5, training=True)
    # p == 1 is input * 0.0 only where the kind allows it (dropout2d does not)
    with pytest.raises(NotImplementedError, match="dropout2d does not support sampling"):
        F.dropout2d(x3, p=1.0, training=True)
    with pytest.raises(RuntimeError, match="device tensors only"):  # the multiply itself needs the device
        F.dropout3d(torch_rs.zeros((1, 1, 1, 1, 2)), p=1.0, training=True)
    # probability arguments
    with pytest.raises(TypeError, match=r"^alpha_dropout\(\): argument 'p' \(position 2\) must be float, not Tensor$"):
        F.alpha_dropout(x3, p=torch_rs.tensor(0.5))
    with pytest.raises(TypeError, match=r"^feature_dropout_\(\): argument 'p' \(position 2\) must be float, "
                                        r"not Tensor$"):
        F.dropout2d(x3, p=torch_rs.tensor([0.5]), inplace=True)
    with pytest.raises(TypeError, match=r"^dropout\(\): argument 'p' \(position 2\) must be float, not Tensor$"):
        F.dropout(x3, p=torch_rs.tensor(0.5, requires_grad=True))
    assert F.dropout(x3, p=np.float32(0.0)) is x3 and F.dropout(x3, p=np.bool_(False)) is x3
    with pytest.raises(TypeError, match=r"^dropout\(\): argument 'p' \(position 2\) must be float, not "
                                        r"test_engine_cpu.SneakyStr$"):
        F.dropout(x3, p=SneakyStr("0.5"))


class SneakyStr(str):  # passes the Python-level range check; not float-like
    def __lt__(self, other):
        return False

    def __gt__(self, other):
        return False


def test_dropout_bridge_cases_on_host():
    F = torch_rs.nn.functional
    x = torch_rs.zeros(4)
    assert F.dropout(x, 0.5, training=False) is x
    assert F.dropout(x, 0.0) is x
    with pytest.raises(ValueError, match="^dropout probability has to be between 0 and 1, but got 1.5$"):
        F.dropout(x, 1.5)
    with pytest.raises(NotImplementedError, match="does not support sampling"):
        F.dropout(x, 0.5)
    with pytest.raises(NotImplementedError, match="inplace=True"):
        F.relu(x, inplace=True)


# ---- fusion tracer --------------------------------------------------------------------------

def test_fusion_tracer_emits_one_rounding_per_op_and_eager_layout():
    f = torch_rs.fuse(lambda x, y, z: ((x * y + z).exp() - 1.0).relu())
    x = torch_rs.zeros(8)
    ir, shape, strides, used = f.trace(x, x, x)
    assert ir == "in f32\nin f32\nin f32\nmul %0 %1\nadd %3 %2\nexp %4\nconst 0x3f800000\nsub %5 %6\nrelu %7\nout %8\n"
    assert shape == (8,) and strides == (1,) and used == [0, 1, 2]
    # (a + b) * c.mT: the planner's contiguous output for config 2's layouts
    g = torch_rs.fuse(lambda a, b, c: (a + b) * c)
    a, b = torch_rs.zeros(64, 1, 8), torch_rs.zeros(1, 16, 8)
    c = torch_rs.zeros(64, 8, 16).mT
    _, shape, strides, _ = g.trace(a, b, c)
    want_shape, want_strides = O.binary_output_layout((64, 16, 8), O.contiguous_strides((64, 16, 8)),
                                                      c.shape, c.stride())
    assert shape == want_shape == (64, 16, 8) and strides == want_strides
    # scalar forms: s - x, s / x -> s * (1 / x), x * s
    h = torch_rs.fuse(lambda x: (2.0 - x) + 3.0 / x + x * 0.5)
    ir, _, _, _ = h.trace(x)
    assert "sub %1 %0" in ir and "div %" in ir and "mul %0 %" in ir


def test_fusion_backward_program_is_the_reverse_mode_of_the_ir():
    """The fused node's backward: one program with one output per input that
    needs a gradient, each the eager VJP's expression (mul: up * other; add:
    up); a division passes no gradient; an input used twice falls back to
    eager autograd (None)."""
    from torch_rs import fusion as F
    x = torch_rs.zeros(4)

    def plan(fn, requires):
        tr, out = torch_rs.fuse(fn)._trace(tuple(x for _ in requires))
        return F._gradient_program(tr, out.vid, requires, out.shape)

    # x*y + z: dx = up*y, dy = up*x, dz = up; arguments x, y, upstream
    assert plan(lambda x, y, z: x * y + z, (True, True, True)) == (
        "in f32\nin f32\nin f32\nmul %2 %1\nmul %2 %0\nout %3\nout %4\nout %2\n", [0, 1, -1], [0, 1, 2])
    assert plan(lambda x, y, z: x * y + z, (False, True, False)) == ("in f32\nin f32\nmul %1 %0\nout %2\n",
                                                                    [0, -1], [1])
    # x reaches the output only through a division: no gradient for x
    assert plan(lambda x, y, z, t: (x * y) / z + t, (True, False, False, True)) == ("in f32\nout %0\n", [-1], [3])
    assert plan(lambda x, y, z, t: (x * y) / z + t, (True, False, False, False)) == F._NO_GRAD
    # a full-shape input with two gradient-carrying uses: its two
    # contributions are summed in the program (x*x: up*x + up*x)
    ir, args, targets = plan(lambda x, y: (x * y).exp() - x.relu(), (True, True))
    assert targets == [0, 1]
    assert plan(lambda x, y: x * x, (True, False)) == ("in f32\nin f32\nmul %1 %0\nmul %1 %0\nadd %2 %3\nout %4\n",
                                                     [0, -1], [0])
    # three uses, or two uses of a broadcast input: eager
    assert plan(lambda x, y: x * x * x, (True, False)) is None
    tr_b, out_b = torch_rs.fuse(lambda x, b: x * b + b)._trace((torch_rs.zeros(4, 3), torch_rs.zeros(3)))
    assert F._gradient_program(tr_b, out_b.vid, (False, True), out_b.shape) is None

    def two_uses(x, y):
        s = x * y
        return s.relu() * s.exp()

    ir, args, targets = plan(two_uses, (True, False))
    assert targets == [0] and args == [0, 1, -1]
    assert "relub" in ir and ir.count("\nout ") == 1


def test_fusion_tracer_declares_broadcast_inputs_first():
    """relu(x + b) with b a row broadcast: b's `in` comes first so kernels load
    it before streaming x; the add still takes x, then b.  This is the IR the
    bench launches for the row-broadcast config."""
    f = torch_rs.fuse(lambda x, b: (x + b).relu())
    ir, shape, _, used = f.trace(torch_rs.zeros(4096, 4096), torch_rs.zeros(4096))
    assert ir == "in f32\nin f32\nadd %1 %0\nrelu %2\nout %3\n" and used == [1, 0] and shape == (4096, 4096)
    g = torch_rs.fuse(lambda a, b, c: (a + b) * c)
    ir, _, _, used = g.trace(torch_rs.zeros(2, 3), torch_rs.zeros(3), torch_rs.zeros(1, 1))
    assert used == [1, 2, 0] and ir == "in f32\nin f32\nin f32\nadd %2 %0\nmul %3 %1\nout %4\n"


def test_fusion_tracer_drops_dead_code_and_unused_inputs():
    f = torch_rs.fuse(lambda x, y, z: (y * 2.0).relu())  # x and z unused
    x, y, z = torch_rs.zeros(5, 7), torch_rs.zeros(3), torch_rs.zeros(9)
    ir, shape, _, used = f.trace(x, y, z)
    assert used == [1] and shape == (3,)
    assert ir == "in f32\nconst 0x40000000\nmul %0 %1\nrelu %2\nout %3\n"
    g = torch_rs.fuse(lambda x, y: ((x + 1.0) * 3.0, y - x)[1])
    ir, _, _, used = g.trace(torch_rs.zeros(4), torch_rs.zeros(4))
    assert used == [0, 1] and "add" not in ir


def test_permute_spellings_negative_dims_and_errors():
    """tests/test_permute.py's forms (variadic, tuple, list, dims=; negative
    dims normalised) and the binding's errors (src/python.rs:9321-9553)."""
    base = torch_rs.zeros(2, 3, 4)
    source = base.transpose(0, 2)[1]  # shape (3, 2), offset view
    for view in (source.permute(-1, -2), source.permute((-1, -2)), source.permute([-1, -2]),
                 source.permute(dims=(-1, -2)), source.permute(dims=[-1, -2])):
        assert view.shape == (2, 3) and view.stride() == (source.stride()[1], source.stride()[0])
        assert view.storage_offset() == source.storage_offset() and view.data_ptr() == source.data_ptr()
    scalar = torch_rs.tensor([2.5, 3.5])[1]
    for view in (scalar.permute(()), scalar.permute([]), scalar.permute(dims=()), scalar.permute(dims=[])):
        assert view.shape == () and view.stride() == () and view.storage_offset() == 1
    empty = torch_rs.zeros(4, 2, 0, 3).transpose(0, 3)[2]
    view = empty.permute(-1, -3, -2)
    assert view.shape == (4, 2, 0) and view.stride() == (empty.stride()[2], empty.stride()[0], empty.stride()[1])
    assert torch_rs.permute(base, dims=(2, 0, 1)).shape == (4, 2, 3)
    leaf = torch_rs.zeros(2, 3, 4).with_requires_grad(True)
    assert leaf.permute(-1, 0, 1)._grad_fn_name == "PermuteBackward0"
    cases = [
        (lambda: base.permute(0, 1), RuntimeError,
         "permute(sparse_coo): number of dimensions in the tensor input does not match the length of the desired "
         "ordering of dimensions i.e. input.dim() = 3 is not equal to len(dims) = 2"),
        (lambda: base.permute(0, 0, 1), RuntimeError, "permute(): duplicate dims are not allowed."),
        (lambda: base.permute(0, -4, 1), IndexError,
         "Dimension out of range (expected to be in range of [-3, 2], but got -4)"),
        (lambda: base.permute(), TypeError, 'permute() missing 1 required positional arguments: "dims"'),
        (lambda: base.permute((0, 1, 2), dims=(0, 1, 2)), TypeError,
         "permute() got multiple values for argument 'dims'"),
        (lambda: base.permute(dims=(0, 1, 2), axes=1), TypeError, "permute() got an unexpected keyword argument 'axes'"),
        (lambda: base.permute("a"), TypeError, "permute(): argument 'dims' (position 1) must be tuple of ints, not str"),
        (lambda: base.permute(("a", 1, 2)), TypeError,
         "permute(): argument 'dims' (position 1) must be tuple of ints, but found element of type str at pos 0"),
        (lambda: base.permute((0, "a", 2)), TypeError,
         "permute(): argument 'dims' failed to unpack the object at pos 2 with error \"type must be tuple of ints,"
         "but got str\""),
        (lambda: base.permute(1.5, 0), TypeError, "permute() takes 1 positional argument but 2 were given"),
    ]
    for call, exc, msg in cases:
        with pytest.raises(exc) as info:
            call()
        assert str(info.value) == msg


def test_requires_grad_arguments_are_builtin_bools():
    """tests/test_autograd.py: tensor() takes an exact bool; zeros/ones/full
    take an exact bool or None, keyword-only (src/python.rs:4189-4215)."""
    class Truthy:
        def __bool__(self):
            return True

    for bad, name in ((np.bool_(True), "numpy.bool"), (1, "int"), (0, "int"), (None, "NoneType"),
                      ("true", "str"), (Truthy(), "Truthy")):
        with pytest.raises(TypeError) as info:
            torch_rs.tensor([1.0], requires_grad=bad)
        assert str(info.value) == f"tensor(): argument 'requires_grad' must be bool, not {name}"
    for fname in ("zeros", "ones"):
        factory = getattr(torch_rs, fname)
        assert not factory((), requires_grad=None).requires_grad
        assert factory((2, 2), requires_grad=True).requires_grad
        for bad, name in ((np.bool_(False), "numpy.bool"), (1, "int"), (1.0, "float"), (object(), "object"),
                          (Truthy(), "Truthy")):
            with pytest.raises(TypeError) as info:
                factory((1,), requires_grad=bad)
            assert str(info.value) == f"{fname}(): argument 'requires_grad' must be bool, not {name}"
        with pytest.raises(TypeError) as info:
            factory((1,), True)
        assert str(info.value) == f"{fname}() takes 1 positional argument but 2 were given"
        assert factory(2, 3).shape == (2, 3) and factory([2, 3]).shape == (2, 3)
    assert torch_rs.full((2,), 1.5, requires_grad=None).shape == (2,)
    with pytest.raises(TypeError, match=r"^full\(\): argument 'requires_grad' must be bool, not int$"):
        torch_rs.full((2,), 1.5, requires_grad=1)


def test_autograd_package_exports_grad_mode():
    """python/torch_rs/autograd/__init__.py:133 and grad_mode.py:81: the
    autograd package exports backward, grad_mode and no_grad, and no_grad is
    one object under every spelling."""
    import importlib
    gm = importlib.import_module("torch_rs.autograd.grad_mode")
    assert torch_rs.autograd.__all__ == ["backward", "grad_mode", "no_grad"]
    assert gm.__all__ == ["no_grad"] and gm.no_grad is torch_rs.no_grad is torch_rs.autograd.no_grad
