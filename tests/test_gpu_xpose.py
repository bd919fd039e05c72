"""GPU parity of the transposing pointwise kernel (pw_xpose) against the oracle.

Layouts whose operand is unit-stride along a dim other than the output's
innermost one (a transposed or permuted view such as c.mT) run pw_xpose:
each lane transposes a 4x4 block in registers.  Fused programs specialise
it on operand roles: operands constant over the outer dims are held in
registers while a block walks several outer tuples, and operands constant
along t are loaded once per tuple.  Every case here is bit-exact against the
oracle's strided restatement (src/tensor.rs:3546-3599 broadcast odometer and
:2701-2708 generic same-shape path), composed op by op; the shapes cover
ragged tiles, unaligned operands (the scalar path), ranks 2-5, walks whose
tuple count is not a multiple of the walk length, byte operands, several
transposed operands and the eager (ahead-of-time) kernels.
"""
import ctypes

import numpy as np
import pytest

import gpu_util as U
import oracle as O
from helpers import assert_bitwise_equal
from trs_backend import abi
from trs_backend.abi import check, layout_of

pytestmark = pytest.mark.gpu

BCAST_MUL_IR = "in f32\nin f32\nin f32\nadd %0 %1\nmul %3 %2\nout %4\n"


def gpu_fused(ir, arrays, layouts, oshape):
    kid = U.fusion_compile(ir)
    devs = [U.dev(a) for a in arrays]
    n = int(np.prod(oshape))
    out = U.out_buffer(n)
    U.fusion_launch(kid, devs, layouts, out, layout_of(oshape))
    return out.to_numpy(count=n)


def oracle_bcast_mul(a, al, b, bl, c, cl, oshape):
    """(a + b) * c in the reference's two passes, each operand a (shape,
    strides, offset) view of its buffer; the output is contiguous."""
    ocs = O.contiguous_strides(oshape)
    s = O.binary(O.ADD, a, *al, b, *bl, oshape, ocs)
    return O.binary(O.MUL, s, oshape, ocs, 0, c, *cl, oshape, ocs)


def transposed_last_two(shape):
    """Strides of the `.mT` view of a contiguous tensor of shape
    shape[:-2] + (shape[-1], shape[-2]), viewed with `shape`."""
    *lead, m, n = shape
    base = tuple(lead) + (n, m)
    cs = O.contiguous_strides(base)
    return tuple(cs[:-2]) + (cs[-1], cs[-2])


# (batch dims, M, N): full 128x64 tiles, ragged tiles in t and x, tiny, and a
# batch whose count is not a multiple of the 8-tuple walk.
SHAPES = [((16,), 256, 128), ((3,), 70, 130), ((1,), 1, 1), ((5,), 9, 3), ((13,), 128, 64), ((20,), 33, 200),
          ((2, 3), 130, 66), ((2, 2, 3), 40, 70)]


@pytest.mark.parametrize("lead,m,n", SHAPES)
def test_fused_broadcast_plus_transposed_view_bit_exact(lead, m, n):
    """(a + b) * c.mT with a [..., 1, N] (constant along t: once per tuple),
    b [1.., M, N] (constant over the batch dims: held for the walk) and c a
    transposed view: the config-3 program at assorted shapes and ranks."""
    rng = np.random.default_rng(sum(lead) * 1000 + m + n)
    oshape = tuple(lead) + (m, n)
    ashape = tuple(lead) + (1, n)
    bshape = (1,) * len(lead) + (m, n)
    a = rng.standard_normal(int(np.prod(ashape))).astype(np.float32)
    b = rng.standard_normal(int(np.prod(bshape))).astype(np.float32)
    c = rng.standard_normal(int(np.prod(oshape))).astype(np.float32)
    al = (ashape, O.contiguous_strides(ashape), 0)
    bl = (bshape, O.contiguous_strides(bshape), 0)
    cl = (oshape, transposed_last_two(oshape), 0)
    got = gpu_fused(BCAST_MUL_IR, [a, b, c], [layout_of(*al[:2]), layout_of(*bl[:2]), layout_of(*cl[:2])], oshape)
    assert_bitwise_equal(got, oracle_bcast_mul(a, al, b, bl, c, cl, oshape))


def test_fused_unaligned_transposed_operand_takes_the_scalar_path_bit_exact():
    """c at storage offset 1 (not 16-byte aligned): every access is scalar
    and bounds-checked; results are unchanged."""
    rng = np.random.default_rng(3)
    B, M, N = 4, 130, 70
    oshape = (B, M, N)
    a = rng.standard_normal(B * N).astype(np.float32)
    b = rng.standard_normal(M * N).astype(np.float32)
    c = rng.standard_normal(B * M * N + 1).astype(np.float32)
    al, bl = ((B, 1, N), (N, N, 1), 0), ((1, M, N), (M * N, N, 1), 0)
    cl = (oshape, (M * N, 1, M), 1)
    lays = [layout_of(*al), layout_of(*bl), layout_of(*cl)]
    got = gpu_fused(BCAST_MUL_IR, [a, b, c], lays, oshape)
    assert_bitwise_equal(got, oracle_bcast_mul(a, al, b, bl, c, cl, oshape))


def test_fused_three_transposed_operands_and_a_held_one():
    """x.mT * y.mT + z.mT * w with w constant over the batch (held): three
    transposed inputs in one kernel (the LDS kernel this replaces took at
    most four), against the oracle op by op."""
    rng = np.random.default_rng(11)
    B, M, N = 6, 100, 72
    oshape = (B, M, N)
    ts = transposed_last_two(oshape)
    ocs = O.contiguous_strides(oshape)
    xs = [rng.standard_normal(B * M * N).astype(np.float32) for _ in range(3)]
    w = rng.standard_normal(M * N).astype(np.float32)
    ir = "in f32\nin f32\nin f32\nin f32\nmul %0 %1\nmul %2 %3\nadd %4 %5\nout %6\n"
    lays = [layout_of(oshape, ts)] * 3 + [layout_of((1, M, N))]
    got = gpu_fused(ir, xs + [w], lays, oshape)
    p = O.binary(O.MUL, xs[0], oshape, ts, 0, xs[1], oshape, ts, 0, oshape, ocs)
    q = O.binary(O.MUL, xs[2], oshape, ts, 0, w, (1, M, N), (M * N, N, 1), 0, oshape, ocs)
    assert_bitwise_equal(got, O.binary(O.ADD, p, oshape, ocs, 0, q, oshape, ocs, 0, oshape, ocs))


def test_fused_transposed_byte_mask():
    """(h * m.mT) * s with the keep-mask a transposed uint8 view (read as 4
    bytes per vector along t) and h contiguous."""
    rng = np.random.default_rng(21)
    B, M, N = 3, 96, 200
    oshape = (B, M, N)
    h = rng.standard_normal(B * M * N).astype(np.float32)
    m = (rng.random(B * M * N) < 0.7).astype(np.uint8)
    ir = "in f32\nin u8\nmul %0 %1\nconst 0x3f8e38e4\nmul %2 %3\nout %4\n"
    ts = transposed_last_two(oshape)
    kid = U.fusion_compile(ir)
    dh = U.dev(h)
    dm = abi.DeviceArray.from_numpy(m)
    out = U.out_buffer(h.size)
    U.fusion_launch(kid, [dh, dm], [layout_of(oshape), layout_of(oshape, ts)], out, layout_of(oshape))
    ocs = O.contiguous_strides(oshape)
    t = O.binary(O.MUL, h, oshape, ocs, 0, m.astype(np.float32), oshape, ts, 0, oshape, ocs)
    want = O.scalar(O.S_MUL, t, oshape, ocs, 0, np.float32(1 / 0.9), ocs)
    assert_bitwise_equal(out.to_numpy(count=h.size), want)


def test_fused_permuted_rank4_view():
    """A rank-4 operand permuted (0, 3, 1, 2): unit stride along a middle dim
    of the output, two outer dims walked, plus a row broadcast."""
    rng = np.random.default_rng(31)
    A, B, C, D = 3, 40, 5, 36
    oshape = (A, B, C, D)
    base = rng.standard_normal(A * C * D * B).astype(np.float32)  # contiguous [A, C, D, B]
    bs = O.contiguous_strides((A, C, D, B))
    pstr = (bs[0], bs[3], bs[1], bs[2])  # the (0, 3, 1, 2) permutation's strides
    row = rng.standard_normal(D).astype(np.float32)
    ir = "in f32\nin f32\nsub %0 %1\nout %2\n"
    got = gpu_fused(ir, [base, row], [layout_of(oshape, pstr), layout_of((D,))], oshape)
    ocs = O.contiguous_strides(oshape)
    want = O.binary(O.SUB, base, oshape, pstr, 0, row, (D,), (1,), 0, oshape, ocs)
    assert_bitwise_equal(got, want)


@pytest.mark.parametrize("which", ["right", "left", "both"])
@pytest.mark.parametrize("shape,offset", [((7, 130, 66), 0), ((2, 64, 128), 0), ((3, 33, 17), 1)])
def test_eager_binary_with_transposed_operands_bit_exact(which, shape, offset):
    """trs_binary_f32 (the ahead-of-time kernels) with the right, left or
    both operands transposed views, aligned and at an odd offset."""
    rng = np.random.default_rng(sum(shape) + offset)
    n = int(np.prod(shape))
    ts = transposed_last_two(shape)
    cs = O.contiguous_strides(shape)
    a = rng.standard_normal(n + offset).astype(np.float32)
    b = rng.standard_normal(n + offset).astype(np.float32)
    la = (shape, ts if which in ("left", "both") else cs, offset)
    lb = (shape, ts if which in ("right", "both") else cs, offset)
    for op in (O.MUL, O.SUB, O.DIV):
        got = U.binary(op, a, *la, b, *lb, shape, cs)
        want = O.binary(op, a, *la, b, *lb, shape, cs)
        assert_bitwise_equal(got, want)


def test_eager_unary_copy_of_transposed_view_bit_exact():
    """contiguous() of a transposed view (COPY through the transposing
    kernel) at a ragged shape."""
    rng = np.random.default_rng(41)
    shape = (5, 131, 67)
    ts = transposed_last_two(shape)
    x = rng.standard_normal(int(np.prod(shape))).astype(np.float32)
    got = U.unary(O.COPY, x, shape, ts, 0, O.contiguous_strides(shape))
    want = O.unary(O.COPY, x, shape, ts, 0, O.contiguous_strides(shape))
    assert_bitwise_equal(got, want)
