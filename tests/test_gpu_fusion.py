"""GPU parity of the pointwise fusion compiler.

A fused program performs the same IEEE operations as the eager chain, so
it is bit-identical to the eager GPU chain (same device expf) and, except
through exp, bit-identical to the CPU oracle; through exp the chain is
within 2 ulp(exp(t)) absolute of the oracle (relu(exp(t) - 1) does not
amplify absolute error).
"""
import numpy as np
import pytest

import gpu_util as U
import oracle as O
from helpers import assert_bitwise_equal, ulp_of
from trs_backend.abi import layout_of

pytestmark = pytest.mark.gpu

CHAIN_IR = "in f32\nin f32\nin f32\nmul %0 %1\nadd %3 %2\nexp %4\nconst 0x3f800000\nsub %5 %6\nrelu %7\nout %8\n"
BCAST_IR = "in f32\nin f32\nin f32\nadd %0 %1\nmul %3 %2\nout %4\n"


def oracle_chain(x, y, z):
    t = O.binary_contig(O.ADD, O.binary_contig(O.MUL, x, y), z)
    e = O.unary_contig(O.EXP, t)
    return O.unary_contig(O.RELU, O.scalar_contig(O.S_SUB, e, 1.0)), t


def gpu_eager_chain(x, y, z):
    n = x.size
    t1 = U.binary(O.MUL, x, (n,), (1,), 0, y, (n,), (1,), 0, (n,), (1,))
    t2 = U.binary(O.ADD, t1, (n,), (1,), 0, z, (n,), (1,), 0, (n,), (1,))
    t3 = U.unary(O.EXP, t2, (n,), (1,), 0, (1,))
    t4 = U.scalar(O.S_SUB, t3, (n,), (1,), 0, 1.0, (1,))
    return U.unary(O.RELU, t4, (n,), (1,), 0, (1,))


def gpu_fused(ir, arrays, layouts, oshape, ostr=None):
    kid = U.fusion_compile(ir)
    devs = [U.dev(a) for a in arrays]
    n = int(np.prod(oshape))
    out = U.out_buffer(n)
    U.fusion_launch(kid, devs, layouts, out, layout_of(oshape, ostr))
    return out.to_numpy(count=n)


@pytest.mark.parametrize("n", [1, 7, 4096, 100_003, 1 << 22])
def test_fused_chain_matches_eager_bitwise_and_oracle_within_exp_bound(n):
    rng = np.random.default_rng(n)
    x, y, z = (rng.uniform(-4, 4, n).astype(np.float32) for _ in range(3))
    lay = [layout_of((n,))] * 3
    fused = gpu_fused(CHAIN_IR, [x, y, z], lay, (n,))
    eager = gpu_eager_chain(x, y, z)
    assert_bitwise_equal(fused, eager)
    want, t = oracle_chain(x, y, z)
    err = np.abs(fused.astype(np.float64) - want.astype(np.float64))
    assert (err <= 2 * ulp_of(np.exp(t.astype(np.float64)).astype(np.float32))).all()


@pytest.mark.parametrize("B,M,N", [(4, 96, 160), (2, 4096, 4096), (2, 4100, 4099)])
def test_fused_broadcast_transposed_chain_bit_exact(B, M, N):
    """(a + b) * c.mT on a config-3-like shape: a [B,1,N], b [1,M,N], c [B,N,M].
    The larger shapes have more tiles per batch than the GPU holds at once
    (diagonal tile order), aligned and ragged."""
    rng = np.random.default_rng(2 + M)
    a = rng.standard_normal(B * N).astype(np.float32)
    b = rng.standard_normal(M * N).astype(np.float32)
    c = rng.standard_normal(B * N * M).astype(np.float32)
    la = layout_of((B, 1, N))
    lb = layout_of((1, M, N))
    lc = layout_of((B, M, N), (N * M, 1, M))  # c.mT
    fused = gpu_fused(BCAST_IR, [a, b, c], [la, lb, lc], (B, M, N))
    # oracle: the reference's two ops, add then mul
    sh1, st1 = O.binary_output_layout((B, 1, N), (N, N, 1), (1, M, N), (M * N, N, 1))
    s = O.binary(O.ADD, a, (B, 1, N), (N, N, 1), 0, b, (1, M, N), (M * N, N, 1), 0, sh1, st1)
    sh2, st2 = O.binary_output_layout(sh1, st1, (B, M, N), (N * M, 1, M))
    want = O.binary(O.MUL, s, sh1, st1, 0, c, (B, M, N), (N * M, 1, M), 0, sh2, st2)
    assert st2 == (M * N, N, 1)
    assert_bitwise_equal(fused, want)


@pytest.mark.parametrize("ash,bsh,osh", [
    ((2, 1, 4, 256), (1, 3, 1, 256), (2, 3, 4, 256)),          # rank 4, fixed-rank rows kernel
    ((4, 1, 6, 2052), (1, 5, 1, 2052), (4, 5, 6, 2052)),       # rank 4, ragged last chunk
    ((2, 1, 3, 1, 128), (1, 2, 1, 4, 128), (2, 2, 3, 4, 128)),  # rank 5, run-time decode
])
def test_fused_rows_of_rank_four_and_five_bit_exact(ash, bsh, osh):
    """(a + b) * c with a and b broadcast so that no dims merge: rows
    launches of rank 4 and 5."""
    rng = np.random.default_rng(sum(osh))
    a = rng.standard_normal(int(np.prod(ash))).astype(np.float32)
    b = rng.standard_normal(int(np.prod(bsh))).astype(np.float32)
    c = rng.standard_normal(int(np.prod(osh))).astype(np.float32)
    ast, bst, ost = O.contiguous_strides(ash), O.contiguous_strides(bsh), O.contiguous_strides(osh)
    fused = gpu_fused(BCAST_IR, [a, b, c], [layout_of(ash), layout_of(bsh), layout_of(osh)], osh)
    sh1, st1 = O.binary_output_layout(ash, ast, bsh, bst)
    s = O.binary(O.ADD, a, ash, ast, 0, b, bsh, bst, 0, sh1, st1)
    want = O.binary(O.MUL, s, sh1, st1, 0, c, osh, ost, 0, osh, ost)
    assert_bitwise_equal(fused, want)


def test_fused_mask_apply_with_u8_input():
    rng = np.random.default_rng(9)
    n = 10_000
    h = rng.standard_normal(n).astype(np.float32)
    m = (rng.random(n) < 0.9).astype(np.uint8)
    ir = f"in f32\nin u8\nmul %0 %1\nconst {np.float32(1 / 0.9).view(np.uint32):#010x}\nmul %2 %3\nout %4\n"
    got = gpu_fused(ir, [h, m], [layout_of((n,)), layout_of((n,))], (n,))
    assert_bitwise_equal(got, O.mask_apply(h, m, float(np.float32(1 / 0.9))))


def test_fused_relu_bias_row_broadcast():
    rng = np.random.default_rng(10)
    R, C = 64, 1000
    x = rng.standard_normal(R * C).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    got = gpu_fused("in f32\nin f32\nadd %0 %1\nrelu %2\nout %3\n", [x, b], [layout_of((R, C)), layout_of((C,))],
                    (R, C))
    want = O.unary_contig(O.RELU, O.row_broadcast(O.ADD, x, b, R, C))
    assert_bitwise_equal(got, want, nan_equal=False)


def _random_program(rng, nin):
    """A random straight-line program over nin inputs: a list of (op, args)."""
    prog = []
    nvals = nin
    for _ in range(int(rng.integers(2, 9))):
        kind = rng.integers(0, 10)
        a = int(rng.integers(0, nvals))
        if kind < 4:
            b = int(rng.integers(0, nvals))
            prog.append((["add", "sub", "mul", "div"][kind], a, b))
        elif kind < 8:
            s = float(rng.choice([0.5, -1.25, 3.0, 1e-3, 2.0]))
            prog.append((["sadd", "ssub", "smul", "rsub"][kind - 4], a, s))
        elif kind == 8:
            prog.append(("relu", a))
        else:
            prog.append(("neg", a))
        nvals += 1
    return prog


def _run_program(prog, args):
    vals = list(args)
    for ins in prog:
        op = ins[0]
        if op in ("add", "sub", "mul", "div"):
            x, y = vals[ins[1]], vals[ins[2]]
            if op == "add":
                vals.append(x + y)
            elif op == "sub":
                vals.append(x - y)
            elif op == "mul":
                vals.append(x * y)
            else:
                vals.append(x / y)
        elif op in ("sadd", "ssub", "smul", "rsub"):
            x, s = vals[ins[1]], ins[2]
            if op == "sadd":
                vals.append(x + s)
            elif op == "ssub":
                vals.append(x - s)
            elif op == "smul":
                vals.append(x * s)
            else:
                vals.append(s - x)
        elif op == "relu":
            vals.append(vals[ins[1]].relu())
        else:
            vals.append(-vals[ins[1]])
    return vals[-1]


def _random_operand(rng, oshape):
    """A device tensor broadcastable to oshape: a suffix of its shape with some
    dims set to 1, laid out contiguously, transposed in its last two dims, or
    as every other column of a wider tensor (stride 2 innermost)."""
    import torch_rs
    r = len(oshape)
    k = int(rng.integers(0, r + 1))
    shape = [1 if rng.random() < 0.25 else d for d in oshape[r - k:]]
    n = int(np.prod(shape)) if shape else 1
    kind = rng.integers(0, 3)
    if kind == 1 and len(shape) >= 2:
        base = rng.standard_normal(n).astype(np.float32).reshape(shape[:-2] + [shape[-1], shape[-2]])
        return torch_rs.tensor(base, device="cuda").mT
    if kind == 2 and len(shape) >= 1:
        base = rng.standard_normal(2 * n).astype(np.float32).reshape(shape[:-1] + [shape[-1], 2])
        t = torch_rs.tensor(base, device="cuda")
        last = len(shape)
        return t.permute(*([last] + list(range(last))))[0]  # select column 0 of each pair
    return torch_rs.tensor(rng.standard_normal(n).astype(np.float32).reshape(shape), device="cuda")


def test_random_programs_fused_equal_eager_bit_for_bit():
    import torch_rs
    rng = np.random.default_rng(77)
    for case in range(40):
        rank = int(rng.integers(1, 4))
        oshape = [int(rng.integers(1, 70)) for _ in range(rank)]
        nin = int(rng.integers(1, 6))
        args = [_random_operand(rng, oshape) for _ in range(nin)]
        # make sure the broadcast result has the full output shape
        args[0] = torch_rs.tensor(rng.standard_normal(int(np.prod(oshape))).astype(np.float32).reshape(oshape),
                                  device="cuda") if rng.random() < 0.5 else \
            torch_rs.tensor(rng.standard_normal(int(np.prod(oshape))).astype(np.float32).reshape(oshape[::-1]),
                            device="cuda").permute(*range(rank - 1, -1, -1))
        prog = _random_program(rng, nin)
        fn = lambda *xs, prog=prog: _run_program(prog, xs)
        eager = fn(*args)
        fused = torch_rs.fuse(fn)(*args)
        assert fused.shape == eager.shape, (case, prog)
        assert fused.stride() == eager.stride(), (case, prog, fused.stride(), eager.stride())
        assert_bitwise_equal(fused.numpy().ravel(), eager.numpy().ravel())


_DISK_CHILD = r"""
import ctypes, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from trs_backend import abi
from trs_backend.abi import DeviceArray, check, layout_of
ir = sys.argv[2]
kid = ctypes.c_uint64()
check(abi.lib.trs_fusion_compile(ir.encode(), len(ir), ctypes.byref(kid)))
hit = ctypes.c_int()
check(abi.lib.trs_fusion_from_disk_cache(kid, ctypes.byref(hit)))
if sys.argv[3] == "launch":
    check(abi.lib.trs_init())
    n = (1 << 20) + 3
    x = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    dx, fused, t1, eager = DeviceArray.from_numpy(x), DeviceArray(n * 4), DeviceArray(n * 4), DeviceArray(n * 4)
    lay = layout_of((n,))
    check(abi.lib.trs_fusion_launch(kid, 1, (ctypes.c_void_p * 1)(dx.addr), (abi.Layout * 1)(lay), fused.ptr,
                                    ctypes.byref(lay)))
    check(abi.lib.trs_binary_scalar_f32(2, dx.ptr, ctypes.byref(lay), ctypes.c_float(np.float32(3.14159274)),
                                        t1.ptr, ctypes.byref(lay)))
    check(abi.lib.trs_unary_f32(2, t1.ptr, ctypes.byref(lay), eager.ptr, ctypes.byref(lay)))
    same = np.array_equal(fused.to_numpy().view(np.uint32), eager.to_numpy().view(np.uint32))
    print(hit.value, int(same))
else:
    print(hit.value, 1)
"""


def test_program_loaded_from_the_disk_cache_runs_bit_exact(tmp_path):
    """A code object written by one process and loaded by another computes
    the same bits as the eager ops: x * f32(pi), then neg."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    ir = "in f32\nconst 0x40490fdb\nmul %0 %1\nneg %2\nout %3\n"
    env = dict(os.environ, TRS_FUSION_CACHE_DIR=str(tmp_path / "fusion"))
    pkg = str(Path(__file__).resolve().parent.parent / "pytorch-rs_amd")

    def child(mode):
        out = subprocess.run([sys.executable, "-c", _DISK_CHILD, pkg, ir, mode], env=env, capture_output=True,
                             text=True, timeout=120)
        assert out.returncode == 0, out.stderr
        return tuple(int(v) for v in out.stdout.split())

    assert child("compile") == (0, 1)
    assert child("launch") == (1, 1)


def _random_program_with_exp(rng, nin):
    """_random_program's ops plus exp of a damped value (x * 0.25, then exp)."""
    prog = []
    nvals = nin
    for _ in range(int(rng.integers(2, 9))):
        a = int(rng.integers(0, nvals))
        if rng.random() < 0.2:
            prog.append(("smul", a, 0.25))
            prog.append(("exp", nvals))
            nvals += 2
            continue
        one = _random_program(np.random.default_rng(int(rng.integers(0, 1 << 30))), nvals)[:1]
        op = one[0][0]
        if op in ("add", "sub", "mul", "div"):
            prog.append((op, a, int(rng.integers(0, nvals))))
        elif op in ("sadd", "ssub", "smul", "rsub"):
            prog.append((op, a, one[0][2]))
        else:
            prog.append((op, a))
        nvals += 1
    return prog


def test_fused_backward_equals_eager_autograd_bit_for_bit():
    """Random programs (add/sub/mul/div, scalar ops, relu, neg, exp) over
    broadcast, transposed and strided operands, with random subsets of the
    inputs requiring grad: the fused node's gradients equal eager autograd's
    bit for bit, its output equals the eager output, and inputs with no
    gradient path stay without a gradient."""
    import torch_rs
    rng = np.random.default_rng(91)
    fused_nodes = 0
    for case in range(40):
        rank = int(rng.integers(1, 4))
        oshape = [int(rng.integers(1, 40)) for _ in range(rank)]
        nin = int(rng.integers(1, 5))
        base = [_random_operand(rng, oshape) for _ in range(nin)]
        base[0] = torch_rs.tensor(rng.standard_normal(int(np.prod(oshape))).astype(np.float32).reshape(oshape),
                                  device="cuda")
        requires = [bool(rng.random() < 0.7) for _ in range(nin)]
        requires[int(rng.integers(0, nin))] = True
        prog = _random_program_with_exp(rng, nin)
        fn = lambda *xs, prog=prog: _eval(prog, xs)
        w = torch_rs.tensor(rng.standard_normal(int(np.prod(oshape))).astype(np.float32).reshape(oshape),
                            device="cuda")

        def leaves():
            return [b.detach().with_requires_grad(r) for b, r in zip(base, requires)]

        le, lf = leaves(), leaves()
        out_e = fn(*le)
        out_f = torch_rs.fuse(fn)(*lf)
        assert_bitwise_equal(out_f.numpy().ravel(), out_e.numpy().ravel())
        assert out_f.requires_grad == out_e.requires_grad, (case, prog)
        if not out_e.requires_grad:
            continue
        fused_nodes += out_f.grad_fn is not None and out_f.grad_fn.name() == "FusedBackward0"
        if tuple(out_e.shape) != tuple(oshape):
            continue  # w would not match; the output is a broadcast of fewer dims
        (out_e * w).sum().backward()
        (out_f * w).sum().backward()
        for i in range(nin):
            ge, gf = le[i].grad, lf[i].grad
            assert (ge is None) == (gf is None), (case, i, prog)
            if ge is not None:
                assert ge.shape == gf.shape, (case, i)
                assert_bitwise_equal(gf.numpy().ravel(), ge.numpy().ravel())
    assert fused_nodes >= 12, fused_nodes  # many programs take the fused backward


def _eval(prog, xs):
    vals = list(xs)
    for ins in prog:
        if ins[0] == "exp":
            vals.append(vals[ins[1]].exp())
        else:
            vals.append(_run_program([ins], vals))
    return vals[-1]


# ---- multi-output programs ----------------------------------------------------

_MULTI_BODY = ("in f32\nin f32\nin f32\nadd %0 %1\nmul %3 %2\nconst 0x3e800000\nmul %4 %5\nexp %6\n"
               "relub %0 %4\n")
_MULTI_OUTS = [4, 7, 8, 3]


def _multi_cases():
    """(name, arrays, input layouts, output shape, output strides): one case
    per kernel variant of the pointwise engine."""
    rng = np.random.default_rng(77)
    n = 100_003
    flat = [rng.standard_normal(n).astype(np.float32) for _ in range(3)]
    yield "flat_contig", flat, [layout_of((n,))] * 3, (n,), None
    shifted = [np.concatenate([[0.0], a]).astype(np.float32) for a in flat]
    yield "flat_unaligned", shifted, [layout_of((n,), (1,), 1)] * 3, (n,), None
    R, C = 64, 1000
    rows = [rng.standard_normal(R * C).astype(np.float32), rng.standard_normal(C).astype(np.float32),
            rng.standard_normal(R * C).astype(np.float32)]
    yield "rows", rows, [layout_of((R, C)), layout_of((C,)), layout_of((R, C))], (R, C), None
    B, M, N = 3, 70, 130
    xpose = [rng.standard_normal(B * N).astype(np.float32), rng.standard_normal(M * N).astype(np.float32),
             rng.standard_normal(B * N * M).astype(np.float32)]
    yield ("xpose", xpose, [layout_of((B, 1, N)), layout_of((1, M, N)), layout_of((B, M, N), (N * M, 1, M))],
           (B, M, N), None)
    A, D = 9, 11
    gen = [rng.standard_normal(A * D * 3).astype(np.float32) for _ in range(3)]
    lays = [layout_of((A, D), (1, A * 3)), layout_of((A, D), (D * 3, 3)), layout_of((A, D), (3, A * 3), 1)]
    yield "generic", gen, lays, (A, D), (1, A)


@pytest.mark.parametrize("case", list(_multi_cases()), ids=lambda c: c[0])
def test_multi_output_program_equals_single_output_programs(case):
    """A four-output program writes, in one launch, exactly what the four
    one-output programs over the same instructions write, on every kernel
    variant (flat, unaligned flat, row broadcast, in-register transpose,
    generic strides)."""
    _, arrays, lays, oshape, ostr = case
    n = int(np.prod(oshape))
    kid = U.fusion_compile(_MULTI_BODY + "".join(f"out %{o}\n" for o in _MULTI_OUTS))
    devs = [U.dev(a) for a in arrays]
    outs = [U.out_buffer(n) for _ in _MULTI_OUTS]
    assert U.fusion_launch_multi(kid, devs, lays, outs, layout_of(oshape, ostr)) == 0
    for o, buf in zip(_MULTI_OUTS, outs):
        single = gpu_fused(_MULTI_BODY + f"out %{o}\n", arrays, lays, oshape, ostr)
        assert_bitwise_equal(buf.to_numpy(count=n), single)


def test_multi_output_launch_rejects_bad_outputs():
    from trs_backend.abi import TRS_E_INVALID_ARGUMENT
    n = 4096
    rng = np.random.default_rng(5)
    arrays = [rng.standard_normal(n).astype(np.float32) for _ in range(3)]
    devs = [U.dev(a) for a in arrays]
    lays = [layout_of((n,))] * 3
    kid = U.fusion_compile(_MULTI_BODY + "out %4\nout %7\n")
    a, b = U.out_buffer(n), U.out_buffer(n)
    lo = layout_of((n,))
    # output count must match the program
    assert U.fusion_launch_multi(kid, devs, lays, [a], lo) == TRS_E_INVALID_ARGUMENT
    assert U.fusion_launch_multi(kid, devs, lays, [a, b, U.out_buffer(n)], lo) == TRS_E_INVALID_ARGUMENT
    ptrs = (U.ctypes.c_void_p * 3)(*[d.addr for d in devs])
    larr = (U.abi.Layout * 3)(*lays)
    assert U.abi.lib.trs_fusion_launch(kid, 3, ptrs, larr, a.ptr, U.ctypes.byref(lo)) == TRS_E_INVALID_ARGUMENT
    # outputs may not share memory with each other
    assert U.fusion_launch_multi(kid, devs, lays, [a, a], lo) == TRS_E_INVALID_ARGUMENT
    # an output may share memory with an input only as the same view
    assert U.fusion_launch_multi(kid, devs, lays, [a, devs[2]], lo) == 0
    half = layout_of((n // 2,))
    assert U.fusion_launch_multi(kid, devs, [layout_of((n // 2,), (1,), 1)] * 3, [a, devs[0]],
                                 half) == TRS_E_INVALID_ARGUMENT
    # the in-place launch above computed from the inputs as they were
    want_7 = gpu_fused(_MULTI_BODY + "out %7\n", arrays, lays, (n,))
    assert_bitwise_equal(devs[2].to_numpy(count=n), want_7)


def test_fused_backward_input_reaching_output_only_through_division():
    """x reaches the output only through a division (which records nothing):
    x gets no gradient, t gets the upstream, as eager autograd gives."""
    import torch_rs
    rng = np.random.default_rng(13)
    shape = (37, 5)
    vals = [rng.standard_normal(shape).astype(np.float32) for _ in range(4)]
    fn = lambda x, y, z, t: (x * y) / z + t

    def run(f):
        x = torch_rs.tensor(vals[0], device="cuda").with_requires_grad(True)
        y = torch_rs.tensor(vals[1], device="cuda")
        z = torch_rs.tensor(vals[2], device="cuda")
        t = torch_rs.tensor(vals[3], device="cuda").with_requires_grad(True)
        out = f(x, y, z, t)
        out.sum().backward()
        return out, x, t

    out_e, xe, te = run(fn)
    out_f, xf, tf = run(torch_rs.fuse(fn))
    assert_bitwise_equal(out_f.numpy().ravel(), out_e.numpy().ravel())
    assert out_f._grad_fn_name == "FusedBackward0"
    assert xe.grad is None and xf.grad is None
    assert_bitwise_equal(tf.grad.numpy().ravel(), te.grad.numpy().ravel())


def test_fused_dropout_activation_with_byte_mask_equals_eager_under_autograd():
    """The MLP's activation, relu(z + b) then dropout-apply with a uint8
    keep-mask, as one fused node reading the mask as bytes: output and
    gradients equal eager F.dropout(relu(z + b), mask=...) bit for bit (the
    backward is (up * f32(1/0.9)) * mask, then relu', as the eager VJPs)."""
    import torch_rs
    F = torch_rs.nn.functional
    rng = np.random.default_rng(31)
    R, C = 96, 257
    zv = rng.standard_normal((R, C)).astype(np.float32)
    zv[0, :4] = [0.0, -0.0, np.nan, np.inf]
    bv = rng.standard_normal(C).astype(np.float32)
    mv = (rng.random((R, C)) < 0.9).astype(np.uint8)
    mask = F.keep_mask(mv, "cuda")
    act = torch_rs.fuse(lambda z, b, m: ((z + b).relu() * m) * (1 / 0.9))

    def run(fused):
        z = torch_rs.tensor(zv, device="cuda").with_requires_grad(True)
        b = torch_rs.tensor(bv, device="cuda")
        w = torch_rs.tensor(rng_w, device="cuda")
        d = act(z, b, mask) if fused else F.dropout((z + b).relu(), 0.1, training=True, mask=mask)
        (d * w).sum().backward()
        return d, z

    rng_w = np.random.default_rng(32).standard_normal((R, C)).astype(np.float32)
    de, ze = run(False)
    df, zf = run(True)
    assert df._grad_fn_name == "FusedBackward0"
    assert_bitwise_equal(df.numpy().ravel(), de.numpy().ravel())
    assert_bitwise_equal(zf.grad.numpy().ravel(), ze.grad.numpy().ravel())
    # the mask stays a byte buffer: a second backward through the node raises
    with pytest.raises(RuntimeError, match="backward through the graph a second time"):
        df.sum().backward()


def test_fused_backward_input_with_two_uses_equals_eager():
    """x feeds two gradient-carrying uses (x*y and the relu): the fused node
    sums the two contributions at full shape, as eager accumulation does."""
    import torch_rs
    rng = np.random.default_rng(17)
    shape = (33, 65)
    xv, yv = (rng.standard_normal(shape).astype(np.float32) for _ in range(2))
    fn = lambda x, y: (x * y).exp() - x.relu() + x * x

    def run(f):
        x = torch_rs.tensor(xv, device="cuda").with_requires_grad(True)
        y = torch_rs.tensor(yv, device="cuda").with_requires_grad(True)
        out = f(x, y)
        out.sum().backward()
        return out, x, y

    oe, xe, ye = run(fn)
    of, xf, yf = run(torch_rs.fuse(lambda x, y: (x * y).exp() - x.relu()))
    assert of._grad_fn_name == "FusedBackward0"
    oe2, xe2, ye2 = run(lambda x, y: (x * y).exp() - x.relu())
    assert_bitwise_equal(of.numpy().ravel(), oe2.numpy().ravel())
    assert_bitwise_equal(xf.grad.numpy().ravel(), xe2.grad.numpy().ravel())
    assert_bitwise_equal(yf.grad.numpy().ravel(), ye2.grad.numpy().ravel())
    sq_e = run(lambda x, y: x * x)
    sq_f = run(torch_rs.fuse(lambda x, y: x * x))
    assert sq_f[0]._grad_fn_name == "FusedBackward0" and sq_f[2].grad is None
    assert_bitwise_equal(sq_f[1].grad.numpy().ravel(), sq_e[1].grad.numpy().ravel())


# ---- the program limits: 8 inputs, 8 outputs ----------------------------------

_EIGHT_IR = ("in f32\n" * 8 + "add %0 %1\nmul %8 %2\nsub %9 %3\nadd %10 %4\nmul %11 %5\ndiv %12 %6\nadd %13 %7\n"
             "relu %14\n" + "".join(f"out %{v}\n" for v in range(8, 16)))
_EIGHT_OPS = [O.ADD, O.MUL, O.SUB, O.ADD, O.MUL, O.DIV, O.ADD]


def _eight_views(rng, oshape):
    """Eight operands of oshape (rank >= 2) in different layouts: contiguous,
    a row broadcast, transposed in its last two dims, a broadcast along the
    second-to-last dim, an offset view transposed in every dim (so no dims
    merge), a scalar, a strided gather and a column broadcast."""
    r = len(oshape)
    lead, (m, k) = oshape[:-2], oshape[-2:]
    views = []

    def add(shape, strides=None, off=0, extra=0):
        strides = O.contiguous_strides(shape) if strides is None else strides
        n = O.storage_size(shape, strides, off) + extra
        views.append((U.special_mix(rng, max(n, 1)), tuple(shape), tuple(strides), off))

    add(oshape)
    add((k,))
    t = O.contiguous_strides(lead + (k, m))
    add(oshape, t[:-2] + (1, m))
    add(lead + (1, k))
    add(oshape, tuple(reversed(O.contiguous_strides(tuple(reversed(oshape))))), off=5)
    add(())
    add(oshape, tuple(2 * s for s in O.contiguous_strides(oshape)))
    add((m, 1))
    assert all(len(v[1]) <= r for v in views)
    return views


@pytest.mark.parametrize("oshape", [(4, 33, 70), (2, 3, 2, 3, 2, 3, 2, 3, 5, 6)])
def test_program_with_eight_inputs_and_eight_outputs(oshape):
    """The most inputs and outputs a program takes, at rank 3 and at rank 10
    (launched in parts): every output equals the eager oracle composition
    bit for bit."""
    from trs_backend import abi
    rng = np.random.default_rng(len(oshape))
    views = _eight_views(rng, oshape)
    lays = [layout_of(*v[1:3], v[3]) for v in views]
    assert abi.pointwise_plan(lays, layout_of(oshape)).split == max(0, len(oshape) - 8)
    n = int(np.prod(oshape))
    ostr = O.contiguous_strides(oshape)
    kid = U.fusion_compile(_EIGHT_IR)
    outs = [U.out_buffer(n) for _ in range(8)]
    rc = U.fusion_launch_multi(kid, [U.dev(v[0]) for v in views], lays, outs, layout_of(oshape))
    assert rc == 0
    buf, sh, st, off = views[0]
    want = []
    for i, op in enumerate(_EIGHT_OPS, start=1):
        b = views[i]
        buf = O.binary(op, buf, sh, st, off, b[0], b[1], b[2], b[3], oshape, ostr)
        sh, st, off = oshape, ostr, 0
        want.append(buf)
    want.append(O.unary(O.RELU, buf, oshape, ostr, 0, ostr))
    for i in range(8):
        assert_bitwise_equal(outs[i].to_numpy(count=n), want[i])


def test_program_limits_are_errors():
    import ctypes
    from trs_backend import abi
    kid = ctypes.c_uint64()
    nine = "in f32\n" * 9 + "add %0 %1\nout %9\n"
    assert abi.lib.trs_fusion_compile(nine.encode(), len(nine), ctypes.byref(kid)) == abi.TRS_E_FUSION
    nine_out = "in f32\n" + "".join(f"neg %{v}\n" for v in range(9)) + "".join(f"out %{v}\n" for v in range(1, 10))
    assert abi.lib.trs_fusion_compile(nine_out.encode(), len(nine_out), ctypes.byref(kid)) == abi.TRS_E_FUSION
