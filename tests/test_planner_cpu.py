"""CPU tests of the pointwise launch planner through trs_pointwise_plan (no
device): how layouts normalise (broadcast alignment, size-1 dims dropped,
contiguous dims merged) and which kernel and compile-time fast case each
launch gets.  The GPU kernels rely on these decisions: a fixed-rank kernel
assumes its rank and 32-bit offsets, the transposing kernel its operand
roles and walk."""
import pytest

from trs_backend import abi
from trs_backend.abi import layout_of

FLAT, ROWS, XPOSE, GENERIC = 1, 2, 3, 4


def plan(*layouts, out, **kw):
    return abi.pointwise_plan(list(layouts), out, **kw)


def test_contiguous_operands_merge_to_one_flat_dim():
    p = plan(layout_of((2, 3, 4)), layout_of((2, 3, 4)), out=layout_of((2, 3, 4)))
    assert (p.variant, p.rank, p.vec) == (FLAT, 1, 1)


def test_size_one_dims_are_dropped_before_merging():
    p = plan(layout_of((1, 64, 1, 32)), layout_of((64, 1, 32)), out=layout_of((1, 64, 1, 32)))
    assert (p.variant, p.rank) == (FLAT, 1)


def test_config0_row_broadcast_is_the_rank2_rows_kernel():
    p = plan(layout_of((4096, 4096)), layout_of((4096,)), out=layout_of((4096, 4096)))
    assert (p.variant, p.rank, p.vec, p.fixed_rank) == (ROWS, 2, 1, 2)
    assert p.grid == 4096 * 16  # one 256-column tile per one-wave block
    assert p.block == 64


def test_rows_blocks_with_streamed_inputs_are_one_wave():
    # The MLP's fused activation: x (f32) and the u8 keep-mask stream, the
    # bias row comes from cache; with the f32 output 9 B per element, so 64
    # lanes of one float4 move 2 KiB through HBM.
    x, mask, b = layout_of((8192, 4096)), layout_of((8192, 4096)), layout_of((4096,))
    p = plan(x, mask, b, out=layout_of((8192, 4096)), elem_bytes=[4, 1, 4])
    assert (p.variant, p.vec, p.block) == (ROWS, 1, 64)
    assert p.grid == 8192 * 16


def test_write_only_rows_blocks_are_wider():
    # a [64,1,1024] + b [1,512,1024]: both from cache, only the output
    # streams (4 B per element), so a block takes 128 lanes (2 KiB): one-wave
    # blocks of 1 KiB are bound by how fast the GPU starts blocks.
    p = plan(layout_of((64, 1, 1024)), layout_of((1, 512, 1024)), out=layout_of((64, 512, 1024)))
    assert (p.variant, p.rank, p.vec, p.fixed_rank) == (ROWS, 3, 1, 3)
    assert p.block == 128
    assert p.grid == 64 * 512 * 2  # 512-column tiles of 1,024-column rows


def test_config2_fused_roles_and_walk():
    a = layout_of((64, 1, 1024))
    b = layout_of((1, 512, 1024))
    c = layout_of((64, 512, 1024), (512 * 1024, 1, 512))  # c.mT
    o = layout_of((64, 512, 1024))
    p = plan(a, b, c, out=o, roles=True)
    assert (p.variant, p.rank, p.vec, p.fixed_rank) == (XPOSE, 3, 1, 3)
    assert (p.trans, p.held, p.once, p.walk, p.skew) == (0b100, 0b010, 0b001, 8, 0)
    assert p.grid == (64 // 8) * (512 // 128) * (1024 // 64)
    eager = plan(a, b, c, out=o)  # the eager launcher takes no roles
    assert (eager.held, eager.once, eager.walk) == (0, 0, 1)


def test_diagonal_tile_order_only_when_a_tuple_outgrows_the_resident_blocks():
    x, y, o = layout_of((8192, 8192)), layout_of((8192, 8192), (1, 8192)), layout_of((8192, 8192))
    assert plan(x, y, out=o).skew == 1                 # 64 x 128 tiles in one tuple, 4 x 256 resident
    assert plan(x, y, out=o, cu_count=4096).skew == 0  # the whole tuple fits at once
    c = layout_of((64, 512, 1024), (512 * 1024, 1, 512))
    assert plan(c, out=layout_of((64, 512, 1024))).skew == 0  # 4 x 16 tiles per tuple


@pytest.mark.parametrize("ashape,bshape,rank,fixed", [
    ((4096, 4096), (4096,), 2, 2),
    ((8, 1, 1024), (96, 1024), 3, 3),
    ((3, 1, 5, 64), (1, 4, 1, 64), 4, 4),
    ((2, 1, 3, 1, 64), (1, 3, 1, 4, 64), 5, 0),  # rank 5: decoded at run time
])
def test_rows_kernels_of_fixed_rank_two_to_four(ashape, bshape, rank, fixed):
    oshape = tuple(max(p, q) for p, q in zip((1,) * (len(bshape) - len(ashape)) + ashape,
                                              (1,) * (len(ashape) - len(bshape)) + bshape))
    p = plan(layout_of(ashape), layout_of(bshape), out=layout_of(oshape))
    assert (p.variant, p.rank, p.fixed_rank) == (ROWS, rank, fixed)


def test_fixed_rank_needs_every_offset_below_two_to_the_32():
    two32 = 1 << 32
    shape, n = (300, 2112), 300 * 2112
    row = layout_of((2112,))
    # the output ends exactly at element 2^32 - 1
    assert plan(layout_of(shape), row, out=layout_of(shape, None, two32 - n)).fixed_rank == 2
    # one element further, or an input past 2^32: 64-bit offsets
    assert plan(layout_of(shape), row, out=layout_of(shape, None, two32 - n + 4)).fixed_rank == 0
    assert plan(layout_of(shape, None, two32), row, out=layout_of(shape)).fixed_rank == 0
    c = layout_of((8, 192, 320), (320 * 192, 1, 192), two32)  # a transposed view past 2^32
    assert plan(c, out=layout_of((8, 192, 320))).fixed_rank == 0
    assert plan(layout_of((8, 192, 320), (320 * 192, 1, 192)), out=layout_of((8, 192, 320))).fixed_rank == 3


def test_vector_access_needs_aligned_bases_and_strides():
    shape = (64, 256)
    assert plan(layout_of(shape), layout_of((256,)), out=layout_of(shape)).vec == 1
    misaligned = plan(layout_of(shape), layout_of((256,)), out=layout_of(shape),
                      bases=[0x20000000004, 0x30000000000])
    assert (misaligned.variant, misaligned.vec) == (ROWS, 0)
    odd_rows = layout_of((64, 255), (256, 1))
    assert plan(odd_rows, out=layout_of((64, 255))).vec == 0


def test_u8_mask_operand_keeps_the_rows_kernel():
    p = plan(layout_of((8192, 4096)), layout_of((8192, 4096)), layout_of((4096,)), out=layout_of((8192, 4096)),
             elem_bytes=[4, 1, 4])
    assert (p.variant, p.vec, p.fixed_rank) == (ROWS, 1, 2)


def test_strided_and_empty_layouts():
    p = plan(layout_of((500,), (3,)), out=layout_of((500,)))
    assert p.variant == GENERIC
    assert plan(layout_of((0, 5)), layout_of((5,)), out=layout_of((0, 5))).variant == 0


def reversed_strides(shape):
    """A view transposed in every dim: no two of its dims merge with a
    contiguous operand's."""
    st, s = [], 1
    for d in shape:  # dim d of the view is dim rank-1-d of the reversed buffer
        st.append(s)
        s *= d
    return tuple(st)


def test_views_above_eight_dims_split_their_smallest_dims_onto_the_host():
    """The kernels index at most 8 dims; a view keeping more after merging is
    launched once per index tuple of its dims with the fewest indices (never
    the innermost), so the launch count is the product of the smallest
    sizes."""
    for shape, launches in [((2, 3) * 5, 2 ** 2), ((2,) * 12 + (1,) * 10 + (3, 1, 2), 2 ** 6), ((2,) * 25, 2 ** 17)]:
        nonunit = sum(1 for d in shape if d != 1)
        p = plan(layout_of(shape), layout_of(shape, reversed_strides(shape)), out=layout_of(shape))
        assert (p.rank, p.split, p.launches) == (8, nonunit - 8, launches)
        assert p.variant == GENERIC  # the reversed operand's unit stride is on a split dim
    # [100000, 2 x 8]: one small dim goes to the host, not the 100,000
    shape = (100000,) + (2,) * 8
    p = plan(layout_of(shape), layout_of(shape, reversed_strides(shape)), out=layout_of(shape))
    assert (p.rank, p.split, p.launches) == (8, 1, 2)
    assert plan(layout_of((4, 5)), out=layout_of((4, 5))).launches == 1
    assert plan(layout_of((0, 5)), out=layout_of((0, 5))).launches == 0


def test_views_above_eight_dims_that_merge_need_no_split():
    shape = (2, 3) * 6
    p = plan(layout_of(shape), layout_of(shape), out=layout_of(shape))
    assert (p.variant, p.rank, p.split, p.vec) == (FLAT, 1, 0, 1)
    # broadcast along the 11 outer dims: the rows kernel over [prod, 3]
    p = plan(layout_of(shape), layout_of((3,)), out=layout_of(shape))
    assert (p.variant, p.rank, p.split) == (ROWS, 2, 0)
    assert plan(layout_of((2, 3)), out=layout_of((2, 3))).split == 0


def test_split_launches_vectorise_only_when_every_part_is_aligned():
    shape = (2,) * 9 + (8,)
    x = layout_of(shape)
    yst = tuple(8 * 2 ** d for d in range(9)) + (1,)  # dims 0-8 reversed, rows of 8 contiguous
    p = plan(x, layout_of(shape, yst), out=layout_of(shape))
    assert (p.variant, p.rank, p.split, p.vec) == (ROWS, 8, 2, 1)
    p = plan(x, layout_of(shape, yst, offset=1), out=layout_of(shape))  # y's base one float off
    assert (p.split, p.vec) == (2, 0)
    # the outermost split dim moves y by 10 floats: the second part of the
    # launch would start 8 bytes off a 16-byte boundary
    p = plan(x, layout_of(shape, (10,) + yst[1:]), out=layout_of(shape))
    assert (p.split, p.vec) == (2, 0)


def test_views_above_the_abi_rank_are_errors():
    lay = abi.Layout()
    lay.rank = abi.MAX_RANK + 1  # refused before any shape entry is read
    with pytest.raises(abi.TrsError) as e:
        plan(layout_of((2,)), out=lay)
    assert e.value.code == abi.TRS_E_INVALID_ARGUMENT
    with pytest.raises(ValueError):
        layout_of((1,) * (abi.MAX_RANK + 1))


def test_shape_mismatch_and_bad_arguments_are_errors():
    with pytest.raises(abi.TrsError) as e:
        plan(layout_of((3, 4)), layout_of((5,)), out=layout_of((3, 4)))
    assert e.value.code == abi.TRS_E_SHAPE_MISMATCH
    with pytest.raises(abi.TrsError):
        plan(layout_of((3, 4)), out=layout_of((3, 4)), cu_count=0)


def test_grid_cap_hook_bounds_every_pointwise_launch_and_resets():
    # trs_debug_pointwise_grid_cap: the tests of the kernels' grid-stride
    # loops plan launches with fewer blocks than tiles through it.
    x, b = layout_of((4096, 4096)), layout_of((4096,))
    c_mt = layout_of((64, 512, 1024), (512 * 1024, 1, 512))
    try:
        abi.check(abi.lib.trs_debug_pointwise_grid_cap(5))
        assert plan(x, b, out=x).grid == 5
        assert plan(layout_of((1 << 20,)), layout_of((1 << 20,)), out=layout_of((1 << 20,))).grid == 5
        assert plan(layout_of((64, 512, 1024)), c_mt, out=layout_of((64, 512, 1024))).grid == 5
        assert abi.lib.trs_debug_pointwise_grid_cap(-1) == abi.TRS_E_INVALID_ARGUMENT
    finally:
        abi.check(abi.lib.trs_debug_pointwise_grid_cap(0))
    assert plan(x, b, out=x).grid == 4096 * 16
    # one-shot up to 2^22 blocks: 2^30 contiguous floats on one-wave blocks
    n = 1 << 30
    assert plan(layout_of((n,)), layout_of((n,)), out=layout_of((n,))).grid == 1 << 22

