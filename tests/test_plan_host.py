"""The launch's plan without a device (charlotte_hip_matmul_plan_launch): which
kernel each shape runs, and the launch's checks, on the CPU.

The reference's launcher is pure and tested without a GPU
(src/core/kernels/interface.h:29-34; tests/kernels_matmul_test.cpp). Here the
plan query runs the same checks as charlotte_hip_matmul_launch, in the same
order, over shape-only weights: descriptors whose sums would wrap 32 or 64
bits are refused before any kernel could read or write outside a weight or an
output; each BASELINE shape gets the kernel the design names for it; AUTO
stays on the bit-exact tile whatever workspace is set; a divided step
(row_divisor, interface.h:270-279) plans its rows.
"""

import pytest

from charlotte_amd import matmul as mm

F32, F16, BF16 = mm.TensorType.F32, mm.TensorType.F16, mm.TensorType.BF16
Q4_0, Q6_K, Q8_0 = mm.TensorType.Q4_0, mm.TensorType.Q6_K, mm.TensorType.Q8_0
K = mm.Kernel
X, Y0, Y1, Y2 = 0x10000, 0x20000, 0x30000, 0x40000  # aligned stand-ins: the plan never touches them
MI355X = mm.Target(compute_units=256)


@pytest.fixture
def shapes():
    made = []

    def make(gtype, rows, columns):
        w = mm.Weight.shape(gtype, rows, columns)
        made.append(w)
        return w

    yield make
    for w in made:
        w.free()


def _write(w, **kw):
    return mm.MatmulLaunch([mm.Member(w)], X, [Y0], **kw)


def _refused(m, tokens, status=mm.Status.INVALID_ARGUMENT, target=MI355X, **kw):
    with pytest.raises(mm.MatmulError) as e:
        mm.plan_launch(m, tokens, target, **kw)
    assert e.value.status == status, str(e.value)
    return str(e.value)


# ---- descriptors that would wrap past a check ------------------------------------


def test_member_row_offset_that_wraps_64_bits_is_refused(shapes):
    w = shapes(Q4_0, 64, 1024)
    # row_offset + rows = 2^64 - 1 + 1 wraps to 0 in 64 bits.
    msg = _refused(mm.MatmulLaunch([mm.Member(w, row_offset=2**64 - 1, rows=1)], X, [Y0]), 1)
    assert "rows past its weight" in msg
    _refused(mm.MatmulLaunch([mm.Member(w, row_offset=64, rows=1)], X, [Y0]), 1)
    _refused(mm.MatmulLaunch([mm.Member(w, row_offset=1, rows=64)], X, [Y0]), 33)
    _refused(mm.MatmulLaunch([mm.Member(w, row_offset=2**63, rows=2**63)], X, [Y0]), 1)
    # The last row alone is inside.
    assert mm.plan_launch(mm.MatmulLaunch([mm.Member(w, row_offset=63, rows=1)], X, [Y0]), 1).kernel != K.NONE


def test_output_rows_that_wrap_32_bits_are_refused(shapes):
    w = shapes(Q4_0, 64, 1024)
    # out_row + rows wraps in 32 bits: 2^32 - 1 + 2.
    m = mm.MatmulLaunch([mm.Member(w, rows=2, output_row=2**32 - 1)], X, [Y0], out_width=2**32 - 1)
    assert "output rows past out_width" in _refused(m, 1)
    # output_row past 2^32 is refused before it could be narrowed.
    m = mm.MatmulLaunch([mm.Member(w, rows=2, output_row=2**32)], X, [Y0], out_width=2**32 - 1)
    assert "output_row" in _refused(m, 1)
    m = mm.MatmulLaunch([mm.Member(w)], X, [Y0], out_width=2**32)
    assert "out_width" in _refused(m, 1)
    # Inside: the member's last output is out_width - 1.
    m = mm.MatmulLaunch([mm.Member(w, output_row=100)], X, [Y0], out_width=164)
    assert mm.plan_launch(m, 2).kernel == K.GEMM_EXACT_SHORT
    _refused(mm.MatmulLaunch([mm.Member(w, output_row=101)], X, [Y0], out_width=164), 2)


def test_descriptor_checks_match_the_launchs(shapes):
    w, v = shapes(Q4_0, 64, 1024), shapes(Q4_0, 64, 2048)
    _refused(mm.MatmulLaunch([mm.Member(w)], 0, [Y0]), 1)  # no input
    _refused(mm.MatmulLaunch([mm.Member(w)], X + 4, [Y0]), 1)  # misaligned input
    _refused(mm.MatmulLaunch([mm.Member(w)], X, [0]), 1)  # no output
    _refused(mm.MatmulLaunch([mm.Member(w), mm.Member(v)], X, [Y0, Y1], epilogue=mm.Epilogue.QKV), 1)
    _refused(_write(w), 0)
    _refused(mm.MatmulLaunch([mm.Member(w)], X, [Y0], epilogue=mm.Epilogue.GatedActivation), 1)
    _refused(mm.MatmulLaunch([mm.Member(w)], X, [Y0], epilogue=mm.Epilogue.QKV, bias=Y1), 1)
    _refused(mm.MatmulLaunch([mm.Member(w)], X, [Y0], epilogue=mm.Epilogue.GatedByInput), 1)


def test_clip_takes_four_bound_words_or_none(shapes):
    """The four bounds are four words of their own, wherever they lie (the
    reference's Constants.clip, a first word each, matmul.cpp:280-281): four
    pointers 32 bytes apart plan as a clipped product, in any order; some but
    not all of them, or one not on a 4-byte word, are refused."""
    w = shapes(Q4_0, 64, 1024)
    span = 0x50000
    apart = [span + 32 * i for i in range(4)]
    assert mm.plan_launch(_write(w, clip=apart), 33).kernel == K.GEMM_EXACT_SHORT
    assert mm.plan_launch(_write(w, clip=apart[::-1]), 1).kernel != K.NONE
    assert mm.plan_launch(_write(w, clip=[span] * 4), 1).kernel != K.NONE
    for partial in ([span, 0, 0, 0], [span, span + 4, span + 8, 0], [0, 0, 0, span]):
        assert "four bounds or none" in _refused(_write(w, clip=partial), 1)
    assert "4-byte" in _refused(_write(w, clip=[span, span + 2, span + 8, span + 12]), 1)
    # An optioned product never splits (matmul.cpp:166-172), whatever the gate.
    assert mm.plan_launch(_write(w, clip=apart), 32, gate=mm.kAlways,
                          range_sums_bytes=1 << 24).kernel == K.GEMM_EXACT_SHORT
    assert mm.plan_launch(_write(w), 32, gate=mm.kAlways, range_sums_bytes=1 << 24).kernel == K.GEMM_EXACT_SPLIT


# ---- the kernel each shape runs --------------------------------------------------


def test_c2_head_is_the_streamed_q6_k_decode(shapes):
    p = mm.plan_launch(_write(shapes(Q6_K, 262144, 1152)), 1)
    assert (p.kernel, p.lanes_a_row, p.groups_a_lane, p.canonical) == (K.GEMV_STREAM, 4, 9, True)
    assert p.tiles == 262144 // 16 and p.workgroups == 2 * 256 and p.launches == 1 and p.rows == 1
    limbs = mm.plan_launch(_write(shapes(Q6_K, 262144, 1152)), 1, mm.Target(256, gemv_path=mm.GemvPath.INT8_LIMBS))
    assert limbs.kernel == K.GEMV_STREAM and not limbs.canonical


@pytest.mark.parametrize("rows,columns", [(151936, 1024), (128256, 2048)])
def test_qwen_and_llama_heads_are_the_streamed_decode_of_k_1024_and_2048(shapes, rows, columns):
    p = mm.plan_launch(_write(shapes(Q6_K, rows, columns)), 1)
    assert p.kernel == K.GEMV_STREAM8 and p.canonical and p.tile_rows == 64 // (columns // 256)


def test_c1_is_the_reference_mapping_in_workgroups_of_one_wave(shapes):
    p = mm.plan_launch(_write(shapes(Q4_0, 3072, 1024)), 1)
    assert (p.kernel, p.lanes_a_row, p.groups_a_lane) == (K.GEMV_RANGES, 32, 1)
    # Two steps a wave (the fewest that would bring four-wave workgroups down to
    # one a CU), the waves as workgroups of one: 2 steps x 2 rows = 4 rows a
    # workgroup, 768 of them over every CU.
    assert (p.steps_a_wave, p.tile_rows, p.tiles) == (2, 4, 768)
    # x staged in LDS (K past 3,072) or 2^20 groups and more: four waves a workgroup
    p = mm.plan_launch(_write(shapes(Q4_0, 3001, 4096)), 1)  # 3,001 rows: not whole streamed steps
    assert p.kernel == K.GEMV_RANGES and p.tile_rows == 4 * p.steps_a_wave * 2
    p = mm.plan_launch(_write(shapes(Q4_0, 32776, 1024)), 1)  # 32,776 rows: not whole streamed steps
    assert p.kernel == K.GEMV_RANGES and p.tile_rows == 4 * p.steps_a_wave * 2
    p = mm.plan_launch(_write(shapes(Q4_0, 32767, 1024)), 1)
    assert p.kernel == K.GEMV_RANGES and p.tile_rows == p.steps_a_wave * 2


def test_large_decodes_balance_their_rounds_of_tiles(shapes):
    """A Q4_1 head of 151,936 rows: at 32 steps a wave, 594 tiles of 256 rows
    on 512 resident workgroups leave 82 with a second round; 8 steps give
    2,374 tiles of 64 rows, 5 rounds, 320 rows on the busiest."""
    p = mm.plan_launch(_write(shapes(mm.TensorType.Q4_1, 151936, 1024)), 1)
    assert (p.kernel, p.steps_a_wave, p.tile_rows, p.tiles) == (K.GEMV_RANGES, 8, 64, 2374)
    # One round already balanced: left as it is.
    p = mm.plan_launch(_write(shapes(Q8_0, 32768, 8192)), 1)
    assert (p.kernel, p.steps_a_wave, p.tiles) == (K.GEMV_RANGES, 8, 512)


def test_k_1152_other_than_whole_streamed_steps_takes_four_lanes_a_row(shapes):
    assert mm.plan_launch(_write(shapes(Q4_0, 1000, 1152)), 1).kernel == K.GEMV_QUARTERS
    assert mm.plan_launch(_write(shapes(Q6_K, 1000, 1152)), 1).kernel == K.GEMV_QUARTERS


@pytest.mark.parametrize("columns,span", [(3072, 3), (4096, 4), (5120, 6), (8192, 8)])
def test_decode_up_to_k_8192_stages_x_whole(shapes, columns, span):
    # 2,049 rows: no whole number of the streamed Q4_0 decode's steps
    p = mm.plan_launch(_write(shapes(Q4_0, 2049, columns)), 1)
    assert (p.kernel, p.groups_a_lane) == (K.GEMV_RANGES, span)
    p = mm.plan_launch(_write(shapes(Q8_0, 2048, columns)), 1)
    assert (p.kernel, p.groups_a_lane) == (K.GEMV_RANGES, span)


@pytest.mark.parametrize("columns,step_rows", [(1024, 16), (2048, 8), (4096, 4), (8192, 2)])
def test_q4_0_k_1024_to_8192_in_whole_steps_is_the_streamed_decode(shapes, columns, step_rows):
    rows = 32768 * 8192 // columns
    p = mm.plan_launch(_write(shapes(Q4_0, rows, columns)), 1)
    assert (p.kernel, p.canonical, p.lanes_a_row, p.groups_a_lane) == (K.GEMV_STREAM4, True, columns // 256, 8)
    assert (p.tile_rows, p.tiles, p.workgroups) == (step_rows, rows // step_rows, 512)
    # INT8_LIMBS: the same kernel's limbs form at K = 1,024 and 2,048; canonical past them
    limbs = mm.plan_launch(_write(shapes(Q4_0, rows, columns)), 1, mm.Target(256, gemv_path=mm.GemvPath.INT8_LIMBS))
    assert limbs.kernel == K.GEMV_STREAM4 and limbs.canonical == (columns > 2048)
    assert (limbs.tile_rows, limbs.tiles, limbs.workgroups) == (step_rows, rows // step_rows, 512)
    # a product under 2^20 groups goes to the 32-lane kernel, canonical whatever the setting
    small = mm.plan_launch(_write(shapes(Q4_0, 2**20 // (columns // 32) - step_rows, columns)), 1,
                           mm.Target(256, gemv_path=mm.GemvPath.INT8_LIMBS))
    assert small.kernel == K.GEMV_RANGES and small.canonical
    w = shapes(Q4_0, 65536, columns)
    big = 2**20 // (columns // 32)  # rows of 2^20 groups: the smallest product streamed
    # a member starting inside a step, or not whole steps long: the reference mapping
    assert mm.plan_launch(mm.MatmulLaunch([mm.Member(w, row_offset=1, rows=big)], X, [Y0]), 1).kernel == \
        K.GEMV_RANGES
    assert mm.plan_launch(mm.MatmulLaunch([mm.Member(w, rows=big + 1)], X, [Y0]), 1).kernel == K.GEMV_RANGES
    # under 2^20 groups: the reference mapping's one-wave workgroups
    p = mm.plan_launch(mm.MatmulLaunch([mm.Member(w, rows=big - step_rows)], X, [Y0]), 1)
    assert p.kernel == K.GEMV_RANGES
    three = [mm.Member(w, rows=big // 2), mm.Member(w, row_offset=big // 2, rows=big // 4),
             mm.Member(w, row_offset=3 * big // 4, rows=big // 4)]
    assert mm.plan_launch(mm.MatmulLaunch(three, X, [Y0, Y1, Y2], epilogue=mm.Epilogue.QKV), 1).kernel == \
        K.GEMV_STREAM4
    # a gated product interleaves its members' rows: the reference mapping
    gated = mm.MatmulLaunch([mm.Member(w), mm.Member(w)], X, [Y0], epilogue=mm.Epilogue.GatedActivation,
                            out_width=65536)
    assert mm.plan_launch(gated, 1).kernel == K.GEMV_RANGES
    # other quantized formats at these K: the reference mapping
    assert mm.plan_launch(_write(shapes(mm.TensorType.Q4_1, 1024, columns)), 1).kernel == K.GEMV_RANGES


@pytest.mark.parametrize("columns", [8192 + 32, 9728, 13824, 17408, 65536])
def test_decode_past_k_8192_stages_x_in_chunks(shapes, columns):
    # Q4_0 past K = 8,192 other than whole 1,024s up to 16,384
    p = mm.plan_launch(_write(shapes(Q4_0, 4096, columns)), 1)
    assert p.kernel == K.GEMV_CHUNKED and p.canonical and p.groups_a_lane == (columns // 32 + 31) // 32
    # other formats at any K past 8,192
    assert mm.plan_launch(_write(shapes(mm.TensorType.Q8_0, 4096, 14336)), 1).kernel == K.GEMV_CHUNKED


@pytest.mark.parametrize("rows,columns", [(4096, 9216), (4096, 14336), (1, 14336), (4097, 16384), (14336, 12288)])
def test_q4_0_k_9216_to_16384_in_whole_1024s_is_the_wide_streamed_decode(shapes, rows, columns):
    """A lane a range (K / 1,024 groups each), two rows a wave step, one
    workgroup of four waves a CU at most."""
    p = mm.plan_launch(_write(shapes(Q4_0, rows, columns)), 1)
    steps = (rows + 1) // 2
    assert (p.kernel, p.canonical, p.lanes_a_row, p.groups_a_lane) == (K.GEMV_WIDE, True, 32, columns // 1024)
    assert (p.tile_rows, p.tiles, p.workgroups) == (2, steps, min(256, (steps + 3) // 4))
    # members anywhere and gated products: rows are copied one at a time
    w = shapes(Q4_0, 2 * rows + 3, columns)
    assert mm.plan_launch(mm.MatmulLaunch([mm.Member(w, row_offset=3, rows=rows)], X, [Y0]), 1).kernel == K.GEMV_WIDE
    gated = mm.MatmulLaunch([mm.Member(w, rows=rows), mm.Member(w, row_offset=rows, rows=rows)], X, [Y0],
                            epilogue=mm.Epilogue.GatedActivation, out_width=rows)
    assert mm.plan_launch(gated, 1).kernel == K.GEMV_WIDE


@pytest.mark.parametrize("gtype,columns,kernel", [
    (F32, 1024, K.GEMV_RANGES), (F32, 2048, K.GEMV_RANGES), (F32, 3072, K.GEMV_CHUNKED),
    (F16, 3072, K.GEMV_RANGES), (F16, 4096, K.GEMV_CHUNKED), (BF16, 1152, K.GEMV_RANGES),
    (BF16, 12288, K.GEMV_CHUNKED),
])
def test_float_formats_decode(shapes, gtype, columns, kernel):
    assert mm.plan_launch(_write(shapes(gtype, 512, columns)), 1).kernel == kernel


def test_last_token_decodes_whatever_the_step(shapes):
    p = mm.plan_launch(_write(shapes(Q6_K, 151936, 1024), rows=mm.Rows.LastToken), 33)
    assert p.kernel == K.GEMV_STREAM8 and p.rows == 1


def test_c4_prefill_is_a_bit_exact_tile_under_auto_with_or_without_a_workspace(shapes):
    """C4 under AUTO: the matrix cores' fused multiply-add tile (1,024 waves of
    64 x 64, the canonical order) whatever workspace is set; CANONICAL: the
    128-row VALU tile."""
    w = shapes(Q4_0, 8192, 2048)
    room = mm.workspace_bytes(512, 2048)
    for target in (MI355X, mm.Target(256, workspace_bytes=room)):
        p = mm.plan_launch(_write(w), 512, target)
        assert (p.kernel, p.canonical, p.tile_tokens, p.tile_rows) == (K.GEMM_EXACT, True, 64, 256), target
        assert p.tiles == 8 * 32
    p = mm.plan_launch(_write(w), 512, mm.Target(256, mm.GemmPath.CANONICAL, workspace_bytes=room))
    assert (p.kernel, p.canonical, p.tile_tokens, p.tile_rows) == (K.GEMM_TILED, True, 64, 128)
    assert p.tiles == 8 * 64
    mfma = mm.plan_launch(_write(w), 512, mm.Target(256, mm.GemmPath.SPLIT_F16_MFMA, workspace_bytes=room))
    assert mfma.kernel == K.GEMM_MFMA and not mfma.canonical and mfma.launches == 2
    assert "workspace" in _refused(_write(w), 512, target=mm.Target(256, mm.GemmPath.SPLIT_F16_MFMA, workspace_bytes=room - 1))


def test_the_matrix_cores_refuse_the_float_formats(shapes):
    w = shapes(F16, 256, 1024)
    target = mm.Target(256, mm.GemmPath.SPLIT_F16_MFMA, workspace_bytes=1 << 30)
    _refused(_write(w), 64, mm.Status.UNSUPPORTED, target=target)
    assert mm.plan_launch(_write(w), 64).kernel == K.GEMM_EXACT_SHORT


def test_short_steps_split_along_k_when_the_gate_and_range_sums_allow(shapes):
    """AUTO splits on the matrix cores' fused multiply-add (GEMM_EXACT_SPLIT),
    CANONICAL on the VALU tile (GEMM_SPLIT): the same range sums, the same
    combine. The exact split cuts the 32 ranges into the fewest chunks (a
    power of two) that give every compute unit two workgroups: 8,192 rows at
    32 tokens are 32 tiles of 256 rows, 16 chunks."""
    w = shapes(Q4_0, 8192, 2048)
    sums = 4 * mm.range_sum_floats(mm.Epilogue.Write, 8192, 2048, mm.kAlways)
    p = mm.plan_launch(_write(w), 32, gate=mm.kAlways, range_sums_bytes=sums)
    assert (p.kernel, p.launches, p.canonical, p.tile_tokens, p.tile_rows) == (K.GEMM_EXACT_SPLIT, 2, True, 32, 256)
    assert (p.tiles, p.chunks, p.workgroups) == (32, 16, 512)
    p = mm.plan_launch(_write(w), 32, mm.Target(256, mm.GemmPath.CANONICAL), gate=mm.kAlways, range_sums_bytes=sums)
    assert (p.kernel, p.launches, p.canonical, p.tile_tokens) == (K.GEMM_SPLIT, 2, True, 32) and p.chunks >= 2
    # C6: 2,048 x 8,192 at 32 tokens: 8 tiles, the most chunks (32); 64 tokens by 64
    down = shapes(Q4_0, 2048, 8192)
    sums = 4 * mm.range_sum_floats(mm.Epilogue.Write, 2048, 8192, mm.kAlways)
    p = mm.plan_launch(_write(down), 32, gate=mm.kAlways, range_sums_bytes=sums)
    assert (p.kernel, p.tiles, p.chunks, p.workgroups) == (K.GEMM_EXACT_SPLIT, 8, 32, 256)
    p = mm.plan_launch(_write(down), 64, gate=mm.kAlways, range_sums_bytes=2 * sums)
    assert (p.kernel, p.tile_tokens, p.tiles, p.chunks) == (K.GEMM_EXACT_SPLIT, 64, 8, 32)
    assert mm.plan_launch(_write(down), 64, mm.Target(128), gate=mm.kAlways, range_sums_bytes=2 * sums).chunks == 32
    assert mm.plan_launch(_write(down), 64, mm.Target(16), gate=mm.kAlways, range_sums_bytes=2 * sums).chunks == 4
    # Range sums too small for the step, no gate, options or a gated product: a
    # short-step tile (on the matrix cores under AUTO, the VALU under CANONICAL).
    canonical = mm.Target(256, mm.GemmPath.CANONICAL)
    for target, kernel in ((MI355X, K.GEMM_EXACT_SHORT), (canonical, K.GEMM_SHORT)):
        assert mm.plan_launch(_write(w), 32, target, gate=mm.kAlways, range_sums_bytes=sums // 64).kernel == kernel
        assert mm.plan_launch(_write(w), 32, target, gate=mm.kNever, range_sums_bytes=sums).kernel == kernel
        assert mm.plan_launch(_write(w, bias=Y1), 32, target, gate=mm.kAlways, range_sums_bytes=sums).kernel == kernel
        g = mm.MatmulLaunch([mm.Member(w), mm.Member(w)], X, [Y0], epilogue=mm.Epilogue.GatedActivation)
        assert mm.plan_launch(g, 32, target, gate=mm.kAlways, range_sums_bytes=2 * sums).kernel == kernel


def test_short_steps_that_do_not_split_take_a_short_step_tile(shapes):
    """AUTO: a step that gives the whole-K matrix-core tile fewer than three
    waves a compute unit runs GEMM_EXACT_SHORT, workgroups of 32 rows x 32
    tokens whose eight waves split K's ranges, or of 16 x 16 where those
    number at most two a compute unit: C6's 32 tokens through 2,048 x 8,192,
    256 of 16 x 16; a 32-token gated gate/up of Llama 3.2 1B (16,384
    interleaved rows), 512 of 32 x 32 (2,048 of 16 x 16 would be eight a
    compute unit). CANONICAL: the VALU short-step tile where the
    128-row tiles would be fewer than the compute units (C6: 16 tiles of 128
    rows on 256 CUs, so 8-row tiles, 256 workgroups; the gated pair 16-row
    tiles, 1,024 workgroups), else the 128-row tile (C4: 512 tiles)."""
    down = shapes(Q4_0, 2048, 8192)
    p = mm.plan_launch(_write(down), 32)
    assert (p.kernel, p.canonical, p.tile_rows, p.tile_tokens, p.workgroups) == (K.GEMM_EXACT_SHORT, True, 16, 16, 256)
    canonical = mm.Target(256, mm.GemmPath.CANONICAL)
    p = mm.plan_launch(_write(down), 32, canonical)
    assert (p.kernel, p.canonical, p.tile_rows, p.tile_tokens, p.workgroups) == (K.GEMM_SHORT, True, 8, 32, 256)
    gate, up = shapes(Q4_0, 8192, 2048), shapes(Q4_0, 8192, 2048)
    g = mm.MatmulLaunch([mm.Member(gate), mm.Member(up)], X, [Y0], epilogue=mm.Epilogue.GatedActivation)
    p = mm.plan_launch(g, 32)
    assert (p.kernel, p.tile_rows, p.workgroups) == (K.GEMM_EXACT_SHORT, 32, 512)
    p = mm.plan_launch(g, 32, canonical)
    assert (p.kernel, p.tile_rows, p.workgroups) == (K.GEMM_SHORT, 16, 1024)
    assert mm.plan_launch(_write(gate), 512).kernel == K.GEMM_EXACT
    assert mm.plan_launch(_write(gate), 512, canonical).kernel == K.GEMM_TILED
    # 100 tokens over 2,048 rows: 64 x 4 workgroups on the matrix cores; on the
    # VALU 32 tiles of 128 rows, so short tiles of 16 rows, 4 x 128 workgroups.
    p = mm.plan_launch(_write(down), 100)
    assert (p.kernel, p.tiles) == (K.GEMM_EXACT_SHORT, 64 * 4)
    p = mm.plan_launch(_write(down), 100, canonical)
    assert (p.kernel, p.tiles, p.tile_rows) == (K.GEMM_SHORT, 4 * 128, 16)


def test_auto_takes_the_exact_matrix_core_tile_from_three_waves_a_compute_unit(shapes):
    """AUTO: GEMM_EXACT where its waves (64 rows by 64 or 32 tokens) number at
    least 3 x the compute units, else the matrix-core short-step tile: 2,048 x
    2,048 at 1,024 tokens is 1,024 waves of 64 x 32, at 512 tokens 512; 2,560
    x 2,048 at 512 tokens 640 (the measured crossing: 91 against 79 us);
    3,072 x 1,024 at 512 tokens 768 (53 against 58 us)."""
    w = shapes(Q4_0, 2048, 2048)
    assert mm.plan_launch(_write(w), 1024).kernel == K.GEMM_EXACT
    assert mm.plan_launch(_write(w), 512).kernel == K.GEMM_EXACT_SHORT
    assert mm.plan_launch(_write(w), 256).kernel == K.GEMM_EXACT_SHORT
    assert mm.plan_launch(_write(shapes(Q4_0, 2560, 2048)), 512).kernel == K.GEMM_EXACT_SHORT  # 640 waves
    assert mm.plan_launch(_write(shapes(Q4_0, 3072, 1024)), 512).kernel == K.GEMM_EXACT  # 768
    assert mm.plan_launch(_write(shapes(Q4_0, 8192, 2048)), 128).kernel == K.GEMM_EXACT_SHORT  # 512 waves
    assert mm.plan_launch(_write(w), 512, mm.Target(128)).kernel == K.GEMM_EXACT  # 512 waves on 128 CUs
    assert mm.plan_launch(_write(w), 256, mm.Target(128)).kernel == K.GEMM_EXACT_SHORT  # 256 of them


def test_exact_mfma_path_takes_every_unsplit_prefill_step(shapes):
    """EXACT_MFMA: every prefill step the gate does not split runs on the matrix
    cores' f32 fused multiply-add (GEMM_EXACT, the canonical order): tiles of
    256 rows by 64 tokens where 64 x 64 waves take no more rounds of the 1,024
    SIMDs than 64 x 32 waves take half-length rounds, else by 32 tokens; decode
    are unchanged, and the split runs on the matrix cores as under AUTO."""
    w = shapes(Q4_0, 2048, 8192)
    exact = mm.Target(256, mm.GemmPath.EXACT_MFMA)
    for tokens in (2, 31, 32, 64, 511, 2048, 4096):
        p = mm.plan_launch(_write(w), tokens, exact)
        rounds64, rounds32 = -(-32 * -(-tokens // 64) // 1024), -(-32 * -(-tokens // 32) // 1024)
        tt = 64 if rounds32 >= 2 * rounds64 else 32
        assert (p.kernel, p.canonical, p.launches, p.tile_rows, p.tile_tokens) == (K.GEMM_EXACT, True, 1, 256, tt)
        assert p.workgroups == 8 * -(-tokens // tt)
    big = shapes(Q4_0, 16384, 2048)
    assert mm.plan_launch(_write(big), 2048, exact).tile_tokens == 64  # C5's gate/up: 8,192 waves of 64 x 64
    assert mm.plan_launch(_write(shapes(Q4_0, 8192, 2048)), 512, exact).tile_tokens == 64  # C4: 1,024 of them
    assert mm.plan_launch(_write(shapes(Q4_0, 4096, 2048)), 512, exact).tile_tokens == 32  # 512 of them
    # Llama 3.2 1B's QKV (3,072 rows) at 2,048 tokens: 1,536 waves of 64 x 64 are two rounds, 3,072 of 64 x 32 three
    # half-length ones
    assert mm.plan_launch(_write(shapes(Q4_0, 3072, 2048)), 2048, exact).tile_tokens == 32
    assert mm.plan_launch(_write(w), 1, exact).kernel == mm.plan_launch(_write(w), 1).kernel == K.GEMV_RANGES
    sums = 4 * mm.range_sum_floats(mm.Epilogue.Write, 2048, 8192, mm.kSplitGate)
    assert mm.plan_launch(_write(w), 32, exact, gate=mm.kSplitGate, range_sums_bytes=sums).kernel == \
        K.GEMM_EXACT_SPLIT
    g = mm.MatmulLaunch([mm.Member(w), mm.Member(w)], X, [Y0], epilogue=mm.Epilogue.GatedActivation)
    assert mm.plan_launch(g, 32, exact).kernel == K.GEMM_EXACT
    f = shapes(F16, 300, 1024)
    assert mm.plan_launch(_write(f), 70, exact).kernel == K.GEMM_EXACT


# ---- row_divisor (interface.h:270-279, 292; program.cpp:382-387) -------------------


def test_a_divided_step_plans_its_rows(shapes):
    w = shapes(Q8_0, 200, 1024)
    for pooled in (1, 2, 7):
        divided = mm.plan_launch(_write(w, row_divisor=9), 9 * pooled)
        plain = mm.plan_launch(_write(w), pooled)
        assert divided == plain and divided.rows == pooled
    # Rounded down, as the reference's step_rows (matmul.wgsl:87-91).
    assert mm.plan_launch(_write(w, row_divisor=9), 20).rows == 2
    nothing = mm.plan_launch(_write(w, row_divisor=9), 8)
    assert (nothing.kernel, nothing.launches) == (K.NONE, 0)
    # 0 is undivided (a zero-initialised descriptor); over the last token, refused.
    assert mm.plan_launch(_write(w, row_divisor=0), 5).rows == 5
    assert "row divisor" in _refused(_write(w, row_divisor=9, rows=mm.Rows.LastToken), 18)
