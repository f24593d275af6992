"""The matrix-core prefill in the canonical order (GEMM_EXACT) against the
128-row VALU tile, bit for bit, at full size.

GEMM_EXACT runs each range's chain on v_mfma_f32_32x32x1_2b_f32, one fused
multiply-add a k, so its outputs are the VALU tile's bits whatever the
inputs. The oracle holds both tiles to the reference order at small sizes
(test_gpu_parity, _formats, _float_formats, _epilogues and _edges run under
EXACT_MFMA too); here the two tiles meet where the oracle would take too long:
the BASELINE prefill shapes in full (C4; C5's QKV, gated gate/up and down at
2,048 tokens), Q6_K products, K past the ranges' count (K = 14,336) and
below it (K = 64: 30 empty ranges), ragged rows and tokens, every epilogue,
on both of its tiles (64 tokens a wave for large steps, 32 for the rest);
and its split along K (GEMM_EXACT_SPLIT) against the VALU's (GEMM_SPLIT).
The reference's own check of the same property: a token's outputs the same
whatever the step (tests/gpu/matmul_test.cpp:257-267).
"""

import numpy as np
import pytest

from tests.support.oracle_lib import F32, Q4_0, Q4_1, Q6_K, Q8_0

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctxs():
    from charlotte_amd import matmul as mm

    exact, tile = mm.Context(0), mm.Context(0)
    exact.set_gemm_path(mm.GemmPath.EXACT_MFMA)
    tile.set_gemm_path(mm.GemmPath.CANONICAL)
    yield exact, tile
    exact.close()
    tile.close()


def _weight(ctx, gtype, rows, columns, stored):
    from charlotte_amd import matmul as mm

    return mm.Weight(ctx, gtype, rows, columns, stored)


def _both(ctxs, members_of, x, tokens, widths, **kw):
    """Run the product on both tiles (members_of(ctx) builds its members)."""
    from tests.support.gpu import Runner

    outs = []
    for ctx in ctxs:
        members, weights = members_of(ctx)
        try:
            outs.append(Runner(ctx).product(members, x, tokens, widths, **kw))
        finally:
            for w in weights:
                w.free()
    return outs


def _same(got, want, what):
    from tests.support.gpu import bits_equal, first_difference

    for g, w in zip(got, want):
        assert not np.isnan(w).all(), f"{what}: nothing written"
        assert bits_equal(g, w), f"{what}: {first_difference(g, w)}"


def _plans(ctx_path, members, tokens):
    from charlotte_amd import matmul as mm

    return mm.plan_launch(mm.MatmulLaunch(members, 16, [16]), tokens, mm.Target(gemm_path=ctx_path)).kernel


@pytest.mark.parametrize("gtype,rows,columns,tokens", [
    (Q4_0, 8192, 2048, 512),     # C4 in full
    (Q4_0, 2048, 8192, 2048),    # C5's down projection
    (Q6_K, 3072, 1152, 300),
    (Q4_0, 1000, 14336, 65),     # 448 groups: 14 a range
    (Q4_0, 333, 64, 129),        # 2 groups: 30 empty ranges
    (Q8_0, 700, 2048, 97),
    (Q4_1, 520, 1024, 70),
    (Q6_K, 16384, 1152, 1024),   # 64-token tiles (4,096 waves of 64 x 64)
    (Q4_0, 16001, 1024, 1001),   # 64-token tiles, ragged rows and tokens
])
def test_write_same_bits_as_the_tile(ctxs, gtype, rows, columns, tokens):
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(rows + columns + tokens)
    stored = synthetic.weight(rng, gtype, rows, columns)
    x = synthetic.activations(rng, tokens, columns)
    assert _plans(mm.GemmPath.EXACT_MFMA, [mm.Member(mm.Weight.shape(gtype, rows, columns))], tokens) == \
        mm.Kernel.GEMM_EXACT

    def members(ctx):
        w = _weight(ctx, gtype, rows, columns, stored)
        return [mm.Member(w)], [w]

    got, want = _both(ctxs, members, x, tokens, [rows])
    _same(got, want, f"type {gtype} {rows}x{columns} tokens={tokens}")


def test_c5_qkv_and_gated_gate_up_same_bits(ctxs):
    """Llama 3.2 1B's fused QKV (2,048 + 512 + 512 rows) and gated gate/up
    (2 x 8,192 rows, SiLU) at 2,048 tokens."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(5)
    tokens, columns = 2048, 2048
    x = synthetic.activations(rng, tokens, columns)
    qkv = [synthetic.weight(rng, Q4_0, r, columns) for r in (2048, 512, 512)]

    def qkv_members(ctx):
        ws = [_weight(ctx, Q4_0, r, columns, s) for r, s in zip((2048, 512, 512), qkv)]
        return [mm.Member(w) for w in ws], ws

    got, want = _both(ctxs, qkv_members, x, tokens, [2048, 512, 512], epilogue=mm.Epilogue.QKV)
    _same(got, want, "qkv")
    gate, up = (synthetic.weight(rng, Q4_0, 8192, columns) for _ in range(2))

    def gated_members(ctx):
        ws = [_weight(ctx, Q4_0, 8192, columns, s) for s in (gate, up)]
        return [mm.Member(w) for w in ws], ws

    got, want = _both(ctxs, gated_members, x, tokens, [8192], epilogue=mm.Epilogue.GatedActivation)
    _same(got, want, "gated gate/up")


@pytest.mark.parametrize("activation", [0, 1, 2])
def test_every_epilogue_and_option_same_bits(ctxs, activation):
    """Ragged rows and tokens through GatedActivation (clipped), GatedByInput,
    a Write with clip, bias and activation, and members placed past row 0."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(40 + activation)
    tokens, columns = 77, 1024
    x = synthetic.activations(rng, tokens, columns)
    a_s, b_s = synthetic.weight(rng, Q4_0, 300, columns), synthetic.weight(rng, Q4_0, 300, columns)
    clip = [-1.5, 1.25, -3.0, 2.5]

    def pair(ctx):
        ws = [_weight(ctx, Q4_0, 300, columns, s) for s in (a_s, b_s)]
        return [mm.Member(w) for w in ws], ws

    got, want = _both(ctxs, pair, x, tokens, [300], epilogue=mm.Epilogue.GatedActivation, activation=activation,
                      clip=clip)
    _same(got, want, f"gated clipped act={activation}")
    u = rng.standard_normal((tokens, 500)).astype(np.float32)

    def one(ctx):
        w = _weight(ctx, Q4_0, 300, columns, a_s)
        return [mm.Member(w, output_row=100)], [w]

    got, want = _both(ctxs, one, x, tokens, [500], epilogue=mm.Epilogue.GatedByInput, activation=activation,
                      out_width=500, gate_input=u, gate_input_stride=500, gate_input_column=50)
    _same(got, want, f"gated by input act={activation}")
    bias = rng.standard_normal(300).astype(np.float32)

    def opts(ctx):
        w = _weight(ctx, Q4_0, 300, columns, b_s)
        return [mm.Member(w)], [w]

    got, want = _both(ctxs, opts, x, tokens, [300], clip=clip, bias=bias, activated=True, activation=activation)
    _same(got, want, f"write with options act={activation}")


@pytest.mark.parametrize("gtype,rows,columns,tokens", [
    (Q4_0, 2048, 8192, 32),      # C6: 8 tiles x 32 chunks
    (Q4_0, 2048, 8192, 64),      # 64-token tiles
    (Q6_K, 3072, 1152, 9),
    (Q4_0, 1000, 14336, 33),     # 448 groups: 14 a range; 64-token tiles, 31 tokens past the step
    (Q4_0, 333, 64, 20),         # 2 groups: 30 empty ranges, chunks holding none
    (Q8_0, 700, 2048, 17),
    (Q4_1, 520, 1024, 5),
    (F32, 300, 1024, 12),
])
def test_split_same_bits_as_the_valu_split(ctxs, gtype, rows, columns, tokens):
    """The split along K (GEMM_EXACT_SPLIT against GEMM_SPLIT): each chunk's
    range sums the VALU split's bits, so the combine's outputs are too."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(rows + columns + tokens + 7)
    if gtype == F32:
        stored = (rng.standard_normal((rows, columns)).astype(np.float32) * np.float32(0.05)).tobytes()
    else:
        stored = synthetic.weight(rng, gtype, rows, columns)
    x = synthetic.activations(rng, tokens, columns)
    sums = 4 * mm.range_sum_floats(mm.Epilogue.Write, rows, columns, mm.kAlways)
    shape = [mm.Member(mm.Weight.shape(gtype, rows, columns))]
    for path, kernel in ((mm.GemmPath.EXACT_MFMA, mm.Kernel.GEMM_EXACT_SPLIT), (mm.GemmPath.CANONICAL,
                                                                                 mm.Kernel.GEMM_SPLIT)):
        assert mm.plan_launch(mm.MatmulLaunch(shape, 16, [16]), tokens, mm.Target(gemm_path=path), gate=mm.kAlways,
                              range_sums_bytes=sums).kernel == kernel

    def members(ctx):
        w = _weight(ctx, gtype, rows, columns, stored)
        return [mm.Member(w)], [w]

    got, want = _both(ctxs, members, x, tokens, [rows], gate=mm.kAlways, sums_bytes=sums)
    _same(got, want, f"split type {gtype} {rows}x{columns} tokens={tokens}")


def test_split_qkv_same_bits_as_the_valu_split(ctxs):
    """A fused QKV step split along K: the combine routes each row to its
    member's output."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(8)
    tokens, columns = 24, 2048
    x = synthetic.activations(rng, tokens, columns)
    parts = [synthetic.weight(rng, Q4_0, r, columns) for r in (2048, 512, 512)]
    sums = 4 * mm.range_sum_floats(mm.Epilogue.QKV, 3072, columns, mm.kAlways)

    def qkv_members(ctx):
        ws = [_weight(ctx, Q4_0, r, columns, s) for r, s in zip((2048, 512, 512), parts)]
        return [mm.Member(w) for w in ws], ws

    got, want = _both(ctxs, qkv_members, x, tokens, [2048, 512, 512], epilogue=mm.Epilogue.QKV, gate=mm.kAlways,
                      sums_bytes=sums)
    _same(got, want, "qkv split")


@pytest.fixture(scope="module")
def short_ctxs():
    """AUTO (the matrix-core short-step tile for short steps) and CANONICAL
    (the VALU short-step tile)."""
    from charlotte_amd import matmul as mm

    auto, tile = mm.Context(0), mm.Context(0)
    tile.set_gemm_path(mm.GemmPath.CANONICAL)
    yield auto, tile
    auto.close()
    tile.close()


@pytest.mark.parametrize("gtype,rows,columns,tokens,tile", [
    (Q4_0, 2048, 8192, 32, 16),  # C6's down projection, unsplit: 64 tiles of 32 x 32, so 256 of 16 x 16
    (Q4_0, 1001, 2048, 45, 16),  # ragged rows and tokens
    (Q6_K, 3072, 1152, 9, 16),
    (Q4_0, 1000, 14336, 33, 16),  # 448 groups: 56 a wave
    (Q4_0, 333, 64, 20, 16),     # 2 groups: 30 empty ranges, waves holding none
    (Q8_0, 700, 2048, 17, 16),
    (Q4_1, 520, 1024, 5, 16),
    (F32, 300, 1024, 12, 16),
    (Q4_0, 640, 1440, 24, 16),   # 45 groups: ranges of 1 and 2, the shorter padded
    (Q6_K, 512, 2816, 16, 16),   # 88 groups: ranges of 2 and 3
    (F32, 200, 1440, 7, 16),
    (Q4_0, 100, 32, 7, 16),      # one group: range 31 alone
    (Q8_0, 70, 96, 40, 16),      # three groups
    (Q4_0, 33, 2080, 3, 16),     # 65 groups: ranges of 2 and 3
    (Q4_0, 8192, 1440, 32, 32),  # 256 tiles of 32 x 32: pairs of unequal ranges
    (Q6_K, 4096, 2816, 64, 32),
    (F32, 8192, 1024, 40, 32),
    (Q4_1, 8200, 2048, 33, 32),  # ragged rows and tokens
    (Q8_0, 8192, 64, 32, 32),    # 2 groups: pairs with an empty range
])
def test_short_step_tile_same_bits_as_the_valu_short_tile(short_ctxs, gtype, rows, columns, tokens, tile):
    """GEMM_EXACT_SHORT against the VALU short-step tile, bit for bit: 32 x 32
    tiles (each wave four of the ranges, two a 32x32x1 two-block instruction)
    where they give every compute unit one, else 16 x 16 (four ranges a
    16x16x1 four-block instruction); the sums combined in LDS."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(rows + columns + tokens + 11)
    if gtype == F32:
        stored = (rng.standard_normal((rows, columns)).astype(np.float32) * np.float32(0.05)).tobytes()
    else:
        stored = synthetic.weight(rng, gtype, rows, columns)
    x = synthetic.activations(rng, tokens, columns)
    shape = mm.MatmulLaunch([mm.Member(mm.Weight.shape(gtype, rows, columns))], 16, [16])
    p = mm.plan_launch(shape, tokens)
    assert (p.kernel, p.tile_rows, p.tile_tokens) == (mm.Kernel.GEMM_EXACT_SHORT, tile, tile)

    def members(ctx):
        w = _weight(ctx, gtype, rows, columns, stored)
        return [mm.Member(w)], [w]

    got, want = _both(short_ctxs, members, x, tokens, [rows])
    _same(got, want, f"short type {gtype} {rows}x{columns} tokens={tokens}")


@pytest.mark.parametrize("rows,tile", [(640, 16), (12288, 32)])
def test_short_step_tile_special_inputs_as_the_valu_short_tile(short_ctxs, rows, tile):
    """Infinite, NaN, huge, subnormal and signed-zero inputs through ranges of
    unequal length (45 groups, a shorter range multiplying -0 by +0 at its
    last step), on both tile sizes: NaN where the VALU short tile has NaN,
    every other output bit for bit."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    columns, tokens = 1440, 5
    rng = np.random.default_rng(45)
    stored = synthetic.weight(rng, Q4_0, rows, columns)
    x = rng.standard_normal((tokens, columns), dtype=np.float32)
    x[0, 3], x[0, 40], x[0, 41], x[0, columns - 1] = 1e28, 1e-40, -1e-42, -0.0
    x[0, 77::97] = np.float32(-1e28)
    x[1, columns // 2] = np.inf
    x[2, 5] = np.nan
    x[3] = (x[3].astype(np.float64) * 1e-39).astype(np.float32)
    x[4, 1400:] = -0.0  # the last groups' inputs all -0: range sums of zero products
    shape = mm.MatmulLaunch([mm.Member(mm.Weight.shape(Q4_0, rows, columns))], 16, [16])
    p = mm.plan_launch(shape, tokens)
    assert (p.kernel, p.tile_rows) == (mm.Kernel.GEMM_EXACT_SHORT, tile)

    def members(ctx):
        w = _weight(ctx, Q4_0, rows, columns, stored)
        return [mm.Member(w)], [w]

    (got,), (want,) = _both(short_ctxs, members, x, tokens, [rows])
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert nan_w.any() and (nan_g == nan_w).all(), "NaN where the VALU tile has NaN"
    assert (got[~nan_w].view(np.uint32) == want[~nan_w].view(np.uint32)).all()


@pytest.mark.parametrize("activation", [0, 1])
def test_short_step_tile_epilogues_same_bits(short_ctxs, activation):
    """A gated gate/up pair (Llama 3.2 1B's, 32 tokens: the 32 x 32 tile; and a
    small ragged one: the 16 x 16), a fused QKV, a Write with clip, bias and
    activation, and GatedByInput, against the VALU short tile."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(60 + activation)
    tokens = 32
    x = synthetic.activations(rng, tokens, 2048)
    gate, up = (synthetic.weight(rng, Q4_0, 8192, 2048) for _ in range(2))

    def gated(ctx):
        ws = [_weight(ctx, Q4_0, 8192, 2048, s) for s in (gate, up)]
        return [mm.Member(w) for w in ws], ws

    got, want = _both(short_ctxs, gated, x, tokens, [8192], epilogue=mm.Epilogue.GatedActivation,
                      activation=activation)
    _same(got, want, f"gated act={activation}")
    # a small gated pair, ragged (2 x 1,000 rows, 13 tokens): the 16 x 16 tile
    small = [synthetic.weight(rng, Q4_0, 1000, 2048) for _ in range(2)]

    def gated_small(ctx):
        ws = [_weight(ctx, Q4_0, 1000, 2048, s) for s in small]
        return [mm.Member(w) for w in ws], ws

    shape = mm.MatmulLaunch([mm.Member(mm.Weight.shape(Q4_0, 1000, 2048))] * 2, 16, [16],
                            epilogue=mm.Epilogue.GatedActivation)
    assert mm.plan_launch(shape, 13).tile_rows == 16
    got, want = _both(short_ctxs, gated_small, x[:13], 13, [1000], epilogue=mm.Epilogue.GatedActivation,
                      activation=activation)
    _same(got, want, f"small gated act={activation}")
    parts = [synthetic.weight(rng, Q4_0, r, 2048) for r in (2048, 512, 512)]

    def qkv(ctx):
        ws = [_weight(ctx, Q4_0, r, 2048, s) for r, s in zip((2048, 512, 512), parts)]
        return [mm.Member(w) for w in ws], ws

    got, want = _both(short_ctxs, qkv, x[:24], 24, [2048, 512, 512], epilogue=mm.Epilogue.QKV)
    _same(got, want, "qkv")
    tokens, columns = 77, 1024
    x = synthetic.activations(rng, tokens, columns)
    a_s = synthetic.weight(rng, Q4_0, 300, columns)
    bias = rng.standard_normal(300).astype(np.float32)

    def opts(ctx):
        w = _weight(ctx, Q4_0, 300, columns, a_s)
        return [mm.Member(w)], [w]

    got, want = _both(short_ctxs, opts, x, tokens, [300], clip=[-1.5, 1.25, -3.0, 2.5], bias=bias, activated=True,
                      activation=activation)
    _same(got, want, f"write with options act={activation}")
    u = rng.standard_normal((tokens, 500)).astype(np.float32)

    def by_input(ctx):
        w = _weight(ctx, Q4_0, 300, columns, a_s)
        return [mm.Member(w, output_row=100)], [w]

    got, want = _both(short_ctxs, by_input, x, tokens, [500], epilogue=mm.Epilogue.GatedByInput,
                      activation=activation, out_width=500, gate_input=u, gate_input_stride=500, gate_input_column=50)
    _same(got, want, f"gated by input act={activation}")
    # the same options and GatedByInput on the 32 x 32 tile (8,200 ragged rows)
    big = synthetic.weight(rng, Q4_0, 8200, columns)
    shape = mm.MatmulLaunch([mm.Member(mm.Weight.shape(Q4_0, 8200, columns))], 16, [16])
    assert mm.plan_launch(shape, tokens).tile_rows == 32
    bias = rng.standard_normal(8200).astype(np.float32)

    def opts_big(ctx):
        w = _weight(ctx, Q4_0, 8200, columns, big)
        return [mm.Member(w)], [w]

    got, want = _both(short_ctxs, opts_big, x, tokens, [8200], clip=[-1.5, 1.25, -3.0, 2.5], bias=bias,
                      activated=True, activation=activation)
    _same(got, want, f"write with options, 32 x 32, act={activation}")
    u = rng.standard_normal((tokens, 8400)).astype(np.float32)

    def by_input_big(ctx):
        w = _weight(ctx, Q4_0, 8200, columns, big)
        return [mm.Member(w, output_row=100)], [w]

    got, want = _both(short_ctxs, by_input_big, x, tokens, [8400], epilogue=mm.Epilogue.GatedByInput,
                      activation=activation, out_width=8400, gate_input=u, gate_input_stride=8400,
                      gate_input_column=50)
    _same(got, want, f"gated by input, 32 x 32, act={activation}")
