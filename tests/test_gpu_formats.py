"""Q4_1, Q8_0 and the embedding gather on the GPU, through the C ABI, against
the CPU oracle bit for bit.

Follows the reference's own GPU tests:
  tests/gpu/unpack_q4_1_test.cpp, unpack_q8_0_test.cpp, unpack_f32_test.cpp —
    unpack bit for bit (Q4_1: its multiply-add rounded twice or fused, which
    are the same bits);
  tests/gpu/matmul_test.cpp:217-267, 462-472 — w_q4_1_1152, w_q4_1_3072 and
    w_q8_0 decoded and prefilled, within gamma(2K) of f64, a token's outputs
    the same bits alone and in any step, split and tiled alike;
  matmul_test.cpp:552-650 — w_q8_0 clamped, biased (bias_q8_0) and activated;
    a GLU over w_glu's halves, sigmoid, clamped;
  tests/gpu/gather_test.cpp:202-300 — every fixture table's rows, a table in
    pieces, Gemma 3's scale, a fed step, step after step.
Beyond them: the media placeholder skipped, the position form, a table of
the listed models' size, and the host's refusals.
"""

import math
import os

import numpy as np
import pytest

from tests.support import blocks as B
from tests.support import gguf_fixture
from tests.support.oracle_lib import F32, Q4_0, Q4_1, Q6_K, Q8_0

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
SILU, GELU, SIGMOID = 0, 1, 2


@pytest.fixture(scope="module", params=["AUTO", "CANONICAL", "EXACT_MFMA"])
def ctx(request):
    """Each test three times: under AUTO (the short-step tile where the 128-row
    tile would leave compute units idle), CANONICAL (always the 128-row tile)
    and EXACT_MFMA (every unsplit step on the matrix cores' f32 fused
    multiply-add)."""
    from charlotte_amd import matmul as mm

    c = mm.Context(0)
    c.set_gemm_path(mm.GemmPath[request.param])
    yield c
    c.close()


@pytest.fixture(scope="module")
def run(ctx):
    from tests.support.gpu import Runner

    return Runner(ctx)


@pytest.fixture(scope="module")
def source(oracle):
    # matmul_test.cpp:141: source rows filled with seed 7, amplitude 1.0.
    return oracle.fill(7, 64 * 3072)


def _check(got, want, what):
    from tests.support.gpu import bits_equal, first_difference

    assert bits_equal(got, want), f"{what}: {first_difference(got, want)}"


# ---- unpack, bit for bit -------------------------------------------------------


@pytest.mark.parametrize("gtype,count", [(Q4_1, 1), (Q4_1, 9), (Q4_1, 257), (Q8_0, 1), (Q8_0, 9), (Q8_0, 257),
                                         (F32, 32), (F32, 8192)])
def test_unpack_decodes_every_block_as_ggml_does(oracle, gtype, count):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    if gtype == F32:
        stored = np.random.default_rng(count).standard_normal(count).astype(np.float32).tobytes()
    else:
        stored = B.q4_1_edge_blocks(count) if gtype == Q4_1 else B.q8_0_edge_blocks(count)
    piece = np.frombuffer(mm.lay_out(gtype, stored, count), np.uint8)
    groups = count // 32 if gtype == F32 else count
    buf = hx.Buffer(16 + piece.size)
    buf.write(np.full(16, 0xA5, np.uint8))
    buf.write(piece, offset=16)
    out = hx.Buffer(groups * 32 * 4)
    hx.unpack(gtype, buf.ptr + 16, count, groups, out.ptr)
    hx.sync()
    got = out.read(np.float32)
    if gtype == Q4_1:
        rounded, fused = oracle.dequantize_q4_1(stored)
        assert (rounded.view(np.uint32) == fused.view(np.uint32)).all()
        want = rounded
    else:
        want = oracle.dequantize(gtype, stored)
    assert (got.view(np.uint32) == want.view(np.uint32)).all(), f"{int((got != want).sum())} weights differ"
    buf.free()
    out.free()


# ---- the fixture's products ------------------------------------------------------


STEPS = [2, 8, 9, 16, 17, 33, 64]
ALONE = [0, 1, 7, 8, 15, 16, 32, 63]


@pytest.mark.parametrize("name", ["w_q4_1_1152", "w_q4_1_3072", "w_q8_0", "w_glu"])
def test_fixture_product_decoded_and_prefilled(oracle, run, source, fixture_tensors, name):
    from tests.support.gpu import bits_equal

    t = fixture_tensors[name]
    w = run.weight(t.type, t.rows, t.columns, t.data)
    x = source[: 64 * t.columns].reshape(64, t.columns)
    want = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x, threads=8)
    y64, bound = oracle.matmul_f64(t.type, t.data, t.rows, t.columns, x)
    prefilled = {}
    for tokens in STEPS:
        got = run.write(w, x, tokens)
        _check(got, want[:tokens], f"{name} tokens={tokens}")
        assert (np.abs(got.astype(np.float64) - y64[:tokens]) <= bound[:tokens]).all()
        prefilled[tokens] = got
    for t_ in ALONE:
        alone = run.write(w, x[t_ : t_ + 1], 1)
        _check(alone[0], want[t_], f"{name} token {t_} decoded")
        for tokens, got in prefilled.items():
            if t_ < tokens:
                assert bits_equal(alone[0], got[t_])
    w.free()


@pytest.mark.parametrize("name", ["w_q4_1_1152", "w_q4_1_3072", "w_q8_0"])
def test_split_is_the_tiled_bits(oracle, run, source, fixture_tensors, name):
    """matmul_test.cpp:462-472: the split along K and its combine give the
    tiled form's bits."""
    from charlotte_amd import matmul as mm

    t = fixture_tensors[name]
    w = run.weight(t.type, t.rows, t.columns, t.data)
    x = source[: 33 * t.columns].reshape(33, t.columns)
    want = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x, threads=8)
    gate = mm.kAlways
    for tokens in (2, 17, 33):
        sums = 32 * tokens * t.rows * 4
        _check(run.write(w, x, tokens, gate=gate, sums_bytes=sums), want[:tokens], f"{name} split tokens={tokens}")
    w.free()


def _f32(t):
    return np.frombuffer(t.data, np.float32)


def test_q8_0_clamped_biased_activated(oracle, run, source, fixture_tensors):
    """matmul_test.cpp:576-606: w_q8_0 with the fixture's bounds, bias_q8_0 and
    SiLU, prefilled over 33 tokens and token 7 alone; the bounds bind both sides."""
    from charlotte_amd import matmul as mm

    t = fixture_tensors["w_q8_0"]
    w = run.weight(t.type, t.rows, 1024, t.data)
    clip = np.array([_f32(fixture_tensors[f"clip_{k}"])[0] for k in ("in_min", "in_max", "out_min", "out_max")])
    bias = _f32(fixture_tensors["bias_q8_0"])
    x = source[: 33 * 1024].reshape(33, 1024)
    xc = oracle.clamp(x, clip[0], clip[1])
    totals = oracle.matmul_f32(t.type, t.data, t.rows, 1024, xc)
    assert (xc != x).any() and ((totals < clip[2]) | (totals > clip[3])).any()
    want = oracle.finish(totals, clip=clip, bias=bias, activated=True, activation=SILU)
    kw = dict(clip=clip, bias=bias, activated=True, activation=SILU)
    _check(run.product([mm.Member(w)], x, 33, [48], **kw)[0], want, "q8_0 options")
    _check(run.product([mm.Member(w)], x[7:8], 1, [48], **kw)[0][0], want[7], "q8_0 options alone")
    w.free()


def test_glu_over_w_glu_halves_sigmoid_clamped(oracle, run, source, fixture_tensors):
    """matmul_test.cpp:622-650: σ(gate) × up over one weight's halves (up the
    first 72 rows, the gate the second), each clamped first."""
    from charlotte_amd import matmul as mm

    t = fixture_tensors["w_glu"]
    w = run.weight(t.type, t.rows, 1024, t.data)
    clip = np.array([_f32(fixture_tensors[f"clip_{k}"])[0] for k in ("in_min", "in_max", "out_min", "out_max")])
    x = source[: 33 * 1024].reshape(33, 1024)
    both = oracle.matmul_f32(t.type, t.data, 144, 1024, oracle.clamp(x, clip[0], clip[1]))
    want = oracle.gated(both[:, 72:], both[:, :72], clip=clip, activation=SIGMOID)
    members = [mm.Member(w, row_offset=72, rows=72), mm.Member(w, row_offset=0, rows=72)]
    kw = dict(epilogue=mm.Epilogue.GatedActivation, activation=SIGMOID, clip=clip)
    _check(run.product(members, x, 33, [72], **kw)[0], want, "GLU prefilled")
    _check(run.product(members, x[5:6], 1, [72], **kw)[0][0], want[5], "GLU alone")
    w.free()


@pytest.mark.parametrize("gtype,columns", [(Q4_1, 1152), (Q4_1, 4096), (Q8_0, 1152), (Q8_0, 2048)])
def test_synthetic_gated_and_by_input(oracle, run, gtype, columns):
    """The fused feed-forward epilogues over the new formats, at a K the
    four-lane decode takes (1,152) and ones the 32-lane decode takes."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(columns + gtype)
    width, tokens = 136, 40
    g_s, u_s = synthetic.weight(rng, gtype, width, columns), synthetic.weight(rng, gtype, width, columns)
    x = synthetic.activations(rng, tokens, columns)
    gate, up = run.weight(gtype, width, columns, g_s), run.weight(gtype, width, columns, u_s)
    g = oracle.matmul_f32(gtype, g_s, width, columns, x, threads=8)
    u = oracle.matmul_f32(gtype, u_s, width, columns, x, threads=8)
    want = oracle.gated(g, u, activation=GELU)
    for t in (1, 9, 40):
        got = run.product([mm.Member(gate), mm.Member(up)], x, t, [width], epilogue=mm.Epilogue.GatedActivation,
                          activation=GELU)[0]
        _check(got, want[:t], f"gated tokens={t}")
    ui = rng.standard_normal((tokens, width + 8)).astype(np.float32)
    want = oracle.gated_by_input(g, ui[:, 8:], activation=SILU)
    got = run.product([mm.Member(gate)], x, tokens, [width], epilogue=mm.Epilogue.GatedByInput, activation=SILU,
                      gate_input=ui, gate_input_stride=width + 8, gate_input_column=8)[0]
    _check(got, want, "gated by input")
    gate.free()
    up.free()


@pytest.mark.parametrize("gtype,rows,columns", [(Q8_0, 4096, 4096), (Q4_1, 3000, 1152), (Q8_0, 262144 // 16, 1152)])
def test_synthetic_decode_at_size(oracle, run, gtype, rows, columns):
    from charlotte_amd import synthetic

    rng = np.random.default_rng(rows)
    stored = synthetic.weight(rng, gtype, rows, columns)
    x = synthetic.activations(rng, 1, columns)
    w = run.weight(gtype, rows, columns, stored)
    _check(run.write(w, x, 1), oracle.matmul_f32(gtype, stored, rows, columns, x, threads=8), "decode")
    w.free()


@pytest.mark.parametrize("name", ["w_q8_0", "w_q4_1_1152", "w_q4_1_3072", "w_glu"])
def test_the_matrix_cores_take_the_fixture_within_tolerance(oracle, run, source, fixture_tensors, name):
    """The split-f16 matrix-core prefill over Q8_0 and Q4_1 (Q4_1's minimum
    through the group's input sum): max |err| / max |y| <= 1e-5 against the
    f64 product. AUTO stays on the bit-exact tile with the workspace set."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    t = fixture_tensors[name]
    w = run.weight(t.type, t.rows, t.columns, t.data)
    x = source[: 64 * t.columns].reshape(64, t.columns)
    y64, _ = oracle.matmul_f64(t.type, t.data, t.rows, t.columns, x)
    exact = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x, threads=8)
    ws = hx.Buffer(mm.workspace_bytes(64, t.columns))
    run.ctx.set_workspace(ws.ptr, mm.workspace_bytes(64, t.columns))
    try:
        path = run.ctx.gemm_path
        run.ctx.set_gemm_path(mm.GemmPath.SPLIT_F16_MFMA)
        for tokens in (16, 33, 64):
            got = run.write(w, x, tokens)
            err = np.abs(got.astype(np.float64) - y64[:tokens]).max()
            assert err <= 1e-5 * np.abs(y64[:tokens]).max(), f"{name} tokens={tokens}: {err}"
            assert (np.argmax(got, 1) == np.argmax(exact[:tokens], 1)).all()
        run.ctx.set_gemm_path(path)
        for tokens in (9, 16, 64):
            _check(run.write(w, x, tokens), exact[:tokens], f"{name} {path.name} {tokens} tokens")
    finally:
        run.ctx.set_gemm_path(path)
        run.ctx.set_workspace(0, 0)
        ws.free()
        w.free()


# ---- the embedding gather (gather.wgsl:21-58) ------------------------------------


EMBEDDINGS = {F32: "embedding_f32", Q4_0: "embedding_q4_0", Q4_1: "embedding_q4_1", Q8_0: "embedding_q8_0",
              Q6_K: "embedding_q6_k"}


def _table(gtype):
    t = gguf_fixture.read(os.path.join(HERE, "golden", "gguf", EMBEDDINGS[gtype] + ".gguf"))["token_embd.weight"]
    assert t.type == gtype
    return t


class _Step:
    """A step's identifiers and hidden rows on the device."""

    def __init__(self, ids, columns, rows=None, fill=0.0):
        from charlotte_amd import harness as hx

        self.ids = hx.Buffer.of(np.asarray(ids if len(ids) else [0], np.uint32))
        self.rows = rows or len(ids) + 1
        self.columns = columns
        self.hidden = hx.Buffer.of(np.full((self.rows, columns), fill, np.float32))

    def read(self):
        from charlotte_amd import harness as hx

        hx.sync()
        return self.hidden.read(np.float32).reshape(self.rows, self.columns)

    def free(self):
        self.ids.free()
        self.hidden.free()


def _expected(oracle, t, ids, rows, first_row=0, row_count=None, fill=0.0, **kw):
    hidden = np.full((rows, t.columns), fill, np.float32)
    row_bytes = len(t.data) // t.rows
    count = t.rows if row_count is None else row_count
    piece = t.data[first_row * row_bytes : (first_row + count) * row_bytes]
    return oracle.gather(t.type, piece, count, t.columns, ids, hidden, first_row=first_row, **kw)


@pytest.mark.parametrize("gtype", sorted(EMBEDDINGS))
def test_gather_every_row_is_its_tokens_row(oracle, run, gtype):
    """gather_test.cpp:202-213: a token twice, the first and last rows; the
    row past the step untouched."""
    from charlotte_amd import matmul as mm

    t = _table(gtype)
    table = run.weight(gtype, t.rows, t.columns, t.data)
    ids = [3, 0, 6, 3, 1]
    s = _Step(ids, t.columns)
    mm.gather(run.ctx, table, s.ids.ptr, len(ids), s.hidden.ptr)
    got = s.read()
    want = _expected(oracle, t, ids, len(ids) + 1)
    _check(got, want, f"gather {EMBEDDINGS[gtype]}")
    assert not got[len(ids)].any()
    s.free()
    table.free()


@pytest.mark.parametrize("gtype", [Q6_K, Q8_0])
def test_gather_a_table_in_pieces(oracle, run, gtype):
    """gather_test.cpp:215-227: rows 0..2, 3..4 and 5..6, one launch a piece,
    identifiers either side of every boundary."""
    from charlotte_amd import matmul as mm

    t = _table(gtype)
    row_bytes = len(t.data) // t.rows
    ids = [2, 3, 4, 5, 0, 6, 4]
    s = _Step(ids, t.columns, fill=7.5)
    want = np.full((len(ids) + 1, t.columns), np.float32(7.5))
    for first, count in ((0, 3), (3, 2), (5, 2)):
        piece = run.weight(gtype, count, t.columns, t.data[first * row_bytes : (first + count) * row_bytes])
        mm.gather(run.ctx, piece, s.ids.ptr, len(ids), s.hidden.ptr, first_row=first)
        oracle.gather(gtype, t.data[first * row_bytes : (first + count) * row_bytes], count, t.columns, ids, want,
                      first_row=first)
        _check(s.read(), want, f"after the piece at {first}")
        piece.free()
    _check(s.read()[: len(ids)], _expected(oracle, t, ids, len(ids)), "every piece")
    s.free()


def test_gather_scale_and_a_decode_step(oracle, run):
    """gather_test.cpp:229-239: Gemma 3's scale sqrt(1152); one row. Decoded,
    then scaled, rounded once: llama.cpp's order, bit for bit."""
    from charlotte_amd import matmul as mm

    t = _table(Q4_0)
    table = run.weight(Q4_0, t.rows, t.columns, t.data)
    scale = float(np.float32(math.sqrt(1152.0)))
    s = _Step([5], t.columns)
    mm.gather(run.ctx, table, s.ids.ptr, 1, s.hidden.ptr, scale=scale)
    _check(s.read(), _expected(oracle, t, [5], 2, scale=scale), "scaled")
    s.free()
    table.free()


def test_gather_fed_step_and_media_rows(oracle, run):
    """gather_test.cpp:241-256: a fed step embeds the draw, not its identifier;
    gather.wgsl:40-45: a media step's placeholder rows are left alone."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    t = _table(Q4_0)
    table = run.weight(Q4_0, t.rows, t.columns, t.data)
    record = hx.Buffer.of(np.array([6, 0, 0, 0], np.uint32))
    s = _Step([2], t.columns, fill=-2.0)
    mm.gather(run.ctx, table, s.ids.ptr, 1, s.hidden.ptr, fed=record.ptr, media=True, media_token=6)
    _check(s.read(), _expected(oracle, t, [2], 2, fill=-2.0, fed=[6]), "fed")
    s.free()
    ids = [1, 4, 4, 0]
    s = _Step(ids, t.columns, fill=-2.0)
    mm.gather(run.ctx, table, s.ids.ptr, len(ids), s.hidden.ptr, media=True, media_token=4)
    got = s.read()
    _check(got, _expected(oracle, t, ids, len(ids) + 1, fill=-2.0, media=True, media_token=4), "media")
    assert (got[1] == -2.0).all() and (got[2] == -2.0).all()
    mm.gather(run.ctx, table, s.ids.ptr, len(ids), s.hidden.ptr, media=False, media_token=4)
    _check(s.read(), _expected(oracle, t, ids, len(ids) + 1, fill=-2.0), "media 0")
    s.free()
    record.free()
    table.free()


def test_gather_step_after_step(oracle, run):
    """gather_test.cpp:258-282: one table, steps of 3, 1 and 2 rows, each
    writing its own rows."""
    from charlotte_amd import matmul as mm

    t = _table(Q8_0)
    table = run.weight(Q8_0, t.rows, t.columns, t.data)
    s = _Step([0] * 3, t.columns, rows=3)
    for ids in ([6, 5, 4], [1], [0, 2]):
        s.ids.write(np.asarray(ids, np.uint32))
        mm.gather(run.ctx, table, s.ids.ptr, len(ids), s.hidden.ptr)
        got = s.read()[: len(ids)]
        _check(got, _expected(oracle, t, ids, len(ids)), f"step {ids}")
    s.free()
    table.free()


@pytest.mark.parametrize("gtype,rows,columns", [(Q6_K, 32768, 1024), (Q8_0, 16384, 1152), (Q4_1, 8192, 2048)])
def test_gather_a_large_table_prefill_step(oracle, run, gtype, rows, columns):
    """A 512-row prefill step (plan.h's block) over a table of thousands of
    rows, random identifiers."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(rows)
    stored = synthetic.weight(rng, gtype, rows, columns)
    table = run.weight(gtype, rows, columns, stored)
    ids = rng.integers(0, rows, 512).astype(np.uint32)
    ids[:2] = [0, rows - 1]
    s = _Step(ids, columns)
    mm.gather(run.ctx, table, s.ids.ptr, 512, s.hidden.ptr)
    want = np.zeros((513, columns), np.float32)
    oracle.gather(gtype, stored, rows, columns, ids, want)
    _check(s.read(), want, "large table")
    s.free()
    table.free()


def test_gather_positions(oracle, run):
    """gather.wgsl:65-84: patch row r is the column row r % columns plus the
    row row positions + r / columns of one F32 table."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    positions, columns, grid, tokens = 16, 256, 12, 12 * 16
    table_f = np.random.default_rng(4).standard_normal((2 * positions, columns)).astype(np.float32)
    table = run.weight(F32, 2 * positions, columns, table_f.tobytes())
    out = hx.Buffer.of(np.zeros((tokens, columns), np.float32))
    mm.gather_positions(run.ctx, table, positions, grid, tokens, out.ptr)
    hx.sync()
    got = out.read(np.float32).reshape(tokens, columns)
    _check(got, oracle.gather_positions(table_f, columns, positions, grid, tokens), "positions")
    out.free()
    table.free()


def test_gather_refusals(run):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    t = _table(F32)
    table = run.weight(F32, t.rows, t.columns, t.data)
    s = _Step([1, 2], t.columns)
    with pytest.raises(mm.MatmulError) as e:
        mm.gather(run.ctx, table, s.ids.ptr, 2, s.hidden.ptr + 4)
    assert e.value.status == mm.Status.INVALID_ARGUMENT and "aligned" in str(e.value)
    with pytest.raises(mm.MatmulError) as e:
        mm.gather(run.ctx, table, s.ids.ptr, 0, s.hidden.ptr)
    assert e.value.status == mm.Status.INVALID_ARGUMENT
    with pytest.raises(mm.MatmulError) as e:
        mm.gather(run.ctx, table, 0, 2, s.hidden.ptr)
    assert e.value.status == mm.Status.INVALID_ARGUMENT and "identifiers" in str(e.value)
    q = _table(Q4_0)
    qt = run.weight(Q4_0, q.rows, q.columns, q.data)
    with pytest.raises(mm.MatmulError) as e:
        mm.gather_positions(run.ctx, qt, 3, 2, 4, s.hidden.ptr)
    assert e.value.status == mm.Status.UNSUPPORTED_TYPE
    with pytest.raises(mm.MatmulError) as e:
        mm.gather_positions(run.ctx, table, 4, 2, 8, s.hidden.ptr)  # 7 rows are not 2 x 4
    assert e.value.status == mm.Status.INVALID_ARGUMENT
    hx.sync()
    s.free()
    qt.free()
    table.free()
