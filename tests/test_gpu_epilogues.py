"""The fused epilogues, the options and the split along K, on the GPU, against
the CPU oracle bit for bit.

Follows the reference's own tests of these launches:
  tests/gpu/matmul_test.cpp:346-435 — the gated feed-forward (gate and up
    fused, SiLU and GELU), a GLU over one weight's halves, GatedByInput;
  matmul_test.cpp:437-514 — the split along K the same bits as the tiled
    form, at K = 64 (30 empty ranges) and K = 1,152 (unequal ranges);
  tests/kernels_matmul_test.cpp — a product with options never splits.
Expected values: the oracle's reference-order f32 totals (over the input
clamped as the product reads it), through the oracle's epilogue.
"""

import numpy as np
import pytest

from tests.support.oracle_lib import Q4_0, Q6_K

pytestmark = pytest.mark.gpu

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


def _data(gtype, rows, columns, tokens, seed):
    from charlotte_amd import synthetic

    rng = np.random.default_rng(seed)
    return synthetic.weight(rng, gtype, rows, columns), synthetic.activations(rng, tokens, columns)


def _check(got, want, what):
    from tests.support.gpu import bits_equal, first_difference

    assert bits_equal(got, want), f"{what}: {first_difference(got, want)}"


# ---- GatedActivation (matmul.wgsl:318-345, 556-573) --------------------------


@pytest.mark.parametrize("gtype,columns", [(Q4_0, 1024), (Q4_0, 3072), (Q6_K, 1152), (Q4_0, 8192), (Q4_0, 64)])
@pytest.mark.parametrize("activation", [SILU, GELU, SIGMOID])
def test_gated_activation_decode_and_prefill(oracle, run, gtype, columns, activation):
    from charlotte_amd import matmul as mm

    width = 200
    gate_s, x = _data(gtype, width, columns, 40, seed=columns + activation)
    up_s, _ = _data(gtype, width, columns, 1, seed=columns + activation + 99)
    gate = run.weight(gtype, width, columns, gate_s)
    up = run.weight(gtype, width, columns, up_s)
    g = oracle.matmul_f32(gtype, gate_s, width, columns, x, threads=8)
    u = oracle.matmul_f32(gtype, up_s, width, columns, x, threads=8)
    want = oracle.gated(g, u, activation=activation)
    for tokens in (1, 7, 33, 40):
        got = run.product([mm.Member(gate), mm.Member(up)], x, tokens, [width], epilogue=mm.Epilogue.GatedActivation,
                          activation=activation)[0]
        _check(got, want[:tokens], f"gated K={columns} act={activation} tokens={tokens}")
    gate.free()
    up.free()


def test_gated_glu_over_one_weights_halves_clipped_and_wide(oracle, run):
    """A GLU over one weight (matmul.h:630-631): up its first half of rows, the
    gate its second; clipped input and outputs; a wider output row."""
    from charlotte_amd import matmul as mm

    half, columns, tokens = 96, 1024, 20
    stored, x = _data(Q4_0, 2 * half, columns, tokens, seed=5)
    w = run.weight(Q4_0, 2 * half, columns, stored)
    clip = np.array([-1.5, 1.25, -0.75, 0.5], np.float32)
    xc = oracle.clamp(x, clip[0], clip[1])
    both = oracle.matmul_f32(Q4_0, stored, 2 * half, columns, xc, threads=8)
    want = oracle.gated(both[:, half:], both[:, :half], clip=clip, activation=SILU)
    members = [mm.Member(w, row_offset=half, rows=half), mm.Member(w, row_offset=0, rows=half)]
    for t in (1, tokens):
        got = run.product(members, x, t, [128], epilogue=mm.Epilogue.GatedActivation, out_width=128, clip=clip)[0]
        _check(got[:, :half], want[:t], f"GLU tokens={t}")
        assert np.isnan(got[:, half:]).all(), "a gated product wrote past its width"
    w.free()


def test_gated_wide_tiles(oracle, run):
    """Enough tiles for the 128-token prefill tile, sampled tokens checked."""
    from charlotte_amd import matmul as mm

    width, columns, tokens = 4096, 1024, 1024
    gate_s, x = _data(Q4_0, width, columns, tokens, seed=11)
    up_s, _ = _data(Q4_0, width, columns, 1, seed=12)
    gate, up = run.weight(Q4_0, width, columns, gate_s), run.weight(Q4_0, width, columns, up_s)
    got = run.product([mm.Member(gate), mm.Member(up)], x, tokens, [width], epilogue=mm.Epilogue.GatedActivation,
                      activation=GELU)[0]
    rows = np.random.default_rng(3).choice(tokens, 48, replace=False)
    g = oracle.matmul_f32(Q4_0, gate_s, width, columns, x[rows], threads=8)
    u = oracle.matmul_f32(Q4_0, up_s, width, columns, x[rows], threads=8)
    _check(got[rows], oracle.gated(g, u, activation=GELU), "gated wide")
    gate.free()
    up.free()


# ---- GatedByInput (matmul.wgsl:347-364, 575-590) -----------------------------


# 300 rows: the ranges and L = 4 decodes; 304 (whole 16-row steps): the
# LDS-streamed Q6_K decodes at K = 1,152, 1,024 and 2,048, and the streamed
# Q4_0 decode at K = 2,048 and 8,192.
@pytest.mark.parametrize("gtype,columns,rows", [(Q4_0, 2048, 300), (Q6_K, 1152, 300), (Q6_K, 1152, 304),
                                                (Q6_K, 1024, 304), (Q6_K, 2048, 304), (Q4_0, 2048, 304),
                                                (Q4_0, 8192, 304)])
def test_gated_by_input(oracle, run, gtype, columns, rows):
    from charlotte_amd import matmul as mm

    tokens, stride, column = 40, 337, 17
    stored, x = _data(gtype, rows, columns, tokens, seed=21)
    w = run.weight(gtype, rows, columns, stored)
    u = np.random.default_rng(22).standard_normal((tokens, stride), dtype=np.float32)
    totals = oracle.matmul_f32(gtype, stored, rows, columns, x, threads=8)
    want = oracle.gated_by_input(totals, u[:, column : column + rows], activation=GELU)
    kw = dict(epilogue=mm.Epilogue.GatedByInput, activation=GELU, gate_input=u, gate_input_stride=stride,
              gate_input_column=column)
    for t in (1, 9, tokens):
        got = run.product([mm.Member(w)], x, t, [rows], **kw)[0]
        _check(got, want[:t], f"GatedByInput tokens={t}")
    # The head's form: the last token's input row and its u row.
    got = run.product([mm.Member(w)], x, 5, [rows], rows=mm.Rows.LastToken, **kw)[0]
    _check(got[0], want[4], "GatedByInput last token")
    w.free()


# ---- a Write's options: clip, bias, activated (matmul.wgsl:117-132, 272-284) --


@pytest.mark.parametrize("gtype,columns", [(Q4_0, 1024), (Q6_K, 1152), (Q4_0, 4096)])
@pytest.mark.parametrize("options", ["clip", "bias", "activated", "all"])
def test_write_options(oracle, run, gtype, columns, options):
    from charlotte_amd import matmul as mm

    rows, tokens = 264, 36
    stored, x = _data(gtype, rows, columns, tokens, seed=31)
    w = run.weight(gtype, rows, columns, stored)
    clip = np.array([-1.0, 0.75, -0.125, 0.25], np.float32) if options in ("clip", "all") else None
    bias = np.random.default_rng(32).standard_normal(rows, dtype=np.float32) * 0.1 if options in ("bias", "all") else None
    activated = options in ("activated", "all")
    xc = x if clip is None else oracle.clamp(x, clip[0], clip[1])
    totals = oracle.matmul_f32(gtype, stored, rows, columns, xc, threads=8)
    want = oracle.finish(totals, clip=clip, bias=bias, activated=activated, activation=SIGMOID)
    for t in (1, 2, tokens):
        got = run.product([mm.Member(w)], x, t, [rows], clip=clip, bias=bias, activated=activated,
                          activation=SIGMOID)[0]
        _check(got, want[:t], f"Write {options} tokens={t}")
    w.free()


# ---- split along K (matmul.wgsl:592-695, matmul_test.cpp:437-514) ------------


def _sums_bytes(tokens, rows):
    return tokens * rows * 32 * 4


@pytest.mark.parametrize("gtype,columns", [(Q4_0, 64), (Q4_0, 1024), (Q6_K, 1152), (Q4_0, 3072)])
def test_split_is_the_tiled_bits(oracle, run, gtype, columns):
    from charlotte_amd import matmul as mm

    rows, tokens = 320, 64
    stored, x = _data(gtype, rows, columns, tokens, seed=41 + columns)
    w = run.weight(gtype, rows, columns, stored)
    want = oracle.matmul_f32(gtype, stored, rows, columns, x, threads=8)
    for t in (2, 5, 32, 33, 64):
        split = run.write(w, x, t, gate=mm.kAlways, sums_bytes=_sums_bytes(t, rows))
        tiled = run.write(w, x, t)
        _check(split, want[:t], f"split K={columns} tokens={t}")
        _check(split, tiled, f"split vs tiled K={columns} tokens={t}")
    w.free()


def test_split_writes_range_sums_range_first(oracle, run):
    """The split form's range sums, [32][tokens][rows], add in order to the outputs."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    rows, columns, tokens = 130, 1152, 9
    stored, x = _data(Q6_K, rows, columns, tokens, seed=51)
    w = run.weight(Q6_K, rows, columns, stored)
    xb, out = hx.Buffer.of(x), hx.Buffer(tokens * rows * 4)
    sums = hx.Buffer(_sums_bytes(tokens, rows))
    sums.fill(0xFF)
    m = mm.MatmulLaunch([mm.Member(w)], xb.ptr, [out.ptr])
    mm.launch(run.ctx, m, tokens, mm.kAlways, sums.ptr, sums.nbytes)
    hx.sync()
    rs = sums.read(np.float32).reshape(32, tokens, rows)
    y = out.read(np.float32).reshape(tokens, rows)
    assert not np.isnan(rs).any()  # G = 36: every range holds a group
    total = np.zeros((tokens, rows), np.float32)
    for r in range(32):
        total = total + rs[r]
    _check(total, y, "range sums added in order")
    _check(y, oracle.matmul_f32(Q6_K, stored, rows, columns, x), "split output")
    for b in (xb, out, sums):
        b.free()
    w.free()


def test_split_qkv_and_gated_by_input(oracle, run):
    from charlotte_amd import matmul as mm

    columns, tokens = 1024, 24
    widths = [128, 64, 64]
    rng_seeds = [61, 62, 63]
    data = [_data(Q4_0, r, columns, tokens, seed=s) for r, s in zip(widths, rng_seeds)]
    x = data[0][1]
    ws = [run.weight(Q4_0, r, columns, d[0]) for r, d in zip(widths, data)]
    rows = sum(widths)
    got = run.product([mm.Member(w) for w in ws], x, tokens, widths, epilogue=mm.Epilogue.QKV, gate=mm.kAlways,
                      sums_bytes=_sums_bytes(tokens, rows))
    for i, (r, d) in enumerate(zip(widths, data)):
        _check(got[i], oracle.matmul_f32(Q4_0, d[0], r, columns, x), f"split QKV member {i}")
    u = np.random.default_rng(64).standard_normal((tokens, 128), dtype=np.float32)
    got = run.product([mm.Member(ws[0])], x, tokens, [128], epilogue=mm.Epilogue.GatedByInput, activation=SILU,
                      gate_input=u, gate_input_stride=128, gate=mm.kAlways, sums_bytes=_sums_bytes(tokens, 128))[0]
    want = oracle.gated_by_input(oracle.matmul_f32(Q4_0, data[0][0], 128, columns, x), u, activation=SILU)
    _check(got, want, "split GatedByInput")
    for w in ws:
        w.free()


def test_split_only_while_range_sums_fit_and_never_with_options(oracle, run):
    from charlotte_amd import matmul as mm

    rows, columns, tokens = 200, 1024, 16
    stored, x = _data(Q4_0, rows, columns, tokens, seed=71)
    w = run.weight(Q4_0, rows, columns, stored)
    want = oracle.matmul_f32(Q4_0, stored, rows, columns, x)
    # Room for 8 tokens' sums: a 16-token step runs tiled, the same bits.
    _check(run.write(w, x, tokens, gate=mm.kAlways, sums_bytes=_sums_bytes(8, rows)), want, "split too small")
    _check(run.write(w, x, 8, gate=mm.kAlways, sums_bytes=_sums_bytes(8, rows)), want[:8], "split fits")
    bias = np.linspace(-1, 1, rows, dtype=np.float32)
    got = run.product([mm.Member(w)], x, tokens, [rows], gate=mm.kAlways, sums_bytes=_sums_bytes(tokens, rows),
                      bias=bias)[0]
    _check(got, oracle.finish(want, bias=bias), "options never split")
    w.free()


def test_write_of_several_pieces_in_one_launch(oracle, run):
    """A weight in pieces as the members of one Write, each at its output row."""
    from charlotte_amd import matmul as mm

    columns, tokens = 1152, 3
    sizes = [72, 68, 60]
    data = [_data(Q6_K, r, columns, tokens, seed=80 + i) for i, r in enumerate(sizes)]
    x = data[0][1]
    ws = [run.weight(Q6_K, r, columns, d[0]) for r, d in zip(sizes, data)]
    firsts = np.cumsum([0] + sizes[:-1])
    members = [mm.Member(w, output_row=int(f)) for w, f in zip(ws, firsts)]
    want = np.concatenate([oracle.matmul_f32(Q6_K, d[0], r, columns, x) for r, d in zip(sizes, data)], axis=1)
    for t in (1, tokens):
        got = run.product(members, x, t, [sum(sizes)])[0]
        _check(got, want[:t], f"pieces tokens={t}")
    for w in ws:
        w.free()


def test_epilogue_argument_errors(run, fixture_tensors):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    t = fixture_tensors["w_q4_0"]
    w = run.weight(t.type, t.rows, t.columns, t.data)
    xb, out = hx.Buffer(4 * t.columns), hx.Buffer(4 * t.rows)
    bad = [
        (dict(members=[mm.Member(w)], epilogue=mm.Epilogue.GatedActivation), "two members"),
        (dict(members=[mm.Member(w, rows=8), mm.Member(w, rows=9)], epilogue=mm.Epilogue.GatedActivation), "rows differ"),
        (dict(members=[mm.Member(w)], epilogue=mm.Epilogue.GatedByInput), "without its input"),
        (dict(members=[mm.Member(w)], epilogue=mm.Epilogue.QKV, bias=xb.ptr), "Write's options"),
        (dict(members=[mm.Member(w)], epilogue=mm.Epilogue.GatedByInput, gate_input=xb.ptr, clip=[xb.ptr] * 4), "clip"),
    ]
    for kw, words in bad:
        m = mm.MatmulLaunch(input=xb.ptr, outputs=[out.ptr], **kw)
        with pytest.raises(mm.MatmulError) as e:
            mm.launch(run.ctx, m, 1)
        assert e.value.status == mm.Status.INVALID_ARGUMENT and words in str(e.value)
    for b in (xb, out):
        b.free()
    w.free()


# ---- the reference fixture's gated and clipped products ----------------------


@pytest.fixture(scope="module")
def source(oracle):
    # matmul_test.cpp:141: source rows filled with seed 7, amplitude 1.0.
    return oracle.fill(7, 64 * 1024).reshape(64, 1024)


def _f32(t):
    return np.frombuffer(t.data, np.float32)


@pytest.mark.parametrize("activation", [SILU, GELU])
def test_fixture_gate_and_up(oracle, run, source, fixture_tensors, activation):
    """matmul_test.cpp:346-389: ffn_gate and ffn_up as one product, 33 tokens,
    tokens 0 and 32 alone and steps of 5 and 12 the same bits."""
    from charlotte_amd import matmul as mm

    g_t, u_t = fixture_tensors["ffn_gate"], fixture_tensors["ffn_up"]
    gate, up = run.weight(g_t.type, g_t.rows, 1024, g_t.data), run.weight(u_t.type, u_t.rows, 1024, u_t.data)
    x = source[:33]
    want = oracle.gated(oracle.matmul_f32(g_t.type, g_t.data, 72, 1024, x),
                        oracle.matmul_f32(u_t.type, u_t.data, 72, 1024, x), activation=activation)
    members = [mm.Member(gate), mm.Member(up)]
    kw = dict(epilogue=mm.Epilogue.GatedActivation, activation=activation)
    prefilled = run.product(members, x, 33, [72], **kw)[0]
    _check(prefilled, want, "fixture gated")
    for t in (0, 32):
        _check(run.product(members, x[t : t + 1], 1, [72], **kw)[0][0], want[t], f"alone {t}")
    for tokens in (5, 12):
        _check(run.product(members, x, tokens, [72], **kw)[0], want[:tokens], f"step {tokens}")
    gate.free()
    up.free()


def test_fixture_gated_by_input_reads_its_row_and_column(oracle, run, source, fixture_tensors):
    """matmul_test.cpp:391-435: u the source rows, stride 1,024, column 100."""
    from charlotte_amd import matmul as mm

    t = fixture_tensors["ffn_gate"]
    w = run.weight(t.type, t.rows, 1024, t.data)
    x = source[:33]
    want = oracle.gated_by_input(oracle.matmul_f32(t.type, t.data, 72, 1024, x), source[:33, 100:172], activation=GELU)
    kw = dict(epilogue=mm.Epilogue.GatedByInput, activation=GELU, gate_input=source, gate_input_stride=1024,
              gate_input_column=100)
    _check(run.product([mm.Member(w)], x, 33, [72], **kw)[0], want, "fixture GatedByInput")
    for t_ in (0, 32):
        # Alone, the step's one token reads u's row 0: pass its own row.
        alone = run.product([mm.Member(w)], x[t_ : t_ + 1], 1, [72], **{**kw, "gate_input": source[t_ : t_ + 1]})[0]
        _check(alone[0], want[t_], f"alone {t_}")
    w.free()


def test_fixture_clip_bounds(oracle, run, source, fixture_tensors):
    """matmul_test.cpp:552-620 with the fixture's bounds on w_q4_0: the bounds
    bind on both sides; bounds no value reaches give the plain product's bits."""
    from charlotte_amd import matmul as mm

    t = fixture_tensors["w_q4_0"]
    w = run.weight(t.type, t.rows, 1024, t.data)
    clip = np.array([_f32(fixture_tensors[f"clip_{k}"])[0] for k in ("in_min", "in_max", "out_min", "out_max")])
    wide = np.array([_f32(fixture_tensors[f"wide_{k}"])[0] for k in ("in_min", "in_max", "out_min", "out_max")])
    x = source[:33]
    xc = oracle.clamp(x, clip[0], clip[1])
    assert (xc != x).any()
    totals = oracle.matmul_f32(t.type, t.data, t.rows, 1024, xc)
    assert ((totals < clip[2]) | (totals > clip[3])).any()
    want = oracle.finish(totals, clip=clip, activated=True, activation=SILU)
    got = run.product([mm.Member(w)], x, 33, [t.rows], clip=clip, activated=True, activation=SILU)[0]
    _check(got, want, "clipped")
    alone = run.product([mm.Member(w)], x[7:8], 1, [t.rows], clip=clip, activated=True, activation=SILU)[0]
    _check(alone[0], want[7], "clipped alone")
    plain = oracle.matmul_f32(t.type, t.data, t.rows, 1024, source[:21])
    _check(run.product([mm.Member(w)], source[:21], 21, [t.rows], clip=wide)[0], plain, "wide bounds")
    w.free()
