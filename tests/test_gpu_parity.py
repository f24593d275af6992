"""The HIP path on the GPU against the CPU oracle, through the C ABI.

Follows the reference's own GPU tests:
  tests/gpu/unpack_q4_0_test.cpp, unpack_q6_k_test.cpp — unpack bit for bit;
  tests/gpu/matmul_test.cpp:217-267 — each format's product decoded and
    prefilled at steps of 2, 8, 9, 16, 17, 33 and 64 tokens, within gamma(2K)
    of f64, and a token's outputs the same bits decoded alone and prefilled;
  matmul_test.cpp:289-299 — the head's last token; 301-344 — QKV.
Beyond them, every output is held to the CPU restatement of the reference's
order of addition bit for bit, and the BASELINE shapes run at full size.
Inputs are the reference tests' fill (fill.h:24-29, seed 7, amplitude 1) or
seeded N(0,1).
"""

import os

import numpy as np
import pytest

from tests.support import blocks as B
from tests.support.oracle_lib import Q4_0, Q6_K

pytestmark = pytest.mark.gpu

TOKENS = 64
WIDEST = 3072
THREADS = max(1, min(16, os.cpu_count() or 1))


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
    return oracle.fill(7, TOKENS * WIDEST)


def _rows_of(source, columns, tokens, first=0):
    return source[first * columns : (first + tokens) * columns].reshape(tokens, columns)


# ---- unpack, bit for bit ------------------------------------------------------


@pytest.mark.parametrize("gtype,count", [(Q4_0, 1), (Q4_0, 9), (Q4_0, 257), (Q6_K, 1), (Q6_K, 9), (Q6_K, 33)])
def test_unpack_decodes_every_block_as_ggml_does(oracle, gtype, count):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    stored = B.q4_0_edge_blocks(count) if gtype == Q4_0 else B.q6_k_edge_blocks(count)
    piece = np.frombuffer(mm.lay_out(gtype, stored, count), np.uint8)
    groups = count if gtype == Q4_0 else 8 * count
    # The piece 16 bytes into its allocation, after bytes no unpack may read
    # (unpack.h:68-86 places it 7 words in; the kernels need 16-byte alignment).
    buf = hx.Buffer(16 + piece.size)
    buf.write(np.full(16, 0xA5, np.uint8))
    buf.write(piece, offset=16)
    out = hx.Buffer(groups * 32 * 4)
    hx.unpack(gtype, buf.ptr + 16, count, groups, out.ptr)
    hx.sync()
    got = out.read(np.float32)
    want = oracle.dequantize(gtype, stored)
    same = (got.view(np.uint32) == want.view(np.uint32)) | ((got == 0) & (want == 0))
    assert same.all(), f"{int((~same).sum())} weights differ"
    buf.free()
    out.free()


# ---- the fixture's products (matmul_test.cpp:217-267) ----------------------


# Every weight of the reference's own product test (matmul_test.cpp:226-227),
# w_f32 among them.
FIXTURE = ["w_q4_0", "w_q6_k", "w_set2", "w_set3", "w_set4", "qkv_q", "ffn_gate", "w_f32", "w_q8_0", "w_q4_1_1152",
           "w_q4_1_3072"]
STEPS = [2, 8, 9, 16, 17, 33, 64]
ALONE = [0, 1, 7, 8, 15, 16, 32, 63]


@pytest.mark.parametrize("name", FIXTURE)
def test_fixture_product_decoded_and_prefilled(oracle, run, source, fixture_tensors, name):
    from tests.support.gpu import bits_equal, first_difference

    t = fixture_tensors[name]
    w = run.weight(t.type, t.rows, t.columns, t.data)
    x = _rows_of(source, t.columns, TOKENS)
    want = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x, threads=8)
    y64, bound = oracle.matmul_f64(t.type, t.data, t.rows, t.columns, x)
    assert (np.abs(want.astype(np.float64) - y64) <= bound).all()
    prefilled = {}
    for tokens in STEPS:
        got = run.write(w, x, tokens)
        assert bits_equal(got, want[:tokens]), f"{name} tokens={tokens}: {first_difference(got, want[:tokens])}"
        assert (np.abs(got.astype(np.float64) - y64[:tokens]) <= bound[:tokens]).all()
        prefilled[tokens] = got
    for t_ in ALONE:
        alone = run.write(w, x[t_ : t_ + 1], 1)
        assert bits_equal(alone[0], want[t_]), f"{name} token {t_} decoded: {first_difference(alone[0], want[t_])}"
        for tokens, got in prefilled.items():
            if t_ < tokens:
                assert bits_equal(alone[0], got[t_])
    w.free()


def test_head_covers_the_last_token_alone(oracle, run, source, fixture_tensors):
    from charlotte_amd import matmul as mm
    from tests.support.gpu import bits_equal

    t = fixture_tensors["w_q6_k"]
    w = run.weight(t.type, t.rows, t.columns, t.data)
    x = _rows_of(source, t.columns, 5)
    last = run.write(w, x, 5, rows=mm.Rows.LastToken)
    alone = run.write(w, x[4:5], 1)
    assert last.shape == (1, t.rows) and bits_equal(last, alone)
    assert bits_equal(last[0], oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x[4:5])[0])
    w.free()


def test_qkv_lands_in_three_buffers(oracle, run, source, fixture_tensors):
    from charlotte_amd import matmul as mm
    from tests.support.gpu import bits_equal

    names = ["qkv_q", "qkv_k", "qkv_v"]
    ts = [fixture_tensors[n] for n in names]
    ws = [run.weight(t.type, t.rows, t.columns, t.data) for t in ts]
    x = _rows_of(source, 1024, 33)
    members = [mm.Member(w) for w in ws]
    for tokens in (1, 5, 12, 33):
        got = run.product(members, x, tokens, [t.rows for t in ts], epilogue=mm.Epilogue.QKV)
        for t, g in zip(ts, got):
            want = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x[:tokens])
            assert bits_equal(g, want), (t.name, tokens)
    for w in ws:
        w.free()


def test_a_weight_in_pieces_writes_its_rows(oracle, run, source, fixture_tensors):
    # matmul_test.cpp:272-287: w_q4_0 as pieces of rows 0..71 and 72..139,
    # each its own weight, each writing its rows of the one output.
    from charlotte_amd import matmul as mm
    from tests.support.gpu import bits_equal

    t = fixture_tensors["w_q4_0"]
    row_bytes = len(t.data) // t.rows
    whole = run.weight(t.type, t.rows, t.columns, t.data)
    parts = [(0, 72), (72, 68)]
    pieces = [run.weight(t.type, n, t.columns, t.data[f * row_bytes : (f + n) * row_bytes]) for f, n in parts]
    x = _rows_of(source, 1024, 33)
    for tokens in (1, 33):
        want = run.write(whole, x, tokens)
        from charlotte_amd import harness as hx

        xb, yb = hx.Buffer.of(x), hx.Buffer(tokens * t.rows * 4)
        for (f, n), p in zip(parts, pieces):
            mm.launch(run.ctx, mm.MatmulLaunch([mm.Member(p, output_row=f)], xb.ptr, [yb.ptr], out_width=t.rows), tokens)
        hx.sync()
        got = yb.read(np.float32).reshape(tokens, t.rows)
        assert bits_equal(got, want)
        xb.free()
        yb.free()
    for w in [whole, *pieces]:
        w.free()


@pytest.mark.parametrize("rows", [2, 18, 130])
def test_q6_k_1152_small_pieces(oracle, run, rows):
    # K = 1,152 (Gemma 3): rows straddle super-blocks; small pieces put the
    # last rows' windows against the piece's end.
    from charlotte_amd import synthetic
    from tests.support.gpu import bits_equal, first_difference

    rng = np.random.default_rng(rows)
    stored = synthetic.q6_k(rng, rows, 1152)
    x = synthetic.activations(rng, 3, 1152)
    w = run.weight(Q6_K, rows, 1152, stored)
    for tokens in (1, 3):
        got = run.write(w, x, tokens)
        want = oracle.matmul_f32(Q6_K, stored, rows, 1152, x[:tokens])
        assert bits_equal(got, want), first_difference(got, want)
    last = run.write(w, x, 3, rows=__import__("charlotte_amd.matmul", fromlist=["Rows"]).Rows.LastToken)
    assert bits_equal(last[0], oracle.matmul_f32(Q6_K, stored, rows, 1152, x[2:3])[0])
    w.free()


# ---- BASELINE shapes at full size ------------------------------------------


def _tolerance_and_argmax(got, y64):
    err = np.abs(got.astype(np.float64) - y64).max()
    assert err / np.abs(y64).max() <= 1e-5
    assert (np.argmax(got, axis=-1) == np.argmax(y64, axis=-1)).all()


def test_c1_q4_0_decode_3072x1024(oracle, run):
    from charlotte_amd import synthetic
    from tests.support.gpu import bits_equal, first_difference

    rng = np.random.default_rng(1)
    stored = synthetic.q4_0(rng, 3072, 1024)
    x = synthetic.activations(rng, 1, 1024)
    w = run.weight(Q4_0, 3072, 1024, stored)
    got = run.write(w, x, 1)
    want = oracle.matmul_f32(Q4_0, stored, 3072, 1024, x, threads=8)
    assert bits_equal(got, want), first_difference(got, want)
    y64, _ = oracle.matmul_f64(Q4_0, stored, 3072, 1024, x)
    _tolerance_and_argmax(got, y64)
    w.free()


def test_c2_in_two_pieces_is_the_whole_weights_bits(run):
    """C2's head as two pieces (the 128 MiB binding splits it, plan.cpp:294-306),
    one launch a piece writing its rows of the one output (matmul.cpp:283-291):
    the pieces' rows are not whole 16-row steps, so they take the L = 4
    decode, and must give the streamed whole weight's bits."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic
    from tests.support.gpu import bits_equal, first_difference

    rng = np.random.default_rng(12)
    rows, columns = 262144, 1152
    stored = synthetic.q6_k(rng, rows, columns)
    x = synthetic.activations(rng, 1, columns)
    whole = run.weight(Q6_K, rows, columns, stored)
    want = run.write(whole, x, 1)
    whole.free()
    parts = [(0, 142030), (142030, rows - 142030)]  # even rows: whole super-blocks
    pieces = [run.weight(Q6_K, n, columns, stored[f * 945 : (f + n) * 945]) for f, n in parts]
    xb, yb = hx.Buffer.of(x), hx.Buffer(rows * 4)
    for (f, n), p in zip(parts, pieces):
        mm.launch(run.ctx, mm.MatmulLaunch([mm.Member(p, output_row=f)], xb.ptr, [yb.ptr], out_width=rows), 1)
    hx.sync()
    got = yb.read(np.float32).reshape(1, rows)
    for b in [xb, yb, *pieces]:
        b.free()
    assert bits_equal(got, want), first_difference(got, want)


def test_c2_q6_k_lm_head_262144x1152(oracle, run):
    from charlotte_amd import synthetic
    from tests.support.gpu import bits_equal, first_difference

    rng = np.random.default_rng(2)
    rows, columns = 262144, 1152
    stored = synthetic.q6_k(rng, rows, columns)
    x = synthetic.activations(rng, 1, columns)
    w = run.weight(Q6_K, rows, columns, stored)
    got = run.write(w, x, 1)
    want = oracle.matmul_f32(Q6_K, stored, rows, columns, x, threads=16)
    assert bits_equal(got, want), first_difference(got, want)
    # f64 on a sample of rows (whole super-blocks: 2 rows are 9 of them)
    for r0 in (0, 131072, rows - 256):
        part = stored[r0 * 945 : (r0 + 256) * 945]
        y64, bound = oracle.matmul_f64(Q6_K, part, 256, columns, x)
        assert (np.abs(got[:, r0 : r0 + 256].astype(np.float64) - y64) <= bound).all()
    w.free()


def test_c4_q4_0_prefill_512x8192x2048(oracle, run):
    """C4 in full: every output the oracle's bits; f64 and the argmax on 64
    sampled token rows over every output row."""
    from charlotte_amd import synthetic
    from tests.support.gpu import bits_equal, first_difference

    rng = np.random.default_rng(4)
    tokens, rows, columns = 512, 8192, 2048
    stored = synthetic.q4_0(rng, rows, columns)
    x = synthetic.activations(rng, tokens, columns)
    w = run.weight(Q4_0, rows, columns, stored)
    got = run.write(w, x, tokens)
    want = oracle.matmul_f32(Q4_0, stored, rows, columns, x, threads=THREADS)
    assert bits_equal(got, want), first_difference(got, want)
    sample = np.sort(np.random.default_rng(40).choice(tokens, 64, replace=False))
    y64, _ = oracle.matmul_f64(Q4_0, stored, rows, columns, x[sample], threads=THREADS)
    _tolerance_and_argmax(got[sample], y64)
    # decode-vs-prefill: the same bits for the same token
    for t_ in (0, 255, 511):
        alone = run.write(w, x[t_ : t_ + 1], 1)
        assert bits_equal(alone[0], got[t_])
    w.free()


def test_c5_layer_products_at_2048_tokens(oracle, run):
    """One Llama 3.2 1B layer at C5's step of 2,048 tokens: QKV (three members,
    2048 + 512 + 512 rows), o (2048 x 2048), gate/up (gated, SiLU, 8192 rows
    each) and down (2048 x 8192), each the oracle's bits on 64 sampled token
    rows over every output row; and the Q6_K head (128,256 x 2,048) on the
    step's last token, in full."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic
    from tests.support.gpu import bits_equal, first_difference

    rng = np.random.default_rng(5)
    tokens, hidden, ffn = 2048, 2048, 8192
    sample = np.sort(np.random.default_rng(50).choice(tokens, 64, replace=False))

    def weight(rows, columns, gtype=Q4_0):
        stored = synthetic.weight(rng, gtype, rows, columns)
        return stored, run.weight(gtype, rows, columns, stored)

    x = synthetic.activations(rng, tokens, hidden)
    qkv = [weight(r, hidden) for r in (2048, 512, 512)]
    got = run.product([mm.Member(w) for _, w in qkv], x, tokens, [2048, 512, 512], epilogue=mm.Epilogue.QKV)
    for (stored, w), g, r in zip(qkv, got, (2048, 512, 512)):
        want = oracle.matmul_f32(Q4_0, stored, r, hidden, x[sample], threads=THREADS)
        assert bits_equal(g[sample], want), first_difference(g[sample], want)
        w.free()
    o_stored, o = weight(hidden, hidden)
    got = run.write(o, x, tokens)
    want = oracle.matmul_f32(Q4_0, o_stored, hidden, hidden, x[sample], threads=THREADS)
    assert bits_equal(got[sample], want), first_difference(got[sample], want)
    o.free()
    (g_stored, gate), (u_stored, up) = weight(ffn, hidden), weight(ffn, hidden)
    got = run.product([mm.Member(gate), mm.Member(up)], x, tokens, [ffn], epilogue=mm.Epilogue.GatedActivation,
                      activation=mm.Activation.SiLU)[0]
    want = oracle.gated(oracle.matmul_f32(Q4_0, g_stored, ffn, hidden, x[sample], threads=THREADS),
                        oracle.matmul_f32(Q4_0, u_stored, ffn, hidden, x[sample], threads=THREADS), activation=0)
    assert bits_equal(got[sample], want), first_difference(got[sample], want)
    gate.free()
    up.free()
    xd = synthetic.activations(rng, tokens, ffn)
    d_stored, down = weight(hidden, ffn)
    got = run.write(down, xd, tokens)
    want = oracle.matmul_f32(Q4_0, d_stored, hidden, ffn, xd[sample], threads=THREADS)
    assert bits_equal(got[sample], want), first_difference(got[sample], want)
    down.free()
    h_stored, head = weight(128256, hidden, Q6_K)
    got = run.write(head, x, tokens, rows=mm.Rows.LastToken)
    want = oracle.matmul_f32(Q6_K, h_stored, 128256, hidden, x[tokens - 1 :], threads=THREADS)
    assert bits_equal(got, want), first_difference(got, want)
    head.free()


# ---- errors the host turns away --------------------------------------------


def test_errors_are_statuses_with_messages(run, fixture_tensors):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    t = fixture_tensors["w_q4_0"]
    with pytest.raises(mm.MatmulError) as e:
        mm.Weight(run.ctx, 6, t.rows, t.columns, t.data)  # Q5_0: no kernels
    assert e.value.status == mm.Status.UNSUPPORTED_TYPE
    with pytest.raises(mm.MatmulError) as e:
        mm.Weight(run.ctx, Q4_0, 18, 1000, bytes(18 * 1000 // 32 * 18))
    assert e.value.status == mm.Status.SHAPE_NOT_GROUPS
    w = run.weight(t.type, t.rows, t.columns, t.data)
    xb, yb = hx.Buffer(4 * 1024 * 2 + 16), hx.Buffer(4 * t.rows * 2)
    with pytest.raises(mm.MatmulError) as e:
        mm.launch(run.ctx, mm.MatmulLaunch([mm.Member(w)], xb.ptr + 4, [yb.ptr]), 1)
    assert e.value.status == mm.Status.INVALID_ARGUMENT and "aligned" in str(e.value)
    with pytest.raises(mm.MatmulError) as e:
        mm.launch(run.ctx, mm.MatmulLaunch([mm.Member(w, row_offset=100, rows=41)], xb.ptr, [yb.ptr]), 1)
    assert e.value.status == mm.Status.INVALID_ARGUMENT and "past" in str(e.value)
    with pytest.raises(mm.MatmulError) as e:
        mm.launch(run.ctx, mm.MatmulLaunch([mm.Member(w)], xb.ptr, [yb.ptr]), 0)
    assert e.value.status == mm.Status.INVALID_ARGUMENT
    hx.sync()
    xb.free()
    yb.free()
    w.free()


# ---- Q6_K at K = 1,152 in whole 16-row steps (the streamed decode) ------------


@pytest.mark.parametrize("rows", [16, 48, 1024, 4096])
def test_q6_k_1152_streamed_steps(oracle, run, rows):
    """Rows a multiple of 16 take the LDS-streamed decode: the same bits as
    the oracle, decoded alone and as the head's last token."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic
    from tests.support.gpu import bits_equal, first_difference

    rng = np.random.default_rng(rows)
    stored = synthetic.q6_k(rng, rows, 1152)
    x = synthetic.activations(rng, 3, 1152)
    w = run.weight(Q6_K, rows, 1152, stored)
    want = oracle.matmul_f32(Q6_K, stored, rows, 1152, x, threads=8)
    got = run.write(w, x[:1], 1)
    assert bits_equal(got[0], want[0]), first_difference(got[0], want[0])
    last = run.write(w, x, 3, rows=mm.Rows.LastToken)
    assert bits_equal(last[0], want[2]), first_difference(last[0], want[2])
    w.free()


def test_q6_k_1152_streamed_members_and_epilogues(oracle, run):
    """QKV of three K = 1,152 weights, members at row offsets, GatedByInput and
    a Write with every option, all through the streamed decode."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic
    from tests.support.gpu import bits_equal, first_difference

    rng = np.random.default_rng(1152)
    sizes = [1024, 256, 256]
    stored = [synthetic.q6_k(rng, r, 1152) for r in sizes]
    x = synthetic.activations(rng, 1, 1152)
    ws = [run.weight(Q6_K, r, 1152, s) for r, s in zip(sizes, stored)]
    want = [oracle.matmul_f32(Q6_K, s, r, 1152, x) for r, s in zip(sizes, stored)]
    got = run.product([mm.Member(w) for w in ws], x, 1, sizes, epilogue=mm.Epilogue.QKV)
    for i in range(3):
        assert bits_equal(got[i], want[i]), f"member {i}: {first_difference(got[i], want[i])}"
    # Rows 32 .. 543 of the first weight, then rows 16 .. 111 of the second, at output rows 0 and 512.
    members = [mm.Member(ws[0], row_offset=32, rows=512), mm.Member(ws[1], row_offset=16, rows=96, output_row=512)]
    got = run.product(members, x, 1, [608])[0]
    expect = np.concatenate([want[0][:, 32:544], want[1][:, 16:112]], axis=1)
    assert bits_equal(got, expect), first_difference(got, expect)
    u = np.random.default_rng(7).standard_normal((1, 1024), dtype=np.float32)
    got = run.product([mm.Member(ws[0])], x, 1, [1024], epilogue=mm.Epilogue.GatedByInput, gate_input=u,
                      gate_input_stride=1024, activation=mm.Activation.GeluTanh)[0]
    expect = oracle.gated_by_input(want[0], u, activation=1)
    assert bits_equal(got, expect), first_difference(got, expect)
    clip = np.array([-1.0, 1.25, -0.02, 0.03], np.float32)
    bias = np.linspace(-0.01, 0.01, 1024, dtype=np.float32)
    got = run.product([mm.Member(ws[0])], x, 1, [1024], clip=clip, bias=bias, activated=True,
                      activation=mm.Activation.SiLU)[0]
    totals = oracle.matmul_f32(Q6_K, stored[0], 1024, 1152, oracle.clamp(x, clip[0], clip[1]))
    expect = oracle.finish(totals, clip=clip, bias=bias, activated=True, activation=0)
    assert bits_equal(got, expect), first_difference(got, expect)
    for w in ws:
        w.free()


# ---- weights read from a GGUF file ----------------------------------------------


def test_weights_uploaded_from_a_gguf_file(oracle, run, source, fixture_tensors):
    """The reference fixture's tensors, read and laid out by the library from
    the file itself, give the oracle's bits."""
    import os

    from charlotte_amd import matmul as mm
    from tests.support.gpu import bits_equal, first_difference

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "matmul_rows.gguf")
    with mm.GgufFile(path) as f:
        for name in ("w_q4_0", "w_q6_k", "qkv_q", "ffn_gate", "w_q4_1_1152", "w_q8_0", "w_f32"):
            t = fixture_tensors[name]
            w = f.upload(run.ctx, name)
            x = _rows_of(source, t.columns, 9)
            want = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x)
            for tokens in (1, 9):
                got = run.write(w, x, tokens)
                assert bits_equal(got, want[:tokens]), f"{name} tokens={tokens}: {first_difference(got, want[:tokens])}"
            w.free()
