"""The oracle's Q4_1, Q8_0 and F32 tables and its embedding gather, pinned
against the reference's own code (oracle/_ref), its tests' blocks and fixture
files, closed forms in numpy and an exhaustive check.

Follows tests/gpu/unpack_q4_1_test.cpp, unpack_q8_0_test.cpp and
gather_test.cpp of the reference.
"""

import math
import os

import numpy as np
import pytest

from tests.support import blocks as B
from tests.support import gguf_fixture
from tests.support.oracle_lib import BF16, BLOCK, F16, F32, Q4_0, Q4_1, Q6_K, Q8_0

HERE = os.path.dirname(os.path.abspath(__file__))
EMBEDDINGS = {F32: "embedding_f32", Q4_0: "embedding_q4_0", Q4_1: "embedding_q4_1", Q8_0: "embedding_q8_0",
              Q6_K: "embedding_q6_k"}


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _table(gtype):
    t = gguf_fixture.read(os.path.join(HERE, "golden", "gguf", EMBEDDINGS[gtype] + ".gguf"))["token_embd.weight"]
    assert t.type == gtype
    return t


# ---- Q4_1 (tests/support/q4_1_reference.h) ------------------------------------


@pytest.mark.parametrize("count", [1, 9, 257])
def test_q4_1_edge_blocks_match_numpy(oracle, count):
    stored = B.q4_1_edge_blocks(count)
    rounded, fused = oracle.dequantize_q4_1(stored)
    assert (_bits(rounded) == _bits(B.numpy_q4_1(stored))).all()
    assert (_bits(oracle.dequantize(Q4_1, stored)) == _bits(rounded)).all()
    if count >= 9:
        # unpack_q4_1_test.cpp:60-73: every edge is some block's d and some block's m.
        b = np.frombuffer(stored, np.uint8).reshape(-1, 20).astype(np.uint16)
        d, m = b[:, 0] | (b[:, 1] << 8), b[:, 2] | (b[:, 3] << 8)
        for edge in B.EDGE_SCALES:
            assert edge in d and edge in m


@pytest.mark.parametrize("count", [1, 9, 257])
def test_q4_1_both_answers_match_the_reference(oracle, reference, count):
    stored = B.q4_1_edge_blocks(count)
    r_o, f_o = oracle.dequantize_q4_1(stored)
    r_r, f_r = reference.dequantize_q4_1(stored)
    assert (_bits(r_o) == _bits(r_r)).all() and (_bits(f_o) == _bits(f_r)).all()


def test_q4_1_code_times_d_is_exact_so_rounded_equals_fused():
    """q (4 bits) times d (fp16, 11 significant bits) is exact in binary32 for
    every finite d: the one rounding left is the add, whichever way the
    multiply-add is evaluated. Exhaustive over all finite fp16 d and all q."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    d = h[(h & 0x7C00) != 0x7C00].view(np.float16).astype(np.float32)
    for q in range(16):
        p32 = (np.float32(q) * d).astype(np.float64)
        assert (p32 == np.float64(q) * d.astype(np.float64)).all(), q


def test_q4_1_weight_is_code_times_d_plus_m(oracle):
    # d = 0.5, m = -3: weight j = (j & 15 for the low, j >> 4 for the high) / 2 - 3.
    qs = bytes(range(0x00, 0x100, 0x11))  # byte j = j | j << 4
    block = bytes([0x00, 0x38, 0x00, 0xC2]) + qs
    w = oracle.dequantize(Q4_1, block)
    assert list(w[:16]) == [j * 0.5 - 3 for j in range(16)]
    assert list(w[16:]) == [j * 0.5 - 3 for j in range(16)]


# ---- Q8_0 (tests/support/q8_0_reference.h) --------------------------------------


@pytest.mark.parametrize("count", [1, 9, 257])
def test_q8_0_edge_blocks_match_numpy_and_the_reference(oracle, reference, count):
    stored = B.q8_0_edge_blocks(count)
    got = oracle.dequantize(Q8_0, stored)
    assert (_bits(got) == _bits(B.numpy_q8_0(stored))).all()
    assert (_bits(got) == _bits(reference.dequantize(Q8_0, stored))).all()


def test_q8_0_codes_are_signed(oracle):
    block = bytes([0x00, 0x3C]) + bytes([0x80, 0x7F, 0xFF, 0x01]) + bytes(28)
    w = oracle.dequantize(Q8_0, block)
    assert list(w[:4]) == [-128.0, 127.0, -1.0, 1.0] and not w[4:].any()


# ---- layouts and unpack (device_layout.h:118-127) ---------------------------------


@pytest.mark.parametrize("count", [1, 2, 9])
def test_q4_1_layout_is_codes_then_d_and_m_words(oracle, count):
    stored = B.q4_1_edge_blocks(count)
    dev = oracle.lay_out(Q4_1, stored)
    assert dev.size == 20 * count
    for b in range(count):
        assert bytes(dev[16 * b : 16 * b + 16]) == stored[20 * b + 4 : 20 * b + 20]
        assert bytes(dev[16 * count + 4 * b : 16 * count + 4 * b + 4]) == stored[20 * b : 20 * b + 4]


@pytest.mark.parametrize("count", [1, 2, 9])
def test_q8_0_layout_is_codes_then_scales_rounded_to_four(oracle, count):
    stored = B.q8_0_edge_blocks(count)
    dev = oracle.lay_out(Q8_0, stored)
    assert dev.size == (34 * count + 3) // 4 * 4
    for b in range(count):
        assert bytes(dev[32 * b : 32 * b + 32]) == stored[34 * b + 2 : 34 * b + 34]
        assert bytes(dev[32 * count + 2 * b : 32 * count + 2 * b + 2]) == stored[34 * b : 34 * b + 2]
    assert not dev[34 * count :].any()


@pytest.mark.parametrize("gtype,count", [(Q4_1, 257), (Q8_0, 257), (F32, 64 * 32)])
def test_unpack_from_the_layout_equals_the_dequant(oracle, gtype, count):
    if gtype == F32:
        stored = np.random.default_rng(3).standard_normal(count).astype(np.float32).tobytes()
    else:
        stored = B.q4_1_edge_blocks(count) if gtype == Q4_1 else B.q8_0_edge_blocks(count)
    dev = oracle.lay_out(gtype, stored)
    want = oracle.dequantize(gtype, stored)
    got = np.concatenate([oracle.unpack_group(gtype, dev, count, g) for g in range(want.size // 32)])
    assert (_bits(got) == _bits(want)).all()


@pytest.mark.parametrize("name", ["w_q4_1_1152", "w_q4_1_3072", "w_q8_0", "w_glu"])
def test_fixture_weights_unpack_as_numpy_decodes(oracle, fixture_tensors, name):
    t = fixture_tensors[name]
    want = B.numpy_q4_1(t.data) if t.type == Q4_1 else B.numpy_q8_0(t.data)
    assert (_bits(oracle.dequantize(t.type, t.data)) == _bits(want)).all()
    n = len(t.data) // BLOCK[t.type][1]
    dev = oracle.lay_out(t.type, t.data)
    for g in (0, 1, n // 2, n - 1):
        assert (_bits(oracle.unpack_group(t.type, dev, n, g)) == _bits(want[32 * g : 32 * g + 32])).all()


@pytest.mark.parametrize("name", ["w_q4_1_1152", "w_q4_1_3072", "w_q8_0", "w_glu"])
def test_f32_product_within_its_bound_of_f64(oracle, fixture_tensors, name):
    t = fixture_tensors[name]
    x = oracle.fill(7, 5 * t.columns)
    y32 = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x, threads=4)
    y64, bound = oracle.matmul_f64(t.type, t.data, t.rows, t.columns, x)
    assert (np.abs(y32.astype(np.float64) - y64) <= bound).all()


# ---- the embedding gather (gather.wgsl:21-58; tests/gpu/gather_test.cpp) -----------


def _rows(oracle, gtype):
    t = _table(gtype)
    return t, oracle.dequantize(gtype, t.data).reshape(t.rows, t.columns)


def _numpy_rows(t):
    if t.type == F32:
        return np.frombuffer(t.data, np.float32).reshape(t.rows, t.columns)
    decode = {Q4_0: B.numpy_q4_0, Q4_1: B.numpy_q4_1, Q8_0: B.numpy_q8_0, Q6_K: B.numpy_q6_k}[t.type]
    return decode(t.data).reshape(t.rows, t.columns)


@pytest.mark.parametrize("gtype", sorted(EMBEDDINGS))
def test_every_row_is_its_tokens_row_decoded(oracle, gtype):
    # gather_test.cpp:202-213: a token twice, the first and last rows; the
    # row past the step untouched.
    t = _table(gtype)
    ids = [3, 0, 6, 3, 1]
    hidden = np.zeros((len(ids) + 1, t.columns), np.float32)
    oracle.gather(gtype, t.data, t.rows, t.columns, ids, hidden)
    want = _numpy_rows(t)
    for i, token in enumerate(ids):
        assert (_bits(hidden[i]) == _bits(want[token])).all(), (i, token)
    assert not hidden[len(ids)].any()


def test_pieces_each_write_their_own_rows(oracle):
    # gather_test.cpp:215-227: rows 0..2, 3..4 and 5..6, ids either side of
    # every boundary; each piece writes only the rows whose token it holds.
    t = _table(Q6_K)
    row_bytes = t.columns // 256 * 210
    ids = [2, 3, 4, 5, 0, 6, 4]
    want = _numpy_rows(t)
    hidden = np.full((len(ids), t.columns), np.float32(7.5))
    for first, count in ((0, 3), (3, 2), (5, 2)):
        piece = t.data[first * row_bytes : (first + count) * row_bytes]
        before = hidden.copy()
        oracle.gather(Q6_K, piece, count, t.columns, ids, hidden, first_row=first)
        for i, token in enumerate(ids):
            mine = first <= token < first + count
            assert (_bits(hidden[i]) == _bits(want[token] if mine else before[i])).all()
    for i, token in enumerate(ids):
        assert (_bits(hidden[i]) == _bits(want[token])).all()


def test_the_scale_multiplies_every_decoded_weight(oracle):
    # gather_test.cpp:229-239: Gemma 3's scale, sqrt(1152) in f32.
    t = _table(Q4_0)
    scale = np.float32(math.sqrt(1152.0))
    hidden = np.zeros((1, t.columns), np.float32)
    oracle.gather(Q4_0, t.data, t.rows, t.columns, [5], hidden, scale=float(scale))
    assert (_bits(hidden[0]) == _bits(_numpy_rows(t)[5] * scale)).all()


def test_a_fed_step_takes_the_draw_and_media_rows_are_skipped(oracle):
    # gather_test.cpp:241-256 (fed), gather.wgsl:40-45 (media).
    t = _table(Q4_0)
    want = _numpy_rows(t)
    hidden = np.full((1, t.columns), np.float32(-2.0))
    oracle.gather(Q4_0, t.data, t.rows, t.columns, [2], hidden, fed=[6, 0, 0, 0])
    assert (_bits(hidden[0]) == _bits(want[6])).all()
    hidden = np.full((4, t.columns), np.float32(-2.0))
    oracle.gather(Q4_0, t.data, t.rows, t.columns, [1, 4, 4, 0], hidden, media=True, media_token=4)
    assert (hidden[1] == -2.0).all() and (hidden[2] == -2.0).all()
    assert (_bits(hidden[0]) == _bits(want[1])).all() and (_bits(hidden[3]) == _bits(want[0])).all()
    # media 0: the placeholder's value is an ordinary token.
    oracle.gather(Q4_0, t.data, t.rows, t.columns, [1, 4, 4, 0], hidden, media=False, media_token=4)
    assert (_bits(hidden[1]) == _bits(want[4])).all()
    # a fed step never compares its token with the placeholder.
    hidden = np.zeros((1, t.columns), np.float32)
    oracle.gather(Q4_0, t.data, t.rows, t.columns, [0], hidden, fed=[4], media=True, media_token=4)
    assert (_bits(hidden[0]) == _bits(want[4])).all()


def test_positions_add_the_column_row_and_the_row_row(oracle):
    rng = np.random.default_rng(11)
    positions, columns, grid = 5, 64, 3
    table = rng.standard_normal((2 * positions, columns)).astype(np.float32)
    out = oracle.gather_positions(table, columns, positions, grid, 13)
    for r in range(13):
        want = table[r % grid] + table[positions + r // grid]
        assert (_bits(out[r]) == _bits(want)).all()


# ---- F16 and BF16 (formats/f16/f16.wgsl, formats/bf16/bf16.wgsl) ------------------


def test_bf16_every_input_is_its_top_half_shift(oracle):
    """ggml_bf16_to_fp32 (unpack_bf16_test.cpp:21): the value's 16 bits are the
    top of an f32, so every input, NaN payloads and -0 included, keeps its bits."""
    every = np.arange(65536, dtype=np.uint16)
    got = oracle.dequantize(BF16, every.tobytes())  # bits straight from C: NaN payloads kept
    want = (every.astype(np.uint32) << 16).view(np.float32)
    assert (_bits(got) == _bits(want)).all()
    # The scalar entry point agrees on every non-NaN input (a float return
    # through Python would quiet a signalling NaN).
    finite = [h for h in range(0, 65536, 7) if (h & 0x7F80) != 0x7F80 or (h & 0x7F) == 0]
    assert all(np.float32(oracle.bf16_to_fp32(h)) == want[h] for h in finite)
    # Known answers: 1.0, -2.0, the largest finite, the smallest subnormal.
    assert oracle.bf16_to_fp32(0x3F80) == 1.0 and oracle.bf16_to_fp32(0xC000) == -2.0
    assert oracle.bf16_to_fp32(0x7F7F) == np.float32(3.3895313892515355e38)
    assert oracle.bf16_to_fp32(0x0001) == np.float32(2.0**-133)


@pytest.mark.parametrize("count", [32, 96, 33 * 32])
def test_f16_values_decode_as_numpy_and_the_reference(oracle, reference, count):
    stored = B.f16_edge_values(count)
    h = np.frombuffer(stored, np.uint16)
    assert list(h[: len(B.F16_EDGES)]) == B.F16_EDGES
    assert not ((h & 0x7C00) == 0x7C00).any()
    got = oracle.dequantize(F16, stored)
    assert (_bits(got) == _bits(h.view(np.float16).astype(np.float32))).all()
    theirs = np.array([reference.fp16_to_fp32(int(v)) for v in h], np.float32)
    assert (_bits(got) == _bits(theirs)).all()


@pytest.mark.parametrize("count", [32, 96, 33 * 32])
def test_bf16_values_decode_as_the_shift(oracle, count):
    stored = B.bf16_edge_values(count)
    h = np.frombuffer(stored, np.uint16)
    assert list(h[: len(B.BF16_EDGES)]) == B.BF16_EDGES
    assert not ((h & 0x7F80) == 0x7F80).any()
    got = oracle.dequantize(BF16, stored)
    assert (_bits(got) == _bits((h.astype(np.uint32) << 16).view(np.float32))).all()
    # -0 keeps its sign; the subnormals keep their value.
    assert _bits(got)[1] == 0x80000000 and got[2] == np.float32(2.0**-133)


@pytest.mark.parametrize("gtype,make", [(F16, B.f16_edge_values), (BF16, B.bf16_edge_values)])
def test_half_layouts_are_the_values_as_stored(oracle, gtype, make):
    """kF16 = kBF16 = {{0, 2}} (device_layout.h:119-120): one stream, the file's
    bytes as they lie; group g is values 32g .. 32g + 31 (f16.wgsl:6-13)."""
    count = 7 * 32
    stored = make(count)
    device = oracle.lay_out(gtype, stored)
    assert device.size == 2 * count and device.tobytes() == stored
    want = oracle.dequantize(gtype, stored)
    for g in range(7):
        assert (_bits(oracle.unpack_group(gtype, device, count, g)) == _bits(want[32 * g : 32 * g + 32])).all()


def _canonical_rows(w, x, groups):
    """The reference's order in exact binary32 arithmetic (fractions), per row."""
    out = []
    for row in w:
        total = np.float32(0.0)
        for r in range(32):
            s = np.float32(0.0)
            for k in range(32 * (r * groups // 32), 32 * ((r + 1) * groups // 32)):
                s = B.fma_f32(row[k], x[k], s)
            total = B.add_f32(total, s)
        out.append(total)
    return np.array(out, np.float32)


@pytest.mark.parametrize("gtype", [F32, F16, BF16])
def test_float_format_products_follow_the_reference_order(oracle, gtype):
    """The F32, F16 and BF16 products (capability.cpp:57-65 composes every
    format with the one matmul): the oracle's bits are the canonical order's,
    computed independently in exact arithmetic, and within gamma(2K) of f64."""
    rng = np.random.default_rng(gtype + 100)
    rows, columns = 3, 96
    w = rng.standard_normal((rows, columns)).astype(np.float32)
    if gtype == F32:
        stored = w.tobytes()
    elif gtype == F16:
        stored = w.astype(np.float16).tobytes()
    else:
        stored = (w.view(np.uint32) >> 16).astype(np.uint16).tobytes()
    wd = oracle.dequantize(gtype, stored).reshape(rows, columns)
    x = (rng.standard_normal((2, columns)) * 1e3).astype(np.float32)
    y = oracle.matmul_f32(gtype, stored, rows, columns, x)
    for t in range(2):
        assert (_bits(y[t]) == _bits(_canonical_rows(wd, x[t], columns // 32))).all()
    y64, bound = oracle.matmul_f64(gtype, stored, rows, columns, x)
    assert (np.abs(y.astype(np.float64) - y64) <= bound).all()
