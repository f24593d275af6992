"""The CPU oracle pinned against the reference's own tests, its own code
(oracle/_ref), closed forms and brute force — before anything trusts it.

Each test names the reference test or file it follows.
"""

import math

import numpy as np
import pytest

from tests.support import blocks as B
from tests.support.oracle_lib import Q4_0, Q6_K


# ---- fp16 (src/core/quant/q4_0.h:66-95; tests/quant_q4_0_test.cpp:41-65) ----


def test_fp16_known_answers(oracle):
    f = oracle.fp16_to_fp32
    assert f(0x0000) == 0.0 and math.copysign(1, f(0x0000)) == 1
    assert f(0x8000) == 0.0 and math.copysign(1, f(0x8000)) == -1
    assert f(0x3C00) == 1.0 and f(0xBC00) == -1.0
    assert f(0x4000) == 2.0 and f(0x3800) == 0.5
    assert f(0x7BFF) == 65504.0
    assert f(0x0001) == 2.0**-24
    assert f(0x0002) == 2.0**-23
    assert f(0x03FF) < f(0x0400)
    assert math.isinf(f(0x7C00)) and math.isinf(f(0xFC00)) and f(0xFC00) < 0
    assert math.isnan(f(0x7E00))


def test_fp16_every_input_matches_numpy_and_the_reference(oracle):
    from tests.support.oracle_lib import reference_or_none

    want = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_fp32(h) for h in range(65536)], np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    ref = reference_or_none()
    if ref is not None:
        theirs = np.array([ref.fp16_to_fp32(h) for h in range(65536)], np.float32)
        assert ((theirs.view(np.uint32) == got.view(np.uint32)) | (np.isnan(got) & np.isnan(theirs))).all()


# ---- Q4_0 dequant (tests/quant_q4_0_test.cpp:87-145) --------------------


def test_q4_0_scale_one_gives_code_minus_eight(oracle):
    nibbles = [i % 16 for i in range(32)]
    out = oracle.dequantize(Q4_0, B.q4_0_block(0x3C00, nibbles))
    assert list(out) == [float(n - 8) for n in nibbles]


def test_q4_0_zero_point_is_eight(oracle):
    out = oracle.dequantize(Q4_0, B.q4_0_block(0x4900, [8] * 32))
    assert (out == 0.0).all()


def test_q4_0_extremes(oracle):
    n = [0] * 32
    n[1] = 15
    out = oracle.dequantize(Q4_0, B.q4_0_block(0x3C00, n))
    assert out[0] == -8.0 and out[1] == 7.0


def test_q4_0_element_16_is_byte_0_high_nibble(oracle):
    n = [8] * 32
    n[16] = 15
    out = oracle.dequantize(Q4_0, B.q4_0_block(0x3C00, n))
    assert out[16] == 7.0 and out[0] == 0.0 and out[1] == 0.0 and out[8] == 0.0


def test_q4_0_scale_is_per_block(oracle):
    data = B.q4_0_block(0x3C00, [9] * 32) + B.q4_0_block(0x4000, [9] * 32)
    out = oracle.dequantize(Q4_0, data)
    assert out[0] == 1.0 and out[32] == 2.0


def _bitwise(got, want):
    """Bit for bit; a zero of either sign equals a zero (tests/gpu/support/unpack.h:90-109)."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    return ((got.view(np.uint32) == want.view(np.uint32)) | ((got == 0) & (want == 0))).all()


@pytest.mark.parametrize("count", [1, 9, 257])
def test_q4_0_edge_blocks_match_closed_form(oracle, count):
    stored = B.q4_0_edge_blocks(count)
    assert _bitwise(oracle.dequantize(Q4_0, stored), B.numpy_q4_0(stored))


@pytest.mark.parametrize("count", [1, 9, 257])
def test_q4_0_edge_blocks_match_the_reference(oracle, reference, count):
    stored = B.q4_0_edge_blocks(count)
    # Every bit, zeros' signs included.
    assert (oracle.dequantize(Q4_0, stored).view(np.uint32) == reference.dequantize(Q4_0, stored).view(np.uint32)).all()


# ---- Q6_K dequant (tests/gpu/unpack_q6_k_test.cpp:24-57) ------------------


@pytest.mark.parametrize("count", [1, 9, 33])
def test_q6_k_edge_blocks_match_closed_form(oracle, count):
    stored = B.q6_k_edge_blocks(count)
    assert _bitwise(oracle.dequantize(Q6_K, stored), B.numpy_q6_k(stored))


@pytest.mark.parametrize("count", [1, 9, 33])
def test_q6_k_edge_blocks_match_the_reference(oracle, reference, count):
    stored = B.q6_k_edge_blocks(count)
    assert (oracle.dequantize(Q6_K, stored).view(np.uint32) == reference.dequantize(Q6_K, stored).view(np.uint32)).all()


def test_q6_k_scale_edges_decode(oracle):
    # Scales -128 and 127 lead every edge block; with d = 1.0 (block 0) the
    # first 16 weights are -128 * (q - 32) and the next 16 are 127 * (q - 32).
    stored = B.q6_k_edge_blocks(1)
    w = oracle.dequantize(Q6_K, stored)
    q = B.q6_k_codes(stored)[0] - 32
    assert (w[:16] == -128.0 * q[:16]).all() and (w[16:32] == 127.0 * q[16:32]).all()


# ---- Q6_K repack (tests/formats_q6_k_repack_test.cpp:24-69) ---------------


def _stored_q(block, k, l):
    h, r = k // 4, k % 4
    ql = block[64 * h + 32 * (r % 2) + l]
    qh = block[128 + 32 * h + l]
    return ((ql >> (4 * (r // 2))) & 0xF) | (((qh >> (2 * r)) & 3) << 4)


def _repacked_q(lo, hi, k, l):
    nibbles = lo[16 * k + l % 16]
    pairs = hi[8 * k + l % 8]
    return ((nibbles >> (4 * (l // 16))) & 0xF) | (((pairs >> (2 * (l // 8))) & 3) << 4)


def test_q6_k_repack_places_every_weight_scale_and_d(oracle):
    stored = B.lcg_bytes(3 * 210)
    lo, hi, sc, d = oracle.repack_q6_k(stored)
    for b in range(3):
        block = stored[210 * b : 210 * b + 210]
        for k in range(8):
            for l in range(32):
                assert _repacked_q(lo[128 * b :], hi[64 * b :], k, l) == _stored_q(block, k, l), (b, k, l)
        assert bytes(sc[16 * b : 16 * b + 16]) == block[192:208]
        assert bytes(d[2 * b : 2 * b + 2]) == block[208:210]


@pytest.mark.parametrize("count", [1, 3, 33])
def test_q6_k_repack_matches_the_reference_byte_for_byte(oracle, reference, count):
    stored = B.lcg_bytes(count * 210, seed=0x2545F491 + count)
    for mine, theirs in zip(oracle.repack_q6_k(stored), reference.repack_q6_k(stored)):
        assert (mine == theirs).all()


# ---- device layout and unpack (device_layout.h:111-136; q4_0.wgsl, q6_k.wgsl) ----


@pytest.mark.parametrize("count", [1, 2, 9])
def test_q4_0_layout_is_codes_then_scales_rounded_to_four(oracle, count):
    stored = B.q4_0_edge_blocks(count)
    dev = oracle.lay_out(Q4_0, stored)
    assert dev.size == (18 * count + 3) // 4 * 4
    for b in range(count):
        assert bytes(dev[16 * b : 16 * b + 16]) == stored[18 * b + 2 : 18 * b + 18]
        assert bytes(dev[16 * count + 2 * b : 16 * count + 2 * b + 2]) == stored[18 * b : 18 * b + 2]


@pytest.mark.parametrize("gtype,count", [(Q4_0, 257), (Q6_K, 33)])
def test_unpack_from_the_layout_equals_the_dequant(oracle, gtype, count):
    stored = B.q4_0_edge_blocks(count) if gtype == Q4_0 else B.q6_k_edge_blocks(count)
    dev = oracle.lay_out(gtype, stored)
    want = oracle.dequantize(gtype, stored)
    groups = want.size // 32
    got = np.concatenate([oracle.unpack_group(gtype, dev, count, g) for g in range(groups)])
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


def test_fixture_weights_unpack_as_they_dequantize(oracle, fixture_tensors):
    for name in ("w_q4_0", "w_q6_k", "qkv_q", "w_set3"):
        t = fixture_tensors[name]
        per, nbytes = (32, 18) if t.type == Q4_0 else (256, 210)
        n = len(t.data) // nbytes
        dev = oracle.lay_out(t.type, t.data)
        want = oracle.dequantize(t.type, t.data)
        for g in (0, 1, want.size // 32 // 2, want.size // 32 - 1):
            assert (oracle.unpack_group(t.type, dev, n, g) == want[32 * g : 32 * g + 32]).all()


# ---- the order of addition (matmul.h:34-50) -------------------------------


@pytest.mark.parametrize("groups", [1, 2, 32, 36, 96])
def test_range_boundaries(oracle, groups):
    # floor(r G / 32); every group in exactly one range, in order.
    los = [oracle.range_lo(r, groups) for r in range(33)]
    assert los[0] == 0 and los[32] == groups
    assert all(a <= b for a, b in zip(los, los[1:]))
    assert all(los[r] == r * groups // 32 for r in range(33))
    if groups == 36:  # Gemma 3's 1,152: ranges 7, 15, 23, 31 hold two groups
        assert [r for r in range(32) if los[r + 1] - los[r] == 2] == [7, 15, 23, 31]


def _canonical(w, x, groups):
    """The reference's order, in exact binary32 arithmetic (independent of C's fmaf)."""
    total = np.float32(0.0)
    for r in range(32):
        s = np.float32(0.0)
        for k in range(32 * (r * groups // 32), 32 * ((r + 1) * groups // 32)):
            s = B.fma_f32(w[k], x[k], s)
        total = B.add_f32(total, s)
    return total


def _one_chain(w, x):
    s = np.float32(0.0)
    for k in range(len(w)):
        s = B.fma_f32(w[k], x[k], s)
    return s


def _mul_add(w, x):
    s = np.float32(0.0)
    for k in range(len(w)):
        s = B.add_f32(s, np.float32(w[k] * x[k]))
    return s


@pytest.mark.parametrize("columns", [64, 1152])
def test_f32_product_is_the_reference_order_bit_for_bit(oracle, columns):
    # A weight whose outputs' bits differ between orders: the canonical one,
    # one long chain, and unfused multiply-adds. The oracle must give the
    # canonical bits for every row, and the other orders must differ on some,
    # so this test would catch a dropped range, a missing fma or a reversed sum.
    rng = np.random.default_rng(columns)
    rows = 6
    q = rng.integers(0, 16, size=(rows * columns // 32, 16), dtype=np.uint8)
    q |= rng.integers(0, 16, size=q.shape, dtype=np.uint8) << 4
    d = (np.abs(rng.standard_normal(q.shape[0])) * 0.02).astype(np.float16).view(np.uint16)
    stored = b"".join(bytes([int(d[i]) & 0xFF, int(d[i]) >> 8]) + q[i].tobytes() for i in range(q.shape[0]))
    x = rng.standard_normal(columns).astype(np.float32) * np.float32(1e3)
    w = oracle.dequantize(Q4_0, stored).reshape(rows, columns)
    y = oracle.matmul_f32(Q4_0, stored, rows, columns, x)[0]
    groups = columns // 32
    differs_chain = differs_unfused = False
    for o in range(rows):
        want = _canonical(w[o], x, groups)
        assert y[o].view(np.uint32) == np.float32(want).view(np.uint32), o
        differs_chain |= _one_chain(w[o], x) != want
        differs_unfused |= _mul_add(w[o], x) != want
    assert differs_chain and differs_unfused


def test_f32_threads_do_not_change_bits(oracle, fixture_tensors):
    t = fixture_tensors["w_q6_k"]
    x = oracle.fill(7, 3 * t.columns)
    one = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x, threads=1)
    many = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x, threads=7)
    assert (one.view(np.uint32) == many.view(np.uint32)).all()


# ---- the f64 oracle and its bound (tests/gpu/matmul_test.cpp:190-211) --------


def test_f64_oracle_is_a_plain_dot_product(oracle, fixture_tensors):
    t = fixture_tensors["w_q4_0"]
    x = oracle.fill(7, 2 * t.columns)
    y, bound = oracle.matmul_f64(t.type, t.data, t.rows, t.columns, x)
    w = oracle.dequantize(t.type, t.data).reshape(t.rows, t.columns).astype(np.float64)
    want = x.reshape(2, -1).astype(np.float64) @ w.T
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12)
    u = 2.0**-24
    gamma = 2 * t.columns * u / (1 - 2 * t.columns * u)
    assert np.allclose(bound, gamma * (np.abs(x.reshape(2, -1)).astype(np.float64) @ np.abs(w).T), rtol=1e-12)


@pytest.mark.parametrize("threads", [2, 3, 8])
def test_f64_threads_split_rows_without_changing_a_value(oracle, fixture_tensors, threads):
    t = fixture_tensors["w_q6_k"]
    x = oracle.fill(11, 3 * t.columns)
    one, b1 = oracle.matmul_f64(t.type, t.data, t.rows, t.columns, x)
    many, bm = oracle.matmul_f64(t.type, t.data, t.rows, t.columns, x, threads=threads)
    assert (one.view(np.uint64) == many.view(np.uint64)).all() and (b1.view(np.uint64) == bm.view(np.uint64)).all()


@pytest.mark.parametrize("name", ["w_q4_0", "w_q6_k", "w_set2", "qkv_q", "ffn_gate"])
def test_f32_within_its_bound_of_f64_on_the_fixture(oracle, fixture_tensors, name):
    t = fixture_tensors[name]
    x = oracle.fill(7, 9 * t.columns)
    y32 = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x)
    y64, bound = oracle.matmul_f64(t.type, t.data, t.rows, t.columns, x)
    assert (np.abs(y32.astype(np.float64) - y64) <= bound).all()


# ---- the reference tests' fill (tests/gpu/support/fill.h:24-29) ----------------


def test_fill_matches_the_hash_recomputed(oracle):
    i = np.arange(7, 7 + 4096, dtype=np.uint64)
    v = (i * 747796405 + 2891336453) & 0xFFFFFFFF
    v = (((v >> ((v >> 28) + 4)) ^ v) * 277803737) & 0xFFFFFFFF
    v = ((v >> 22) ^ v) & 0xFFFFFFFF
    want = (v >> 8).astype(np.float32) / np.float32(8388608.0) - np.float32(1.0)
    got = oracle.fill(7, 4096)
    assert (got == want).all() and got.min() >= -1.0 and got.max() < 1.0


# ---- activations (matmul.wgsl:169-205), for the fused epilogues ----------------


def test_exp_nonpositive_within_its_stated_error(oracle):
    for x in np.linspace(-87.0, 0.0, 20001, dtype=np.float32):
        e = oracle.exp_nonpositive(float(x))
        want = math.exp(float(x))
        assert abs(e - want) <= 2.0**-21 * want + 1e-38
    assert oracle.exp_nonpositive(-200.0) == pytest.approx(math.exp(-100.0), rel=1e-5)


@pytest.mark.parametrize("activation", [0, 1, 2])
def test_activations_near_their_definitions(oracle, activation):
    for g in np.linspace(-30, 30, 6001, dtype=np.float32):
        g = float(g)
        if activation == 0:
            want = g / (1 + math.exp(-g))
        elif activation == 2:
            want = 1 / (1 + math.exp(-g))
        else:
            want = 0.5 * g * (1 + math.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g**3)))
        # GELU's 1 + tanh cancels in its negative tail, so its error there is
        # absolute, a few units of |g| 2^-24, not relative.
        tail = 2.0**-21 * abs(g) if activation == 1 else 0.0
        assert abs(oracle.activate(activation, g) - want) <= 2.0**-16 * abs(want) + tail + 2.0**-30


# ---- epilogues (matmul.wgsl:117-132, 272-351) ---------------------------------


def _silu(g):
    return g / (1 + math.exp(-g))


def _gelu(g):
    return 0.5 * g * (1 + math.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g**3)))


def test_clamp_is_min_of_max(oracle):
    x = np.array([-5.0, -1.0, -0.5, 0.25, 1.0, 7.0], np.float32)
    assert oracle.clamp(x, -1.0, 1.0).tolist() == [-1.0, -1.0, -0.5, 0.25, 1.0, 1.0]


def test_finish_orders_clamp_then_bias_then_activation(oracle):
    # total 3 clamped to [-1, 1] is 1; the bias 0.5 makes 1.5; SiLU last. Any
    # other order gives another value: bias first 3.5 -> 1 -> SiLU(1) = 0.731;
    # activation before the bias SiLU(1) + 0.5 = 1.231.
    clip = [-9.0, 9.0, -1.0, 1.0]
    got = oracle.finish(np.array([[3.0]]), clip=clip, bias=[0.5], activated=True, activation=0)[0, 0]
    assert got == pytest.approx(_silu(1.5), rel=2e-6)
    assert abs(got - _silu(1.0)) > 0.4 and abs(got - (_silu(1.0) + 0.5)) > 4e-3
    # Each option alone, and the bias indexed by output row.
    t = np.array([[2.0, -3.0, 0.5], [-0.25, 4.0, 1.5]], np.float32)
    assert (oracle.finish(t) == t).all()
    assert oracle.finish(t, clip=[0, 0, -1.0, 1.0]).tolist() == [[1.0, -1.0, 0.5], [-0.25, 1.0, 1.0]]
    assert oracle.finish(t, bias=[1.0, 10.0, 100.0]).tolist() == [[3.0, 7.0, 100.5], [0.75, 14.0, 101.5]]
    got = oracle.finish(t, activated=True, activation=1)
    for a, b in zip(got.ravel(), t.ravel()):
        # GELU's negative tail: absolute error, as in the activation test.
        assert a == pytest.approx(_gelu(float(b)), rel=1e-5, abs=2.0**-21 * abs(float(b)))


def test_gated_is_activated_gate_times_up(oracle):
    gate = np.array([-3.0, 0.5, 2.0], np.float32)
    up = np.array([5.0, -4.0, 0.25], np.float32)
    got = oracle.gated(gate, up, activation=0)
    for a, g, u in zip(got, gate, up):
        assert a == pytest.approx(_silu(float(g)) * float(u), rel=2e-6)
    # Gate and up are not interchangeable: SiLU(5) * -3 is far from SiLU(-3) * 5.
    assert abs(got[0] - _silu(5.0) * -3.0) > 10
    # Clipped: both totals clamped to the output bounds before the activation.
    got = oracle.gated(gate, up, clip=[0, 0, -2.0, 2.0], activation=2)
    want = [1 / (1 + math.exp(2.0)) * 2.0, 1 / (1 + math.exp(-0.5)) * -2.0, 1 / (1 + math.exp(-2.0)) * 0.25]
    assert got.tolist() == pytest.approx(want, rel=2e-6)


def test_gated_by_input_is_activated_total_times_u(oracle):
    t = np.array([0.7, -1.25, 3.0], np.float32)
    u = np.array([2.0, -0.5, 0.125], np.float32)
    got = oracle.gated_by_input(t, u, activation=1)
    for a, g, v in zip(got, t, u):
        assert a == pytest.approx(_gelu(float(g)) * float(v), rel=1e-5, abs=2.0**-21 * abs(float(g * v)))
