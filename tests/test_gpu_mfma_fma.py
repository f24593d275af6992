"""The matrix-core instruction the canonical-order prefill tiles (GEMM_EXACT,
GEMM_EXACT_SHORT, GEMM_EXACT_SPLIT) are built on, v_mfma_f32_32x32x1_2b_f32,
and its four-block K = 1 sibling v_mfma_f32_16x16x1_4b_f32 are, element by
element, one fused multiply-add, d = fmaf(a, b, c), bit for bit; and their
lane layouts.

GEMM_EXACT's outputs are the reference order's bits only because of that, so
the property itself is held here, on the harness's probes (harness.hip):
mfma_fma_check gives every lane of a wave one a and one b and 2,048
accumulators c, so every element of the result is c + a b whatever its place,
and compares each with fmaf on the VALU; mfma_c_probe checks that each
accumulator comes back in its own place (a = b = 0). Operands: random
magnitudes over 2^+-20, products cancelling their accumulator, sums on and
next to halfway points of the accumulator's ulp, denormal operands and
results, infinities, NaNs and signed zeros, and overflow.

The K = 2 and K = 4 f32 shapes (32x32x2, 16x16x4) against fmaf applied in k
order (mfma_chain_check), on operands whose two products nearly cancel with a
small accumulator: there the sequential sum and a once-rounded one differ for
most elements (counted exactly on the CPU below), so agreement shows the
instruction rounds after each product.
"""

import numpy as np
import pytest

PAIRS = 2048
F32 = np.float32


def _classes(rng):
    n = PAIRS

    def random():
        a = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(F32)
        b = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(F32)
        ab = np.abs(a.astype(np.float64) * b)
        c = rng.standard_normal((n, 2048)) * ab[:, None] * 2.0 ** rng.integers(-30, 30, (n, 2048))
        return a, b, c.astype(F32)

    def cancel():
        a, b = rng.standard_normal(n).astype(F32), rng.standard_normal(n).astype(F32)
        ab = a.astype(np.float64) * b
        rel = rng.standard_normal((n, 2048)) * 2.0 ** rng.integers(-30, -1, (n, 2048))
        return a, b, (-(ab[:, None]) * (1 + rel)).astype(F32)

    def halfway():
        # a b = (2j + 1) 2^(e - 24 - k), c a 24-bit integer times 2^(e - 23):
        # the sum on (k = 0) or near a halfway point of c's ulp
        e = rng.integers(-20, 20, n)
        j, k = rng.integers(0, 1 << 10, n), rng.integers(0, 3, n)
        a = ((2 * j + 1) * 2.0 ** (e - 34 - k)).astype(F32)
        b = np.full(n, 2.0 ** 10, F32)
        m = rng.integers(1 << 23, 1 << 24, (n, 2048)) * rng.choice([-1.0, 1.0], (n, 2048))
        return a, b, (m * 2.0 ** (e[:, None] - 23)).astype(F32)

    def denormal():
        a = (rng.standard_normal(n) * 2.0 ** rng.integers(-80, -60, n)).astype(F32)
        b = (rng.standard_normal(n) * 2.0 ** rng.integers(-80, -60, n)).astype(F32)
        c = rng.standard_normal((n, 2048)) * 2.0 ** rng.integers(-150, -120, (n, 2048))
        return a, b, c.astype(F32)

    def denormal_operand():
        a = (rng.standard_normal(n) * 2.0 ** rng.integers(-140, -127, n)).astype(F32)
        b = (rng.standard_normal(n) * 2.0 ** rng.integers(0, 40, n)).astype(F32)
        ab = np.abs(a.astype(np.float64) * b)
        c = rng.standard_normal((n, 2048)) * ab[:, None] * 2.0 ** rng.integers(-10, 10, (n, 2048))
        return a, b, c.astype(F32)

    def special():
        vals = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 3.4e38, -3.4e38, 1e-45, -1e-45,
                         1.17549435e-38], F32)
        return rng.choice(vals, n).astype(F32), rng.choice(vals, n).astype(F32), rng.choice(vals, (n, 2048))

    def overflow():
        a = (rng.standard_normal(n) * 2.0 ** rng.integers(60, 64, n)).astype(F32)
        b = (rng.standard_normal(n) * 2.0 ** rng.integers(60, 64, n)).astype(F32)
        c = rng.standard_normal((n, 2048)) * 2.0 ** rng.integers(110, 125, (n, 2048))
        return a, b, c.astype(F32)

    return {"random": random, "cancel": cancel, "halfway": halfway, "denormal": denormal,
            "denormal_operand": denormal_operand, "special": special, "overflow": overflow}


@pytest.mark.gpu
@pytest.mark.parametrize("shape,registers", [(5, 32), (6, 16)])
@pytest.mark.parametrize("name", ["random", "cancel", "halfway", "denormal", "denormal_operand", "special",
                                  "overflow"])
def test_k1_f32_instruction_is_fmaf_bit_for_bit(name, shape, registers):
    """Shape 5: v_mfma_f32_32x32x1_2b_f32; 6: v_mfma_f32_16x16x1_4b_f32."""
    from charlotte_amd import harness as hx

    a, b, c = _classes(np.random.default_rng(sum(map(ord, name))))[name]()
    ab = hx.Buffer.of(np.stack([a, b], 1).astype(F32).ravel())
    cb = hx.Buffer.of(np.ascontiguousarray(c, F32).ravel())
    out = hx.Buffer(nbytes=(2 + 256) * 4)
    s = hx.Stream()
    try:
        hx.mfma_fma_check(ab.ptr, cb.ptr, PAIRS, 1024, out.ptr, s, shape=shape)
        s.sync()
        o = out.read(np.uint32)
        assert o[1] == PAIRS * 64 * registers, "every element compared"
        assert o[0] == 0, f"{name}: {o[0]} of {o[1]} differ; first (pair, element, mfma, fmaf): {o[2:6].tolist()}"
    finally:
        for buf in (ab, cb, out):
            buf.free()
        s.destroy()


@pytest.mark.gpu
@pytest.mark.parametrize("shape,registers", [(5, 32), (6, 16), (7, 16), (8, 4), (9, 4), (1, 16)])
def test_accumulators_come_back_in_their_places(shape, registers):
    """a = b = 0: D = C, each accumulator in its own register and lane (the
    f32 K = 1, 2 and 4 shapes, and the f16 32 x 32 x 16 one)."""
    from charlotte_amd import harness as hx

    ids = (np.arange(2048) + 1).astype(F32)
    cb, ob = hx.Buffer.of(ids), hx.Buffer(nbytes=2048 * 4)
    s = hx.Stream()
    try:
        hx.mfma_c_probe(shape, cb.ptr, ob.ptr, s)
        s.sync()
        got = ob.read(np.float32)[: 64 * registers]
        assert (got == ids[: 64 * registers]).all()
    finally:
        cb.free()
        ob.free()
        s.destroy()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [5, 6])
def test_k1_f32_instruction_layout(shape):
    """The places the exact prefill tiles read results from. 32x32x1 (two
    blocks, 32 registers): register v of lane l is block v / 16, its row 8
    ((v % 16) / 4) + 4 (l / 32) + v % 4 (a from lane 32 (v / 16) + that row),
    its column l % 32 (b from lane 32 (v / 16) + l % 32). 16x16x1 (four
    blocks, 16 registers): block v / 4, row 4 (l / 16) + v % 4, column l % 16,
    a and b from lanes 16 (v / 4) + row and + column."""
    from charlotte_amd import harness as hx

    registers = 32 if shape == 5 else 16
    out = hx.Buffer(nbytes=2 * 64 * registers * 4)
    s = hx.Stream()
    try:
        hx.mfma_layout(out.ptr, s, shape=shape)
        s.sync()
        got = out.read(np.float32).reshape(2, registers, 64)
    finally:
        out.free()
        s.destroy()
    v = np.arange(registers)[:, None]
    lane = np.arange(64)[None, :]
    if shape == 5:
        block, row, col = v // 16, 8 * ((v % 16) // 4) + 4 * (lane // 32) + v % 4, lane % 32
        width = 32
    else:
        block, row, col = v // 4, 4 * (lane // 16) + v % 4, lane % 16
        width = 16
    assert (got[0] == width * block + row + 1).all(), "rows"
    assert (got[1] == width * block + col + 1).all(), "columns"


def _mixed(rng, n, k, registers):
    """k products a pair, the second cancelling the first to its rounding, and
    small accumulators: c + a0 b0 rounded, then + a1 b1, is far from the once-
    rounded sum for most elements."""
    a = (rng.standard_normal((n, k)) * 2.0 ** rng.integers(-10, 10, (n, k))).astype(F32)
    b = (rng.standard_normal((n, k)) * 2.0 ** rng.integers(-10, 10, (n, k))).astype(F32)
    b[:, 1] = (-(a[:, 0].astype(np.float64) * b[:, 0]) / a[:, 1]).astype(F32)
    c = (rng.standard_normal((n, 64 * registers)) * 2.0 ** rng.integers(-30, 0, (n, 64 * registers))).astype(F32)
    return a, b, c


def _round_f32(x):
    """A Fraction to the nearest binary32, ties to even (finite, normal range)."""
    from fractions import Fraction

    f = np.float32(float(x))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    return min(cands, key=lambda v: (abs(Fraction(float(v)) - x), int(np.array([v]).view(np.uint32)[0]) & 1))


def test_mixed_operands_tell_sequential_from_once_rounded_sums():
    """On the CPU, exactly: the mixed operands separate the two semantics, so
    the GPU check below can tell them apart."""
    from fractions import Fraction as Fr

    a, b, c = _mixed(np.random.default_rng(3), 200, 2, 1)
    differ = total = 0
    for p in range(200):
        for e in range(4):
            p0, p1 = Fr(float(a[p, 0])) * Fr(float(b[p, 0])), Fr(float(a[p, 1])) * Fr(float(b[p, 1]))
            seq = _round_f32(p1 + Fr(float(_round_f32(p0 + Fr(float(c[p, e]))))))
            once = _round_f32(p0 + p1 + Fr(float(c[p, e])))
            differ += int(seq != once)
            total += 1
    assert differ > total // 2, f"{differ} of {total}"


@pytest.mark.gpu
@pytest.mark.parametrize("k,registers", [(2, 16), (4, 4)])
@pytest.mark.parametrize("kind", ["random", "cancel", "mixed"])
def test_k2_and_k4_f32_instructions_are_fmaf_in_k_order(k, registers, kind):
    from charlotte_amd import harness as hx

    rng = np.random.default_rng(10 * k + len(kind))
    n = PAIRS
    if kind == "mixed":
        a, b, c = _mixed(rng, n, k, registers)
    else:
        a = (rng.standard_normal((n, k)) * 2.0 ** rng.integers(-10, 10, (n, k))).astype(F32)
        b = (rng.standard_normal((n, k)) * 2.0 ** rng.integers(-10, 10, (n, k))).astype(F32)
        if kind == "random":
            c = rng.standard_normal((n, 64 * registers)) * 2.0 ** rng.integers(-20, 20, (n, 64 * registers))
        else:
            ab = (a.astype(np.float64) * b).sum(1)
            rel = rng.standard_normal((n, 64 * registers)) * 2.0 ** rng.integers(-30, -1, (n, 64 * registers))
            c = -(ab[:, None]) * (1 + rel)
        c = c.astype(F32)
    abuf = hx.Buffer.of(np.stack([a, b], 2).astype(F32).ravel())
    cbuf = hx.Buffer.of(np.ascontiguousarray(c, F32).ravel())
    out = hx.Buffer(nbytes=(2 + 256) * 4)
    s = hx.Stream()
    try:
        hx.mfma_chain_check(k, abuf.ptr, cbuf.ptr, n, 1024, out.ptr, s)
        s.sync()
        o = out.read(np.uint32)
        assert o[1] == n * 64 * registers
        assert o[0] == 0, f"K={k} {kind}: {o[0]} of {o[1]} differ; first: {o[2:6].tolist()}"
    finally:
        for buf in (abuf, cbuf, out):
            buf.free()
        s.destroy()
