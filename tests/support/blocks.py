"""Stored blocks the reference's own tests build, restated (test infrastructure).

- q4_0_edge_blocks: tests/gpu/unpack_q4_0_test.cpp:24-37 — scales 1, -1, +0,
  -0, the smallest subnormal, the largest subnormal, +-65504 and 0x2E66 first,
  then LCG scales (never inf/NaN); LCG codes throughout.
- q6_k_edge_blocks: tests/gpu/unpack_q6_k_test.cpp:24-41 — LCG ql/qh, scales
  with -128 and 127 first, the same d edges.
- q4_1_edge_blocks: tests/gpu/unpack_q4_1_test.cpp:24-46 — every edge as d and,
  four apart, as m; then LCG d and m; LCG codes.
- q8_0_edge_blocks: tests/gpu/unpack_q8_0_test.cpp:22-39 — the same d edges,
  codes -128 and 127 first in every block, LCG codes.
- f16_edge_values / bf16_edge_values: tests/gpu/unpack_f16_test.cpp:24-35 and
  unpack_bf16_test.cpp:29-40 — +-0, the smallest and largest subnormals, the
  smallest normal, the largest finite of either sign, 1 (and -2 for BF16),
  then LCG values, never inf or NaN.
- lcg_bytes: tests/formats_q6_k_repack_test.cpp:44-49's stored bytes.
- q4_0_block: tests/quant_q4_0_test.cpp:70-84's make_block.

Also an exact f32 fused multiply-add (for pinning the order of addition
independently of any C library), and independent numpy decoders.
"""

from fractions import Fraction

import numpy as np

EDGE_SCALES = [0x3C00, 0xBC00, 0x0000, 0x8000, 0x0001, 0x03FF, 0x7BFF, 0xFBFF, 0x2E66]


class Lcg:
    def __init__(self, state):
        self.state = state & 0xFFFFFFFF

    def next(self):
        self.state = (self.state * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.state


def _scale(b, lcg):
    d = EDGE_SCALES[b] if b < len(EDGE_SCALES) else (lcg.next() >> 16)
    if (d & 0x7C00) == 0x7C00:
        d &= 0xBBFF
    return d


def q4_0_edge_blocks(count, seed=0x2545F491):
    lcg = Lcg(seed)
    out = bytearray()
    for b in range(count):
        d = _scale(b, lcg)
        out += bytes([d & 0xFF, d >> 8])
        out += bytes((lcg.next() >> 24) & 0xFF for _ in range(16))
    return bytes(out)


def q6_k_edge_blocks(count, seed=0x7F4A7C15):
    lcg = Lcg(seed)
    out = bytearray()
    for b in range(count):
        out += bytes((lcg.next() >> 24) & 0xFF for _ in range(192))
        for i in range(16):
            s = (lcg.next() >> 24) & 0xFF
            out.append(0x80 if i == 0 else 0x7F if i == 1 else s)
        d = _scale(b, lcg)
        out += bytes([d & 0xFF, d >> 8])
    return bytes(out)


def _finite(h):
    return h & 0xBBFF if (h & 0x7C00) == 0x7C00 else h


def q4_1_edge_blocks(count, seed=0x9E3779B9):
    lcg = Lcg(seed)
    n = len(EDGE_SCALES)

    def finite(i):
        return _finite(EDGE_SCALES[i] if i < n else (lcg.next() >> 16))

    out = bytearray()
    for b in range(count):
        d = finite(b)
        m = finite((b + 4) % n if b < n else b)
        for h in (d, m):
            out += bytes([h & 0xFF, h >> 8])
        out += bytes((lcg.next() >> 24) & 0xFF for _ in range(16))
    return bytes(out)


def q8_0_edge_blocks(count, seed=0x1B873593):
    lcg = Lcg(seed)
    out = bytearray()
    for b in range(count):
        d = _finite(EDGE_SCALES[b] if b < len(EDGE_SCALES) else (lcg.next() >> 16))
        out += bytes([d & 0xFF, d >> 8])
        for j in range(32):
            q = (lcg.next() >> 24) & 0xFF
            out.append(0x80 if j == 0 else 0x7F if j == 1 else q)
    return bytes(out)


def lcg_bytes(count, seed=0x2545F491):
    lcg = Lcg(seed)
    return bytes((lcg.next() >> 24) & 0xFF for _ in range(count))


def q4_0_block(scale_fp16, nibbles):
    assert len(nibbles) == 32
    block = bytearray([scale_fp16 & 0xFF, scale_fp16 >> 8])
    for j in range(16):
        block.append((nibbles[j] & 0x0F) | ((nibbles[j + 16] & 0x0F) << 4))
    return bytes(block)


# ---- independent numpy decoders (closed forms, numpy's own fp16) ----------


def half(u16):
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float32)


def numpy_q4_0(blocks):
    b = np.frombuffer(blocks, np.uint8).reshape(-1, 18)
    d = half(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    qs = b[:, 2:]
    codes = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.int32) - 8
    return (codes.astype(np.float32) * d[:, None]).reshape(-1)


def numpy_q4_1(blocks):
    """ggml's block_q4_1 (d, m, qs[16]) in numpy float32: the product and the
    sum each rounded (numpy never fuses)."""
    b = np.frombuffer(blocks, np.uint8).reshape(-1, 20)
    d = half(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    m = half(b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << 8))
    qs = b[:, 4:]
    codes = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.float32)
    return ((codes * d[:, None]).astype(np.float32) + m[:, None]).astype(np.float32).reshape(-1)


def numpy_q8_0(blocks):
    b = np.frombuffer(blocks, np.uint8).reshape(-1, 34)
    d = half(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    codes = b[:, 2:].view(np.int8).astype(np.float32)
    return (codes * d[:, None]).astype(np.float32).reshape(-1)


def q6_k_codes(blocks):
    """[n, 256] six-bit codes of stored Q6_K blocks, from ggml's block_q6_K
    field definitions (ql low nibbles for weights 0..63 of each half, high
    nibbles for 64..127; qh pairs at bits 0, 2, 4, 6 for the four 32-weight
    quarters of each half)."""
    b = np.frombuffer(blocks, np.uint8).reshape(-1, 210)
    out = np.empty((b.shape[0], 256), np.int32)
    for half_ in range(2):
        ql = b[:, 64 * half_ : 64 * half_ + 64].astype(np.int32)
        qh = b[:, 128 + 32 * half_ : 128 + 32 * half_ + 32].astype(np.int32)
        for quarter in range(4):
            low = (ql[:, 32 * (quarter % 2) : 32 * (quarter % 2) + 32] >> (4 * (quarter // 2))) & 0xF
            high = (qh >> (2 * quarter)) & 3
            out[:, 128 * half_ + 32 * quarter : 128 * half_ + 32 * quarter + 32] = low | (high << 4)
    return out


def numpy_q6_k(blocks):
    b = np.frombuffer(blocks, np.uint8).reshape(-1, 210)
    d = half(b[:, 208].astype(np.uint16) | (b[:, 209].astype(np.uint16) << 8))
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    q = (q6_k_codes(blocks) - 32).astype(np.float32)
    scale = np.repeat(sc, 16, axis=1)  # scale i covers weights 16i .. 16i + 15
    return ((d[:, None] * scale) * q).reshape(-1).astype(np.float32)


# ---- exact f32 arithmetic ----------------------------------------------


def round_f32(v):
    """The binary32 nearest the rational v, ties to even (finite, normal or
    subnormal; no overflow handling needed here)."""
    if v == 0:
        return np.float32(0.0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)  # subnormals share the smallest normal's quantum
    quantum = Fraction(2) ** (e - 23)
    q, rem = divmod(a, quantum)
    q = int(q)
    if rem * 2 > quantum or (rem * 2 == quantum and q % 2 == 1):
        q += 1
    return np.float32(sign * float(q * quantum))


def fma_f32(a, b, c):
    """fl(a * b + c) with one rounding: IEEE fusedMultiplyAdd in binary32."""
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def add_f32(a, b):
    return round_f32(Fraction(float(a)) + Fraction(float(b)))


F16_EDGES = [0x0000, 0x8000, 0x0001, 0x83FF, 0x0400, 0x7BFF, 0xFBFF, 0x3C00]
BF16_EDGES = [0x0000, 0x8000, 0x0001, 0x807F, 0x0080, 0x7F7F, 0xFF7F, 0x3F80, 0xC000]


def _half_values(count, seed, edges, exponent_mask):
    lcg = Lcg(seed)
    out = np.empty(count, np.uint16)
    for i in range(count):
        state = lcg.next()
        h = edges[i] if i < len(edges) else state >> 16
        if (h & exponent_mask) == exponent_mask:  # never infinity or NaN
            h &= 0xBFFF
        out[i] = h
    return out


def f16_edge_values(count):
    """F16 values as stored (little-endian bytes), unpack_f16_test.cpp:24-35."""
    return _half_values(count, 0x6C078965, F16_EDGES, 0x7C00).tobytes()


def bf16_edge_values(count):
    """BF16 values as stored (little-endian bytes), unpack_bf16_test.cpp:29-40."""
    return _half_values(count, 0x2545F491, BF16_EDGES, 0x7F80).tobytes()
