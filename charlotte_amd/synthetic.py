"""Seeded synthetic weights and activations of the benchmark's configurations
(the distributions BASELINE's configs state), as stored GGUF blocks in file
order — what a GGUF file holds and charlotte_hip_matmul_weight_upload takes.

  Q4_0: d = fp16(|N(0,1)| * 0.02), codes uniform 0..15 (offset 8);
        block = d (2 bytes, little-endian) then 16 code bytes, byte j holding
        weight j (low nibble) and j + 16 (high nibble).
  Q6_K: codes uniform 0..63, int8 scales uniform -64..63,
        d = fp16(|N(0,1)| * 0.001); block = ql[128] qh[64] scales[16] d,
        weight l of group k = 4h + r low nibble at nibble r/2 of
        ql[64h + 32(r%2) + l], high pair at bits 2r of qh[32h + l] (ggml's
        block_q6_K).
  Q4_1: d = fp16(|N(0,1)| * 0.02), m = fp16(-8 d), codes uniform 0..15;
        block = d, m, then 16 code bytes as Q4_0's.
  Q8_0: d = fp16(|N(0,1)| * 0.0005), codes uniform -128..127;
        block = d then 32 int8 codes.
  x:    f32 N(0,1).
"""

import numpy as np


def q4_0(rng: np.random.Generator, rows: int, columns: int) -> bytes:
    n = rows * columns // 32
    d = (np.abs(rng.standard_normal(n, dtype=np.float32)) * np.float32(0.02)).astype(np.float16)
    codes = rng.integers(0, 16, size=(n, 32), dtype=np.uint8)
    blocks = np.empty((n, 18), np.uint8)
    blocks[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blocks[:, 2:18] = codes[:, :16] | (codes[:, 16:] << 4)
    return blocks.tobytes()


def q6_k_from_codes(codes: np.ndarray, scales: np.ndarray, d: np.ndarray) -> bytes:
    """Stored Q6_K blocks of codes [n, 256] (0..63), scales [n, 16] (int8), d [n] (fp16)."""
    n = codes.shape[0]
    blocks = np.zeros((n, 210), np.uint8)
    for h in range(2):
        for r in range(4):
            c = codes[:, 128 * h + 32 * r : 128 * h + 32 * r + 32].astype(np.uint8)
            q = 64 * h + 32 * (r % 2)
            blocks[:, q : q + 32] |= (c & 0xF) << (4 * (r // 2))
            blocks[:, 128 + 32 * h : 160 + 32 * h] |= (c >> 4) << (2 * r)
    blocks[:, 192:208] = scales.astype(np.int8).view(np.uint8)
    blocks[:, 208:210] = d.astype(np.float16).view(np.uint8).reshape(n, 2)
    return blocks.tobytes()


def q6_k(rng: np.random.Generator, rows: int, columns: int) -> bytes:
    n = rows * columns // 256
    codes = rng.integers(0, 64, size=(n, 256), dtype=np.uint8)
    scales = rng.integers(-64, 64, size=(n, 16), dtype=np.int16)
    d = (np.abs(rng.standard_normal(n, dtype=np.float32)) * np.float32(0.001)).astype(np.float16)
    return q6_k_from_codes(codes, scales, d)


def q4_1(rng: np.random.Generator, rows: int, columns: int) -> bytes:
    n = rows * columns // 32
    d = (np.abs(rng.standard_normal(n, dtype=np.float32)) * np.float32(0.02)).astype(np.float16)
    m = (d.astype(np.float32) * np.float32(-8.0)).astype(np.float16)
    codes = rng.integers(0, 16, size=(n, 32), dtype=np.uint8)
    blocks = np.empty((n, 20), np.uint8)
    blocks[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blocks[:, 2:4] = m.view(np.uint8).reshape(n, 2)
    blocks[:, 4:20] = codes[:, :16] | (codes[:, 16:] << 4)
    return blocks.tobytes()


def q8_0(rng: np.random.Generator, rows: int, columns: int) -> bytes:
    n = rows * columns // 32
    d = (np.abs(rng.standard_normal(n, dtype=np.float32)) * np.float32(0.0005)).astype(np.float16)
    blocks = np.empty((n, 34), np.uint8)
    blocks[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blocks[:, 2:34] = rng.integers(-128, 128, size=(n, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    return blocks.tobytes()


def f32(rng: np.random.Generator, rows: int, columns: int) -> bytes:
    return (rng.standard_normal((rows, columns)).astype(np.float32) * np.float32(0.05)).tobytes()


def f16(rng: np.random.Generator, rows: int, columns: int) -> bytes:
    return (rng.standard_normal((rows, columns)) * 0.05).astype(np.float16).tobytes()


def bf16(rng: np.random.Generator, rows: int, columns: int) -> bytes:
    bits = (rng.standard_normal((rows, columns)).astype(np.float32) * np.float32(0.05)).view(np.uint32)
    return (bits >> 16).astype(np.uint16).tobytes()  # the upper halves: bf16 by truncation


_MAKERS = {0: f32, 1: f16, 2: q4_0, 3: q4_1, 8: q8_0, 14: q6_k, 30: bf16}
_BLOCKS = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 8: (32, 34), 14: (256, 210), 30: (1, 2)}


def weight(rng, gguf_type: int, rows: int, columns: int) -> bytes:
    return _MAKERS[gguf_type](rng, rows, columns)


def activations(rng: np.random.Generator, tokens: int, columns: int) -> np.ndarray:
    return rng.standard_normal((tokens, columns), dtype=np.float32)


def stored_bytes(gguf_type: int, rows: int, columns: int) -> int:
    per, nbytes = _BLOCKS[gguf_type]
    return rows * columns // per * nbytes
