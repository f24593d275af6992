"""ctypes bindings to the CPU oracle (oracle/liborc.so) and, where it was
built, oracle/_ref/libref.so (the reference's own dequant/repack code).

Test infrastructure only: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg load these, as the checker.
"""

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
ORACLE_DIR = os.path.join(ROOT, "oracle")

F32, F16, Q4_0, Q4_1, Q8_0, Q6_K, BF16 = 0, 1, 2, 3, 8, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34), Q6_K: (256, 210)}

_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u32p = ctypes.POINTER(ctypes.c_uint32)


def _ptr(a, t):
    return a.ctypes.data_as(t)


def _bytes(b):
    return np.frombuffer(b, dtype=np.uint8) if isinstance(b, (bytes, bytearray)) else np.ascontiguousarray(b, np.uint8)


class Oracle:
    def __init__(self, path=None):
        path = path or os.path.join(ORACLE_DIR, "liborc.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build() or make -C oracle")
        lib = ctypes.CDLL(path)
        lib.orc_fp16_to_fp32.restype = ctypes.c_float
        lib.orc_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        lib.orc_bf16_to_fp32.restype = ctypes.c_float
        lib.orc_bf16_to_fp32.argtypes = [ctypes.c_uint16]
        for f in (lib.orc_dequantize_q4_0, lib.orc_dequantize_q6_k, lib.orc_dequantize_q8_0):
            f.argtypes = [_u8p, ctypes.c_uint64, _f32p]
        lib.orc_dequantize_q4_1.argtypes = [_u8p, ctypes.c_uint64, _f32p, _f32p]
        lib.orc_gather.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, _u32p,
                                   ctypes.c_uint32, _u32p, ctypes.c_int, ctypes.c_uint32, ctypes.c_float, _f32p]
        lib.orc_gather_positions.argtypes = [_f32p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                             ctypes.c_uint32, _f32p]
        lib.orc_dequantize_range.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64, _f32p]
        lib.orc_layout_bytes.restype = ctypes.c_uint64
        lib.orc_layout_bytes.argtypes = [ctypes.c_uint32, ctypes.c_uint64]
        lib.orc_lay_out.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, _u8p]
        lib.orc_repack_q6_k.argtypes = [_u8p, ctypes.c_uint64, _u8p, _u8p, _u8p, _u8p]
        lib.orc_unpack_group.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64, _f32p]
        lib.orc_range_lo.restype = ctypes.c_uint64
        lib.orc_range_lo.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        lib.orc_matmul_f32.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64, _f32p,
                                       ctypes.c_uint32, _f32p, ctypes.c_uint32]
        lib.orc_matmul_f64.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64, _f32p,
                                       ctypes.c_uint32, _f64p, _f64p]
        lib.orc_matmul_f64_threads.argtypes = [ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_uint64, _f32p,
                                               ctypes.c_uint32, _f64p, _f64p, ctypes.c_uint32]
        lib.orc_fill_unit.restype = ctypes.c_float
        lib.orc_fill_unit.argtypes = [ctypes.c_uint32]
        lib.orc_fill.argtypes = [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, _f32p]
        lib.orc_exp_nonpositive.restype = ctypes.c_float
        lib.orc_exp_nonpositive.argtypes = [ctypes.c_float]
        lib.orc_activate.restype = ctypes.c_float
        lib.orc_activate.argtypes = [ctypes.c_uint32, ctypes.c_float]
        lib.orc_now.restype = ctypes.c_double
        lib.orc_clamp.argtypes = [_f32p, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, _f32p]
        lib.orc_finish.argtypes = [_f32p, ctypes.c_uint64, ctypes.c_uint64, _f32p, _f32p, ctypes.c_int,
                                   ctypes.c_uint32, _f32p]
        lib.orc_gated.argtypes = [_f32p, _f32p, ctypes.c_uint64, _f32p, ctypes.c_uint32, _f32p]
        lib.orc_gated_by_input.argtypes = [_f32p, _f32p, ctypes.c_uint64, ctypes.c_uint32, _f32p]
        self.lib = lib

    def fp16_to_fp32(self, h):
        return self.lib.orc_fp16_to_fp32(h)

    def bf16_to_fp32(self, h):
        return self.lib.orc_bf16_to_fp32(h)

    def dequantize(self, gtype, blocks):
        """File-order blocks -> weights (Q4_1: its rounded answer)."""
        b = _bytes(blocks)
        per, nbytes = BLOCK[gtype]
        n = b.size // nbytes
        out = np.empty(n * per, np.float32)
        if gtype in (F16, BF16):
            assert self.lib.orc_dequantize_range(gtype, _ptr(b, _u8p), 0, n, _ptr(out, _f32p)) == 0
            return out
        if gtype == Q4_1:
            self.lib.orc_dequantize_q4_1(_ptr(b, _u8p), n, _ptr(out, _f32p), None)
            return out
        f = {F32: None, Q4_0: self.lib.orc_dequantize_q4_0, Q8_0: self.lib.orc_dequantize_q8_0,
             Q6_K: self.lib.orc_dequantize_q6_k}[gtype]
        if f is None:
            return np.frombuffer(b.tobytes(), np.float32).copy()
        f(_ptr(b, _u8p), n, _ptr(out, _f32p))
        return out

    def dequantize_q4_1(self, blocks):
        """Q4_1's two answers: (rounded, fused)."""
        b = _bytes(blocks)
        n = b.size // 20
        rounded, fused = np.empty(n * 32, np.float32), np.empty(n * 32, np.float32)
        self.lib.orc_dequantize_q4_1(_ptr(b, _u8p), n, _ptr(rounded, _f32p), _ptr(fused, _f32p))
        return rounded, fused

    def gather(self, gtype, stored_rows, row_count, columns, ids, hidden, first_row=0, fed=None, media=False,
               media_token=0, scale=1.0):
        """Writes the step's rows into `hidden` (float32 [tokens][columns]) in place."""
        b = _bytes(stored_rows)
        ids = np.ascontiguousarray(ids, np.uint32)
        f = None if fed is None else np.ascontiguousarray(fed, np.uint32)
        assert hidden.dtype == np.float32 and hidden.flags.c_contiguous and hidden.size >= ids.size * columns
        assert self.lib.orc_gather(gtype, _ptr(b, _u8p), row_count, columns, first_row, _ptr(ids, _u32p), ids.size,
                                   None if f is None else _ptr(f, _u32p), int(media), media_token, scale,
                                   _ptr(hidden, _f32p)) == 0
        return hidden

    def gather_positions(self, table, columns, positions, grid_columns, tokens):
        t = np.ascontiguousarray(table, np.float32)
        out = np.zeros((tokens, columns), np.float32)
        assert self.lib.orc_gather_positions(_ptr(t, _f32p), columns, positions, grid_columns, tokens,
                                             _ptr(out, _f32p)) == 0
        return out

    def layout_bytes(self, gtype, nblocks):
        return self.lib.orc_layout_bytes(gtype, nblocks)

    def lay_out(self, gtype, blocks):
        b = _bytes(blocks)
        n = b.size // BLOCK[gtype][1]
        out = np.zeros(self.layout_bytes(gtype, n), np.uint8)
        assert self.lib.orc_lay_out(gtype, _ptr(b, _u8p), n, _ptr(out, _u8p)) == 0
        return out

    def repack_q6_k(self, blocks):
        b = _bytes(blocks)
        n = b.size // 210
        lo, hi = np.zeros(128 * n, np.uint8), np.zeros(64 * n, np.uint8)
        sc, d = np.zeros(16 * n, np.uint8), np.zeros(2 * n, np.uint8)
        self.lib.orc_repack_q6_k(_ptr(b, _u8p), n, _ptr(lo, _u8p), _ptr(hi, _u8p), _ptr(sc, _u8p), _ptr(d, _u8p))
        return lo, hi, sc, d

    def unpack_group(self, gtype, device, blocks_in_piece, group):
        out = np.empty(32, np.float32)
        assert self.lib.orc_unpack_group(gtype, _ptr(device, _u8p), blocks_in_piece, group, _ptr(out, _f32p)) == 0
        return out

    def range_lo(self, r, groups):
        return self.lib.orc_range_lo(r, groups)

    def matmul_f32(self, gtype, blocks, rows, columns, x, threads=1):
        b = _bytes(blocks)
        x = np.ascontiguousarray(x, np.float32).reshape(-1, columns)
        y = np.empty((x.shape[0], rows), np.float32)
        assert self.lib.orc_matmul_f32(gtype, _ptr(b, _u8p), rows, columns, _ptr(x, _f32p), x.shape[0],
                                       _ptr(y, _f32p), threads) == 0
        return y

    def matmul_f64(self, gtype, blocks, rows, columns, x, threads=1):
        b = _bytes(blocks)
        x = np.ascontiguousarray(x, np.float32).reshape(-1, columns)
        y = np.empty((x.shape[0], rows), np.float64)
        bound = np.empty_like(y)
        if threads == 1:
            status = self.lib.orc_matmul_f64(gtype, _ptr(b, _u8p), rows, columns, _ptr(x, _f32p), x.shape[0],
                                             _ptr(y, _f64p), _ptr(bound, _f64p))
        else:
            status = self.lib.orc_matmul_f64_threads(gtype, _ptr(b, _u8p), rows, columns, _ptr(x, _f32p),
                                                     x.shape[0], _ptr(y, _f64p), _ptr(bound, _f64p), threads)
        assert status == 0
        return y, bound

    def fill(self, seed, count, amplitude=1.0):
        out = np.empty(count, np.float32)
        self.lib.orc_fill(seed, count, amplitude, _ptr(out, _f32p))
        return out

    def activate(self, activation, g):
        return self.lib.orc_activate(activation, g)

    def exp_nonpositive(self, x):
        return self.lib.orc_exp_nonpositive(x)

    # Epilogues over arrays (matmul.wgsl:117-132, 272-351).
    @staticmethod
    def _f32(a):
        return np.ascontiguousarray(a, np.float32)

    def clamp(self, x, lo, hi):
        x = self._f32(x)
        out = np.empty_like(x)
        self.lib.orc_clamp(_ptr(x, _f32p), x.size, lo, hi, _ptr(out, _f32p))
        return out

    def finish(self, totals, clip=None, bias=None, activated=False, activation=0):
        t = self._f32(totals)
        tokens, rows = t.reshape(-1, t.shape[-1]).shape
        c = None if clip is None else self._f32(clip)
        b = None if bias is None else self._f32(bias)
        out = np.empty_like(t)
        self.lib.orc_finish(_ptr(t, _f32p), tokens, rows, None if c is None else _ptr(c, _f32p),
                            None if b is None else _ptr(b, _f32p), int(activated), activation, _ptr(out, _f32p))
        return out

    def gated(self, gate, up, clip=None, activation=0):
        g, u = self._f32(gate), self._f32(up)
        assert g.shape == u.shape
        c = None if clip is None else self._f32(clip)
        out = np.empty_like(g)
        self.lib.orc_gated(_ptr(g, _f32p), _ptr(u, _f32p), g.size, None if c is None else _ptr(c, _f32p),
                           activation, _ptr(out, _f32p))
        return out

    def gated_by_input(self, totals, u, activation=0):
        t, u = self._f32(totals), self._f32(u)
        assert t.shape == u.shape
        out = np.empty_like(t)
        self.lib.orc_gated_by_input(_ptr(t, _f32p), _ptr(u, _f32p), t.size, activation, _ptr(out, _f32p))
        return out


class Reference:
    """The reference's own code (oracle/_ref/libref.so), built here only."""

    def __init__(self, path=None):
        path = path or os.path.join(ORACLE_DIR, "_ref", "libref.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        lib = ctypes.CDLL(path)
        lib.ref_fp16_to_fp32.restype = ctypes.c_float
        lib.ref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        for f in (lib.ref_dequantize_q4_0, lib.ref_dequantize_q6_k, lib.ref_dequantize_q8_0):
            f.argtypes = [_u8p, ctypes.c_uint64, _f32p]
        lib.ref_dequantize_q4_1.argtypes = [_u8p, ctypes.c_uint64, _f32p, _f32p]
        lib.ref_repack_q6_k.argtypes = [_u8p, ctypes.c_uint64, _u8p, _u8p, _u8p, _u8p]
        self.lib = lib

    def fp16_to_fp32(self, h):
        return self.lib.ref_fp16_to_fp32(h)

    def dequantize(self, gtype, blocks):
        b = _bytes(blocks)
        per, nbytes = BLOCK[gtype]
        n = b.size // nbytes
        out = np.empty(n * per, np.float32)
        f = {Q4_0: self.lib.ref_dequantize_q4_0, Q8_0: self.lib.ref_dequantize_q8_0,
             Q6_K: self.lib.ref_dequantize_q6_k}[gtype]
        f(_ptr(b, _u8p), n, _ptr(out, _f32p))
        return out

    def dequantize_q4_1(self, blocks):
        b = _bytes(blocks)
        n = b.size // 20
        rounded, fused = np.empty(n * 32, np.float32), np.empty(n * 32, np.float32)
        self.lib.ref_dequantize_q4_1(_ptr(b, _u8p), n, _ptr(rounded, _f32p), _ptr(fused, _f32p))
        return rounded, fused

    def repack_q6_k(self, blocks):
        b = _bytes(blocks)
        n = b.size // 210
        lo, hi = np.zeros(128 * n, np.uint8), np.zeros(64 * n, np.uint8)
        sc, d = np.zeros(16 * n, np.uint8), np.zeros(2 * n, np.uint8)
        self.lib.ref_repack_q6_k(_ptr(b, _u8p), n, _ptr(lo, _u8p), _ptr(hi, _u8p), _ptr(sc, _u8p), _ptr(d, _u8p))
        return lo, hi, sc, d


def reference_or_none():
    try:
        return Reference()
    except (FileNotFoundError, OSError):
        return None
