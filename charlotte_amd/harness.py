"""Device memory, streams, events and graphs for tests and the benchmark,
over libcharlotte_hip_harness.so (charlotte_amd/csrc/harness.hip) — plain
HIP, so GPU processes need no framework. Not part of the product's ABI.
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libcharlotte_hip_harness.so")

_c = ctypes
_SIGS = {
    "chx_device_count": (_c.c_int, []),
    "chx_set_device": (_c.c_int, [_c.c_int]),
    "chx_device_name": (_c.c_int, [_c.c_int, _c.c_char_p, _c.c_int]),
    "chx_error_string": (_c.c_char_p, [_c.c_int]),
    "chx_malloc": (_c.c_int, [_c.POINTER(_c.c_void_p), _c.c_uint64]),
    "chx_free": (_c.c_int, [_c.c_void_p]),
    "chx_h2d": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_uint64]),
    "chx_d2h": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_uint64]),
    "chx_d2d": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_uint64]),
    "chx_memset": (_c.c_int, [_c.c_void_p, _c.c_int, _c.c_uint64]),
    "chx_sync": (_c.c_int, []),
    "chx_last_error": (_c.c_int, []),
    "chx_stream_create": (_c.c_int, [_c.POINTER(_c.c_void_p)]),
    "chx_stream_destroy": (_c.c_int, [_c.c_void_p]),
    "chx_stream_sync": (_c.c_int, [_c.c_void_p]),
    "chx_event_create": (_c.c_int, [_c.POINTER(_c.c_void_p)]),
    "chx_event_destroy": (_c.c_int, [_c.c_void_p]),
    "chx_event_record": (_c.c_int, [_c.c_void_p, _c.c_void_p]),
    "chx_event_sync": (_c.c_int, [_c.c_void_p]),
    "chx_event_elapsed_ms": (_c.c_int, [_c.POINTER(_c.c_float), _c.c_void_p, _c.c_void_p]),
    "chx_capture_begin": (_c.c_int, [_c.c_void_p]),
    "chx_capture_begin_global": (_c.c_int, [_c.c_void_p]),
    "chx_capture_end": (_c.c_int, [_c.c_void_p, _c.POINTER(_c.c_void_p)]),
    "chx_graph_launch": (_c.c_int, [_c.c_void_p, _c.c_void_p]),
    "chx_graph_destroy": (_c.c_int, [_c.c_void_p]),
    "chx_unpack": (_c.c_int, [_c.c_uint32, _c.c_void_p, _c.c_uint64, _c.c_uint64, _c.c_void_p, _c.c_void_p]),
    "chx_copy": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_uint64, _c.c_void_p]),
    "chx_null": (_c.c_int, [_c.c_void_p]),
    "chx_read_sink_bytes": (_c.c_int, [_c.POINTER(_c.c_uint64)]),
    "chx_read": (_c.c_int, [_c.c_void_p, _c.c_uint64, _c.c_void_p, _c.c_uint64, _c.c_void_p]),
    "chx_touch": (_c.c_int, [_c.c_void_p, _c.c_uint32, _c.c_uint32, _c.c_void_p, _c.c_uint64, _c.c_void_p]),
    "chx_mfma_rate": (_c.c_int, [_c.c_int, _c.c_int, _c.c_uint32, _c.c_uint32, _c.c_void_p, _c.c_uint64, _c.c_void_p]),
    "chx_read_sweep": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_uint32, _c.c_uint32, _c.c_void_p,
                                  _c.c_uint64, _c.c_void_p, _c.c_uint64, _c.c_void_p]),
    "chx_mfma_fma_check": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_void_p, _c.c_uint32, _c.c_uint32, _c.c_void_p,
                                      _c.c_void_p]),
    "chx_mfma_layout": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_void_p]),
    "chx_mfma_c_probe": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_void_p, _c.c_void_p]),
    "chx_mfma_chain_check": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_void_p, _c.c_uint32, _c.c_uint32, _c.c_void_p,
                                        _c.c_void_p]),
}


def _load():
    if not os.path.exists(LIBRARY):
        raise ImportError(f"{LIBRARY} is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(LIBRARY)
    for name, (restype, argtypes) in _SIGS.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = restype, argtypes
    return lib


lib = _load()


class HipError(RuntimeError):
    pass


def check(e, what=""):
    if e != 0:
        raise HipError(f"{what}: {lib.chx_error_string(e).decode()} ({e})")


def device_count():
    return lib.chx_device_count()


def device_name(d=0):
    buf = ctypes.create_string_buffer(512)
    check(lib.chx_device_name(d, buf, 512), "device name")
    return buf.value.decode()


def sync():
    check(lib.chx_sync(), "device synchronize")


class Buffer:
    """Device memory of `nbytes` bytes."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib.chx_malloc(ctypes.byref(p), max(self.nbytes, 16)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def of(cls, array):
        a = np.ascontiguousarray(array)
        b = cls(a.nbytes)
        b.write(a)
        return b

    def write(self, array, offset=0):
        a = np.ascontiguousarray(array)
        check(lib.chx_h2d(self.ptr + offset, a.ctypes.data, a.nbytes), "h2d")

    def read(self, dtype=np.float32, count=None, offset=0):
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if count is None else count
        out = np.empty(count, dtype)
        check(lib.chx_d2h(out.ctypes.data, self.ptr + offset, out.nbytes), "d2h")
        return out

    def fill(self, byte):
        check(lib.chx_memset(self.ptr, byte, self.nbytes), "memset")

    def free(self):
        if self.ptr:
            check(lib.chx_free(self.ptr), "hipFree")
            self.ptr = None


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        check(lib.chx_stream_create(ctypes.byref(s)), "stream create")
        self.handle = s.value

    def sync(self):
        check(lib.chx_stream_sync(self.handle), "stream sync")

    def destroy(self):
        if self.handle:
            lib.chx_stream_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(lib.chx_event_create(ctypes.byref(e)), "event create")
        self.handle = e.value

    def record(self, stream=None):
        check(lib.chx_event_record(self.handle, stream.handle if isinstance(stream, Stream) else stream), "event record")

    def sync(self):
        check(lib.chx_event_sync(self.handle), "event sync")

    def elapsed_ms(self, later):
        ms = ctypes.c_float()
        check(lib.chx_event_elapsed_ms(ctypes.byref(ms), self.handle, later.handle), "event elapsed")
        return ms.value

    def destroy(self):
        if self.handle:
            lib.chx_event_destroy(self.handle)
            self.handle = None


class Graph:
    """The launches a callable makes on `stream`, captured once, replayable."""

    def __init__(self, stream: Stream, body, global_mode=False):
        """global_mode: capture in hipStreamCaptureModeGlobal, under which any
        allocation, free or synchronous copy the body makes fails the capture."""
        begin = lib.chx_capture_begin_global if global_mode else lib.chx_capture_begin
        check(begin(stream.handle), "capture begin")
        try:
            body()
        finally:
            exe = ctypes.c_void_p()
            e = lib.chx_capture_end(stream.handle, ctypes.byref(exe))
        check(e, "capture end")
        self.exec = exe.value
        self.stream = stream

    def launch(self):
        check(lib.chx_graph_launch(self.exec, self.stream.handle), "graph launch")

    def destroy(self):
        if self.exec:
            lib.chx_graph_destroy(self.exec)
            self.exec = None


def unpack(gguf_type, piece_ptr, blocks_in_piece, groups, out_ptr, stream=None):
    check(lib.chx_unpack(int(gguf_type), piece_ptr, blocks_in_piece, groups, out_ptr,
                         stream.handle if isinstance(stream, Stream) else stream), "unpack")


def copy(src_ptr, dst_ptr, nbytes, stream=None):
    check(lib.chx_copy(src_ptr, dst_ptr, nbytes, stream.handle if isinstance(stream, Stream) else stream), "copy")


def read_sink_bytes():
    n = _c.c_uint64()
    check(lib.chx_read_sink_bytes(_c.byref(n)), "read sink bytes")
    return n.value


def read(src_ptr, nbytes, sink_ptr, sink_bytes, stream=None):
    """A streaming read of nbytes (whole KB) and nothing else: the copy
    pattern of the LDS-streamed decodes with their arithmetic taken away."""
    check(lib.chx_read(src_ptr, nbytes, sink_ptr, sink_bytes, stream.handle if isinstance(stream, Stream) else stream),
          "read")


def read_sweep(form, u, nt, depth, blocks, threads, src_ptr, nbytes, sink_ptr, sink_bytes, stream=None):
    """One form of the pure-read sweep (chx_read_sweep): 0 registers grid-strided, 1 registers a chunk a
    workgroup (u loads in flight a lane, nt non-temporal), 2 the LDS copy (u KB a wave step, depth steps)."""
    check(lib.chx_read_sweep(form, u, int(nt), depth, blocks, threads, src_ptr, nbytes, sink_ptr, sink_bytes,
                             stream.handle if isinstance(stream, Stream) else stream), "read sweep")


def mfma_rate(shape, chains, blocks, iters, sink_ptr, sink_bytes, stream=None):
    """The matrix-core rate probe (chx_mfma_rate): shape 0 f16 16x16x32, 1 f16 32x32x16, 2 bf16 16x16x32,
    3 i8 16x16x64, 4 i8 32x32x32, 5 f32 32x32x1 (two blocks), 6 f32 16x16x1 (four blocks), 7 f32 32x32x2,
    8 f32 16x16x4; `chains` independent accumulators a wave (at most 4 for shape 5)."""
    check(lib.chx_mfma_rate(shape, chains, blocks, iters, sink_ptr, sink_bytes,
                            stream.handle if isinstance(stream, Stream) else stream), "mfma rate")


def mfma_fma_check(ab_ptr, c_ptr, pairs, blocks, out_ptr, stream=None, shape=5):
    """chx_mfma_fma_check: a K = 1 f32 matrix instruction (shape 5 the 32x32x1 two-block, 6 the 16x16x1
    four-block) against fmaf, bit for bit; out (2 + 256 words): differing, compared, then (pair, element,
    instruction bits, fmaf bits) for the first 64 differing."""
    check(lib.chx_mfma_fma_check(shape, ab_ptr, c_ptr, pairs, blocks, out_ptr,
                                 stream.handle if isinstance(stream, Stream) else stream), "mfma fma check")


def mfma_chain_check(k, ab_ptr, c_ptr, pairs, blocks, out_ptr, stream=None):
    """chx_mfma_chain_check: the K = 2 (32x32x2) or K = 4 (16x16x4) f32 shape against fmaf in k order;
    ab 2 k floats a pair, c 1,024 (k = 2) or 256 (k = 4) a pair; out as mfma_fma_check's."""
    check(lib.chx_mfma_chain_check(k, ab_ptr, c_ptr, pairs, blocks, out_ptr,
                                   stream.handle if isinstance(stream, Stream) else stream), "mfma chain check")


def mfma_layout(out_ptr, stream=None, shape=5):
    """chx_mfma_layout: the lane (+1) each result of a K = 1 f32 shape (5 the 32x32x1, 32 registers; 6 the
    16x16x1, 16) took its a from, then its b: 2 x 64 x registers floats, [64 v + lane]."""
    check(lib.chx_mfma_layout(shape, out_ptr, stream.handle if isinstance(stream, Stream) else stream),
          "mfma layout")


def mfma_c_probe(shape, c_ptr, out_ptr, stream=None):
    """chx_mfma_c_probe: D of a = b = 0 and C = c (2,048 floats, c[64 v + lane]) written at C's places."""
    check(lib.chx_mfma_c_probe(shape, c_ptr, out_ptr, stream.handle if isinstance(stream, Stream) else stream),
          "mfma c probe")


def touch(src_ptr, waves, kib, sink_ptr, sink_bytes, stream=None):
    """`waves` one-wave workgroups each reading `kib` KB and writing a word:
    a small decode's dispatch and round trip with nothing decoded."""
    check(lib.chx_touch(src_ptr, waves, kib, sink_ptr, sink_bytes,
                        stream.handle if isinstance(stream, Stream) else stream), "touch")


def null(stream=None):
    check(lib.chx_null(stream.handle if isinstance(stream, Stream) else stream), "null kernel")
