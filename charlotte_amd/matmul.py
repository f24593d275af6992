"""The matrix product's operator interface, over the C ABI
(include/charlotte_hip_matmul.h, libcharlotte_hip_matmul.so).

It mirrors the reference's operator surface for this path
(src/core/kernels/matmul/matmul.h:594-673): ``Epilogue``, ``MatmulLaunch``,
``SplitGate``, ``split_tokens`` and ``range_sum_floats``. A launch takes
device pointers (ints) for its input and outputs, as the reference's
BufferRanges name device buffers, and runs on a HIP stream. Errors raise
``MatmulError`` carrying the status and the library's message; the library
itself never throws across its ABI.

The native library must be built (``__graft_entry__.build()``); importing
this module without it raises, so nothing can silently run elsewhere.
"""

import ctypes
import enum
import os
from dataclasses import dataclass, field
from typing import Optional, Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
# CHARLOTTE_HIP_MATMUL_LIBRARY names another build of the same ABI.
LIBRARY = os.environ.get("CHARLOTTE_HIP_MATMUL_LIBRARY") or os.path.join(HERE, "libcharlotte_hip_matmul.so")


class Status(enum.IntEnum):
    OK = 0
    INVALID_ARGUMENT = 1
    UNSUPPORTED_TYPE = 2
    SHAPE_NOT_GROUPS = 3
    OUT_OF_MEMORY = 4
    HIP_ERROR = 5
    NO_DEVICE = 6
    UNSUPPORTED = 7
    BAD_FILE = 8
    IO_ERROR = 9


class TensorType(enum.IntEnum):
    """The reference's format table (src/core/capability/capability.cpp:57-65)."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q8_0 = 8
    Q6_K = 14
    BF16 = 30


# Weights a block of each type (src/core/gguf/types.h:65-101).
BLOCK_WEIGHTS = {TensorType.F32: 1, TensorType.F16: 1, TensorType.BF16: 1, TensorType.Q4_0: 32, TensorType.Q4_1: 32,
                 TensorType.Q8_0: 32, TensorType.Q6_K: 256}


class Epilogue(enum.IntEnum):
    Write = 0
    QKV = 1
    GatedActivation = 2
    GatedByInput = 3


class Activation(enum.IntEnum):
    SiLU = 0
    GeluTanh = 1
    Sigmoid = 2


class Rows(enum.IntEnum):
    EveryToken = 0
    LastToken = 1


class GemmPath(enum.IntEnum):
    """The prefill kernel: AUTO (the default), CANONICAL and EXACT_MFMA are
    bit-exact — AUTO runs the matrix cores' f32 fused multiply-add, whole
    (GEMM_EXACT) from three waves a compute unit, else split in the workgroup
    (GEMM_EXACT_SHORT), and its split along K (GEMM_EXACT_SPLIT); CANONICAL
    keeps to the VALU (the 128-row tile, the short-step tile GEMM_SHORT where
    the 128-row tiles would leave compute units idle, GEMM_SPLIT); EXACT_MFMA
    runs every step that does not split on GEMM_EXACT; SPLIT_F16_MFMA, only
    when asked for, the matrix cores within 1e-5."""

    AUTO = 0
    CANONICAL = 1
    SPLIT_F16_MFMA = 2
    EXACT_MFMA = 3


class Kernel(enum.IntEnum):
    """charlotte_hip_matmul_kernel: the kernel a launch's plan runs."""

    NONE = 0
    GEMV_RANGES = 1
    GEMV_QUARTERS = 2
    GEMV_STREAM = 3
    GEMV_STREAM8 = 4
    GEMV_CHUNKED = 5
    GEMV_STREAM4 = 6
    GEMV_WIDE = 7
    GEMM_TILED = 16
    GEMM_SPLIT = 17
    GEMM_MFMA = 18
    GEMM_SHORT = 19
    GEMM_EXACT = 20
    GEMM_EXACT_SPLIT = 21
    GEMM_EXACT_SHORT = 22


class GemvPath(enum.IntEnum):
    """The decode kernel: CANONICAL (bit-exact, the default) or INT8_LIMBS (x as
    three int8 limbs on the dot instructions, within 1e-5; built for the streamed
    shapes: Q6_K at K = 1,024 or 1,152 with rows in 16s and K = 2,048 with rows
    in 8s, Q4_0 at K = 1,024 or 2,048 in products of 2^20 groups or more; other
    shapes decode canonically)."""

    CANONICAL = 0
    INT8_LIMBS = 1


class MatmulError(RuntimeError):
    def __init__(self, status, message=""):
        self.status = Status(status)
        super().__init__(f"{self.status.name}: {message}")


@dataclass(frozen=True)
class SplitGate:
    """kernels::SplitGate (matmul.h:634-646)."""

    numerator: int
    denominator: int
    max_workgroups: int


# The reference's test gates (tests/kernels_matmul_test.cpp:36-39) and its
# measured value (matmul.h:646).
kNever = SplitGate(0, 1, 0)
kAlways = SplitGate(1024, 1, 1024)
kSplitGate = SplitGate(2, 1, 64)


class _Gate(ctypes.Structure):
    _fields_ = [("numerator", ctypes.c_uint32), ("denominator", ctypes.c_uint32), ("max_workgroups", ctypes.c_uint32)]


class _Member(ctypes.Structure):
    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("row_offset", ctypes.c_uint64),
        ("rows", ctypes.c_uint64),
        ("output_row", ctypes.c_uint64),
    ]


class _Desc(ctypes.Structure):
    _fields_ = [
        ("members", _Member * 3),
        ("member_count", ctypes.c_uint32),
        ("epilogue", ctypes.c_uint32),
        ("activation", ctypes.c_uint32),
        ("rows", ctypes.c_uint32),
        ("input", ctypes.c_void_p),
        ("outputs", ctypes.c_void_p * 3),
        ("out_width", ctypes.c_uint64),
        ("gate_input", ctypes.c_void_p),
        ("gate_input_stride", ctypes.c_uint32),
        ("gate_input_column", ctypes.c_uint32),
        ("clip", ctypes.c_void_p * 4),
        ("bias", ctypes.c_void_p),
        ("activated", ctypes.c_uint32),
        ("row_divisor", ctypes.c_uint32),
    ]


class _Target(ctypes.Structure):
    _fields_ = [("compute_units", ctypes.c_uint32), ("gemm_path", ctypes.c_uint32), ("gemv_path", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32), ("workspace_bytes", ctypes.c_uint64)]


class _Plan(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_uint32), ("launches", ctypes.c_uint32), ("canonical", ctypes.c_uint32),
                ("rows", ctypes.c_uint32), ("lanes_a_row", ctypes.c_uint32), ("groups_a_lane", ctypes.c_uint32),
                ("steps_a_wave", ctypes.c_uint32), ("tile_tokens", ctypes.c_uint32), ("tile_rows", ctypes.c_uint32),
                ("chunks", ctypes.c_uint32), ("tiles", ctypes.c_uint64), ("workgroups", ctypes.c_uint64)]


class _GatherDesc(ctypes.Structure):
    _fields_ = [
        ("table", ctypes.c_void_p),
        ("first_row", ctypes.c_uint64),
        ("ids", ctypes.c_void_p),
        ("fed", ctypes.c_void_p),
        ("media", ctypes.c_uint32),
        ("media_token", ctypes.c_uint32),
        ("scale", ctypes.c_float),
        ("hidden", ctypes.c_void_p),
    ]


class _GgufTensor(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("gguf_type", ctypes.c_uint32),
        ("dimension_count", ctypes.c_uint32),
        ("dimensions", ctypes.c_uint64 * 4),
        ("element_count", ctypes.c_uint64),
        ("offset", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
    ]


# Every symbol the header declares, with its ctypes signature.
_c = ctypes
SIGNATURES = {
    "charlotte_hip_matmul_context_create": (_c.c_int, [_c.c_int, _c.POINTER(_c.c_void_p)]),
    "charlotte_hip_matmul_context_destroy": (_c.c_int, [_c.c_void_p]),
    "charlotte_hip_matmul_last_error": (_c.c_char_p, [_c.c_void_p]),
    "charlotte_hip_matmul_set_gemm_path": (_c.c_int, [_c.c_void_p, _c.c_int]),
    "charlotte_hip_matmul_set_gemv_path": (_c.c_int, [_c.c_void_p, _c.c_int]),
    "charlotte_hip_matmul_set_workspace": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_uint64]),
    "charlotte_hip_matmul_workspace_bytes": (_c.c_uint64, [_c.c_uint32, _c.c_uint64]),
    "charlotte_hip_matmul_layout_bytes": (_c.c_uint64, [_c.c_uint32, _c.c_uint64, _c.c_uint64]),
    "charlotte_hip_matmul_lay_out": (_c.c_int, [_c.c_uint32, _c.c_void_p, _c.c_uint64, _c.c_void_p]),
    "charlotte_hip_matmul_repack_q6_k": (_c.c_int, [_c.c_void_p, _c.c_uint64, _c.POINTER(_c.c_void_p)]),
    "charlotte_hip_matmul_weight_upload": (
        _c.c_int,
        [_c.c_void_p, _c.c_uint32, _c.c_uint64, _c.c_uint64, _c.c_void_p, _c.c_uint64, _c.POINTER(_c.c_void_p)],
    ),
    "charlotte_hip_matmul_weight_wrap": (
        _c.c_int,
        [_c.c_void_p, _c.c_uint32, _c.c_uint64, _c.c_uint64, _c.c_void_p, _c.c_uint64, _c.POINTER(_c.c_void_p)],
    ),
    "charlotte_hip_matmul_weight_shape": (
        _c.c_int, [_c.c_uint32, _c.c_uint64, _c.c_uint64, _c.POINTER(_c.c_void_p)]),
    "charlotte_hip_matmul_weight_free": (_c.c_int, [_c.c_void_p]),
    "charlotte_hip_matmul_weight_device": (_c.c_void_p, [_c.c_void_p]),
    "charlotte_hip_matmul_launch": (
        _c.c_int,
        [_c.c_void_p, _c.POINTER(_Desc), _Gate, _c.c_void_p, _c.c_uint64, _c.c_uint32, _c.c_void_p],
    ),
    "charlotte_hip_matmul_launch_static": (
        _c.c_int, [_c.c_void_p, _c.POINTER(_Desc), _Gate, _c.c_uint32, _c.c_void_p]),
    "charlotte_hip_matmul_plan_launch": (
        _c.c_int,
        [_c.POINTER(_Desc), _c.POINTER(_Target), _Gate, _c.c_uint64, _c.c_uint32, _c.POINTER(_Plan), _c.c_char_p,
         _c.c_uint64],
    ),
    "charlotte_hip_matmul_split_tokens": (_c.c_uint32, [_c.c_uint32, _c.c_uint64, _c.c_uint64, _Gate]),
    "charlotte_hip_matmul_range_sum_floats": (_c.c_uint64, [_c.c_uint32, _c.c_uint64, _c.c_uint64, _Gate]),
    "charlotte_hip_matmul_gather": (_c.c_int, [_c.c_void_p, _c.POINTER(_GatherDesc), _c.c_uint32, _c.c_void_p]),
    "charlotte_hip_matmul_gather_positions": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_void_p, _c.c_void_p],
    ),
    "charlotte_hip_matmul_gguf_open": (_c.c_int, [_c.c_char_p, _c.POINTER(_c.c_void_p), _c.POINTER(_c.c_uint32)]),
    "charlotte_hip_matmul_gguf_read": (
        _c.c_int,
        [_c.c_void_p, _c.c_uint64, _c.POINTER(_c.c_void_p), _c.POINTER(_c.c_uint32)],
    ),
    "charlotte_hip_matmul_gguf_error_string": (_c.c_char_p, [_c.c_uint32]),
    "charlotte_hip_matmul_gguf_close": (_c.c_int, [_c.c_void_p]),
    "charlotte_hip_matmul_gguf_tensor_count": (_c.c_uint64, [_c.c_void_p]),
    "charlotte_hip_matmul_gguf_tensor_at": (_c.c_int, [_c.c_void_p, _c.c_uint64, _c.POINTER(_GgufTensor)]),
    "charlotte_hip_matmul_gguf_find": (_c.c_int64, [_c.c_void_p, _c.c_char_p]),
    "charlotte_hip_matmul_gguf_bytes": (_c.c_void_p, [_c.c_void_p]),
    "charlotte_hip_matmul_gguf_upload": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_uint64, _c.POINTER(_c.c_void_p)],
    ),
}


def _load():
    if not os.path.exists(LIBRARY):
        raise ImportError(f"{LIBRARY} is not built: run __graft_entry__.build() (make -C charlotte_amd/csrc)")
    lib = ctypes.CDLL(LIBRARY)
    for name, (restype, argtypes) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = restype
        f.argtypes = argtypes
    return lib


lib = _load()


def _gate(g: SplitGate):
    return _Gate(g.numerator, g.denominator, g.max_workgroups)


def split_tokens(epilogue, rows, columns, gate: SplitGate):
    return lib.charlotte_hip_matmul_split_tokens(int(epilogue), rows, columns, _gate(gate))


def range_sum_floats(epilogue, rows, columns, gate: SplitGate):
    return lib.charlotte_hip_matmul_range_sum_floats(int(epilogue), rows, columns, _gate(gate))


def workspace_bytes(tokens, columns):
    return lib.charlotte_hip_matmul_workspace_bytes(tokens, columns)


def layout_bytes(gguf_type, rows, columns):
    return lib.charlotte_hip_matmul_layout_bytes(int(gguf_type), rows, columns)


def lay_out(gguf_type, stored: bytes, blocks: int) -> bytes:
    """File-order blocks -> the device layout, on the host."""
    per = BLOCK_WEIGHTS[TensorType(gguf_type)]
    out = ctypes.create_string_buffer(layout_bytes(gguf_type, 1, per * blocks) if blocks else 0)
    src = ctypes.create_string_buffer(bytes(stored), len(stored))
    s = lib.charlotte_hip_matmul_lay_out(int(gguf_type), src, blocks, out)
    if s != 0:
        raise MatmulError(s, "lay_out")
    return out.raw


def repack_q6_k(stored: bytes, blocks: int):
    bufs = [ctypes.create_string_buffer(w * blocks) for w in (128, 64, 16, 2)]
    arr = (ctypes.c_void_p * 4)(*[ctypes.cast(b, ctypes.c_void_p) for b in bufs])
    src = ctypes.create_string_buffer(bytes(stored), len(stored))
    s = lib.charlotte_hip_matmul_repack_q6_k(src, blocks, arr)
    if s != 0:
        raise MatmulError(s, "repack_q6_k")
    return [b.raw for b in bufs]


class Context:
    """One device (charlotte_hip_matmul_context)."""

    def __init__(self, device=0):
        h = ctypes.c_void_p()
        s = lib.charlotte_hip_matmul_context_create(device, ctypes.byref(h))
        if s != 0:
            raise MatmulError(s, f"context on device {device}")
        self.handle = h

    def error(self):
        return (lib.charlotte_hip_matmul_last_error(self.handle) or b"").decode()

    def check(self, status):
        if status != 0:
            raise MatmulError(status, self.error())

    gemm_path = GemmPath.AUTO

    def set_gemm_path(self, path: GemmPath):
        self.check(lib.charlotte_hip_matmul_set_gemm_path(self.handle, int(path)))
        self.gemm_path = GemmPath(path)

    def set_gemv_path(self, path: GemvPath):
        self.check(lib.charlotte_hip_matmul_set_gemv_path(self.handle, int(path)))

    def set_workspace(self, device_ptr, nbytes):
        """The matrix-core path's working memory (device pointer, bytes); 0, 0 unsets it."""
        self.check(lib.charlotte_hip_matmul_set_workspace(self.handle, device_ptr or None, nbytes))

    def close(self):
        if self.handle:
            lib.charlotte_hip_matmul_context_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Weight:
    """A weight in the device layout (residency::WeightView of one piece)."""

    def __init__(self, ctx: Context, gguf_type, rows, columns, stored: Optional[bytes] = None, device_piece=None,
                 nbytes=None):
        h = ctypes.c_void_p()
        if device_piece is None:
            buf = ctypes.create_string_buffer(bytes(stored), len(stored)) if not isinstance(stored, ctypes.Array) else stored
            ctx.check(lib.charlotte_hip_matmul_weight_upload(ctx.handle, int(gguf_type), rows, columns, buf,
                                                             len(stored), ctypes.byref(h)))
        else:
            ctx.check(lib.charlotte_hip_matmul_weight_wrap(ctx.handle, int(gguf_type), rows, columns, device_piece,
                                                           nbytes, ctypes.byref(h)))
        self.ctx, self.type, self.rows, self.columns, self.handle = ctx, TensorType(gguf_type), rows, columns, h

    @classmethod
    def shape(cls, gguf_type, rows, columns):
        """A shape-only weight (no device memory), for plans: charlotte_hip_matmul_weight_shape."""
        h = ctypes.c_void_p()
        s = lib.charlotte_hip_matmul_weight_shape(int(gguf_type), rows, columns, ctypes.byref(h))
        if s != 0:
            raise MatmulError(s, f"weight shape {gguf_type} {rows}x{columns}")
        w = cls.__new__(cls)
        w.ctx, w.type, w.rows, w.columns, w.handle = None, TensorType(gguf_type), rows, columns, h
        return w

    @property
    def device(self):
        return lib.charlotte_hip_matmul_weight_device(self.handle)

    def free(self):
        if self.handle:
            lib.charlotte_hip_matmul_weight_free(self.handle)
            self.handle = None


@dataclass
class Member:
    weight: Weight
    row_offset: int = 0
    rows: Optional[int] = None
    output_row: int = 0


@dataclass
class MatmulLaunch:
    """kernels::MatmulLaunch (matmul.h:602-632) with device pointers."""

    members: Sequence[Member]
    input: int
    outputs: Sequence[int]
    epilogue: Epilogue = Epilogue.Write
    activation: Activation = Activation.SiLU
    rows: Rows = Rows.EveryToken
    out_width: int = 0
    gate_input: int = 0
    gate_input_stride: int = 0
    gate_input_column: int = 0
    clip: Sequence[int] = ()  # four device pointers: in_min, in_max, out_min, out_max (or none)
    bias: int = 0
    activated: bool = False
    row_divisor: int = 1
    _desc: Optional[_Desc] = field(default=None, repr=False)

    def desc(self):
        d = _Desc()
        for i, m in enumerate(self.members):
            d.members[i] = _Member(m.weight.handle, m.row_offset, m.weight.rows - m.row_offset if m.rows is None else m.rows,
                                   m.output_row)
        d.member_count = len(self.members)
        d.epilogue, d.activation, d.rows = int(self.epilogue), int(self.activation), int(self.rows)
        d.input = self.input
        for i, o in enumerate(self.outputs):
            d.outputs[i] = o
        d.out_width = self.out_width
        d.gate_input, d.gate_input_stride, d.gate_input_column = self.gate_input, self.gate_input_stride, self.gate_input_column
        for i, bound in enumerate(self.clip):
            d.clip[i] = bound
        d.bias, d.activated = self.bias, int(self.activated)
        d.row_divisor = self.row_divisor
        return d


def launch(ctx: Context, m: MatmulLaunch, tokens: int, gate: SplitGate = kNever, range_sums=0, range_sums_bytes=0,
           stream=None):
    """One product over a step of `tokens` tokens, asynchronous on `stream`."""
    if m._desc is None:
        m._desc = m.desc()
    ctx.check(lib.charlotte_hip_matmul_launch(ctx.handle, ctypes.byref(m._desc), _gate(gate), range_sums,
                                              range_sums_bytes, tokens, stream))


@dataclass(frozen=True)
class Target:
    """What a plan is made for: charlotte_hip_matmul_target."""

    compute_units: int = 256
    gemm_path: GemmPath = GemmPath.AUTO
    gemv_path: GemvPath = GemvPath.CANONICAL
    workspace_bytes: int = 0


@dataclass(frozen=True)
class Plan:
    """charlotte_hip_matmul_plan: the kernel a launch runs and its shape."""

    kernel: Kernel
    launches: int
    canonical: bool
    rows: int
    lanes_a_row: int
    groups_a_lane: int
    steps_a_wave: int
    tile_tokens: int
    tile_rows: int
    chunks: int
    tiles: int
    workgroups: int


def plan_launch(m: MatmulLaunch, tokens: int, target: Target = Target(), gate: SplitGate = kNever,
                range_sums_bytes=0) -> Plan:
    """The plan charlotte_hip_matmul_launch would follow, without a device (the
    reference's pure kernels::matmul_launches, matmul.h:661-673). Raises
    MatmulError with the launch's status and message where the launch would fail."""
    t = _Target(target.compute_units, int(target.gemm_path), int(target.gemv_path), 0, target.workspace_bytes)
    p = _Plan()
    msg = ctypes.create_string_buffer(512)
    s = lib.charlotte_hip_matmul_plan_launch(ctypes.byref(m.desc()), ctypes.byref(t), _gate(gate), range_sums_bytes,
                                             tokens, ctypes.byref(p), msg, len(msg))
    if s != 0:
        raise MatmulError(s, msg.value.decode())
    return Plan(Kernel(p.kernel), p.launches, bool(p.canonical), p.rows, p.lanes_a_row, p.groups_a_lane,
                p.steps_a_wave, p.tile_tokens, p.tile_rows, p.chunks, p.tiles, p.workgroups)


# The allocation-free launch's static range sums, a device (the header's constant).
STATIC_SCRATCH_BYTES = 16 * 1024 * 1024


def launch_static(ctx: Context, m: MatmulLaunch, tokens: int, gate: SplitGate = kNever, stream=None):
    """charlotte_hip_matmul_launch_static: the launch with the split's range sums
    in the library's static array (no allocation, no caller buffer). Calls that
    overlap on one GPU race."""
    if m._desc is None:
        m._desc = m.desc()
    ctx.check(lib.charlotte_hip_matmul_launch_static(ctx.handle, ctypes.byref(m._desc), _gate(gate), tokens, stream))


# ---- the embedding gather (src/core/kernels/gather/gather.h:126-145) ------------


def gather(ctx: Context, table: Weight, ids: int, tokens: int, hidden: int, first_row=0, fed=0, media=False,
           media_token=0, scale=1.0, stream=None):
    """Rows of `hidden` from the table rows of the step's tokens (gather.wgsl:21-58).

    `ids`, `fed` and `hidden` are device pointers; `fed` (or 0) is a fed step's
    draw record, whose first word is every row's token."""
    d = _GatherDesc(table.handle, first_row, ids, fed, int(bool(media)), media_token, scale, hidden)
    ctx.check(lib.charlotte_hip_matmul_gather(ctx.handle, ctypes.byref(d), tokens, stream))


def gather_positions(ctx: Context, table: Weight, positions: int, grid_columns: int, tokens: int, output: int,
                     stream=None):
    """A vision step's learned positions (gather.wgsl:65-84): row r is table row
    r % grid_columns plus table row positions + r // grid_columns."""
    ctx.check(lib.charlotte_hip_matmul_gather_positions(ctx.handle, table.handle, positions, grid_columns, tokens,
                                                        output, stream))


# ---- GGUF files (gguf::read_index, src/core/gguf/reader.cpp) -----------------

# gguf::ReadError (src/core/gguf/types.h:112-141), numbered alike.
class ReadError(enum.IntEnum):
    Ok = 0
    NeedMoreBytes = 1
    ShortRead = 2
    BadMagic = 3
    UnsupportedVersion = 4
    CountTooLarge = 5
    StringTooLong = 6
    ArrayTooLong = 7
    UnknownValueType = 8
    UnknownTensorType = 9
    RowNotWholeBlocks = 10
    TooManyDimensions = 11
    NegativeDimension = 12
    ElementCountOverflow = 13
    OffsetOverflow = 14
    TensorDataOutOfBounds = 15
    DuplicateTensorName = 16
    TensorNameTooLong = 17
    MisalignedTensorData = 18
    OverlappingTensorData = 19
    BadAlignment = 20
    EmptyKey = 21
    DuplicateMetadataKey = 22
    NestedArray = 23
    WrongElementType = 24


class GgufError(RuntimeError):
    def __init__(self, status, read_error):
        self.status = Status(status)
        self.read_error = ReadError(read_error)
        super().__init__(f"{self.status.name}: {self.read_error.name}: "
                         f"{lib.charlotte_hip_matmul_gguf_error_string(read_error).decode()}")


@dataclass(frozen=True)
class GgufTensor:
    """gguf::TensorEntry (src/core/gguf/types.h:191-243): offsets absolute."""

    index: int
    name: str
    gguf_type: int
    dimensions: tuple
    element_count: int
    offset: int
    bytes: int


class GgufFile:
    """A GGUF v3 file's validated tensor index (charlotte_hip_matmul_gguf_*):
    opened from a path (mapped) or read from bytes in memory."""

    def __init__(self, path=None, data: Optional[bytes] = None):
        h = ctypes.c_void_p()
        err = ctypes.c_uint32()
        if path is not None:
            s = lib.charlotte_hip_matmul_gguf_open(os.fsencode(path), ctypes.byref(h), ctypes.byref(err))
        else:
            self._data = ctypes.create_string_buffer(bytes(data), len(data)) if len(data) else None
            s = lib.charlotte_hip_matmul_gguf_read(self._data, len(data), ctypes.byref(h), ctypes.byref(err))
        if s != 0:
            raise GgufError(s, err.value)
        self.handle = h
        self.tensors = []
        for i in range(lib.charlotte_hip_matmul_gguf_tensor_count(h)):
            t = _GgufTensor()
            assert lib.charlotte_hip_matmul_gguf_tensor_at(h, i, ctypes.byref(t)) == 0
            self.tensors.append(GgufTensor(i, t.name.decode(), t.gguf_type, tuple(t.dimensions[: t.dimension_count]),
                                           t.element_count, t.offset, t.bytes))

    def find(self, name) -> int:
        return lib.charlotte_hip_matmul_gguf_find(self.handle, name.encode())

    def data(self, tensor: GgufTensor) -> bytes:
        base = lib.charlotte_hip_matmul_gguf_bytes(self.handle)
        return ctypes.string_at(base + tensor.offset, tensor.bytes)

    def upload(self, ctx: "Context", name) -> "Weight":
        i = self.find(name)
        if i < 0:
            raise KeyError(name)
        t = self.tensors[i]
        h = ctypes.c_void_p()
        ctx.check(lib.charlotte_hip_matmul_gguf_upload(ctx.handle, self.handle, i, ctypes.byref(h)))
        w = Weight.__new__(Weight)
        w.ctx, w.type, w.rows, w.columns, w.handle = ctx, TensorType(t.gguf_type), t.element_count // t.dimensions[0], \
            t.dimensions[0], h
        return w

    def close(self):
        if self.handle:
            lib.charlotte_hip_matmul_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
