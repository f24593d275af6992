"""A product's bounds and bias read where the file keeps them.

The reference keeps a clipped product's four bounds as four F32 scalars beside
its weight, and its bias as an F32 row, all in one buffer (the product span),
and its kernels read each bound from its own word of that span: the launch's
constants carry one word offset per bound (`clip: vec4<u32>`,
src/core/kernels/matmul/matmul.cpp:280-281, matmul.h:275-277). Its test binds
the whole weights buffer as the span and points at the fixture's `clip_*`,
`wide_*` and `bias_q8_0` tensors in place (tests/gpu/matmul_test.cpp:552-650).

Here the whole of matmul_rows.gguf goes to one device buffer, byte for byte, so
every F32 scalar sits at its file offset, 32 bytes from the next (the file's
alignment); each bound is passed as its own pointer into that buffer and the
bias as a pointer to its row there. The weights are uploaded through the GGUF
reader (laid out). Outputs must be the oracle's bits, decoded and prefilled.
"""

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "matmul_rows.gguf")
SILU, SIGMOID = 0, 2


@pytest.fixture(scope="module")
def ctx():
    from charlotte_amd import matmul as mm

    c = mm.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def span():
    """The file's bytes on the device (one buffer), and its tensor index."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    raw = np.fromfile(FIXTURE, np.uint8)
    buf = hx.Buffer.of(raw)
    f = mm.GgufFile(FIXTURE)
    yield buf, f, raw
    f.close()
    buf.free()


@pytest.fixture(scope="module")
def source(oracle):
    # matmul_test.cpp:141: source rows filled with seed 7, amplitude 1.0.
    return oracle.fill(7, 64 * 1024).reshape(64, 1024)


def _tensor(f, name):
    return f.tensors[f.find(name)]


def _scalar(raw, t):
    return np.frombuffer(raw[t.offset : t.offset + 4].tobytes(), np.float32)[0]


def _bounds(span, prefix):
    """Pointers to the four bounds in place, and their values read from the file."""
    buf, f, raw = span
    ts = [_tensor(f, f"{prefix}{k}") for k in ("in_min", "in_max", "out_min", "out_max")]
    return [buf.ptr + t.offset for t in ts], np.array([_scalar(raw, t) for t in ts], np.float32), ts


def _run(ctx, m, x, tokens, width, gate=None, sums_bytes=0):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    xb = hx.Buffer.of(np.ascontiguousarray(x[:tokens], np.float32))
    out = hx.Buffer(tokens * width * 4)
    out.fill(0xFF)
    sums = hx.Buffer(sums_bytes) if sums_bytes else None
    try:
        m.input, m.outputs, m._desc = xb.ptr, [out.ptr], None
        mm.launch(ctx, m, tokens, gate or mm.kNever, sums.ptr if sums else 0, sums_bytes)
        hx.sync()
        return out.read(np.float32).reshape(tokens, width)
    finally:
        for b in (xb, out, sums):
            if b:
                b.free()


def _check(got, want, what):
    from tests.support.gpu import bits_equal, first_difference

    assert bits_equal(got, want), f"{what}: {first_difference(got, want)}"


def test_bounds_lie_apart_in_the_file(span):
    """The layout the ABI must bind: four scalars 32 bytes apart, not one vector."""
    _, f, _ = span
    for prefix in ("clip_", "wide_"):
        _, _, ts = _bounds(span, prefix)
        offsets = [t.offset for t in ts]
        assert [b - a for a, b in zip(offsets, offsets[1:])] == [32, 32, 32]
        assert all(t.gguf_type == 0 and t.bytes == 4 for t in ts)


def test_write_clamped_biased_activated_in_place(oracle, ctx, span, source):
    """matmul_test.cpp:576-606: w_q8_0 with clip_* and bias_q8_0 read in place,
    SiLU; 33 tokens prefilled under a gate that would split any other product
    (an optioned product never splits, matmul.cpp:166-172), token 7 alone the
    same bits; the bounds bind on both sides."""
    from charlotte_amd import matmul as mm

    buf, f, raw = span
    w = f.upload(ctx, "w_q8_0")
    t = _tensor(f, "w_q8_0")
    bias_t = _tensor(f, "bias_q8_0")
    ptrs, clip, _ = _bounds(span, "clip_")
    bias = np.frombuffer(raw[bias_t.offset : bias_t.offset + bias_t.bytes].tobytes(), np.float32)
    x = source[:33]
    xc = oracle.clamp(x, clip[0], clip[1])
    totals = oracle.matmul_f32(t.gguf_type, f.data(t), 48, 1024, xc)
    assert (xc != x).any() and ((totals < clip[2]) | (totals > clip[3])).any()
    want = oracle.finish(totals, clip=clip, bias=bias, activated=True, activation=SILU)
    m = mm.MatmulLaunch([mm.Member(w)], 0x10000, [0x20000], clip=ptrs, bias=buf.ptr + bias_t.offset, activated=True,
                        activation=mm.Activation.SiLU)
    plan = mm.plan_launch(m, 33, gate=mm.kAlways, range_sums_bytes=1 << 24)
    assert plan.kernel == mm.Kernel.GEMM_EXACT_SHORT
    _check(_run(ctx, m, x, 33, 48, gate=mm.kAlways, sums_bytes=1 << 24), want, "prefilled")
    _check(_run(ctx, m, x[7:8], 1, 48)[0], want[7], "token 7 decoded")
    w.free()


def test_wide_bounds_give_the_plain_bits(oracle, ctx, span, source):
    """matmul_test.cpp:608-620: bounds no value reaches, read in place, leave
    the unclamped product's bits."""
    from charlotte_amd import matmul as mm

    _, f, _ = span
    w = f.upload(ctx, "w_q8_0")
    t = _tensor(f, "w_q8_0")
    ptrs, _, _ = _bounds(span, "wide_")
    plain = oracle.matmul_f32(t.gguf_type, f.data(t), 48, 1024, source[:21])
    m = mm.MatmulLaunch([mm.Member(w)], 0, [0], clip=ptrs)
    _check(_run(ctx, m, source, 21, 48), plain, "wide bounds prefilled")
    _check(_run(ctx, m, source[4:5], 1, 48)[0], plain[4], "wide bounds decoded")
    w.free()


def test_glu_halves_clamped_in_place(oracle, ctx, span, source):
    """matmul_test.cpp:622-650: sigmoid(gate) x up over w_glu's halves (up its
    first 72 rows, the gate the second), each clamped to the in-place bounds."""
    from charlotte_amd import matmul as mm

    _, f, _ = span
    w = f.upload(ctx, "w_glu")
    t = _tensor(f, "w_glu")
    ptrs, clip, _ = _bounds(span, "clip_")
    x = source[:33]
    both = oracle.matmul_f32(t.gguf_type, f.data(t), 144, 1024, oracle.clamp(x, clip[0], clip[1]))
    want = oracle.gated(both[:, 72:], both[:, :72], clip=clip, activation=SIGMOID)
    m = mm.MatmulLaunch([mm.Member(w, row_offset=72, rows=72), mm.Member(w, row_offset=0, rows=72)], 0, [0],
                        epilogue=mm.Epilogue.GatedActivation, activation=mm.Activation.Sigmoid, clip=ptrs)
    _check(_run(ctx, m, x, 33, 72), want, "GLU prefilled")
    _check(_run(ctx, m, x[5:6], 1, 72)[0], want[5], "GLU decoded")
    w.free()
