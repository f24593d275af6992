"""The allocation-free launch (charlotte_hip_matmul_launch_static) against the
ordinary launch with the caller's range sums: the same bits, and the CPU
oracle's, on two calls in a row — the second smaller, reading what the first
left in the library's static array — a decode, a step whose range sums would
pass the array (tiled instead, as the ordinary launch tiles it with a buffer of
that size), and launches captured in a HIP graph in global capture mode, where
any allocation would fail the capture, replayed with changed inputs."""

import numpy as np
import pytest

from tests.support.oracle_lib import Q4_0, Q6_K

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from charlotte_amd import matmul as mm

    c = mm.Context(0)
    yield c
    c.close()


def _both(ctx, gtype, rows, columns, tokens, seed, oracle, gate=None):
    """The same product through launch (range sums in a caller buffer) and
    launch_static; returns both outputs and the oracle's."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    gate = gate or mm.kAlways
    rng = np.random.default_rng(seed)
    stored = synthetic.weight(rng, gtype, rows, columns)
    x = synthetic.activations(rng, tokens, columns)
    w = mm.Weight(ctx, gtype, rows, columns, stored)
    xb = hx.Buffer.of(x)
    ya, yb = hx.Buffer(4 * tokens * rows), hx.Buffer(4 * tokens * rows)
    ya.fill(0xFF)
    yb.fill(0xFF)
    sums_bytes = 4 * 32 * tokens * rows
    sums = hx.Buffer(sums_bytes)
    m_a = mm.MatmulLaunch([mm.Member(w)], xb.ptr, [ya.ptr])
    m_b = mm.MatmulLaunch([mm.Member(w)], xb.ptr, [yb.ptr])
    plan = mm.plan_launch(m_a, tokens, gate=gate, range_sums_bytes=sums_bytes)
    mm.launch(ctx, m_a, tokens, gate, sums.ptr, sums_bytes)
    mm.launch_static(ctx, m_b, tokens, gate)
    hx.sync()
    got_a = ya.read(np.float32).reshape(tokens, rows)
    got_b = yb.read(np.float32).reshape(tokens, rows)
    want = oracle.matmul_f32(gtype, stored, rows, columns, x, threads=16)
    for b in (xb, ya, yb, sums):
        b.free()
    w.free()
    return plan, got_a, got_b, want


def _same(a, b):
    return (np.ascontiguousarray(a).view(np.uint32) == np.ascontiguousarray(b).view(np.uint32)).all()


def test_static_launch_matches_the_launch_on_two_calls_the_second_smaller(ctx, oracle):
    from charlotte_amd import matmul as mm

    print("no-alloc: call 1, Q4_0 2048 x 2048, 32 tokens, split", flush=True)
    plan, a, b, want = _both(ctx, Q4_0, 2048, 2048, 32, 1, oracle)
    assert plan.kernel == mm.Kernel.GEMM_EXACT_SPLIT
    assert _same(a, want) and _same(b, a)
    print("no-alloc: call 2, Q6_K 512 x 1024, 9 tokens, split", flush=True)
    plan, a, b, want = _both(ctx, Q6_K, 512, 1024, 9, 2, oracle)
    assert plan.kernel == mm.Kernel.GEMM_EXACT_SPLIT
    assert _same(a, want) and _same(b, a)


def test_static_launch_decodes_and_tiles_as_the_launch(ctx, oracle):
    from charlotte_amd import matmul as mm

    print("no-alloc: decode, Q4_0 3072 x 1024", flush=True)
    plan, a, b, want = _both(ctx, Q4_0, 3072, 1024, 1, 3, oracle)
    assert plan.kernel == mm.Kernel.GEMV_RANGES and _same(a, want) and _same(b, a)
    print("no-alloc: tiled (no split gate), Q4_0 256 x 1024, 100 tokens", flush=True)
    plan, a, b, want = _both(ctx, Q4_0, 256, 1024, 100, 4, oracle, gate=mm.kNever)
    assert plan.kernel == mm.Kernel.GEMM_EXACT_SHORT and _same(a, want) and _same(b, a)


def test_static_launch_tiles_a_split_past_its_array(ctx, oracle):
    """A step the gate would split, whose range sums (32 MiB) pass the static
    array, runs the tiled form — what the ordinary launch runs with a buffer of
    the array's size — with the same bits as the split."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rows, columns, tokens = 8192, 2048, 32
    assert 4 * 32 * tokens * rows > mm.STATIC_SCRATCH_BYTES
    print("no-alloc: Q4_0 8192 x 2048, 32 tokens, past the static array", flush=True)
    rng = np.random.default_rng(5)
    stored = synthetic.weight(rng, Q4_0, rows, columns)
    x = synthetic.activations(rng, tokens, columns)
    w = mm.Weight(ctx, Q4_0, rows, columns, stored)
    xb, yb = hx.Buffer.of(x), hx.Buffer(4 * tokens * rows)
    yb.fill(0xFF)
    m = mm.MatmulLaunch([mm.Member(w)], xb.ptr, [yb.ptr])
    assert mm.plan_launch(m, tokens, gate=mm.kAlways, range_sums_bytes=1 << 40).kernel == mm.Kernel.GEMM_EXACT_SPLIT
    assert mm.plan_launch(m, tokens, gate=mm.kAlways,
                          range_sums_bytes=mm.STATIC_SCRATCH_BYTES).kernel == mm.Kernel.GEMM_EXACT_SHORT
    mm.launch_static(ctx, m, tokens, mm.kAlways)
    hx.sync()
    got = yb.read(np.float32).reshape(tokens, rows)
    want = oracle.matmul_f32(Q4_0, stored, rows, columns, x, threads=16)
    for b in (xb, yb):
        b.free()
    w.free()
    assert _same(got, want)


def test_static_launch_replays_from_a_graph_captured_in_global_mode(ctx, oracle):
    """launch_static of a split step and of a decode captured on a stream in
    global capture mode (an allocation, free or synchronous copy anywhere in
    the process would fail it), then replayed three times with the inputs
    changed between replays and the program's own eager launch_static calls
    in between, which leave other contents in the static array: every replay
    is the oracle's bits."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    print("no-alloc: graph capture (global mode) of a split step and a decode", flush=True)
    rng = np.random.default_rng(6)
    shapes = [(Q4_0, 2048, 2048, 32), (Q6_K, 4096, 1152, 1)]
    stored = [synthetic.weight(rng, g, r, c) for g, r, c, _ in shapes]
    inputs = [[synthetic.activations(rng, t, c) for _ in range(2)] for _, _, c, t in shapes]
    ws = [mm.Weight(ctx, g, r, c, s) for (g, r, c, _), s in zip(shapes, stored)]
    xs = [hx.Buffer.of(i[0]) for i in inputs]
    ys = [hx.Buffer(4 * t * r) for _, r, _, t in shapes]
    other_w = mm.Weight(ctx, Q4_0, 512, 1024, synthetic.weight(rng, Q4_0, 512, 1024))
    other_x, other_y = hx.Buffer.of(synthetic.activations(rng, 24, 1024)), hx.Buffer(4 * 24 * 512)
    stream = hx.Stream()
    ms = [mm.MatmulLaunch([mm.Member(w)], x.ptr, [y.ptr]) for w, x, y in zip(ws, xs, ys)]
    other = mm.MatmulLaunch([mm.Member(other_w)], other_x.ptr, [other_y.ptr])
    assert mm.plan_launch(ms[0], 32, gate=mm.kAlways,
                          range_sums_bytes=mm.STATIC_SCRATCH_BYTES).kernel == mm.Kernel.GEMM_EXACT_SPLIT
    want = [[oracle.matmul_f32(g, s, r, c, i, threads=16) for i in ins]
            for (g, r, c, _), s, ins in zip(shapes, stored, inputs)]

    def body():
        for m, (_, _, _, t) in zip(ms, shapes):
            mm.launch_static(ctx, m, t, mm.kAlways, stream=stream.handle)

    graph = hx.Graph(stream, body, global_mode=True)
    try:
        for r in range(3):
            which = (r + 1) % 2
            for x, ins in zip(xs, inputs):
                x.write(ins[which])
            for y in ys:
                y.fill(0xFF)
            hx.sync()
            graph.launch()
            stream.sync()
            for k, (y, (_, rows, _, t)) in enumerate(zip(ys, shapes)):
                got = y.read(np.float32).reshape(t, rows)
                assert _same(got, want[k][which]), f"replay {r}: product {k} differs"
            # eager allocation-free work between replays, through the same static array
            mm.launch_static(ctx, other, 24, mm.kAlways, stream=stream.handle)
            stream.sync()
    finally:
        graph.destroy()
        stream.destroy()
        for b in (*xs, *ys, other_x, other_y):
            b.free()
        for w in (*ws, other_w):
            w.free()
