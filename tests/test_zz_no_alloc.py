"""The allocation-free launch (charlotte_hip_matmul_launch_static) against the
ordinary launch with the caller's range sums: the same bits, and the CPU
oracle's, on two calls in a row — the second smaller, reading what the first
left in the library's static array — a decode, and a step whose range sums
would pass the array (refused)."""

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
    assert plan.kernel == mm.Kernel.GEMM_SPLIT
    assert _same(a, want) and _same(b, a)
    print("no-alloc: call 2, Q6_K 512 x 1024, 9 tokens, split", flush=True)
    plan, a, b, want = _both(ctx, Q6_K, 512, 1024, 9, 2, oracle)
    assert plan.kernel == mm.Kernel.GEMM_SPLIT
    assert _same(a, want) and _same(b, a)


def test_static_launch_decodes_and_tiles_as_the_launch(ctx, oracle):
    from charlotte_amd import matmul as mm

    print("no-alloc: decode, Q4_0 3072 x 1024", flush=True)
    plan, a, b, want = _both(ctx, Q4_0, 3072, 1024, 1, 3, oracle)
    assert plan.kernel == mm.Kernel.GEMV_RANGES and _same(a, want) and _same(b, a)
    print("no-alloc: tiled (no split gate), Q4_0 256 x 1024, 100 tokens", flush=True)
    plan, a, b, want = _both(ctx, Q4_0, 256, 1024, 100, 4, oracle, gate=mm.kNever)
    assert plan.kernel == mm.Kernel.GEMM_TILED and _same(a, want) and _same(b, a)


def test_static_launch_refuses_range_sums_past_its_array(ctx):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    rows, columns, tokens = 8192, 2048, 32  # 32 MiB of range sums
    assert 4 * 32 * tokens * rows > mm.STATIC_SCRATCH_BYTES
    xb, yb = hx.Buffer(4 * tokens * columns), hx.Buffer(4 * tokens * rows)
    real = mm.Weight(ctx, Q4_0, rows, columns, bytes(rows * columns // 32 * 18))
    m = mm.MatmulLaunch([mm.Member(real)], xb.ptr, [yb.ptr])
    assert mm.plan_launch(m, tokens, gate=mm.kAlways, range_sums_bytes=1 << 40).kernel == mm.Kernel.GEMM_SPLIT
    with pytest.raises(mm.MatmulError) as e:
        mm.launch_static(ctx, m, tokens, mm.kAlways)
    assert e.value.status == mm.Status.INVALID_ARGUMENT and "static scratch" in str(e.value)
    # Without a split gate the same step tiles, and runs.
    mm.launch_static(ctx, m, tokens, mm.kNever)
    hx.sync()
    for b in (xb, yb):
        b.free()
    real.free()
