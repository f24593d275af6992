"""The drop-in boundary on the GPU: a divided step (row_divisor), the default
prefill path's bits with a workspace set, and weights a launch refuses.

Follows the reference's tests/gpu/matmul_test.cpp:516-537 ("a product over
the step's tokens divided writes those rows' bits, as a step of that many")
over w_q8_0 and w_f32, and its decode = prefill contract
(matmul_test.cpp:257-267) for the default path.
"""

import numpy as np
import pytest

from tests.support.oracle_lib import Q4_0

pytestmark = pytest.mark.gpu

TOKENS = 64
WIDEST = 3072


@pytest.fixture(scope="module")
def ctx():
    from charlotte_amd import matmul as mm

    c = mm.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def source(oracle):
    return oracle.fill(7, TOKENS * WIDEST)


def _run(ctx, m_kwargs, weight, x, tokens, out_rows):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    xb = hx.Buffer.of(np.ascontiguousarray(x, np.float32))
    yb = hx.Buffer(4 * weight.rows * max(out_rows, 1) + 4 * weight.rows)
    yb.fill(0xFF)
    mm.launch(ctx, mm.MatmulLaunch([mm.Member(weight)], xb.ptr, [yb.ptr], **m_kwargs), tokens)
    hx.sync()
    y = yb.read(np.float32).reshape(-1, weight.rows)
    xb.free()
    yb.free()
    return y


@pytest.mark.parametrize("name", ["w_q8_0", "w_f32"])
def test_a_divided_step_writes_the_bits_of_a_step_of_that_many_rows(oracle, ctx, source, fixture_tensors, name):
    from charlotte_amd import matmul as mm

    t = fixture_tensors[name]
    w = mm.Weight(ctx, t.type, t.rows, t.columns, t.data)
    x = source[: 63 * t.columns].reshape(63, t.columns)
    want = oracle.matmul_f32(t.type, t.data, t.rows, t.columns, x)
    for pooled in (1, 2, 7):
        plain = _run(ctx, {}, w, x[:pooled], pooled, pooled)
        divided = _run(ctx, {"row_divisor": 9}, w, x[: 9 * pooled], 9 * pooled, pooled)
        assert (plain[:pooled].view(np.uint32) == want[:pooled].view(np.uint32)).all()
        assert (divided[:pooled].view(np.uint32) == plain[:pooled].view(np.uint32)).all(), f"{name} pooled {pooled}"
        assert np.isnan(divided[pooled:]).all(), "a divided step wrote past its rows"
    # Fewer tokens than the divisor: nothing runs, nothing is written.
    assert np.isnan(_run(ctx, {"row_divisor": 9}, w, x[:8], 8, 1)).all()
    w.free()


def test_auto_with_a_workspace_keeps_the_bit_exact_tile(oracle, ctx):
    """A drop-in caller that sets a workspace and leaves the path at its default
    gets the reference's bits, decoded and prefilled alike."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(16)
    rows, columns, tokens = 1024, 2048, 64
    stored = synthetic.q4_0(rng, rows, columns)
    x = synthetic.activations(rng, tokens, columns)
    want = oracle.matmul_f32(Q4_0, stored, rows, columns, x, threads=16)
    ws = hx.Buffer(mm.workspace_bytes(tokens, columns))
    ctx.set_workspace(ws.ptr, ws.nbytes)
    try:
        w = mm.Weight(ctx, Q4_0, rows, columns, stored)
        for steps in (16, 33, 64):
            got = _run(ctx, {}, w, x[:steps], steps, steps)[:steps]
            assert (got.view(np.uint32) == want[:steps].view(np.uint32)).all(), f"AUTO {steps} tokens"
        alone = _run(ctx, {}, w, x[40:41], 1, 1)[0]
        assert (alone.view(np.uint32) == want[40].view(np.uint32)).all()
        w.free()
    finally:
        ctx.set_workspace(0, 0)
        ws.free()


def test_a_launch_refuses_a_shape_only_weight(ctx):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    w = mm.Weight.shape(Q4_0, 64, 1024)
    xb, yb = hx.Buffer(4 * 1024), hx.Buffer(4 * 64)
    with pytest.raises(mm.MatmulError) as e:
        mm.launch(ctx, mm.MatmulLaunch([mm.Member(w)], xb.ptr, [yb.ptr]), 1)
    assert e.value.status == mm.Status.INVALID_ARGUMENT and "shape-only" in str(e.value)
    # The same descriptor plans.
    assert mm.plan_launch(mm.MatmulLaunch([mm.Member(w)], xb.ptr, [yb.ptr]), 1).kernel == mm.Kernel.GEMV_RANGES
    hx.sync()
    xb.free()
    yb.free()
    w.free()

