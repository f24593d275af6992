"""The streamed Q6_K decode at K = 1,024 and 2,048 (gemv_stream8.hip) on the
GPU: the oracle's bits at every shape it takes — from one step to the LM heads
of Qwen3 0.6B (151,936 x 1,024) and Llama 3.2 1B (128,256 x 2,048) — through
members, epilogues and the head's last token; a token's decode the same bits
as its prefill; and its INT8_LIMBS form within the stated tolerance.
"""

import os

import numpy as np
import pytest

from tests.support.oracle_lib import Q6_K

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def ctx():
    from charlotte_amd import matmul as mm

    c = mm.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def run(ctx):
    from tests.support.gpu import Runner

    return Runner(ctx)


@pytest.fixture(scope="module")
def limbs_run():
    from charlotte_amd import matmul as mm
    from tests.support.gpu import Runner

    c = mm.Context(0)
    c.set_gemv_path(mm.GemvPath.INT8_LIMBS)
    yield Runner(c)
    c.close()


def _data(rows, columns, seed, tokens=1):
    from charlotte_amd import synthetic

    rng = np.random.default_rng(seed)
    return synthetic.q6_k(rng, rows, columns), synthetic.activations(rng, tokens, columns)


SHAPES = [(16, 1024), (48, 1024), (4096, 1024), (151936, 1024), (8, 2048), (24, 2048), (4096, 2048), (128256, 2048)]


@pytest.mark.parametrize("rows,columns", SHAPES)
def test_stream8_decode_is_the_oracles_bits(oracle, run, rows, columns):
    from tests.support.gpu import bits_equal, first_difference

    stored, x = _data(rows, columns, seed=rows + columns)
    w = run.weight(Q6_K, rows, columns, stored)
    got = run.write(w, x, 1)
    want = oracle.matmul_f32(Q6_K, stored, rows, columns, x, threads=THREADS)
    assert bits_equal(got, want), first_difference(got, want)
    w.free()


@pytest.mark.parametrize("columns", [1024, 2048])
def test_stream8_members_epilogues_and_the_head(oracle, run, columns):
    """QKV members at their output rows, Write with clip, bias and activation,
    and the last of three token rows: the oracle's bits."""
    from charlotte_amd import matmul as mm
    from tests.support.gpu import bits_equal, first_difference

    widths = [256, 64, 64]
    data = [_data(r, columns, seed=70 + i + columns) for i, r in enumerate(widths)]
    x = data[0][1]
    ws = [run.weight(Q6_K, r, columns, d[0]) for r, d in zip(widths, data)]
    got = run.product([mm.Member(w) for w in ws], x, 1, widths, epilogue=mm.Epilogue.QKV)
    for i, (r, d) in enumerate(zip(widths, data)):
        want = oracle.matmul_f32(Q6_K, d[0], r, columns, x)
        assert bits_equal(got[i], want), f"member {i}: " + str(first_difference(got[i], want))
    clip = np.array([-1.0, 1.5, -3.0, 2.5], np.float32)
    bias = np.linspace(-0.5, 0.5, 256, dtype=np.float32)
    for activation in (mm.Activation.SiLU, mm.Activation.GeluTanh, mm.Activation.Sigmoid):
        got = run.product([mm.Member(ws[0])], x, 1, [256], clip=clip, bias=bias, activated=True,
                          activation=activation)[0]
        totals = oracle.matmul_f32(Q6_K, data[0][0], 256, columns, oracle.clamp(x, clip[0], clip[1]))
        want = oracle.finish(totals, clip=clip, bias=bias, activated=True, activation=int(activation))
        assert bits_equal(got, want), f"{activation.name}: " + str(first_difference(got, want))
    xs = np.concatenate([np.random.default_rng(9).standard_normal((2, columns), dtype=np.float32), x])
    got = run.write(ws[0], xs, 3, rows=mm.Rows.LastToken)
    want = oracle.matmul_f32(Q6_K, data[0][0], 256, columns, x)
    assert bits_equal(got, want), first_difference(got, want)
    for w in ws:
        w.free()


@pytest.mark.parametrize("rows,columns", [(4096, 1024), (2048, 2048)])
def test_stream8_decode_matches_prefill(run, rows, columns):
    """A token decoded alone and the same token prefilled in a step of 5: the
    same bits (the consistency the reference tracks)."""
    from tests.support.gpu import bits_equal, first_difference

    stored, x = _data(rows, columns, seed=3 * rows, tokens=5)
    w = run.weight(Q6_K, rows, columns, stored)
    prefill = run.write(w, x, 5)
    for t in (0, 4):
        alone = run.write(w, x[t : t + 1], 1)
        assert bits_equal(alone[0], prefill[t]), first_difference(alone[0], prefill[t])
    w.free()


@pytest.mark.parametrize("rows,columns", [(4096, 1024), (151936, 1024), (4096, 2048), (128256, 2048)])
def test_stream8_limbs_within_tolerance(oracle, limbs_run, rows, columns):
    stored, x = _data(rows, columns, seed=rows + 7 * columns)
    w = limbs_run.weight(Q6_K, rows, columns, stored)
    got = limbs_run.write(w, x, 1)
    w.free()
    assert np.isfinite(got).all()
    canonical = oracle.matmul_f32(Q6_K, stored, rows, columns, x, threads=THREADS)
    if rows <= 4096:
        y64, _ = oracle.matmul_f64(Q6_K, stored, rows, columns, x, threads=THREADS)
    else:
        y64 = canonical.astype(np.float64)  # the reference order, itself within gamma(2K) of f64
    err = np.abs(got.astype(np.float64) - y64).max()
    top = np.abs(y64).max()
    assert err <= 1e-5 * top, f"{err:.3e} vs {top:.3e} ({err / top:.2e})"
    a, b = int(np.argmax(got)), int(np.argmax(canonical))
    if a != b:
        s = np.sort(y64[0])
        assert s[-1] - s[-2] <= 2 * err


@pytest.mark.parametrize("columns", [1024, 2048])
def test_stream8_limbs_members_epilogues_and_the_head(oracle, limbs_run, columns):
    """The INT8_LIMBS form through QKV members, Write with clip, bias and
    activation, and the head's last token: within the bar of the f64 totals
    the epilogue is applied to."""
    from charlotte_amd import matmul as mm

    def within(got, want64, what):
        err = np.abs(got.astype(np.float64) - want64).max()
        top = np.abs(want64).max()
        assert np.isfinite(got).all() and err <= 1e-5 * top, f"{what}: {err:.3e} vs {top:.3e}"

    widths = [256, 64, 64]
    data = [_data(r, columns, seed=90 + i + columns) for i, r in enumerate(widths)]
    x = data[0][1]
    ws = [limbs_run.weight(Q6_K, r, columns, d[0]) for r, d in zip(widths, data)]
    got = limbs_run.product([mm.Member(w) for w in ws], x, 1, widths, epilogue=mm.Epilogue.QKV)
    for i, (r, d) in enumerate(zip(widths, data)):
        within(got[i], oracle.matmul_f64(Q6_K, d[0], r, columns, x)[0], f"member {i}")
    clip = np.array([-1.0, 1.5, -3.0, 2.5], np.float32)
    bias = np.linspace(-0.5, 0.5, 256, dtype=np.float32)
    t64, _ = oracle.matmul_f64(Q6_K, data[0][0], 256, columns, oracle.clamp(x, clip[0], clip[1]))
    got = limbs_run.product([mm.Member(ws[0])], x, 1, [256], clip=clip, bias=bias, activated=True,
                            activation=mm.Activation.SiLU)[0]
    want = oracle.finish(t64.astype(np.float32), clip=clip, bias=bias, activated=True, activation=0)
    within(got, want.astype(np.float64), "Write with options")
    xs = np.concatenate([np.random.default_rng(9).standard_normal((2, columns), dtype=np.float32), x])
    got = limbs_run.write(ws[0], xs, 3, rows=mm.Rows.LastToken)
    within(got, oracle.matmul_f64(Q6_K, data[0][0], 256, columns, x)[0], "last token")
    for w in ws:
        w.free()
