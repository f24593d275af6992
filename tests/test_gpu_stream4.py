"""The streamed Q4_0 decode at K = 1,024, 2,048, 4,096 and 8,192 (gemv_stream4.hip)
on the GPU: the oracle's bits at every shape it takes — from its smallest
product, 2^20 groups, to 32,768 x 8,192 — through members at row offsets,
epilogues and the head's last token; smaller products, and rows that are
not whole steps, go to the reference's mapping, the same bits; a token's
decode the same bits as its prefill.
"""

import os

import numpy as np
import pytest

from tests.support.oracle_lib import Q4_0

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


def _data(rows, columns, seed, tokens=1):
    from charlotte_amd import synthetic

    rng = np.random.default_rng(seed)
    return synthetic.weight(rng, Q4_0, rows, columns), synthetic.activations(rng, tokens, columns)


def _kernel(w, rows=None):
    from charlotte_amd import matmul as mm

    rows = w.rows if rows is None else rows
    return mm.plan_launch(mm.MatmulLaunch([mm.Member(w, rows=rows)], 16, [16]), 1).kernel


def _smallest(columns):
    """Rows of the smallest streamed product at this K: 2^20 groups."""
    return 2**20 // (columns // 32)


# Steps are 16, 8, 4 and 2 rows at K = 1,024, 2,048, 4,096 and 8,192; the
# smallest streamed products are 32,768, 16,384, 8,192 and 4,096 rows.
SHAPES = [(32768, 1024), (32784, 1024), (151936, 1024), (262144, 1024), (16384, 2048), (16392, 2048), (8192, 4096), (8196, 4096), (14336, 4096), (4096, 8192), (4098, 8192),
          (32768, 8192)]
SMALL = [(16, 1024), (32752, 1024), (8, 2048), (24, 2048), (8192, 2048), (16376, 2048), (4, 4096), (4100, 4096), (2, 8192), (6, 8192),
         (4094, 8192)]


@pytest.mark.parametrize("rows,columns", SHAPES)
def test_stream4_decode_is_the_oracles_bits(oracle, run, rows, columns):
    from charlotte_amd import matmul as mm
    from tests.support.gpu import bits_equal, first_difference

    stored, x = _data(rows, columns, seed=rows + columns)
    w = run.weight(Q4_0, rows, columns, stored)
    assert _kernel(w) == mm.Kernel.GEMV_STREAM4
    got = run.write(w, x, 1)
    want = oracle.matmul_f32(Q4_0, stored, rows, columns, x, threads=THREADS)
    assert bits_equal(got, want), first_difference(got, want)
    w.free()


@pytest.mark.parametrize("rows,columns", SMALL)
def test_products_under_2_20_groups_take_the_reference_mapping(oracle, run, rows, columns):
    from charlotte_amd import matmul as mm
    from tests.support.gpu import bits_equal, first_difference

    stored, x = _data(rows, columns, seed=rows + columns)
    w = run.weight(Q4_0, rows, columns, stored)
    assert _kernel(w) == mm.Kernel.GEMV_RANGES
    got = run.write(w, x, 1)
    want = oracle.matmul_f32(Q4_0, stored, rows, columns, x, threads=THREADS)
    assert bits_equal(got, want), first_difference(got, want)
    w.free()


@pytest.mark.parametrize("rows,columns", [(32776, 1024), (16388, 2048), (8194, 4096), (4097, 8192)])
def test_rows_not_whole_steps_take_the_reference_mapping(oracle, run, rows, columns):
    from charlotte_amd import matmul as mm
    from tests.support.gpu import bits_equal, first_difference

    stored, x = _data(rows, columns, seed=5 * rows + columns)
    w = run.weight(Q4_0, rows, columns, stored)
    assert _kernel(w) == mm.Kernel.GEMV_RANGES
    got = run.write(w, x, 1)
    want = oracle.matmul_f32(Q4_0, stored, rows, columns, x, threads=THREADS)
    assert bits_equal(got, want), first_difference(got, want)
    w.free()


@pytest.mark.parametrize("columns", [1024, 2048, 4096, 8192])
def test_stream4_members_epilogues_and_the_head(oracle, run, columns):
    """QKV members — one of them rows 64..191 of a larger weight — at their
    output rows, Write with clip, bias and activation, and the last of three
    token rows: the oracle's bits."""
    from charlotte_amd import matmul as mm
    from tests.support.gpu import bits_equal, first_difference

    big = _smallest(columns)
    widths = [big, 64]
    data = [_data(r, columns, seed=70 + i + columns) for i, r in enumerate(widths)]
    x = data[0][1]
    ws = [run.weight(Q4_0, r, columns, d[0]) for r, d in zip(widths, data)]
    members = [mm.Member(ws[0]), mm.Member(ws[1]), mm.Member(ws[0], row_offset=64, rows=128)]
    assert mm.plan_launch(mm.MatmulLaunch(members, 16, [16, 16, 16], epilogue=mm.Epilogue.QKV), 1).kernel == \
        mm.Kernel.GEMV_STREAM4
    got = run.product(members, x, 1, [big, 64, 128], epilogue=mm.Epilogue.QKV)
    full = oracle.matmul_f32(Q4_0, data[0][0], big, columns, x, threads=THREADS)
    wants = [full, oracle.matmul_f32(Q4_0, data[1][0], 64, columns, x), full[:, 64:192]]
    for i, want in enumerate(wants):
        assert bits_equal(got[i], want), f"member {i}: " + str(first_difference(got[i], want))
    clip = np.array([-1.0, 1.5, -3.0, 2.5], np.float32)
    bias = np.linspace(-0.5, 0.5, big, dtype=np.float32)
    assert _kernel(ws[0]) == mm.Kernel.GEMV_STREAM4
    for activation in (mm.Activation.SiLU, mm.Activation.GeluTanh, mm.Activation.Sigmoid):
        got = run.product([mm.Member(ws[0])], x, 1, [big], clip=clip, bias=bias, activated=True,
                          activation=activation)[0]
        totals = oracle.matmul_f32(Q4_0, data[0][0], big, columns, oracle.clamp(x, clip[0], clip[1]),
                                   threads=THREADS)
        want = oracle.finish(totals, clip=clip, bias=bias, activated=True, activation=int(activation))
        assert bits_equal(got, want), f"{activation.name}: " + str(first_difference(got, want))
    xs = np.concatenate([np.random.default_rng(9).standard_normal((2, columns), dtype=np.float32), x])
    got = run.write(ws[0], xs, 3, rows=mm.Rows.LastToken)
    assert bits_equal(got, full), first_difference(got, full)
    for w in ws:
        w.free()


@pytest.mark.parametrize("rows,columns", [(151936, 1024), (16384, 2048), (14336, 4096), (32768, 8192)])
def test_stream4_decode_matches_prefill(run, rows, columns):
    """A token decoded alone and the same token prefilled in a step of 5: the
    same bits (the consistency the reference tracks), at full size."""
    from tests.support.gpu import bits_equal, first_difference

    from charlotte_amd import matmul as mm

    stored, x = _data(rows, columns, seed=3 * rows, tokens=5)
    w = run.weight(Q4_0, rows, columns, stored)
    assert _kernel(w) == mm.Kernel.GEMV_STREAM4
    prefill = run.write(w, x, 5)
    for t in (0, 4):
        alone = run.write(w, x[t : t + 1], 1)
        assert bits_equal(alone[0], prefill[t]), first_difference(alone[0], prefill[t])
    w.free()
