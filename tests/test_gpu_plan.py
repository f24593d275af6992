"""The decode plan's launch shapes on the GPU: Q4_0 and Q6_K products whose
row counts straddle every boundary of the steps-a-wave rule (one, two, four,
eight ... steps a wave; a batch of loads of each size; one workgroup a CU or
two past 2^20 groups; grids that loop over row tiles) at K = 1,024 (x in
registers, one group a lane), 2,048, 3,072, 4,096 and 8,192 (x staged in LDS),
each against the oracle's bits — the order of addition is the canonical one
whatever the shape, so the plan may change speed but never a bit.
"""

import os

import numpy as np
import pytest

from tests.support.oracle_lib import Q4_0, Q6_K

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def run():
    from charlotte_amd import matmul as mm
    from tests.support.gpu import Runner

    c = mm.Context(0)
    yield Runner(c)
    c.close()


def _check(oracle, run, gtype, rows, columns, seed):
    from charlotte_amd import synthetic
    from tests.support.gpu import bits_equal, first_difference

    rng = np.random.default_rng(seed)
    stored = synthetic.weight(rng, gtype, rows, columns)
    x = synthetic.activations(rng, 1, columns)
    w = run.weight(gtype, rows, columns, stored)
    try:
        got = run.write(w, x, 1)
    finally:
        w.free()
    want = oracle.matmul_f32(gtype, stored, rows, columns, x, threads=THREADS)
    assert bits_equal(got, want), f"{rows} x {columns}: " + str(first_difference(got, want))


# Rows either side of the step boundaries for 256 CUs (one workgroup a CU holds
# 2,048 rows at one step a wave), a ragged last tile, and 2^20 groups.
@pytest.mark.parametrize("rows", [7, 2047, 2048, 2049, 4095, 4097, 8200, 16385, 32768, 40000])
def test_q4_0_k1024_rows_across_the_plan(oracle, run, rows):
    _check(oracle, run, Q4_0, rows, 1024, seed=rows)


@pytest.mark.parametrize("rows,columns", [(2049, 2048), (8193, 2048), (16384, 2048), (4097, 3072), (12000, 3072),
                                          (3000, 4096), (9000, 4096), (1500, 8192), (4096, 8192), (5000, 8192)])
def test_q4_0_wider_k_across_the_plan(oracle, run, rows, columns):
    _check(oracle, run, Q4_0, rows, columns, seed=rows + columns)


def test_q4_0_largest_steps_and_looping_grid(oracle, run):
    """262,136 rows at K = 1,024 (not whole 16-row steps of the streamed
    kernel): 32 steps a wave in batches of 8, more row tiles than the grid
    holds, so each workgroup loops."""
    _check(oracle, run, Q4_0, 262136, 1024, seed=5)


@pytest.mark.parametrize("rows,columns", [(2050, 2048), (9000, 3072), (3000, 8192)])
def test_q6_k_across_the_plan(oracle, run, rows, columns):
    """Q6_K shapes the streamed kernels leave to the ranges kernel."""
    _check(oracle, run, Q6_K, rows, columns, seed=3 * rows + columns)
