"""Extreme values through every canonical decode kernel and the prefill tile,
against the oracle: weights whose block scales take the reference tests' edge
values (+-0, the smallest and largest subnormal, +-65504; Q6_K sub-block
scales -128 and 127), and inputs holding +inf, NaN, +-1e28, subnormals and -0,
one kind of special a token, and a token whose inputs are all subnormal
(reading them as zero would change its bits). Finite outputs must be the oracle's bits and
NaN outputs NaN (a NaN's payload is not part of the order of addition).
"""

import os

import numpy as np
import pytest

from tests.support import blocks as B
from tests.support.oracle_lib import Q4_0, Q6_K

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))
BLOCK_BYTES = {Q4_0: 18, Q6_K: 210}
D_OFFSET = {Q4_0: 0, Q6_K: 208}  # where a block's fp16 d lies
WEIGHTS_A_BLOCK = {Q4_0: 32, Q6_K: 256}


@pytest.fixture(scope="module", params=["AUTO", "CANONICAL", "EXACT_MFMA"])
def run(request):
    """The prefill under AUTO (the short-step tile for these small steps),
    CANONICAL (the 128-row tile) and EXACT_MFMA (the matrix cores' f32 fused
    multiply-add)."""
    from charlotte_amd import matmul as mm
    from tests.support.gpu import Runner

    c = mm.Context(0)
    c.set_gemm_path(mm.GemmPath[request.param])
    yield Runner(c)
    c.close()


def _edge_weight(gtype, rows, columns, seed=None):
    """The format's edge blocks (their codes and later scales from the LCG at
    `seed`), and every fifth block's d set to one of the edge scales in turn.
    Past 8,192 blocks the first 8,192 repeat (the LCG in Python is slow), the
    edge scales still every fifth block over the whole weight."""
    count = rows * columns // WEIGHTS_A_BLOCK[gtype]
    n = min(count, 8192)
    make = B.q4_0_edge_blocks if gtype == Q4_0 else B.q6_k_edge_blocks
    size, at = BLOCK_BYTES[gtype], D_OFFSET[gtype]
    base = np.frombuffer(make(n) if seed is None else make(n, seed=seed), np.uint8).reshape(n, size)
    stored = np.tile(base, (-(-count // n), 1))[:count].copy()
    scales = np.array(B.EDGE_SCALES, "<u2")[np.arange(-(-count // 5)) % len(B.EDGE_SCALES)]
    stored[::5, at : at + 2] = scales.view(np.uint8).reshape(-1, 2)
    return stored.tobytes()


def _special_inputs(columns, seed):
    """Five tokens: huge (1e28, so most products stay finite against the
    largest weights), subnormal and -0 values; one +inf (inf or NaN where its
    weight is 0); one NaN; plain N(0, 1); N(0, 1) x 1e-39, every input
    subnormal."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((5, columns), dtype=np.float32)
    x[4] = (x[4].astype(np.float64) * 1e-39).astype(np.float32)
    x[0, 3], x[0, 40], x[0, 41], x[0, columns - 1] = 1e28, 1e-40, -1e-42, -0.0
    x[0, 77::97] = np.float32(-1e28)
    x[0, 13::61] = np.float32(3e-39)
    x[1, columns // 2] = np.inf
    x[2, 5] = np.nan
    return x


def _check(got, want, what):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    nan_w, nan_g = np.isnan(want), np.isnan(got)
    assert (nan_w == nan_g).all(), f"{what}: NaN at {np.argwhere(nan_w != nan_g)[:4].tolist()}"
    gb, wb = got[~nan_w].view(np.uint32), want[~nan_w].view(np.uint32)
    bad = np.flatnonzero(gb != wb)
    assert bad.size == 0, f"{what}: {bad.size} differ; first got {got[~nan_w][bad[0]]!r} want {want[~nan_w][bad[0]]!r}"


# (format, rows, K, the decode kernel the plan names): the ranges kernel with
# x in registers and staged in LDS, the L = 4 kernel (rows not whole 16-row
# steps), the streamed K = 1,152 and K = 1,024 / 2,048 Q6_K kernels; the
# streamed Q4_0 kernel at K = 1,024 with its dealing's turn (4,096 steps over
# 2,048 waves: the last round's steps go to the first half of the grid) and
# at K = 8,192; the wide Q4_0 kernel (K = 9,216, an odd number of two-row
# steps' rows); the chunked kernel past K = 8,192.
CASES = [(Q4_0, 256, 1024, "GEMV_RANGES"), (Q4_0, 96, 4096, "GEMV_RANGES"), (Q6_K, 70, 1152, "GEMV_QUARTERS"),
         (Q6_K, 64, 1152, "GEMV_STREAM"), (Q6_K, 64, 1024, "GEMV_STREAM8"), (Q6_K, 48, 2048, "GEMV_STREAM8"),
         (Q4_0, 65536, 1024, "GEMV_STREAM4"), (Q4_0, 4096, 8192, "GEMV_STREAM4"), (Q4_0, 66, 9216, "GEMV_WIDE"),
         (Q6_K, 64, 9216, "GEMV_CHUNKED")]


def _kernel_of(m, tokens=1):
    from charlotte_amd import matmul as mm

    return mm.plan_launch(m, tokens).kernel.name


@pytest.mark.parametrize("gtype,rows,columns,kernel", CASES)
def test_edges_decoded_and_prefilled(oracle, run, gtype, rows, columns, kernel):
    from charlotte_amd import matmul as mm

    stored = _edge_weight(gtype, rows, columns)
    x = _special_inputs(columns, seed=rows + columns)
    w = run.weight(gtype, rows, columns, stored)
    try:
        assert _kernel_of(mm.MatmulLaunch([mm.Member(w)], 0x10000, [0x20000])) == kernel
        want = oracle.matmul_f32(gtype, stored, rows, columns, x, threads=THREADS)
        assert np.isfinite(want[0]).mean() > 0.5 and np.isfinite(want[3]).mean() > 0.5 and np.isnan(want[2]).all()
        for t in range(5):
            got = run.write(w, x[t : t + 1], 1)
            _check(got[0], want[t], f"decode token {t}")
        got = run.write(w, x, 5)
        _check(got, want, "prefill")
    finally:
        w.free()


@pytest.mark.parametrize("gtype,rows,columns,kernels", [
    (Q4_0, 128, 1024, ("GEMV_RANGES", "GEMV_RANGES")), (Q6_K, 64, 1152, ("GEMV_QUARTERS", "GEMV_STREAM")),
    (Q4_0, 66, 9216, ("GEMV_WIDE", "GEMV_WIDE")), (Q4_0, 32768, 1024, ("GEMV_RANGES", "GEMV_STREAM4"))])
def test_edges_through_the_epilogues(oracle, run, gtype, rows, columns, kernels):
    """The same weights and inputs through GatedActivation (SiLU) and Write
    with bias and GELU-tanh: the activations of huge, infinite and NaN
    totals, decoded and prefilled. `kernels`: the decodes of the gated
    product and of the Write, by the plan."""
    from charlotte_amd import matmul as mm

    stored = [_edge_weight(gtype, rows, columns), _edge_weight(gtype, rows, columns, seed=0x68E31DA4)]
    x = _special_inputs(columns, seed=7 * columns)
    ws = [run.weight(gtype, rows, columns, s) for s in stored]
    try:
        gated = mm.MatmulLaunch([mm.Member(ws[0]), mm.Member(ws[1])], 0x10000, [0x20000],
                                epilogue=mm.Epilogue.GatedActivation)
        write = mm.MatmulLaunch([mm.Member(ws[0])], 0x10000, [0x20000], bias=0x30000, activated=True)
        assert (_kernel_of(gated), _kernel_of(write)) == kernels
        gate = oracle.matmul_f32(gtype, stored[0], rows, columns, x, threads=THREADS)
        up = oracle.matmul_f32(gtype, stored[1], rows, columns, x, threads=THREADS)
        want_gated = oracle.gated(gate, up, activation=0)
        bias = np.linspace(-3.0, 3.0, rows, dtype=np.float32)
        want_write = oracle.finish(gate, bias=bias, activated=True, activation=1)
        for t in (0, 1, 3, 4):
            got = run.product([mm.Member(ws[0]), mm.Member(ws[1])], x[t : t + 1], 1, [rows],
                              epilogue=mm.Epilogue.GatedActivation, activation=mm.Activation.SiLU)[0]
            _check(got[0], want_gated[t], f"gated decode token {t}")
            got = run.product([mm.Member(ws[0])], x[t : t + 1], 1, [rows], bias=bias, activated=True,
                              activation=mm.Activation.GeluTanh)[0]
            _check(got[0], want_write[t], f"write decode token {t}")
        got = run.product([mm.Member(ws[0]), mm.Member(ws[1])], x, 5, [rows], epilogue=mm.Epilogue.GatedActivation,
                          activation=mm.Activation.SiLU)[0]
        _check(got, want_gated, "gated prefill")
        got = run.product([mm.Member(ws[0])], x, 5, [rows], bias=bias, activated=True,
                          activation=mm.Activation.GeluTanh)[0]
        _check(got, want_write, "write prefill")
    finally:
        for w in ws:
            w.free()
