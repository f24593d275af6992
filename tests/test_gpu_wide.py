"""The streamed Q4_0 decode at K = 9,216 .. 16,384 in whole 1,024s
(gemv_wide.hip) on the GPU, against the CPU oracle bit for bit: every span
of groups a range from 9 to 16, rows odd and even, one row, Llama 3 8B's down
projection in full; a token decoded alone the same bits as the token
prefilled; the head's last token; members at any row offset, QKV, gated,
GatedByInput and a clipped, biased, activated Write.
"""

import numpy as np
import pytest

from tests.support.oracle_lib import Q4_0

pytestmark = pytest.mark.gpu

SILU = 0


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


def _check(got, want, what):
    from tests.support.gpu import bits_equal, first_difference

    assert bits_equal(got, want), f"{what}: {first_difference(got, want)}"


def _kernel(w):
    from charlotte_amd import matmul as mm

    return mm.plan_launch(mm.MatmulLaunch([mm.Member(w)], 16, [16]), 1).kernel


@pytest.mark.parametrize("rows,columns", [
    (333, 9216), (1001, 10240), (513, 11264), (2050, 12288), (129, 13312), (77, 14336), (4096, 14336),
    (65, 15360), (1, 16384), (2, 16384),
])
def test_wide_decode_is_the_oracles_bits_and_prefills(oracle, run, rows, columns):
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(rows * 17 + columns)
    stored = synthetic.q4_0(rng, rows, columns)
    x = synthetic.activations(rng, 3, columns)
    w = run.weight(Q4_0, rows, columns, stored)
    assert _kernel(w) == mm.Kernel.GEMV_WIDE
    want = oracle.matmul_f32(Q4_0, stored, rows, columns, x, threads=16)
    for t in (0, 2):
        _check(run.write(w, x[t : t + 1], 1)[0], want[t], f"{rows}x{columns} token {t} decoded")
    _check(run.write(w, x, 3), want, f"{rows}x{columns} prefill")
    _check(run.write(w, x, 3, rows=mm.Rows.LastToken)[0], want[2], "the last token of 3")
    w.free()


def test_wide_members_and_epilogues(oracle, run):
    """At K = 14,336: QKV members, members at odd row offsets, gated,
    GatedByInput and a clipped, biased, activated Write, decoded."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(14336 * 3)
    columns = 14336
    sizes = [256, 129, 129]
    stored = [synthetic.q4_0(rng, r, columns) for r in sizes]
    x = synthetic.activations(rng, 1, columns)
    ws = [run.weight(Q4_0, r, columns, s) for r, s in zip(sizes, stored)]
    totals = [oracle.matmul_f32(Q4_0, s, r, columns, x, threads=16) for r, s in zip(sizes, stored)]
    qkv = mm.MatmulLaunch([mm.Member(w) for w in ws], 16, [16, 16, 16], epilogue=mm.Epilogue.QKV)
    assert mm.plan_launch(qkv, 1).kernel == mm.Kernel.GEMV_WIDE
    got = run.product([mm.Member(w) for w in ws], x, 1, sizes, epilogue=mm.Epilogue.QKV)
    for i in range(3):
        _check(got[i], totals[i], f"QKV member {i}")
    got = run.product([mm.Member(ws[0], row_offset=65, rows=101), mm.Member(ws[1], row_offset=3, rows=20, output_row=101)],
                      x, 1, [121])[0]
    _check(got, np.concatenate([totals[0][:, 65:166], totals[1][:, 3:23]], axis=1), "members at odd offsets")
    got = run.product([mm.Member(ws[1]), mm.Member(ws[2])], x, 1, [129], epilogue=mm.Epilogue.GatedActivation)[0]
    _check(got, oracle.gated(totals[1], totals[2], activation=SILU), "gated")
    u = rng.standard_normal((1, 256), dtype=np.float32)
    got = run.product([mm.Member(ws[0])], x, 1, [256], epilogue=mm.Epilogue.GatedByInput, gate_input=u,
                      gate_input_stride=256)[0]
    _check(got, oracle.gated_by_input(totals[0], u, activation=SILU), "GatedByInput")
    clip = np.array([-1.0, 1.5, -2.0, 2.5], np.float32)
    bias = np.linspace(-1, 1, 256, dtype=np.float32)
    got = run.product([mm.Member(ws[0])], x, 1, [256], clip=clip, bias=bias, activated=True,
                      activation=mm.Activation.GeluTanh)[0]
    clipped = oracle.matmul_f32(Q4_0, stored[0], 256, columns, oracle.clamp(x, clip[0], clip[1]), threads=16)
    _check(got, oracle.finish(clipped, clip=clip, bias=bias, activated=True, activation=1), "options")
    for w in ws:
        w.free()
