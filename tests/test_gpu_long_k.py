"""Decode past K = 8,192 on the GPU, against the CPU oracle bit for bit.

The reference decodes any K of whole 32-weight groups (matmul.h:661-671; the
ranges of matmul.wgsl:134-137 are defined for every G). Past 8,192 x no
longer fits the LDS stage the shorter decodes use, so the kernel stages it a
chunk of groups at a time and every row's chains run on across chunks; the
order of addition is unchanged, so decode is still prefill's bits. Shapes:
just past 8,192, K = 9,728, 13,824 and 14,336 (Llama 3 8B's down
projection, 4,096 x 14,336 in full — Q4_0 there runs the streamed kernel of
gemv_wide.hip, tests/test_gpu_wide.py), rows not whole tiles, every format,
the fused epilogues, the head's last token.
"""

import numpy as np
import pytest

from tests.support.oracle_lib import BF16, F16, Q4_0, Q4_1, Q6_K, Q8_0

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


def _weight(gtype, rows, columns, rng):
    from charlotte_amd import synthetic

    if gtype in (F16, BF16):
        w = rng.standard_normal((rows, columns), dtype=np.float32) * np.float32(0.05)
        return w.astype(np.float16).tobytes() if gtype == F16 else (w.view(np.uint32) >> 16).astype(np.uint16).tobytes()
    return synthetic.weight(rng, gtype, rows, columns)


def _check(got, want, what):
    from tests.support.gpu import bits_equal, first_difference

    assert bits_equal(got, want), f"{what}: {first_difference(got, want)}"


@pytest.mark.parametrize("gtype,rows,columns", [
    (Q4_0, 300, 8224), (Q4_0, 1001, 9728), (Q4_0, 77, 13824), (Q6_K, 512, 9728), (Q6_K, 333, 14336),
    (Q8_0, 300, 9728), (Q4_1, 200, 14336), (F16, 160, 14336), (BF16, 96, 9728), (Q4_0, 1, 17408),
])
def test_long_k_decode_is_the_oracles_bits_and_prefills(oracle, run, gtype, rows, columns):
    from charlotte_amd import matmul as mm

    rng = np.random.default_rng(rows * 31 + columns)
    stored = _weight(gtype, rows, columns, rng)
    x = rng.standard_normal((5, columns), dtype=np.float32)
    w = run.weight(gtype, rows, columns, stored)
    assert mm.plan_launch(mm.MatmulLaunch([mm.Member(w)], 16, [16]), 1).kernel == mm.Kernel.GEMV_CHUNKED
    want = oracle.matmul_f32(gtype, stored, rows, columns, x, threads=16)
    prefilled = run.write(w, x, 5)
    _check(prefilled, want, f"{gtype} {rows}x{columns} prefill")
    for t in (0, 3, 4):
        _check(run.write(w, x[t : t + 1], 1)[0], want[t], f"{gtype} {rows}x{columns} token {t} decoded")
    last = run.write(w, x, 5, rows=mm.Rows.LastToken)
    _check(last[0], want[4], "the last token of 5")
    w.free()


def test_llama_3_8b_down_projection_in_full(oracle, run):
    """4,096 rows x K = 14,336, Q4_0: one decode, every output the oracle's bits."""
    from charlotte_amd import synthetic

    rng = np.random.default_rng(14336)
    stored = synthetic.q4_0(rng, 4096, 14336)
    x = synthetic.activations(rng, 1, 14336)
    w = run.weight(Q4_0, 4096, 14336, stored)
    _check(run.write(w, x, 1), oracle.matmul_f32(Q4_0, stored, 4096, 14336, x, threads=16), "4096 x 14336")
    w.free()


def test_long_k_fused_epilogues(oracle, run):
    """QKV with members at row offsets, gated, GatedByInput and a clipped,
    biased, activated Write at K = 9,728, decoded."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(9728)
    columns = 9728
    sizes = [256, 128, 128]
    stored = [synthetic.q4_0(rng, r, columns) for r in sizes]
    x = synthetic.activations(rng, 1, columns)
    ws = [run.weight(Q4_0, r, columns, s) for r, s in zip(sizes, stored)]
    totals = [oracle.matmul_f32(Q4_0, s, r, columns, x, threads=16) for r, s in zip(sizes, stored)]
    got = run.product([mm.Member(w) for w in ws], x, 1, sizes, epilogue=mm.Epilogue.QKV)
    for i in range(3):
        _check(got[i], totals[i], f"QKV member {i}")
    got = run.product([mm.Member(ws[0], row_offset=64, rows=100), mm.Member(ws[1], row_offset=3, rows=20, output_row=100)],
                      x, 1, [120])[0]
    _check(got, np.concatenate([totals[0][:, 64:164], totals[1][:, 3:23]], axis=1), "members at offsets")
    got = run.product([mm.Member(ws[1]), mm.Member(ws[2])], x, 1, [128], epilogue=mm.Epilogue.GatedActivation)[0]
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
