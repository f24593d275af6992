"""F32, F16 and BF16 weights on the GPU, against the CPU oracle bit for bit.

The reference's format table registers them beside the quantized formats
(src/core/capability/capability.cpp:57-65) and every product composes with
any format's unpack (format.h:172-191): its own product test runs the w_f32
fixture decoded and prefilled (tests/gpu/matmul_test.cpp:222-268, run in
test_gpu_parity.py's fixture list), and its unpack tests hold F16 and BF16 to
every value bit for bit (tests/gpu/unpack_f16_test.cpp, unpack_bf16_test.cpp).
Here: those unpacks; products of each format decoded and prefilled across K
(x held in registers, staged whole, staged in chunks), decode = prefill, the
fused epilogues and the split along K; the gather over F16 and BF16 tables.
"""

import numpy as np
import pytest

from tests.support import blocks as B
from tests.support.oracle_lib import BF16, F16, F32

pytestmark = pytest.mark.gpu

SILU, GELU = 0, 1


@pytest.fixture(scope="module", params=["AUTO", "CANONICAL", "EXACT_MFMA"])
def ctx(request):
    """Each test three times: under AUTO (the short-step tile where the 128-row
    tile would leave compute units idle), CANONICAL (always the 128-row tile)
    and EXACT_MFMA (every unsplit step on the matrix cores' f32 fused
    multiply-add)."""
    from charlotte_amd import matmul as mm

    c = mm.Context(0)
    c.set_gemm_path(mm.GemmPath[request.param])
    yield c
    c.close()


@pytest.fixture(scope="module")
def run(ctx):
    from tests.support.gpu import Runner

    return Runner(ctx)


def _stored(gtype, values):
    """Values as the file stores them in `gtype`."""
    v = np.ascontiguousarray(values, np.float32)
    if gtype == F32:
        return v.tobytes()
    if gtype == F16:
        return v.astype(np.float16).tobytes()
    return (v.view(np.uint32) >> 16).astype(np.uint16).tobytes()  # bf16 by truncation: any bits are a value


def _data(gtype, rows, columns, tokens, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((rows, columns), dtype=np.float32) * np.float32(0.05)
    return _stored(gtype, w), rng.standard_normal((tokens, columns), dtype=np.float32)


def _check(got, want, what):
    from tests.support.gpu import bits_equal, first_difference

    assert bits_equal(got, want), f"{what}: {first_difference(got, want)}"


@pytest.mark.parametrize("gtype,make", [(F16, B.f16_edge_values), (BF16, B.bf16_edge_values)])
@pytest.mark.parametrize("groups", [1, 3, 33])
def test_unpack_returns_every_value_exactly(oracle, gtype, make, groups):
    """unpack_f16_test.cpp / unpack_bf16_test.cpp: +-0, subnormals, the largest
    finite, then LCG values; every weight bit for bit, -0 included, from a
    piece at a nonzero offset in its allocation."""
    from charlotte_amd import harness as hx

    stored = make(groups * 32)
    buf = hx.Buffer(16 + len(stored))
    buf.write(np.full(16, 0xA5, np.uint8))
    buf.write(np.frombuffer(stored, np.uint8), offset=16)
    out = hx.Buffer(groups * 32 * 4)
    hx.unpack(gtype, buf.ptr + 16, groups * 32, groups, out.ptr)
    hx.sync()
    got = out.read(np.float32)
    want = oracle.dequantize(gtype, stored)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    buf.free()
    out.free()


# K = 64 (30 empty ranges), 1,024 and 2,048 (x in registers), 1,152 (unequal
# ranges), 3,072, then past each format's register budget (x in chunks).
SHAPES = [(F32, 64), (F32, 1024), (F32, 1152), (F32, 2048), (F32, 3072), (F32, 9728),
          (F16, 64), (F16, 1024), (F16, 1152), (F16, 3072), (F16, 4096), (F16, 14336),
          (BF16, 64), (BF16, 1024), (BF16, 1152), (BF16, 3072), (BF16, 12288)]


@pytest.mark.parametrize("gtype,columns", SHAPES)
def test_product_decoded_and_prefilled_is_the_oracles_bits(oracle, run, gtype, columns):
    rows, tokens = 300, 33
    stored, x = _data(gtype, rows, columns, tokens, seed=gtype * 7919 + columns)
    w = run.weight(gtype, rows, columns, stored)
    want = oracle.matmul_f32(gtype, stored, rows, columns, x, threads=16)
    y64, bound = oracle.matmul_f64(gtype, stored, rows, columns, x, threads=16)
    assert (np.abs(want.astype(np.float64) - y64) <= bound).all()
    for steps in (2, 17, 33):
        _check(run.write(w, x, steps), want[:steps], f"type {gtype} K={columns} tokens={steps}")
    for t in (0, 16, 32):
        _check(run.write(w, x[t : t + 1], 1)[0], want[t], f"type {gtype} K={columns} token {t} decoded")
    w.free()


@pytest.mark.parametrize("gtype", [F32, F16, BF16])
def test_epilogues_over_float_weights(oracle, run, gtype):
    """QKV, the gated feed-forward, GatedByInput and a Write with every option,
    decoded and prefilled."""
    from charlotte_amd import matmul as mm

    columns = 1024
    sizes = [256, 128, 128]
    data = [_data(gtype, r, columns, 9, seed=50 + i) for i, r in enumerate(sizes)]
    x = data[0][1]
    ws = [run.weight(gtype, r, columns, s) for r, (s, _) in zip(sizes, data)]
    totals = [oracle.matmul_f32(gtype, s, r, columns, x) for r, (s, _) in zip(sizes, data)]
    for tokens in (1, 9):
        got = run.product([mm.Member(w) for w in ws], x, tokens, sizes, epilogue=mm.Epilogue.QKV)
        for i in range(3):
            _check(got[i], totals[i][:tokens], f"QKV member {i} tokens={tokens}")
        got = run.product([mm.Member(ws[1]), mm.Member(ws[2])], x, tokens, [128],
                          epilogue=mm.Epilogue.GatedActivation, activation=mm.Activation.GeluTanh)[0]
        _check(got, oracle.gated(totals[1], totals[2], activation=GELU)[:tokens], f"gated tokens={tokens}")
        u = np.random.default_rng(3).standard_normal((tokens, 512), dtype=np.float32)
        got = run.product([mm.Member(ws[0])], x, tokens, [256], epilogue=mm.Epilogue.GatedByInput, gate_input=u,
                          gate_input_stride=512, gate_input_column=100)[0]
        _check(got, oracle.gated_by_input(totals[0][:tokens], u[:, 100:356], activation=SILU), "GatedByInput")
        clip = np.array([-1.5, 1.25, -0.3, 0.4], np.float32)
        bias = np.linspace(-0.1, 0.1, 256, dtype=np.float32)
        got = run.product([mm.Member(ws[0])], x, tokens, [256], clip=clip, bias=bias, activated=True)[0]
        clipped = oracle.matmul_f32(gtype, data[0][0], 256, columns, oracle.clamp(x, clip[0], clip[1]))
        _check(got, oracle.finish(clipped, clip=clip, bias=bias, activated=True, activation=SILU)[:tokens],
               f"options tokens={tokens}")
    for w in ws:
        w.free()


@pytest.mark.parametrize("gtype", [F16, BF16, F32])
def test_split_along_k_gives_the_tiled_bits(oracle, run, gtype):
    from charlotte_amd import matmul as mm

    rows, columns = 1000, 2048
    stored, x = _data(gtype, rows, columns, 32, seed=77)
    w = run.weight(gtype, rows, columns, stored)
    want = oracle.matmul_f32(gtype, stored, rows, columns, x, threads=16)
    sums = 4 * mm.range_sum_floats(mm.Epilogue.Write, rows, columns, mm.kAlways)
    assert mm.plan_launch(mm.MatmulLaunch([mm.Member(w)], 16, [16]), 32, gate=mm.kAlways,
                          range_sums_bytes=sums).kernel == mm.Kernel.GEMM_EXACT_SPLIT  # AUTO's plan
    _check(run.write(w, x, 32, gate=mm.kAlways, sums_bytes=sums), want, "split")
    w.free()


@pytest.mark.parametrize("gtype", [F16, BF16, F32])
def test_gather_over_a_float_table(oracle, ctx, gtype):
    """gather.wgsl:21-58 through the table's format: each row exact, scaled."""
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm

    rows, columns, tokens = 500, 1024, 40
    stored, _ = _data(gtype, rows, columns, 1, seed=9)
    table = mm.Weight(ctx, gtype, rows, columns, stored)
    ids = np.random.default_rng(5).integers(0, rows, tokens).astype(np.uint32)
    ib, hb = hx.Buffer.of(ids), hx.Buffer(tokens * columns * 4)
    for scale in (1.0, 0.125, 3.0):
        hb.fill(0xFF)
        mm.gather(ctx, table, ib.ptr, tokens, hb.ptr, scale=scale)
        hx.sync()
        want = oracle.gather(gtype, stored, rows, columns, ids, np.full((tokens, columns), np.nan, np.float32),
                             scale=scale)
        _check(hb.read(np.float32).reshape(tokens, columns), want, f"gather scale {scale}")
    ib.free()
    hb.free()
    table.free()
