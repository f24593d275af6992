"""C3 as a workload: Qwen3 0.6B's decode step, every product at its fused
shape, on the GPU against the CPU oracle bit for bit, then the same token
prefilled as the last of four through every product, bit for bit with its
decode.

The step is what the reference's graph launches for one token
(src/core/graph/graph.cpp:216-287): per layer QKV as one product of three
members (q 2,048, k 1,024, v 1,024 rows at K = 1,024, matmul.wgsl:298-314),
o 1,024 x 2,048, gate and up as one gated product (2 x 3,072 at K = 1,024,
SiLU, matmul.wgsl:318-345), down 1,024 x 3,072; 28 layers; then the tied
Q6_K head 151,936 x 1,024. 113 launches. Weights are seeded Q4_0 (Q6_K for
the head) with BASELINE's distributions (charlotte_amd/synthetic.py), x
N(0, 1).

Decode = prefill is the consistency the reference tracks
(tests/gpu/matmul_test.cpp:257-267, forward_test.cpp:67-80).
"""

import numpy as np
import pytest

from tests.support.oracle_lib import Q4_0, Q6_K

pytestmark = pytest.mark.gpu

LAYERS = 28
HIDDEN, Q_ROWS, KV_ROWS, FFN = 1024, 2048, 1024, 3072
HEAD_ROWS = 151936
PREFILL_TOKENS = 4
SILU = 0


@pytest.fixture(scope="module")
def ctx():
    from charlotte_amd import matmul as mm

    c = mm.Context(0)
    yield c
    c.close()


class _Product:
    """One launch of the step: its launch descriptor over device buffers, and
    what the oracle needs to compute its outputs."""

    def __init__(self, kind, weights, stored, shapes, launch, outs, widths):
        self.kind, self.weights, self.stored, self.shapes = kind, weights, stored, shapes
        self.launch, self.outs, self.widths = launch, outs, widths


def _build(ctx, rng, hx, mm, synthetic, xs):
    """The 113 products of one decode step, reading xs[K] (one token)."""
    products = []

    def weight(gtype, rows, columns):
        stored = synthetic.weight(rng, gtype, rows, columns)
        return mm.Weight(ctx, gtype, rows, columns, stored), stored

    for _ in range(LAYERS):
        # QKV: three members, each writing its own output.
        ws, st = zip(*(weight(Q4_0, r, HIDDEN) for r in (Q_ROWS, KV_ROWS, KV_ROWS)))
        outs = [hx.Buffer(4 * r) for r in (Q_ROWS, KV_ROWS, KV_ROWS)]
        launch = mm.MatmulLaunch([mm.Member(w) for w in ws], xs[HIDDEN].ptr, [o.ptr for o in outs],
                                 epilogue=mm.Epilogue.QKV)
        products.append(_Product("qkv", ws, st, [(r, HIDDEN) for r in (Q_ROWS, KV_ROWS, KV_ROWS)], launch, outs,
                                 [Q_ROWS, KV_ROWS, KV_ROWS]))
        # o: 1,024 rows over K = 2,048.
        w, s = weight(Q4_0, HIDDEN, Q_ROWS)
        out = hx.Buffer(4 * HIDDEN)
        products.append(_Product("write", [w], [s], [(HIDDEN, Q_ROWS)],
                                 mm.MatmulLaunch([mm.Member(w)], xs[Q_ROWS].ptr, [out.ptr]), [out], [HIDDEN]))
        # gate and up: one gated product, SiLU(gate) * up.
        ws, st = zip(*(weight(Q4_0, FFN, HIDDEN) for _ in range(2)))
        out = hx.Buffer(4 * FFN)
        launch = mm.MatmulLaunch([mm.Member(w) for w in ws], xs[HIDDEN].ptr, [out.ptr],
                                 epilogue=mm.Epilogue.GatedActivation, activation=mm.Activation.SiLU)
        products.append(_Product("gated", ws, st, [(FFN, HIDDEN)] * 2, launch, [out], [FFN]))
        # down: 1,024 rows over K = 3,072.
        w, s = weight(Q4_0, HIDDEN, FFN)
        out = hx.Buffer(4 * HIDDEN)
        products.append(_Product("write", [w], [s], [(HIDDEN, FFN)],
                                 mm.MatmulLaunch([mm.Member(w)], xs[FFN].ptr, [out.ptr]), [out], [HIDDEN]))
    # The tied head.
    w, s = weight(Q6_K, HEAD_ROWS, HIDDEN)
    out = hx.Buffer(4 * HEAD_ROWS)
    products.append(_Product("write", [w], [s], [(HEAD_ROWS, HIDDEN)],
                             mm.MatmulLaunch([mm.Member(w)], xs[HIDDEN].ptr, [out.ptr]), [out], [HEAD_ROWS]))
    return products


def _oracle_outputs(oracle, p, x):
    """The product's outputs for input rows x [tokens, K], as the oracle computes them."""
    gtype = Q6_K if p.shapes[0] == (HEAD_ROWS, HIDDEN) else Q4_0
    totals = [oracle.matmul_f32(gtype, s, r, c, x, threads=16) for s, (r, c) in zip(p.stored, p.shapes)]
    if p.kind == "gated":
        return [oracle.gated(totals[0], totals[1], activation=SILU)]
    return totals


def test_c3_decode_step_bits_and_prefill_consistency(oracle, ctx):
    from charlotte_amd import harness as hx
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    rng = np.random.default_rng(0xC3C3)
    x1 = {k: synthetic.activations(rng, 1, k) for k in (HIDDEN, Q_ROWS, FFN)}
    xs = {k: hx.Buffer.of(v) for k, v in x1.items()}
    products = _build(ctx, rng, hx, mm, synthetic, xs)
    assert len(products) == 4 * LAYERS + 1
    assert sum(len(p.shapes) for p in products) == 7 * LAYERS + 1  # the 197 unfused GEMVs
    for p in products:
        for o in p.outs:
            o.fill(0xFF)
    # The step, in order on one stream, as the bench launches it.
    for p in products:
        mm.launch(ctx, p.launch, 1)
    hx.sync()
    decoded = [[o.read(np.float32) for o in p.outs] for p in products]
    for i, p in enumerate(products):
        columns = p.shapes[0][1]
        want = _oracle_outputs(oracle, p, x1[columns])
        for m, (got, w) in enumerate(zip(decoded[i], want)):
            assert (got.view(np.uint32) == w[0].view(np.uint32)).all(), \
                f"product {i} ({p.kind}, {p.shapes[m]}) output {m}: {int((got != w[0]).sum())} differ from the oracle"

    # The same token as the last of four, through every product.
    rows = {k: np.concatenate([synthetic.activations(rng, PREFILL_TOKENS - 1, k), v]) for k, v in x1.items()}
    prefill_x = {k: hx.Buffer.of(v) for k, v in rows.items()}
    compared = 0
    for i, p in enumerate(products):
        columns = p.shapes[0][1]
        outs = [hx.Buffer(4 * w * PREFILL_TOKENS) for w in p.widths]
        launch = mm.MatmulLaunch(p.launch.members, prefill_x[columns].ptr, [o.ptr for o in outs],
                                 epilogue=p.launch.epilogue, activation=p.launch.activation)
        mm.launch(ctx, launch, PREFILL_TOKENS)
        hx.sync()
        for m, (o, w) in enumerate(zip(outs, p.widths)):
            last = o.read(np.float32).reshape(PREFILL_TOKENS, w)[-1]
            assert (last.view(np.uint32) == decoded[i][m].view(np.uint32)).all(), \
                f"product {i} ({p.kind}) output {m}: prefilled differs from decoded in {int((last != decoded[i][m]).sum())}"
            compared += w
            o.free()
    assert compared == 28 * (Q_ROWS + 2 * KV_ROWS + HIDDEN + FFN + HIDDEN) + HEAD_ROWS  # 409,984
    for p in products:
        for w in p.weights:
            w.free()
        for o in p.outs:
            o.free()
    for b in (*xs.values(), *prefill_x.values()):
        b.free()
