"""A step's products captured once into a HIP graph and replayed: every replay
the eager launches' bits.

The launches allocate nothing and clear nothing, so a graph of them holds only
kernel nodes; this checks that replays see the buffers as they stand at each
replay (the input changed between replays), that the range sums and the
matrix-core workspace carry nothing from one replay or eager launch to the
next, and that eager work on the same buffers between replays leaves the graph
correct. Every kernel family runs in the step: the ranges and quarters decodes
(one member, QKV, gated), the LDS-streamed Q6_K decodes at K = 1,152 and
1,024, the INT8_LIMBS decode, the split along K, the canonical tile, the
matrix-core prefill and the embedding gather.
"""

import numpy as np
import pytest

from tests.support.oracle_lib import Q4_0, Q6_K

pytestmark = pytest.mark.gpu

REPLAYS = 4


class Step:
    """Weights, inputs and outputs of one step, and the launches that run it."""

    def __init__(self):
        from charlotte_amd import harness as hx
        from charlotte_amd import matmul as mm
        from charlotte_amd import synthetic

        self.hx, self.mm = hx, mm
        rng = np.random.default_rng(20)
        self.ctx = mm.Context(0)
        self.ws = hx.Buffer(mm.workspace_bytes(32, 1152))
        self.ctx.set_workspace(self.ws.ptr, self.ws.nbytes)
        self.limbs = mm.Context(0)
        self.limbs.set_gemv_path(mm.GemvPath.INT8_LIMBS)
        self.stream = hx.Stream()
        self.owned = []
        self.weights = []
        self.outputs = []
        self.calls = []

        def weight(ctx, gtype, rows, columns):
            w = mm.Weight(ctx, gtype, rows, columns, synthetic.weight(rng, gtype, rows, columns))
            self.weights.append(w)
            return w

        def out(floats):
            b = hx.Buffer(floats * 4)
            self.outputs.append(b)
            return b.ptr

        self.x = {}
        self.inputs = {}
        for columns in (1024, 1152, 3072):
            tokens = 32
            self.inputs[columns] = [synthetic.activations(rng, tokens, columns) for _ in range(2)]
            self.x[columns] = hx.Buffer.of(self.inputs[columns][0])
            self.owned.append(self.x[columns])

        def product(ctx, members, columns, tokens, widths, gate=mm.kNever, sums=0, **kw):
            outs = [out(tokens * w) for w in widths]
            m = mm.MatmulLaunch(members, self.x[columns].ptr, outs, **kw)
            nbytes = 0
            if sums:
                b = hx.Buffer(sums)
                self.owned.append(b)
                sums, nbytes = b.ptr, b.nbytes
            self.calls.append(lambda: mm.launch(ctx, m, tokens, gate, sums, nbytes, stream=self.stream.handle))

        c = self.ctx
        product(c, [mm.Member(weight(c, Q4_0, 1024, 1024))], 1024, 1, [1024])
        qkv = [weight(c, Q4_0, r, 1024) for r in (256, 64, 64)]
        product(c, [mm.Member(w) for w in qkv], 1024, 1, [256, 64, 64], epilogue=mm.Epilogue.QKV)
        gated = [weight(c, Q4_0, 512, 1024) for _ in range(2)]
        product(c, [mm.Member(w) for w in gated], 1024, 1, [512], epilogue=mm.Epilogue.GatedActivation)
        product(c, [mm.Member(weight(c, Q4_0, 256, 3072))], 3072, 1, [256])
        product(c, [mm.Member(weight(c, Q6_K, 4096, 1152))], 1152, 1, [4096])
        product(c, [mm.Member(weight(c, Q6_K, 4096, 1024))], 1024, 1, [4096])
        product(self.limbs, [mm.Member(weight(self.limbs, Q6_K, 4096, 1152))], 1152, 1, [4096])
        product(c, [mm.Member(weight(c, Q4_0, 320, 1024))], 1024, 5, [320], gate=mm.kAlways,
                sums=5 * 320 * 32 * 4)
        product(c, [mm.Member(weight(c, Q4_0, 256, 1024))], 1024, 8, [256])
        product(c, [mm.Member(weight(c, Q6_K, 256, 1152))], 1152, 32, [256])
        # the short-step tile's 32 x 32 form, and the whole-K matrix-core tile
        product(c, [mm.Member(weight(c, Q4_0, 8192, 1024))], 1024, 32, [8192])
        product(c, [mm.Member(weight(c, Q4_0, 49152, 1024))], 1024, 32, [49152])
        table = weight(c, Q4_0, 64, 1024)
        ids = hx.Buffer.of(np.array([3, 0, 63, 3, 17], np.uint32))
        self.owned.append(ids)
        hidden = out(5 * 1024)
        self.calls.append(lambda: mm.gather(c, table, ids.ptr, 5, hidden, stream=self.stream.handle))

    def body(self):
        for call in self.calls:
            call()

    def set_input(self, which):
        for columns, b in self.x.items():
            b.write(self.inputs[columns][which])

    def clear(self):
        for o in self.outputs:
            o.fill(0xFF)
        self.hx.sync()

    def read(self):
        self.stream.sync()
        return [o.read(np.uint32) for o in self.outputs]

    def eager(self, which):
        self.set_input(which)
        self.clear()
        self.body()
        return self.read()

    def close(self):
        for b in self.owned + self.outputs:
            b.free()
        for w in self.weights:
            w.free()
        self.stream.destroy()
        self.ctx.close()
        self.limbs.close()
        self.ws.free()


def _same(got, want, what):
    for i, (g, w) in enumerate(zip(got, want)):
        n = int((g != w).sum())
        assert n == 0, f"{what}: output {i} differs in {n} of {w.size} words"


def test_graph_replays_are_the_eager_bits():
    from charlotte_amd import harness as hx

    s = Step()
    try:
        want = [s.eager(0), s.eager(1)]
        for which in (0, 1):
            for o in want[which]:
                assert not (o == 0xFFFFFFFF).all(), "an output was left unwritten"
        _same(s.eager(0), want[0], "eager again")
        s.set_input(0)
        graph = hx.Graph(s.stream, s.body)
        try:
            for r in range(REPLAYS):
                which = r % 2
                s.set_input(which)
                s.clear()
                graph.launch()
                _same(s.read(), want[which], f"replay {r} (input {which})")
                # the program's own eager work on the same buffers between replays
                _same(s.eager(1 - which), want[1 - which], f"eager between replays {r}")
        finally:
            graph.destroy()
    finally:
        s.close()
