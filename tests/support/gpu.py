"""GPU test helpers: upload a weight, run a product through the C ABI, read
the outputs back (test infrastructure)."""

import numpy as np

from charlotte_amd import harness as hx
from charlotte_amd import matmul as mm


class Runner:
    def __init__(self, ctx: mm.Context):
        self.ctx = ctx

    def weight(self, gtype, rows, columns, stored):
        return mm.Weight(self.ctx, gtype, rows, columns, stored)

    def product(self, members, x, tokens, out_widths, epilogue=mm.Epilogue.Write, rows=mm.Rows.EveryToken,
                out_width=0, gate=mm.kNever, sums_bytes=0, activation=mm.Activation.SiLU, gate_input=None,
                gate_input_stride=0, gate_input_column=0, clip=None, bias=None, activated=False):
        """Run one product over the first `tokens` rows of x; return each output as [rows_written, width].

        gate_input, clip and bias are host arrays, copied to the device for the launch. The
        four clip bounds go to words 32 bytes apart in one buffer, each bound its own
        pointer, as the reference's file keeps them (matmul_rows.gguf's clip_* tensors)."""
        x = np.ascontiguousarray(x, np.float32)
        xb = hx.Buffer.of(x)
        out_rows = 1 if rows == mm.Rows.LastToken else tokens
        outs = [hx.Buffer(out_rows * w * 4) for w in out_widths]
        for o in outs:
            o.fill(0xFF)  # NaN: an output left unwritten shows
        extra = {}
        owned = [xb, *outs]
        for name, value in (("gate_input", gate_input), ("bias", bias)):
            if value is not None:
                b = hx.Buffer.of(np.asarray(value, np.float32))
                extra[name] = b.ptr
                owned.append(b)
        if clip is not None:
            spaced = np.full((4, 8), np.nan, np.float32)  # padding words read as NaN if ever misread
            spaced[:, 0] = np.asarray(clip, np.float32)
            b = hx.Buffer.of(spaced)
            extra["clip"] = [b.ptr + 32 * i for i in range(4)]
            owned.append(b)
        sums = hx.Buffer(sums_bytes) if sums_bytes else None
        if sums:
            sums.fill(0xFF)
            owned.append(sums)
        m = mm.MatmulLaunch(members, xb.ptr, [o.ptr for o in outs], epilogue=epilogue, rows=rows, out_width=out_width,
                            activation=activation, gate_input_stride=gate_input_stride,
                            gate_input_column=gate_input_column, activated=activated, **extra)
        try:
            mm.launch(self.ctx, m, tokens, gate, sums.ptr if sums else 0, sums_bytes)
            hx.sync()
            return [o.read(np.float32).reshape(out_rows, w) for o, w in zip(outs, out_widths)]
        finally:
            for b in owned:
                b.free()

    def write(self, w, x, tokens, rows=mm.Rows.EveryToken, **kw):
        return self.product([mm.Member(w)], x, tokens, [w.rows], rows=rows, **kw)[0]


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


def first_difference(a, b):
    idx = np.argwhere(np.ascontiguousarray(a, np.float32).view(np.uint32) != np.ascontiguousarray(b, np.float32).view(np.uint32))
    if idx.size == 0:
        return None
    i = tuple(idx[0])
    return f"{len(idx)} differ; first at {i}: got {a[i]!r} want {b[i]!r}"
