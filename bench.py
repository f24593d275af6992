"""Benchmark of the quantized GGUF matmul path on one MI355X.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c1,c2,...]

A step is one pass of the hot path over one batch of synthetic input:
  c1  Q4_0 decode GEMV 3072x1024 (Qwen3-0.6B FFN up)
  c2  Q6_K LM-head GEMV 262144x1152, repacked (Gemma-3-1B)   <- the headline,
      canonical order (bit-exact); again on the INT8_LIMBS decode (x as three
      int8 limbs on the dot instructions, within 1e-5) as c2_limbs
  c3  Qwen3-0.6B decode sweep: 28 layers x 7 Q4_0 GEMVs + Q6_K head 151936x1024,
      launched as the reference's graph does (QKV and gate/up fused: 113 launches)
      and unfused (197)
  c4  Q4_0 prefill GEMM M=512, N=8192, K=2048 (Llama-3.2-1B gate/up)
  c5  Llama-3.2-1B prefill, M=2048, 16 layers x 7 Q4_0 GEMMs (fused as c3) + Q6_K
      head on the last row
  c4, c5 run on the matrix cores (split-f16, within tolerance), again in the
  canonical order as a drop-in caller gets it (AUTO, bit-exact: the matrix
  cores' f32 fused multiply-add tile at these sizes), reported as c4_canonical,
  c5_canonical, and on the 128-row VALU tile (the same bits) as c4_tile128,
  c5_tile128.
  c6  a short prefill step, 32 tokens through Llama-3.2-1B's down projection
      (2048x8192 Q4_0): split along K on the matrix cores' fused multiply-add
      (c6_split, AUTO) and on the VALU (c6_split128); unsplit on the matrix-core
      short-step tile (c6_tiled, AUTO) and the VALU one (c6_tiled_valu); the
      split-f16 matrix cores
  c7  the embedding gather from Qwen3-0.6B's Q6_K table (151936x1024): a
      512-token step and a decode step
  c8  large Q4_0 decodes: a Q4_0 LM head 151936x1024 and a 32768x8192 product
c2 and c8 also time a read floor: the same bytes read by the streamed decodes'
copy (global_load_lds_dwordx4, 9 KB a wave a step) with nothing decoded, the
practical ceiling under the 8 TB/s peak; frac_of_read_floor is the decode's
rate over it.
Every row carries a roofline in the unit its kernel runs on: HBM GB/s for the
decodes; TFLOP/s for the prefills, the VALU tiles and the f32 fused
multiply-add tile against the FP32 peak, the split-f16 matrix cores against
the dense FP16 peak and that design's useful half of it.
Inputs are seeded synthetic data (BASELINE's distributions) resident in HBM
before timing; a GEMV's weights rotate over copies totalling > 2x the 256 MB
MALL so every step reads HBM. Each config's launches are captured once in a
HIP graph and replayed; HIP events on the launch stream bracket the K timed
steps, five times over, and the median is reported, after --settle-ms (200) of
untimed replays: from idle the GPU takes ~60 ms of sustained load to reach its
steady speed, and the timed replays are meant to show that steady state (the
replay straight after idle is kept as ms_first_replay; C1-C3 are also timed
eagerly, one launch at a time: ms_single_launch). One JSON line on stdout; progress on
stderr. `--cpu-table` instead times the CPU baseline table of C1-C5 (host only).
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
FP32_PEAK_TFLOPS = 157.3   # MI355X FP32 (vector and matrix)
F16_PEAK_TFLOPS = 2516.6   # MI355X FP16 dense matrix
MALL_BYTES = 256 << 20
SETTLE_MS = 200.0  # untimed replays before the timed ones (Setup.time_graph)
METRIC = "GEMV HBM GB/s (% of 8 TB/s); prefill GEMM TFLOP/s (% peak); host-CPU baseline"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(gtype, rows, columns):
    from charlotte_amd import synthetic

    return synthetic.stored_bytes(gtype, rows, columns) + 4 * columns + 4 * rows


class Setup:
    def __init__(self):
        from charlotte_amd import harness as hx
        from charlotte_amd import matmul as mm

        self.hx, self.mm = hx, mm
        self.ctx = mm.Context(0)
        self.stream = hx.Stream()
        self.buffers = []
        self.weights = []
        self.settle_ms = SETTLE_MS
        self.settle_replays = None  # a count of untimed replays in place of settle_ms (bounded under a tracer)
        self.last_first = None

    def buffer(self, array=None, nbytes=None):
        b = self.hx.Buffer.of(array) if array is not None else self.hx.Buffer(nbytes)
        self.buffers.append(b)
        return b

    def weight_copies(self, gtype, rows, columns, stored, copies):
        """`copies` device copies of one weight, laid out once and copied on the device."""
        mm = self.mm
        first = mm.Weight(self.ctx, gtype, rows, columns, stored)
        self.weights.append(first)
        out = [first]
        nbytes = mm.layout_bytes(gtype, rows, columns)
        for _ in range(copies - 1):
            b = self.buffer(nbytes=nbytes)
            self.hx.check(self.hx.lib.chx_d2d(b.ptr, first.device, nbytes), "d2d")
            w = mm.Weight(self.ctx, gtype, rows, columns, device_piece=b.ptr, nbytes=nbytes)
            self.weights.append(w)
            out.append(w)
        return out

    def time_graph(self, body, steps, warmup, reps=5):
        """Capture body() (one step's launches) `steps` times into a graph; replay it
        once untimed (warmup), once timed from a GPU that has just been idle (kept
        as self.last_first), then untimed for `self.settle_ms` of wall time, then
        `reps` times timed, each between HIP events on the launch stream; return
        the median ms per step (the spread is kept in self.last_reps).

        The settling: from idle, a sustained decode runs 15-25% slower for its
        first ~60 ms (its replays' times fall steadily over that span and then
        stay level), so the timed replays follow the
        GPU's steady state, the state a serving loop runs in."""
        hx = self.hx
        # warmup, eager
        for _ in range(warmup):
            body()
        self.stream.sync()
        graph = hx.Graph(self.stream, lambda: [body() for _ in range(steps)])
        graph.launch()  # untimed replay: first-launch costs
        self.stream.sync()
        start, stop = hx.Event(), hx.Event()
        start.record(self.stream)
        graph.launch()
        stop.record(self.stream)
        stop.sync()
        self.last_first = start.elapsed_ms(stop) / steps
        # replays in batches of ~10 ms, so the queue never drains while settling
        batch = max(1, int(10.0 / max(self.last_first * steps, 1e-3)))
        if self.settle_replays is not None:
            # a fixed count (--settle-replays): a tracer records a bounded number of dispatches
            left = self.settle_replays
            while left > 0:
                for _ in range(min(batch, left)):
                    graph.launch()
                left -= min(batch, left)
                self.stream.sync()
        else:
            t0 = time.time()
            while time.time() - t0 < self.settle_ms / 1e3:
                for _ in range(batch):
                    graph.launch()
                self.stream.sync()
        times = []
        for _ in range(reps):
            start.record(self.stream)
            graph.launch()
            stop.record(self.stream)
            stop.sync()
            times.append(start.elapsed_ms(stop) / steps)
        graph.destroy()
        start.destroy()
        stop.destroy()
        self.last_reps = times
        return float(np.median(times))

    def time_single(self, body, reps=20):
        """body() launched eagerly (no graph), each time between HIP events and
        synchronized: the single-launch figure, launch cost included; median ms."""
        hx = self.hx
        body()
        self.stream.sync()
        start, stop = hx.Event(), hx.Event()
        times = []
        for _ in range(reps):
            start.record(self.stream)
            body()
            stop.record(self.stream)
            stop.sync()
            times.append(start.elapsed_ms(stop))
        start.destroy()
        stop.destroy()
        return float(np.median(times))

    def close(self):
        for w in self.weights:
            w.free()
        for b in self.buffers:
            b.free()
        self.stream.destroy()
        self.ctx.close()


def run_gemv(S, name, gtype, rows, columns, steps, warmup, rng, copies=None):
    from charlotte_amd import synthetic

    mm = S.mm
    wbytes = synthetic.stored_bytes(gtype, rows, columns)
    copies = copies or max(2, -(-2 * MALL_BYTES // wbytes))
    t0 = time.time()
    stored = synthetic.weight(rng, gtype, rows, columns)
    ws = S.weight_copies(gtype, rows, columns, stored, copies)
    x = S.buffer(synthetic.activations(rng, 1, columns))
    y = S.buffer(nbytes=4 * rows)
    launches = [mm.MatmulLaunch([mm.Member(w)], x.ptr, [y.ptr]) for w in ws]
    state = {"i": 0}

    def body():
        m = launches[state["i"] % len(launches)]
        state["i"] += 1
        mm.launch(S.ctx, m, 1, stream=S.stream.handle)

    log(f"{name}: {rows}x{columns} {mm.TensorType(gtype).name}, {copies} copies, setup {time.time() - t0:.1f}s")
    ms = S.time_graph(body, steps, warmup)
    spread = [round(t * 1e3, 2) for t in S.last_reps]
    single = S.time_single(body)
    nbytes = gemv_bytes(gtype, rows, columns)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"{name}: {ms * 1e3:.2f} us/launch (median of {spread} us), {gbs:.0f} GB/s "
        f"({100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s); single launch {single * 1e3:.2f} us")
    return {"ms_per_step": ms, "bytes": nbytes, "GB/s": gbs, "frac": gbs / HBM_PEAK_GBS, "copies": copies,
            "ms_first_replay": S.last_first, "ms_single_launch": single, "stored": stored, "x": x, "weights": ws,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": gemv_traffic(name)}}


def parse_shapes(spec):
    """ROWSxCOLUMNS[:TYPE],... -> [(rows, columns, gguf_type)], Q4_0 (2) when
    no type is given."""
    shapes = []
    for item in spec.split(","):
        shape, _, t = item.strip().partition(":")
        rows, columns = (int(v) for v in shape.lower().split("x"))
        shapes.append((rows, columns, int(t or 2)))
    return shapes


def time_decode_shapes(spec, steps, warmup, settle_ms, limbs=False):
    """One decode product a shape, timed as the configs are (weights rotated
    past the MALL, graph replays): {"ROWSxCOLUMNS:TYPE": {us, GB/s, frac}};
    `limbs` decodes on the INT8_LIMBS path where it applies."""
    S = Setup()
    S.settle_ms = settle_ms
    if limbs:
        S.ctx.set_gemv_path(S.mm.GemvPath.INT8_LIMBS)
    rng = np.random.default_rng(1)
    out = {}
    try:
        for rows, columns, gtype in parse_shapes(spec):
            tag = f"{rows}x{columns}:{gtype}"
            r = run_gemv(S, tag, gtype, rows, columns, steps, warmup, rng)
            out[tag] = {"us": round(r["ms_per_step"] * 1e3, 2), "GB/s": round(r["GB/s"], 1),
                        "frac": round(r["frac"], 4), "bytes": r["bytes"]}
    finally:
        S.close()
    return out


PREFILL_TYPES = {"f32": 0, "f16": 1, "q4_0": 2, "q4_1": 3, "q8_0": 8, "q6_k": 14, "bf16": 30}


def parse_prefill_shapes(spec):
    """--prefill's comma list of [TYPE:]ROWSxKxTOKENS as (item, GGUF type, rows,
    K, tokens); SystemExit naming the item that does not parse."""
    shapes = []
    for item in spec.split(","):
        kind, _, dims = item.strip().lower().rpartition(":")
        if kind and kind not in PREFILL_TYPES:
            raise SystemExit(f"--prefill {item}: the type is one of {', '.join(PREFILL_TYPES)}")
        try:
            rows, columns, tokens = (int(v) for v in dims.split("x"))
        except ValueError:
            raise SystemExit(f"--prefill {item}: not [TYPE:]ROWSxKxTOKENS") from None
        shapes.append((item.strip(), PREFILL_TYPES[kind or "q4_0"], rows, columns, tokens))
    return shapes


def time_prefill_shapes(spec, steps, warmup, settle_ms):
    """One prefill product a shape [TYPE:]ROWSxKxTOKENS (TYPE a key of
    PREFILL_TYPES, Q4_0 when absent), timed as the configs are, on each
    bit-exact path (CANONICAL: the 128-row tile; AUTO; EXACT_MFMA: the matrix
    cores' fused multiply-add): {"[TYPE:]ROWSxKxTOKENS": {path: {us, TFLOP/s,
    kernel}}}. The figures that choose AUTO's kernel."""
    shapes = parse_prefill_shapes(spec)
    S = Setup()
    S.settle_ms = settle_ms
    rng = np.random.default_rng(2)
    out = {}
    try:
        for item, gtype, rows, columns, tokens in shapes:
            row = {}
            for path in (S.mm.GemmPath.CANONICAL, S.mm.GemmPath.AUTO, S.mm.GemmPath.EXACT_MFMA):
                r = run_gemm(S, f"{item} {path.name}", [("write", [(rows, columns)])], tokens, steps, warmup, rng,
                             path, gtype=gtype)
                row[path.name] = {"us": round(r["ms_per_step"] * 1e3, 2), "TFLOP/s": round(r["TFLOP/s"], 1),
                                  "kernel": r["kernels"][0]}
            out[item] = row
    finally:
        S.close()
    return out


def run_read_floor(S, name, nbytes, copies, steps, warmup):
    """The same bytes read and nothing else (harness chx_read: the LDS-streamed
    decodes' copy, 9 KB a wave a step, with no decode), over `copies` buffers
    rotated as the decode's weight copies are: the rate the decode would reach
    were its arithmetic free — the practical ceiling under the 8 TB/s peak."""
    hx = S.hx
    nbytes = nbytes // 1024 * 1024
    bufs = [S.buffer(nbytes=nbytes) for _ in range(copies)]
    sink = S.buffer(nbytes=hx.read_sink_bytes())
    state = {"i": 0}

    def body():
        b = bufs[state["i"] % len(bufs)]
        state["i"] += 1
        hx.read(b.ptr, nbytes, sink.ptr, sink.nbytes, S.stream)

    ms = S.time_graph(body, steps, warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"{name}: {ms * 1e3:.2f} us/launch, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s), "
        f"{nbytes} bytes read, nothing decoded")
    for b in bufs + [sink]:
        b.free()
        S.buffers.remove(b)
    return {"kernel": "harness read_kernel: global_load_lds_dwordx4 nt, 9 KB a wave a step, no decode",
            "bytes": nbytes, "ms_per_step": ms, "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


def read_sweep(steps, warmup, settle_ms):
    """The ceiling of a pure read of C2's bytes on this part: every form of
    chx_read_sweep (registers grid-strided or a chunk a workgroup, 4-16 loads
    in flight a lane, plain or non-temporal, 8-32 waves a CU; the LDS copy at
    4, 9 and 16 KB a wave step, one or two steps in flight, plain or
    non-temporal) over the same
    three rotated copies as c2, each timed as c2 is (graph replays, median of
    5). One JSON object: each form's us and TB/s, fastest first."""
    from charlotte_amd import synthetic

    S = Setup()
    S.settle_ms = settle_ms
    hx = S.hx
    cus = int(hx.device_name(0).split("cus=")[1].split("|")[0])
    nbytes = synthetic.stored_bytes(14, 262144, 1152) // 1024 * 1024
    bufs = [S.buffer(nbytes=nbytes) for _ in range(3)]
    for b in bufs:
        b.fill(0x5A)
    forms = []
    for per_cu in (2, 4, 8):
        for u in (4, 8, 16):
            for nt in (False, True):
                forms.append((f"regs strided u{u}{' nt' if nt else ''} {per_cu * 4} waves/CU", 0, u, nt, 1,
                              cus * per_cu, 256))
    for per_cu, threads in ((4, 256), (8, 256), (2, 1024)):
        for nt in (False, True):
            forms.append((f"regs chunk u8{' nt' if nt else ''} {per_cu * threads // 64} waves/CU "
                          f"({per_cu} x {threads} lanes)", 1, 8, nt, 1, cus * per_cu, threads))
    for kb in (4, 9, 16):
        for depth in (1, 2):
            for nt in (False, True):
                per_cu = 1 if kb * depth > 16 else 2
                forms.append((f"lds {kb} KB x{depth}{' nt' if nt else ''} {per_cu * 4} waves/CU", 2, kb, nt, depth,
                              cus * per_cu, 256))
    sink_bytes = max(f[5] * f[6] for f in forms) * 4
    sink = S.buffer(nbytes=sink_bytes)
    rows = []
    try:
        for name, form, u, nt, depth, blocks, threads in forms:
            state = {"i": 0}

            def body():
                b = bufs[state["i"] % len(bufs)]
                state["i"] += 1
                hx.read_sweep(form, u, nt, depth, blocks, threads, b.ptr, nbytes, sink.ptr, sink_bytes, S.stream)

            ms = S.time_graph(body, steps, warmup)
            tbs = nbytes / (ms * 1e-3) / 1e12
            rows.append({"form": name, "us": round(ms * 1e3, 2), "TB/s": round(tbs, 3),
                         "frac": round(tbs * 1e3 / HBM_PEAK_GBS, 4)})
            log(f"read {name}: {ms * 1e3:.2f} us, {tbs:.3f} TB/s")
    finally:
        S.close()
    rows.sort(key=lambda r: r["us"])
    return {"bytes": nbytes, "copies": 3, "steps": steps, "forms": rows}


# (probe shape, name, operations an instruction, the shape's dense peak TOP/s, chain counts timed)
MFMA_SHAPES = ((0, "f16 16x16x32", 2 * 16 * 16 * 32, F16_PEAK_TFLOPS, (1, 8)),
               (1, "f16 32x32x16", 2 * 32 * 32 * 16, F16_PEAK_TFLOPS, (1, 8)),
               (2, "bf16 16x16x32", 2 * 16 * 16 * 32, F16_PEAK_TFLOPS, (1, 8)),
               (3, "i8 16x16x64", 2 * 16 * 16 * 64, 2 * F16_PEAK_TFLOPS, (1, 8)),
               (4, "i8 32x32x32", 2 * 32 * 32 * 32, 2 * F16_PEAK_TFLOPS, (1, 8)),
               (5, "f32 32x32x1 (2 blocks)", 2 * 32 * 32 * 2, FP32_PEAK_TFLOPS, (1, 4)),
               (6, "f32 16x16x1 (4 blocks)", 2 * 16 * 16 * 4, FP32_PEAK_TFLOPS, (1, 8)),
               (7, "f32 32x32x2", 2 * 32 * 32 * 2, FP32_PEAK_TFLOPS, (1, 8)),
               (8, "f32 16x16x4", 2 * 16 * 16 * 4, FP32_PEAK_TFLOPS, (1, 8)))


def mfma_rate(iters=2000, shapes=None):
    """Each matrix-core shape the prefill could use (`shapes`: probe numbers,
    default all), issued back to back by every wave of the GPU
    (chx_mfma_rate), a few independent accumulators a wave, 1, 2 or 4 waves a
    SIMD: the sustained rate against the shape's dense peak, and the time a
    SIMD spends on one instruction (ns; x the clock for cycles). Single
    launches between HIP events, median of 5."""
    S = Setup()
    hx = S.hx
    cus = int(hx.device_name(0).split("cus=")[1].split("|")[0])
    sink = S.buffer(nbytes=cus * 4 * 256 * 4)
    rows = []
    try:
        for shape, name, ops, peak, chain_counts in MFMA_SHAPES:
            if shapes is not None and shape not in shapes:
                continue
            for chains in chain_counts:
                for per_simd in (1, 2, 4):
                    blocks = cus * per_simd

                    def body():
                        hx.mfma_rate(shape, chains, blocks, iters, sink.ptr, sink.nbytes, S.stream)

                    ms = S.time_single(body, reps=5)
                    count = blocks * 4 * iters * chains
                    rate = count * ops / (ms * 1e-3) / 1e12
                    ns = ms * 1e6 / (count / (cus * 4))
                    rows.append({"shape": name, "chains": chains, "waves_a_simd": per_simd,
                                 "TOP/s": round(rate, 1), "frac_of_dense_peak": round(rate / peak, 3),
                                 "ns_an_instruction_a_simd": round(ns, 2)})
                    log(f"mfma {name} chains {chains} waves/SIMD {per_simd}: {rate:.0f} TOP/s "
                        f"({100 * rate / peak:.0f}% of {peak:.0f}), {ns:.2f} ns an instruction a SIMD")
    finally:
        S.close()
    return {"iters": iters, "rows": rows}


def build_products(S, rng, plan, tokens, gtype=2):
    """Weights, inputs and outputs for a list of products. plan: (kind, [(rows, columns), ...]) with kind
    "write" (one member), "qkv" (three members, three outputs) or "gated" (gate, up; one output of their rows).
    Returns launches, algorithmic GEMV bytes of one pass, flops of one pass at `tokens` tokens."""
    from charlotte_amd import synthetic

    mm = S.mm
    widths = sorted({c for _, members in plan for _, c in members})
    xs = {c: S.buffer(synthetic.activations(rng, tokens, c)) for c in widths}
    launches, nbytes, flops = [], 0, 0
    for kind, members in plan:
        ws = []
        for rows, columns in members:
            w = mm.Weight(S.ctx, gtype, rows, columns, synthetic.weight(rng, gtype, rows, columns))
            S.weights.append(w)
            ws.append(w)
            nbytes += synthetic.stored_bytes(gtype, rows, columns)
            flops += 2 * tokens * rows * columns
        columns = members[0][1]
        nbytes += 4 * columns
        if kind == "qkv":
            outs = [S.buffer(nbytes=4 * r * tokens) for r, _ in members]
            nbytes += 4 * sum(r for r, _ in members)
            m = mm.MatmulLaunch([mm.Member(w) for w in ws], xs[columns].ptr, [o.ptr for o in outs],
                                epilogue=mm.Epilogue.QKV)
        elif kind == "gated":
            out = S.buffer(nbytes=4 * members[0][0] * tokens)
            nbytes += 4 * members[0][0]
            m = mm.MatmulLaunch([mm.Member(w) for w in ws], xs[columns].ptr, [out.ptr],
                                epilogue=mm.Epilogue.GatedActivation, activation=mm.Activation.SiLU)
        else:
            out = S.buffer(nbytes=4 * members[0][0] * tokens)
            nbytes += 4 * members[0][0]
            m = mm.MatmulLaunch([mm.Member(ws[0])], xs[columns].ptr, [out.ptr])
        launches.append(m)
    return launches, xs, nbytes, flops


def layer_plan(q, kv, hidden, ffn, fused):
    """One transformer layer's products: q/k/v, o, gate/up, down."""
    if fused:
        return [("qkv", [(q, hidden), (kv, hidden), (kv, hidden)]), ("write", [(hidden, q)]),
                ("gated", [(ffn, hidden), (ffn, hidden)]), ("write", [(hidden, ffn)])]
    return [("write", [(q, hidden)]), ("write", [(kv, hidden)]), ("write", [(kv, hidden)]), ("write", [(hidden, q)]),
            ("write", [(ffn, hidden)]), ("write", [(ffn, hidden)]), ("write", [(hidden, ffn)])]


def run_c3(S, steps, warmup, rng, fused=True):
    """Qwen3-0.6B decode step: 28 layers x (q, k, v, o, gate, up, down) + the Q6_K head. Fused as the
    reference's graph launches them (QKV one product, gate and up one gated product): 113 launches;
    unfused: 197."""
    from charlotte_amd import synthetic

    mm = S.mm
    t0 = time.time()
    plan = layer_plan(2048, 1024, 1024, 3072, fused) * 28
    launches, xs, total, _ = build_products(S, rng, plan, 1)
    head = mm.Weight(S.ctx, 14, 151936, 1024, synthetic.q6_k(rng, 151936, 1024))
    S.weights.append(head)
    yh = S.buffer(nbytes=4 * 151936)
    launches.append(mm.MatmulLaunch([mm.Member(head)], xs[1024].ptr, [yh.ptr]))
    total += gemv_bytes(14, 151936, 1024)
    tag = "c3" if fused else "c3_unfused"
    log(f"{tag}: {len(launches)} launches, {total / 1e6:.1f} MB, setup {time.time() - t0:.1f}s")

    def body():
        for m in launches:
            mm.launch(S.ctx, m, 1, stream=S.stream.handle)

    ms = S.time_graph(body, steps, warmup)
    single = S.time_single(body, reps=5)
    gbs = total / (ms * 1e-3) / 1e9
    log(f"{tag}: {ms * 1e3:.1f} us/step, {gbs:.0f} GB/s aggregate, {1e3 / ms:.0f} tokens/s; "
        f"launched eagerly {single * 1e3:.1f} us/step")
    out = {"ms_per_step": ms, "ms_first_replay": S.last_first, "bytes": total, "GB/s": gbs, "frac": gbs / HBM_PEAK_GBS, "launches": len(launches),
           "tokens_per_s": 1e3 / ms, "ms_single_launch": single,
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}}
    if fused:
        out["floors"] = c3_floors(S, launches, steps, warmup)
        out["breakdown"] = c3_breakdown(S, launches, ms, steps, warmup)
        out.update(decode_matches_prefill(S, launches, xs, rng))
    return out


C3_KINDS = ("qkv", "o", "gate_up", "down", "head")


def prefix_breakdown(S, calls, kind_of, names, step_ms, steps, warmup, reads_of=None):
    """Each kind of launch in a step timed in place, as the reference's
    forward profile times a launch where timestamps inside a pass are not
    granted (bench/forward_profile.cpp:44-68): a prefix's time T, and a
    launch's time the difference of two prefixes' medians. Here the prefix
    runs through kind k of every layer (the layers' launches of kinds < k, in
    step order, each layer's weights its own, so the step's traffic through
    the caches is kept), and the last kind (the head) is the whole step less
    all layers:
        launch of kind k = (T(kinds <= k) - T(kinds < k)) / its launches,
    each T the median of 5 settled, timed replays of its graph, reported with
    the spread (least and most) of the replays. Beside each kind: the same
    launches alone back to back and, with `reads_of`, their reads-alone floor
    in place (the products' bytes read in their launch shapes, nothing
    decoded). calls: one launcher a launch, in step order; kind_of: each
    launch's kind (an index into names)."""

    def body_of(keep):
        chosen = [c for c, k in zip(calls, kind_of) if k in keep]

        def body():
            for c in chosen:
                c()
        return body

    def timed(body):
        ms = S.time_graph(body, steps, warmup)
        return ms * 1e3, [round(t * 1e3, 1) for t in (min(S.last_reps), max(S.last_reps))]

    last = len(names) - 1
    prefix = [(0.0, [0.0, 0.0])]
    for k in range(1, last + 1):
        prefix.append(timed(body_of(set(range(k)))))
    prefix.append((step_ms * 1e3, None))
    rows = {}
    for k, name in enumerate(names):
        count = sum(1 for kk in kind_of if kk == k)
        in_place = (prefix[k + 1][0] - prefix[k][0]) / count
        alone, alone_spread = timed(body_of({k}))
        rows[name] = {"launches": count, "us_in_place": round(in_place, 2), "us_alone": round(alone / count, 2),
                      "prefix_us": round(prefix[k + 1][0], 1), "prefix_spread_us": prefix[k + 1][1],
                      "alone_spread_us": alone_spread}
        line = (f"{name}: {count} launches, {in_place:.2f} us each in place (prefix {prefix[k][0]:.1f} -> "
                f"{prefix[k + 1][0]:.1f} us), {alone / count:.2f} alone")
        if reads_of is not None:
            reads, _ = timed(reads_of({k}))
            rows[name]["us_reads_alone"] = round(reads / count, 2)
            line += f", reads alone {reads / count:.2f}"
        log("  breakdown " + line)
    return {"method": "prefix through kind k of every layer; median of 5 settled replays a prefix", "kinds": rows}


def c3_breakdown(S, launches, step_ms, steps, warmup):
    """The decode step's kinds (QKV, o, gate/up, down, head) timed in place
    (prefix_breakdown), each beside its reads-alone floor."""
    hx, mm = S.hx, S.mm
    layers = (len(launches) - 1) // 4
    kind_of = [i % 4 if i < 4 * layers else 4 for i in range(len(launches))]
    calls = [lambda m=m: mm.launch(S.ctx, m, 1, stream=S.stream.handle) for m in launches]
    # the reads-alone stand-ins, each at its place in the step's walk through memory
    parts = floor_parts(mm, launches)
    offsets, at = [], 0
    for k, a, c in parts:
        offsets.append(at)
        at += a if k == "read" else a * c * 1024
    buf = S.buffer(nbytes=max(at, 2 * MALL_BYTES) + (1 << 20))
    sink_bytes = max(hx.read_sink_bytes(), 64 * 4 * max(a for k, a, c in parts if k == "touch"))
    sink = S.buffer(nbytes=sink_bytes)

    def reads_of(keep):
        chosen = [(p, o) for p, o, k in zip(parts, offsets, kind_of) if k in keep]

        def body():
            for (k, a, c), o in chosen:
                if k == "read":
                    hx.read(buf.ptr + o, a, sink.ptr, sink_bytes, S.stream)
                else:
                    hx.touch(buf.ptr + o, a, c, sink.ptr, sink_bytes, S.stream)
        return body

    log("c3 breakdown (a launch of each kind in place, us):")
    out = prefix_breakdown(S, calls, kind_of, C3_KINDS, step_ms, steps, warmup, reads_of)
    for b in (buf, sink):
        b.free()
        S.buffers.remove(b)
    out["head_placement"] = c3_head_placement(S, launches, steps, warmup)
    return out


def c3_head_placement(S, launches, steps, warmup):
    """What the head adds where it stands, each a graph of settled replays timed
    one after another: the layers; the step (the layers, then the head); the
    step with a second head after the first (its own copy of the weights, so
    none of the first head's bytes come from a cache); the layers, 20 empty
    launches, then the head; and the head and the 20 empty launches alone.
    A prefix difference holds a launch's own time only if the launches around
    it run as they do alone."""
    from charlotte_amd import synthetic

    mm, hx = S.mm, S.hx
    head = launches[-1]
    w = head.members[0].weight
    twin_w = mm.Weight(S.ctx, int(w.type), w.rows, w.columns,
                       synthetic.q6_k(np.random.default_rng(0x4EAD), w.rows, w.columns))
    S.weights.append(twin_w)
    twin = mm.MatmulLaunch([mm.Member(twin_w)], head.input, list(head.outputs))

    def run(ms):
        for m in ms:
            mm.launch(S.ctx, m, 1, stream=S.stream.handle)

    def empties():
        for _ in range(20):
            hx.null(S.stream)

    layers = launches[:-1]
    cases = (("layers", lambda: run(layers)),
             ("step", lambda: run(launches)),
             ("step, head twice", lambda: run(launches + [twin])),
             ("layers, 20 empty, head", lambda: (run(layers), empties(), run([head]))),
             ("head alone", lambda: run([head])),
             ("20 empty alone", empties))
    out = {}
    for name, body in cases:
        ms = S.time_graph(body, steps, warmup)
        out[name] = round(ms * 1e3, 1)
    log("c3 head in place (us a step): " + ", ".join(f"{k} {v:.1f}" for k, v in out.items()))
    return out


def floor_parts(mm, launches):
    """Each launch's reads-alone stand-in: ("read", bytes, 0) for a streamed
    product (its stored bytes, whole KB), ("touch", waves, kib) for the
    others — the plan's waves, each reading kib whole KB of the product's
    stored bytes (never more than them)."""
    from charlotte_amd import synthetic

    parts = []
    for m in launches:
        p = mm.plan_launch(m, 1)
        nbytes = sum(synthetic.stored_bytes(int(x.weight.type), x.rows or x.weight.rows, x.weight.columns)
                     for x in m.members)
        if p.kernel in (mm.Kernel.GEMV_STREAM, mm.Kernel.GEMV_STREAM8, mm.Kernel.GEMV_STREAM4):
            parts.append(("read", nbytes // 1024 * 1024, 0))
        else:
            waves = p.tile_rows // (p.steps_a_wave * (64 // p.lanes_a_row)) * min(p.tiles, p.workgroups)
            kib = max(1, nbytes // (waves * 1024))
            waves = min(waves, nbytes // (kib * 1024))
            parts.append(("touch", waves, kib))
    return parts


def c3_floors(S, launches, steps, warmup):
    """Two floors under a decode step's launches, each timed as a graph of as
    many launches as the step: `launch_us`, an empty kernel of one workgroup
    a launch (what launching costs); `memory_us`, each product's bytes read
    in its own launch shape with nothing decoded — the 32-lane products'
    one-wave workgroups (chx_touch: as many waves as the plan's, the
    product's stored bytes split among them), the streamed products by the
    streamed copy (chx_read). Reads walk one buffer longer than the MALL, a
    product's bytes after the last's, as the step's weights do."""
    hx = S.hx
    parts = floor_parts(S.mm, launches)
    total = sum(a if k == "read" else a * c * 1024 for k, a, c in parts)
    buf = S.buffer(nbytes=max(total, 2 * MALL_BYTES) + (1 << 20))
    sink_bytes = max(hx.read_sink_bytes(), 64 * 4 * max(a for k, a, c in parts if k == "touch"))
    sink = S.buffer(nbytes=sink_bytes)

    def memory():
        at = 0
        for k, a, c in parts:
            if k == "read":
                hx.read(buf.ptr + at, a, sink.ptr, sink_bytes, S.stream)
                at += a
            else:
                hx.touch(buf.ptr + at, a, c, sink.ptr, sink_bytes, S.stream)
                at += a * c * 1024

    def empty():
        for _ in parts:
            hx.null(S.stream)

    launch_ms = S.time_graph(empty, steps, warmup)
    memory_ms = S.time_graph(memory, steps, warmup)
    log(f"c3 floors: {len(parts)} empty launches {launch_ms * 1e3:.1f} us; the products' reads alone "
        f"{memory_ms * 1e3:.1f} us ({total / 1e6:.1f} MB)")
    for b in (buf, sink):
        b.free()
        S.buffers.remove(b)
    return {"launch_us": round(launch_ms * 1e3, 1), "memory_us": round(memory_ms * 1e3, 1), "memory_bytes": total}


def c3_cached(steps, warmup, settle_ms):
    """c3's 112 layer launches (the step without its head) as graphs, with
    every layer's own weights (235 MB, the step as it runs) and with the first
    7, 3 and 1 layers' weights cycled through the same 112 launches (59, 25
    and 8.4 MB: inside the MALL; the L2s' 32 MB; one layer's, L2-resident):
    what a launch would save with its weights already cached. Two rounds,
    us a step and a launch."""
    S = Setup()
    S.settle_ms = settle_ms
    mm = S.mm
    rng = np.random.default_rng(3)
    out = {}
    try:
        launches, _, _, _ = build_products(S, rng, layer_plan(2048, 1024, 1024, 3072, True) * 28, 1)
        cases = [("28 layers", launches), ("7 layers cycled", launches[:28] * 4),
                 ("3 layers cycled", (launches[:12] * 10)[:112]), ("1 layer cycled", launches[:4] * 28)]
        for rnd in range(2):
            for name, ls in cases:
                def body(ls=ls):
                    for m in ls:
                        mm.launch(S.ctx, m, 1, stream=S.stream.handle)
                us = S.time_graph(body, steps, warmup) * 1e3
                log(f"c3 cached, {name}: {us:.1f} us for {len(ls)} launches, {us / len(ls):.2f} us a launch")
                out.setdefault(name, []).append({"us": round(us, 1), "us_a_launch": round(us / len(ls), 3)})
    finally:
        S.close()
    return out


def decode_matches_prefill(S, launches, xs, rng, tokens=4):
    """The step's token decoded alone (the outputs the timed launches wrote) against the same token
    prefilled as the last of `tokens`: every product, bit for bit (the consistency the reference tracks,
    tests/gpu/matmul_test.cpp:257-267)."""
    from charlotte_amd import synthetic

    mm = S.mm
    S.stream.sync()
    prefill_x = {}
    for c, b in xs.items():
        rows = np.concatenate([synthetic.activations(rng, tokens - 1, c), b.read(np.float32).reshape(1, c)])
        prefill_x[c] = S.buffer(rows)
    compared = differing = 0
    for m in launches:
        columns = m.members[0].weight.columns
        if m.epilogue == mm.Epilogue.QKV:
            widths = [mem.weight.rows for mem in m.members]
        else:
            widths = [m.members[0].weight.rows]
        outs = [S.buffer(nbytes=4 * w * tokens) for w in widths]
        p = mm.MatmulLaunch(m.members, prefill_x[columns].ptr, [o.ptr for o in outs], epilogue=m.epilogue,
                            activation=m.activation)
        mm.launch(S.ctx, p, tokens, stream=S.stream.handle)
        S.stream.sync()
        for ptr, o, w in zip(m.outputs, outs, widths):
            decoded = np.empty(w, np.float32)
            S.hx.check(S.hx.lib.chx_d2h(decoded.ctypes.data, ptr, 4 * w), "d2h")
            last = o.read(np.uint32).reshape(tokens, w)[-1]
            compared += w
            differing += int((decoded.view(np.uint32) != last).sum())
    log(f"decode vs prefill (token {tokens} of {tokens}): {compared} outputs of {len(launches)} products, "
        f"{differing} differ")
    return {"decode_prefill_outputs_compared": compared, "decode_prefill_bits_equal": differing == 0}


def run_gemm(S, name, plan, tokens, steps, warmup, rng, path, head=None, gate=None, breakdown=False, gtype=2):
    """plan: products (build_products, weights of GGUF type `gtype`) over `tokens` tokens, on prefill path `path`; with `gate`, the
    split along K where the gate takes the step (range sums sized for the largest product). With
    `breakdown`, a step of layers of four products and a head: each kind timed in place."""
    from charlotte_amd import synthetic

    mm = S.mm
    t0 = time.time()
    S.ctx.set_gemm_path(path)
    launches, xs, _, flops = build_products(S, rng, plan, tokens, gtype)
    launches = [(m, tokens) for m in launches]
    gate = gate or mm.kNever
    sums, sums_bytes = 0, 0
    if gate is not mm.kNever:
        sums_bytes = 4 * 32 * tokens * max(sum(mem.rows or mem.weight.rows for mem in m.members) for m, _ in launches)
        sums = S.buffer(nbytes=sums_bytes).ptr
    head_bytes = 0
    if head is not None:
        rows, columns = head
        w = mm.Weight(S.ctx, 14, rows, columns, synthetic.q6_k(rng, rows, columns))
        S.weights.append(w)
        y = S.buffer(nbytes=4 * rows)
        launches.append((mm.MatmulLaunch([mm.Member(w)], xs[columns].ptr, [y.ptr], rows=mm.Rows.LastToken), tokens))
        head_bytes = gemv_bytes(14, rows, columns)
    log(f"{name}: {len(launches)} launches, {flops / 1e9:.1f} GFLOP, path {path.name}, setup {time.time() - t0:.1f}s")

    def body():
        for m, t in launches:
            mm.launch(S.ctx, m, t, gate, sums, sums_bytes, stream=S.stream.handle)

    ms = S.time_graph(body, steps, warmup)
    tflops = flops / (ms * 1e-3) / 1e12
    target = mm.Target(256, path, workspace_bytes=1 << 40)
    kernels = sorted({mm.plan_launch(m, t, target, gate, sums_bytes).kernel.name for m, t in launches})
    roof = gemm_roofline(tflops, path, name, kernels)
    log(f"{name}: {ms:.3f} ms/step, {tflops:.1f} TFLOP/s ({100 * roof['frac']:.1f}% of its unit's peak, "
        f"{roof['peak']} TFLOP/s {roof['bound']}); kernels {','.join(kernels)}")
    out = {"ms_per_step": ms, "ms_first_replay": S.last_first, "flops": flops, "TFLOP/s": tflops, "path": path.name,
           "kernels": kernels, "roofline": roof, "tokens_per_s": tokens / (ms * 1e-3), "launches": len(launches),
           "head_gemv_bytes": head_bytes}
    if breakdown and head is not None:
        layers = (len(launches) - 1) // 4
        kind_of = [i % 4 if i < 4 * layers else 4 for i in range(len(launches))]
        calls = [lambda m=m, t=t: mm.launch(S.ctx, m, t, gate, sums, sums_bytes, stream=S.stream.handle)
                 for m, t in launches]
        log(f"{name} breakdown (a launch of each kind in place, us):")
        out["breakdown"] = prefix_breakdown(S, calls, kind_of, C3_KINDS, ms, steps, warmup)
    return out


def gemm_roofline(tflops, path, name, kernels):
    """The roofline of a prefill row in the unit its kernel runs on: the
    canonical order on the matrix cores' f32 fused multiply-add (GEMM_EXACT)
    against their FP32 peak; the VALU tiles against the FP32 peak; the
    split-f16 matrix cores against the dense FP16 peak, and against the useful
    ceiling of that design (two f16 products an output product: half the
    peak). Counter traffic where profiles/traffic_c4.json holds it (c4)."""
    if path.name == "SPLIT_F16_MFMA":
        roof = {"bound": "mfma", "achieved": round(tflops, 1), "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / F16_PEAK_TFLOPS, 4), "useful_peak": F16_PEAK_TFLOPS / 2,
                "frac_of_useful": round(tflops / (F16_PEAK_TFLOPS / 2), 4)}
        kind = "mfma"
    elif any(k.startswith("GEMM_EXACT") for k in kernels):
        roof = {"bound": "mfma", "achieved": round(tflops, 1), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / FP32_PEAK_TFLOPS, 4)}
        kind = "exact"
    else:
        roof = {"bound": "valu", "achieved": round(tflops, 1), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / FP32_PEAK_TFLOPS, 4)}
        kind = "canonical"
    roof["traffic"] = gemm_traffic(name, kind)
    return roof


def gemm_traffic(name, kind):
    """HBM bytes a step of c4 from the counter runs in profiles/traffic_c4.json
    (FETCH_SIZE and WRITE_SIZE, KiB a dispatch, scaled as traffic_c2.json's)
    for its kernel kind (mfma: the split-f16 step, with prepare_x's; exact;
    canonical: the 128-row tile). None for other configs or kinds absent."""
    file = os.path.join(ROOT, "profiles", "traffic_c4.json")
    if not name.startswith("c4") or not os.path.exists(file):
        return None
    t = json.load(open(file))
    k = t["kernels"]

    def b(e):
        return (e["fetch_kib"] * t["fetch_scale"] + e["write_kib"] * t["write_scale"]) * 1024

    if kind == "mfma":
        return int(round(b(k["mfma"]) + b(k["prepare_x"])))
    return int(round(b(k[kind]))) if kind in k else None


def gemv_traffic(name):
    """HBM bytes a launch of a c1 or c8 decode from the counter runs in
    profiles/traffic_c1.json and traffic_c8.json (FETCH_SIZE and WRITE_SIZE,
    KiB a dispatch, scaled as traffic_c2.json's); None for other configs or
    when absent."""
    file = os.path.join(ROOT, "profiles", "traffic_c1.json" if name == "c1" else "traffic_c8.json")
    if not os.path.exists(file):
        return None
    t = json.load(open(file))
    k = t["kernels"].get(name)
    if k is None:
        return None
    return int(round((k["fetch_kib"] * t["fetch_scale"] + k["write_kib"] * t["write_scale"]) * 1024))


def run_gather(S, name, gtype, rows, columns, tokens, steps, warmup, rng):
    """The embedding gather of a step of `tokens` identifiers from a table of `rows` x `columns`:
    bytes = the rows read (stored size) + the hidden rows written (4 a weight)."""
    from charlotte_amd import synthetic

    mm = S.mm
    t0 = time.time()
    table = mm.Weight(S.ctx, gtype, rows, columns, synthetic.weight(rng, gtype, rows, columns))
    S.weights.append(table)
    ids = S.buffer(rng.integers(0, rows, tokens).astype(np.uint32))
    hidden = S.buffer(nbytes=4 * tokens * columns)

    def body():
        mm.gather(S.ctx, table, ids.ptr, tokens, hidden.ptr, stream=S.stream.handle)

    ms = S.time_graph(body, steps, warmup)
    nbytes = tokens * (synthetic.stored_bytes(gtype, 1, columns) + 4 * columns + 4)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"{name}: {tokens} rows of {rows}x{columns} (type {gtype}), setup {time.time() - t0:.1f}s: "
        f"{ms * 1e3:.2f} us/step, {gbs:.0f} GB/s")
    return {"ms_per_step": ms, "ms_first_replay": S.last_first, "bytes": nbytes, "GB/s": gbs, "frac": gbs / HBM_PEAK_GBS, "tokens": tokens,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}}


def cpu_baseline_c2(stored, x, rows, columns, seconds=10.0):
    """The oracle's reference-order f32 GEMV (the CPU restatement of the
    reference's order of addition, oracle/liborc.so) over all of C2 on the
    host's cores, repeated for about `seconds`; the median run."""
    from tests.support.oracle_lib import Oracle

    oracle = Oracle()
    threads = min(os.cpu_count() or 1, 16)
    oracle.matmul_f32(14, stored, rows, columns, x, threads=threads)  # warm-up
    times = []
    t_end = time.time() + seconds
    while (time.time() < t_end and len(times) < 200) or len(times) < 5:
        t0 = time.time()
        oracle.matmul_f32(14, stored, rows, columns, x, threads=threads)
        times.append(time.time() - t0)
    t = float(np.median(times))
    nbytes = gemv_bytes(14, rows, columns)
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"all of C2 ({rows}x{columns} Q6_K), reference-order f32 fma, median of {len(times)} runs "
                      f"of {t * 1e3:.1f} ms; oracle/liborc.so on {threads} threads"}


def cpu_table(threads_all):
    """The CPU baseline table: the oracle's reference-order f32 product and its
    f64 product (the reference tests' check) for C1-C5, on one thread and on
    `threads_all`, median of the runs made. C1-C4 run in full; C5 is one layer
    timed on 128 of its 2,048 token rows, scaled by 16 (tokens) and 16
    (layers; the head, a GEMV, is left out); single-thread C4 and C5 are one
    run each. Host only: no GPU call."""
    from charlotte_amd import synthetic
    from tests.support.oracle_lib import Oracle

    oracle = Oracle()
    rng = np.random.default_rng(0xC9)

    def timed(fn, reps):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    def products(shapes, tokens):
        out = []
        for gtype, rows, columns, count in shapes:
            out.append((gtype, rows, columns, synthetic.weight(rng, gtype, rows, columns),
                        synthetic.activations(rng, tokens, columns), count))
        return out

    def run(kind, prods, threads, reps):
        # each distinct product timed; products that repeat (layers) count `count` times
        total = 0.0
        for prod in prods:
            one = [prod]
            def fn_one(one=one):
                gtype, rows, columns, stored, x, _ = one[0]
                if kind == "f32":
                    oracle.matmul_f32(gtype, stored, rows, columns, x, threads=threads)
                else:
                    oracle.matmul_f64(gtype, stored, rows, columns, x, threads=threads)
            total += timed(fn_one, reps) * prod[5]
        return total

    c3_layer = [(2, 2048, 1024, 28), (2, 1024, 1024, 56), (2, 1024, 2048, 28), (2, 3072, 1024, 56), (2, 1024, 3072, 28)]
    c5_layer = [(2, 2048, 2048, 32), (2, 512, 2048, 32), (2, 8192, 2048, 32), (2, 2048, 8192, 16)]
    configs = [
        ("c1", products([(2, 3072, 1024, 1)], 1), "GB/s", gemv_bytes(2, 3072, 1024), 1.0, 1),
        ("c2", products([(14, 262144, 1152, 1)], 1), "GB/s", gemv_bytes(14, 262144, 1152), 1.0, 1),
        ("c3", products(c3_layer + [(14, 151936, 1024, 1)], 1), "GB/s",
         sum(gemv_bytes(g, r, c) * n for g, r, c, n in c3_layer) + gemv_bytes(14, 151936, 1024), 1.0, 1),
        ("c4", products([(2, 8192, 2048, 1)], 512), "TFLOP/s", 2 * 512 * 8192 * 2048, 1.0, 0),
        ("c5", products(c5_layer, 128), "TFLOP/s", 2 * 2048 * sum(r * c * n for _, r, c, n in c5_layer), 16.0, 0),
    ]
    rows_out = []
    for name, prods, unit, work, scale, small in configs:
        for kind in ("f32", "f64"):
            for threads in (1, threads_all):
                reps = 5 if small or threads > 1 else 1
                t = run(kind, prods, threads, reps) * scale
                value = work / t / (1e9 if unit == "GB/s" else 1e12)
                rows_out.append({"config": name, "kind": kind, "threads": threads, "seconds": t, "value": value,
                                 "unit": unit, "runs": reps,
                                 "note": "one layer on 128 of 2048 token rows, x16 tokens x16 layers" if name == "c5"
                                 else "in full"})
                log(f"cpu {name} {kind} {threads} thread(s): {t:.4f} s, {value:.3f} {unit}")
    model = ""
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"cpu_table": rows_out, "host": {"cpus": os.cpu_count(), "threads_used": threads_all, "model": model}}


def run_copy(S, nbytes=256 << 20, reps=5):
    """A plain device copy of known size: the yardstick the HBM counters
    (rocprofv3 FETCH_SIZE / WRITE_SIZE) are scaled by."""
    hx = S.hx
    a, b = S.buffer(nbytes=nbytes), S.buffer(nbytes=nbytes)
    for _ in range(reps):
        hx.copy(a.ptr, b.ptr, nbytes, S.stream)
    S.stream.sync()
    log(f"copy: {reps} x {nbytes >> 20} MiB")


def measured_traffic(limbs=False):
    """HBM bytes per launch of the headline kernel (or of its INT8_LIMBS form),
    from the rocprofv3 counter runs recorded in profiles/traffic_c2.json
    (FETCH_SIZE and WRITE_SIZE in KiB per dispatch, each scaled by what the
    counter reads for a copy of known size); None when absent."""
    path = os.path.join(ROOT, "profiles", "traffic_c2.json")
    if not os.path.exists(path):
        return None
    t = json.load(open(path))
    k = t.get("limbs") if limbs else t
    if k is None:
        return None
    return int(round((k["fetch_kib"] * t["fetch_scale"] + k["write_kib"] * t["write_scale"]) * 1024))


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                   help="untimed replays of each config's graph, in ms of wall time, before its timed replays")
    p.add_argument("--settle-replays", type=int, default=None,
                   help="settle with this many untimed replays of each graph instead of --settle-ms of wall time "
                        "(for runs under a tracer: the dispatches it records stay bounded)")
    p.add_argument("--only", default="c1,c2,c3,c4,c5,c6,c7,c8")
    p.add_argument("--breakdown", action="store_true",
                   help="also time each kind of c5's launches in place (prefixes of its graph)")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-table", action="store_true",
                   help="time the CPU baseline table (C1-C5, f32 and f64, 1 and all threads) and exit")
    p.add_argument("--decode", metavar="SHAPES",
                   help="time decode products of the given shapes and exit: a comma list of ROWSxCOLUMNS[:TYPE], "
                        "TYPE a GGUF type number (2 Q4_0, default; 3 Q4_1; 8 Q8_0; 14 Q6_K, repacked)")
    p.add_argument("--limbs", action="store_true", help="with --decode: the INT8_LIMBS decode path")
    p.add_argument("--prefill", metavar="SHAPES",
                   help="time prefill products [TYPE:]ROWSxKxTOKENS (a comma list; TYPE f32, f16, bf16, q4_0 (the "
                        "default), q4_1, q8_0 or q6_k) on each bit-exact path and exit")
    p.add_argument("--mfma-rate", nargs="?", const="all", default=None,
                   help="time each matrix-core instruction shape's sustained rate (a probe) and exit; "
                        "optionally a comma list of probe shape numbers (0-8)")
    p.add_argument("--read-sweep", action="store_true",
                   help="time every pure-read form over C2's bytes (the read ceiling) and exit")
    p.add_argument("--c3-cached", action="store_true",
                   help="time c3's 112 layer launches with 28, 7, 3 and 1 layers' weights (cycled) and exit")
    args = p.parse_args()
    if args.cpu_table:
        print(json.dumps(cpu_table(min(os.cpu_count() or 1, 16))), flush=True)
        return
    if args.mfma_rate:
        shapes = None if args.mfma_rate == "all" else {int(x) for x in args.mfma_rate.split(",")}
        print(json.dumps(mfma_rate(shapes=shapes)), flush=True)
        return
    if args.read_sweep:
        print(json.dumps(read_sweep(max(args.steps, 20), args.warmup, args.settle_ms)), flush=True)
        return
    if args.c3_cached:
        print(json.dumps(c3_cached(args.steps, args.warmup, args.settle_ms)), flush=True)
        return
    if args.decode:
        print(json.dumps(time_decode_shapes(args.decode, args.steps, args.warmup, args.settle_ms, args.limbs)),
              flush=True)
        return
    if args.prefill:
        print(json.dumps(time_prefill_shapes(args.prefill, args.steps, args.warmup, args.settle_ms)), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (this path is measured on one MI355X); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    only = set(args.only.split(","))
    from charlotte_amd import harness as hx

    log("device:", hx.device_name(0))
    S = Setup()
    S.settle_ms = args.settle_ms
    S.settle_replays = args.settle_replays
    out = {}
    rng = np.random.default_rng(0xC4A7)
    c2 = None
    c2_x = None
    try:
        if "copy" in only:
            run_copy(S)
        if "c2" in only:
            c2 = run_gemv(S, "c2", 14, 262144, 1152, max(args.steps, 20), args.warmup, np.random.default_rng(2))
            c2_x = c2["x"].read(np.float32)
            S.ctx.set_gemv_path(S.mm.GemvPath.INT8_LIMBS)
            r = run_gemv(S, "c2_limbs", 14, 262144, 1152, max(args.steps, 20), args.warmup,
                         np.random.default_rng(2))
            S.ctx.set_gemv_path(S.mm.GemvPath.CANONICAL)
            out["c2_limbs"] = {k: v for k, v in r.items() if k not in ("stored", "x", "weights")}
            out["c2_limbs"]["path"] = "INT8_LIMBS: within 1e-5 of the canonical order, not its bits"
            out["c2_limbs"]["roofline"]["traffic"] = measured_traffic(limbs=True)
            floor = run_read_floor(S, "c2_read_floor", c2["bytes"], c2["copies"], max(args.steps, 20), args.warmup)
            out["c2_read_floor"] = floor
            for r in (c2, out["c2_limbs"]):
                r["frac_of_read_floor"] = round(r["GB/s"] / floor["GB/s"], 4)
        if "c1" in only:
            r = run_gemv(S, "c1", 2, 3072, 1024, max(args.steps, 100), args.warmup, np.random.default_rng(1))
            out["c1"] = {k: v for k, v in r.items() if k not in ("stored", "x", "weights")}
        if "c8" in only:
            # Large Q4_0 decodes: a Q4_0 LM head (151,936 x 1,024) and a wide
            # product (32,768 x 8,192), weights rotated past the MALL.
            for tag, rows, columns in (("c8_q4_0_head", 151936, 1024), ("c8_q4_0_wide", 32768, 8192)):
                r = run_gemv(S, tag, 2, rows, columns, max(args.steps, 20), args.warmup, np.random.default_rng(8))
                out[tag] = {k: v for k, v in r.items() if k not in ("stored", "x", "weights")}
                floor = run_read_floor(S, tag + "_read_floor", r["bytes"], r["copies"], max(args.steps, 20),
                                       args.warmup)
                out[tag]["read_floor"] = floor
                out[tag]["frac_of_read_floor"] = round(r["GB/s"] / floor["GB/s"], 4)
                if columns > 2048:
                    continue  # the INT8_LIMBS form is built for K = 1,024 and 2,048
                S.ctx.set_gemv_path(S.mm.GemvPath.INT8_LIMBS)
                r = run_gemv(S, tag + "_limbs", 2, rows, columns, max(args.steps, 20), args.warmup,
                             np.random.default_rng(8))
                S.ctx.set_gemv_path(S.mm.GemvPath.CANONICAL)
                out[tag + "_limbs"] = {k: v for k, v in r.items() if k not in ("stored", "x", "weights")}
                out[tag + "_limbs"]["path"] = "INT8_LIMBS: within 1e-5 of the canonical order, not its bits"
                out[tag + "_limbs"]["frac_of_read_floor"] = round(r["GB/s"] / floor["GB/s"], 4)
        if "c3" in only:
            out["c3"] = run_c3(S, max(args.steps // 4, 3), args.warmup, rng)
            out["c3_unfused"] = run_c3(S, max(args.steps // 4, 3), args.warmup, rng, fused=False)
        # Prefill: the matrix cores (split-f16, within tolerance) and the
        # canonical VALU tile (bit-exact), each on the same shapes.
        ws = S.buffer(nbytes=S.mm.workspace_bytes(2048, 8192))
        S.ctx.set_workspace(ws.ptr, ws.nbytes)
        # The split-f16 matrix cores (within 1e-5, opt-in); the bit-exact
        # default (AUTO: the matrix cores' fused multiply-add tile at these
        # sizes); the 128-row VALU tile (CANONICAL), the same bits.
        paths = [("", S.mm.GemmPath.SPLIT_F16_MFMA), ("_canonical", S.mm.GemmPath.AUTO),
                 ("_tile128", S.mm.GemmPath.CANONICAL)]
        if "c4" in only:
            for tag, path in paths:
                out["c4" + tag] = run_gemm(S, "c4" + tag, [("write", [(8192, 2048)])], 512, args.steps, args.warmup,
                                           rng, path)
        if "c5" in only:
            for tag, path in paths:
                out["c5" + tag] = run_gemm(S, "c5" + tag, layer_plan(2048, 512, 2048, 8192, True) * 16, 2048,
                                           max(args.steps // 4, 3), args.warmup, rng, path, head=(128256, 2048),
                                           breakdown=args.breakdown)
        if "c6" in only:
            # A short prefill step (32 tokens) through Llama 3.2 1B's down
            # projection: split along K (the reference's measured gate, 2/1 up
            # to 64 workgroups) as AUTO runs it, on the matrix cores' fused
            # multiply-add, and on the VALU tile; unsplit, as a product with
            # options or without range sums runs, on the matrix-core short-step
            # tile AUTO takes (32 rows x 32 tokens, K split among a workgroup's
            # eight waves: 64 workgroups) and on the VALU short-step tile
            # CANONICAL takes (8 rows x 32 tokens: 256 workgroups); on the
            # split-f16 matrix cores. Then the same step's gated gate/up
            # product, which never splits, on both short-step tiles.
            plan = [("write", [(2048, 8192)])]
            out["c6_split"] = run_gemm(S, "c6_split", plan, 32, args.steps, args.warmup, rng,
                                       S.mm.GemmPath.AUTO, gate=S.mm.kSplitGate)
            out["c6_split128"] = run_gemm(S, "c6_split128", plan, 32, args.steps, args.warmup, rng,
                                          S.mm.GemmPath.CANONICAL, gate=S.mm.kSplitGate)
            out["c6_tiled"] = run_gemm(S, "c6_tiled", plan, 32, args.steps, args.warmup, rng, S.mm.GemmPath.AUTO)
            out["c6_tiled_valu"] = run_gemm(S, "c6_tiled_valu", plan, 32, args.steps, args.warmup, rng,
                                            S.mm.GemmPath.CANONICAL)
            out["c6_mfma"] = run_gemm(S, "c6_mfma", plan, 32, args.steps, args.warmup, rng,
                                      S.mm.GemmPath.SPLIT_F16_MFMA)
            gated = [("gated", [(8192, 2048), (8192, 2048)])]
            out["c6_gated"] = run_gemm(S, "c6_gated", gated, 32, args.steps, args.warmup, rng, S.mm.GemmPath.AUTO)
            out["c6_gated_valu"] = run_gemm(S, "c6_gated_valu", gated, 32, args.steps, args.warmup, rng,
                                            S.mm.GemmPath.CANONICAL)
        if "c7" in only:
            # The embedding gather of Qwen3 0.6B's tied Q6_K table: a
            # 512-token prefill step and a decode step.
            for tokens in (512, 1):
                out[f"c7_gather_{tokens}"] = run_gather(S, f"c7_gather_{tokens}", 14, 151936, 1024, tokens,
                                                        args.steps, args.warmup, rng)
    finally:
        S.close()

    result = {"metric": METRIC, "unit": "GB/s", "higher_is_better": True, "n_gpus": 1, "scaling": "weak",
              "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded; BASELINE distributions)"}
    if c2 is not None:
        cpu = None
        if not args.no_cpu:
            log("cpu baseline: oracle f32 on a sample of c2 ...")
            cpu = cpu_baseline_c2(c2["stored"], c2_x, 262144, 1152)
            log(f"cpu baseline: {cpu['value']:.1f} GB/s on {cpu['cores']} threads")
        result.update({
            "value": round(c2["GB/s"], 1), "steps": max(args.steps, 20), "warmup": args.warmup,
            "settle_ms": args.settle_ms,
            "ms_per_step": c2["ms_per_step"],
            "config": {"workload": "c2: Q6_K LM-head GEMV y[1,262144] = x[1,1152] W^T (Gemma-3-1B), repacked Q6_K",
                       "weights": "Q6_K (repacked), x and y f32", "rows": 262144, "columns": 1152,
                       "weight_copies": c2["copies"]},
            "roofline": {"bound": "hbm", "achieved": round(c2["GB/s"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(c2["frac"], 4), "traffic": measured_traffic()},
            "cpu_baseline": cpu,
            "read_floor": out.get("c2_read_floor"),
            "frac_of_read_floor": c2.get("frac_of_read_floor"),
        })
    result["configs"] = out
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
