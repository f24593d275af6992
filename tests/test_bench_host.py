"""bench.py's host side, without a GPU: the algorithmic bytes its rooflines
divide by (the figures the measurement plan fixes for C1-C3), the CPU
baseline's fields on a small sample, and its refusal of more than one GPU.
"""

import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_gemv_bytes_are_the_algorithmic_figures():
    # stored weight bytes + 4 K (x) + 4 N (y)
    assert bench.gemv_bytes(2, 3072, 1024) == 1_785_856  # C1
    assert bench.gemv_bytes(14, 262144, 1152) == 248_779_264  # C2
    # C3 unfused: 28 layers of seven Q4_0 products and the Q6_K head, 197 launches
    layer = [(2048, 1024), (1024, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (3072, 1024), (1024, 3072)]
    total = 28 * sum(bench.gemv_bytes(2, r, c) for r, c in layer) + bench.gemv_bytes(14, 151936, 1024)
    assert total == 378_487_296


def test_decode_step_floor_reads_each_product_in_its_launch_shape():
    """The reads-alone floor of the Qwen3 0.6B step: each 32-lane product's
    plan's waves reading whole KB of its stored bytes (never more), the Q6_K
    head by the streamed copy."""
    from charlotte_amd import matmul as mm
    from charlotte_amd import synthetic

    Q4_0, Q6_K = mm.TensorType.Q4_0, mm.TensorType.Q6_K
    made = []

    def w(gtype, rows, columns):
        made.append(mm.Weight.shape(gtype, rows, columns))
        return made[-1]

    X, Y = 16, 16
    launches = [
        mm.MatmulLaunch([mm.Member(w(Q4_0, 2048, 1024)), mm.Member(w(Q4_0, 1024, 1024)),
                         mm.Member(w(Q4_0, 1024, 1024))], X, [Y, Y, Y], epilogue=mm.Epilogue.QKV),
        mm.MatmulLaunch([mm.Member(w(Q4_0, 1024, 2048))], X, [Y]),
        mm.MatmulLaunch([mm.Member(w(Q4_0, 3072, 1024)), mm.Member(w(Q4_0, 3072, 1024))], X, [Y],
                        epilogue=mm.Epilogue.GatedActivation),
        mm.MatmulLaunch([mm.Member(w(Q4_0, 1024, 3072))], X, [Y]),
        mm.MatmulLaunch([mm.Member(w(Q6_K, 151936, 1024))], X, [Y]),
    ]
    try:
        parts = bench.floor_parts(mm, launches)
        assert [k for k, _, _ in parts] == ["touch"] * 4 + ["read"]
        for m, (kind, a, c) in zip(launches, parts):
            stored = sum(synthetic.stored_bytes(int(x.weight.type), x.weight.rows, x.weight.columns) for x in m.members)
            if kind == "read":
                assert a == stored // 1024 * 1024
            else:
                p = mm.plan_launch(m, 1)
                assert a == p.workgroups  # one-wave workgroups, one a tile
                assert 0 < a * c * 1024 <= stored < (a + 1) * (c + 1) * 1024
    finally:
        for x in made:
            x.free()


def test_cpu_baseline_reports_its_fields_on_a_sample():
    from charlotte_amd import synthetic

    rng = np.random.default_rng(1)
    rows, columns = 256, 1152
    stored = synthetic.q6_k(rng, rows, columns)
    x = synthetic.activations(rng, 1, columns)
    r = bench.cpu_baseline_c2(stored, x, rows, columns, seconds=0.05)
    assert set(r) == {"value", "unit", "cores", "kind", "sample"}
    assert r["unit"] == "GB/s" and r["kind"] == "port" and r["cores"] >= 1 and r["value"] > 0


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr


def test_decode_shapes_parse_with_q4_0_by_default():
    assert bench.parse_shapes("4096x14336,151936x1024:14, 3072X1024:8") == [
        (4096, 14336, 2), (151936, 1024, 14), (3072, 1024, 8)]


def test_prefill_shapes_parse_with_an_optional_weight_type():
    """--prefill's list: Q4_0 where no type is given, the GGUF type where one
    is; an unknown type or a malformed shape stops with the item named."""
    assert bench.parse_prefill_shapes("2048x8192x32, f32:300x1024x12,q6_k:512x2816x16") == [
        ("2048x8192x32", 2, 2048, 8192, 32), ("f32:300x1024x12", 0, 300, 1024, 12),
        ("q6_k:512x2816x16", 14, 512, 2816, 16)]
    for bad in ("q5_k:64x256x2", "64x256", "64xKx2"):
        try:
            bench.parse_prefill_shapes(bad)
        except SystemExit as e:
            assert bad in str(e)
        else:
            raise AssertionError(bad)
