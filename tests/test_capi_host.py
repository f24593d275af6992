"""The C ABI on the CPU: the library loads and exports what the header
declares; the host-side layout and repack agree with the oracle and the
reference's own code; the split planning mirrors the reference's tables
(tests/kernels_matmul_test.cpp:211-285); the synthetic generators encode what
they claim. No kernel runs here.
"""

import ctypes
import os
import re

import numpy as np
import pytest

from tests.support import blocks as B
from tests.support.oracle_lib import F32, Q4_0, Q4_1, Q6_K, Q8_0

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(charlotte_hip_matmul_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from charlotte_amd import matmul as mm

    names = _declared("charlotte_hip_matmul.h")
    assert len(names) >= 14
    lib = ctypes.CDLL(mm.LIBRARY)
    for name in names:
        assert hasattr(lib, name), name
    # and the Python mirror binds each one with a signature
    assert set(names) <= set(mm.SIGNATURES)


def test_harness_library_loads():
    from charlotte_amd import harness

    assert callable(harness.lib.chx_malloc)


def test_layout_bytes():
    from charlotte_amd import matmul as mm

    assert mm.layout_bytes(Q4_0, 3072, 1024) == 3072 * 32 * 18
    assert mm.layout_bytes(Q4_0, 1, 32) == 20  # 18 rounded up to 4
    assert mm.layout_bytes(Q6_K, 262144, 1152) == 262144 * 1152 // 256 * 210
    assert mm.layout_bytes(Q6_K, 1, 1152) == 0  # 4.5 super-blocks: not whole blocks
    assert mm.layout_bytes(Q4_0, 4, 1000) == 0  # not whole groups
    assert mm.layout_bytes(99, 4, 1024) == 0
    assert mm.layout_bytes(Q4_1, 40, 3072) == 40 * 96 * 20
    assert mm.layout_bytes(Q8_0, 1, 32) == 36  # 34 rounded up to 4
    assert mm.layout_bytes(F32, 7, 256) == 7 * 256 * 4


def _edge_blocks(gtype, count):
    if gtype == F32:
        return np.random.default_rng(count).standard_normal(count).astype(np.float32).tobytes()
    return {Q4_0: B.q4_0_edge_blocks, Q4_1: B.q4_1_edge_blocks, Q8_0: B.q8_0_edge_blocks,
            Q6_K: B.q6_k_edge_blocks}[gtype](count)


@pytest.mark.parametrize("gtype,count", [(Q4_0, 1), (Q4_0, 257), (Q6_K, 1), (Q6_K, 33), (Q4_1, 1), (Q4_1, 257),
                                         (Q8_0, 1), (Q8_0, 257), (F32, 32), (F32, 4096)])
def test_lay_out_matches_the_oracle(oracle, gtype, count):
    from charlotte_amd import matmul as mm

    stored = _edge_blocks(gtype, count)
    assert np.frombuffer(mm.lay_out(gtype, stored, count), np.uint8).tolist() == oracle.lay_out(gtype, stored).tolist()


def test_lay_out_many_blocks_threads(oracle):
    from charlotte_amd import matmul as mm

    stored = B.lcg_bytes(210 * 70000, seed=11)  # enough blocks for the threaded path
    assert mm.lay_out(Q6_K, stored, 70000) == oracle.lay_out(Q6_K, stored).tobytes()


@pytest.mark.parametrize("gtype", [Q4_1, Q8_0])
def test_lay_out_of_many_blocks_is_the_oracles(oracle, gtype):
    from charlotte_amd import matmul as mm

    n = 70000
    stored = B.lcg_bytes(n * {Q4_1: 20, Q8_0: 34}[gtype], seed=5)
    assert mm.lay_out(gtype, stored, n) == oracle.lay_out(gtype, stored).tobytes()


def test_repack_matches_the_reference(reference):
    from charlotte_amd import matmul as mm

    stored = B.lcg_bytes(210 * 33, seed=5)
    mine = mm.repack_q6_k(stored, 33)
    theirs = reference.repack_q6_k(stored)
    for a, b in zip(mine, theirs):
        assert a == b.tobytes()


def test_split_tokens_at_each_listed_models_products():
    # tests/kernels_matmul_test.cpp:211-245.
    from charlotte_amd import matmul as mm

    E = mm.Epilogue
    cases = [
        (E.Write, 512, 2048, 256), (E.Write, 512, 1024, 256), (E.GatedByInput, 512, 512, 128),
        (E.QKV, 2048, 512, 32), (E.QKV, 3072, 512, 1), (E.GatedActivation, 4096, 512, 1),
        (E.Write, 1024, 3072, 128), (E.Write, 1024, 2048, 128), (E.QKV, 4096, 1024, 32),
        (E.Write, 2048, 8192, 64), (E.QKV, 3072, 2048, 32), (E.Write, 2048, 2048, 64),
        (E.QKV, 1536, 1152, 64), (E.Write, 1152, 1024, 96), (E.Write, 1152, 6912, 96),
    ]
    for epilogue, rows, columns, want in cases:
        split = mm.split_tokens(epilogue, rows, columns, mm.kSplitGate)
        assert split == want, (epilogue, rows, columns)
        need = mm.range_sum_floats(epilogue, rows, columns, mm.kSplitGate)
        assert need == (0 if split < 2 else split * rows * 32)
        assert need * 4 <= 16 << 20


def test_split_gate_boundaries():
    # tests/kernels_matmul_test.cpp:272-285.
    from charlotte_amd import matmul as mm

    W, G = mm.Epilogue.Write, mm.Epilogue.GatedActivation
    assert mm.split_tokens(W, 512, 1024, mm.SplitGate(1, 4, 128)) == 32
    assert mm.split_tokens(W, 512, 1024, mm.SplitGate(1, 5, 128)) == 1
    assert mm.split_tokens(W, 512, 1024, mm.SplitGate(2, 1, 8)) == 32
    assert mm.split_tokens(W, 512, 1024, mm.SplitGate(2, 1, 7)) == 1
    assert mm.split_tokens(W, 512, 1024, mm.SplitGate(2, 1, 16)) == 64
    assert mm.split_tokens(W, 64, 8192, mm.kAlways) == 512
    assert mm.split_tokens(G, 64, 8192, mm.kAlways) == 1
    assert mm.split_tokens(W, 64, 8192, mm.kNever) == 1


def test_context_without_a_device_is_refused():
    from charlotte_amd import harness
    from charlotte_amd import matmul as mm

    if harness.device_count() > 0:
        pytest.skip("a device is present")
    with pytest.raises(mm.MatmulError) as e:
        mm.Context(0)
    assert e.value.status == mm.Status.NO_DEVICE


def test_synthetic_q6_k_encodes_its_codes_scales_and_d(oracle):
    from charlotte_amd import synthetic

    rng = np.random.default_rng(3)
    codes = rng.integers(0, 64, size=(5, 256), dtype=np.uint8)
    scales = rng.integers(-64, 64, size=(5, 16), dtype=np.int16)
    d = (np.abs(rng.standard_normal(5)) * 0.001).astype(np.float16)
    stored = synthetic.q6_k_from_codes(codes, scales, d)
    assert (B.q6_k_codes(stored) == codes).all()
    w = oracle.dequantize(Q6_K, stored).reshape(5, 256)
    want = (d.astype(np.float32)[:, None] * np.repeat(scales.astype(np.float32), 16, axis=1)) * (
        codes.astype(np.float32) - 32)
    assert (w == want).all()


def test_synthetic_q4_0_distribution(oracle):
    from charlotte_amd import synthetic

    rng = np.random.default_rng(4)
    stored = synthetic.q4_0(rng, 64, 1024)
    b = np.frombuffer(stored, np.uint8).reshape(-1, 18)
    d = b[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    assert (d >= 0).all() and 0.01 < d.mean() < 0.02  # |N(0,1)| * 0.02 has mean 0.016
    codes = np.concatenate([b[:, 2:] & 0xF, b[:, 2:] >> 4], axis=1)
    assert codes.min() == 0 and codes.max() == 15
