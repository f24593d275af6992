"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer
(oracle/Makefile's `sanitize` target, host code only): every entry point the
tests use runs over the reference's fixture tensors and each format's edge
blocks in a child process with the ASan runtime preloaded, reports fatal; the
child must finish clean.
"""

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import os, sys
sys.path.insert(0, os.environ["ORACLE_ROOT"])
import numpy as np
from tests.support import blocks as B
from tests.support import gguf_fixture
from tests.support.oracle_lib import F32, Q4_0, Q4_1, Q8_0, Q6_K, Oracle

o = Oracle(os.path.join(os.environ["ORACLE_ROOT"], "oracle", "_san", "liborc_san.so"))
for h in range(0, 65536, 7):
    o.fp16_to_fp32(h)
edges = {Q4_0: B.q4_0_edge_blocks(37), Q6_K: B.q6_k_edge_blocks(9), Q4_1: B.q4_1_edge_blocks(37),
         Q8_0: B.q8_0_edge_blocks(37)}
for t, blocks in edges.items():
    o.dequantize(t, blocks)
    device = o.lay_out(t, blocks)
    n = len(blocks) // {Q4_0: 18, Q6_K: 210, Q4_1: 20, Q8_0: 34}[t]
    for g in range(n * (8 if t == Q6_K else 1)):
        o.unpack_group(t, device, n, g)
o.repack_q6_k(edges[Q6_K])
tensors = gguf_fixture.read(os.path.join(os.environ["ORACLE_ROOT"], "tests", "golden", "matmul_rows.gguf"))
for name, t in tensors.items():
    if t.type not in (Q4_0, Q6_K, Q4_1, Q8_0):
        continue
    x = o.fill(7, 3 * t.columns)
    for threads in (1, 3):
        o.matmul_f32(t.type, t.data, t.rows, t.columns, x, threads=threads)
        o.matmul_f64(t.type, t.data, t.rows, t.columns, x, threads=threads)
    totals = o.matmul_f32(t.type, t.data, t.rows, t.columns, x)
    o.finish(totals, clip=np.array([-1, 1, -2, 2], np.float32), bias=np.zeros(t.rows, np.float32),
             activated=True, activation=1)
    o.gated(totals, totals, activation=0)
    o.gated_by_input(totals, totals, activation=2)
    ids = np.arange(min(t.rows, 5), dtype=np.uint32)
    hidden = np.zeros((ids.size, t.columns), np.float32)
    o.gather(t.type, t.data, t.rows, t.columns, ids, hidden, scale=0.5)
table = np.random.default_rng(1).standard_normal((6, 64), dtype=np.float32)
o.gather_positions(table, 64, 3, 3, 6)
print("sanitized oracle ok", flush=True)
"""


def test_oracle_is_clean_under_asan_and_ubsan():
    if shutil.which("gcc") is None or shutil.which("make") is None:
        pytest.skip("no host compiler")
    build = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "sanitize"], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-2000:]
    libasan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(libasan) or not os.path.exists(libasan):
        pytest.skip("no AddressSanitizer runtime")
    env = dict(os.environ, ORACLE_ROOT=ROOT, LD_PRELOAD=libasan,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-c", SCRIPT], env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0 and "sanitized oracle ok" in r.stdout, (r.stdout[-2000:], r.stderr[-4000:])
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
