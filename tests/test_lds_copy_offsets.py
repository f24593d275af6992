"""The LDS DMA copies (`__builtin_amdgcn_global_load_lds`) and their immediate
offset. The instruction's offset field is 13 bits, signed; this image's
compiler puts the builtin's offset argument into it without a range check, so
an offset of 4,096 is encoded as -4,096 and 8,192 as 0 — the copy then reads 4
KB before (or at) its base instead of past it, outside the buffer at the start
of an allocation, and lands at the same wrong distance from its LDS address.
Every copy in the library therefore passes its full address and an offset of
0. CPU only: the first test reads the sources, the second compiles a probe to
assembly (no GPU)."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "charlotte_amd", "csrc")


def _call_arguments(text, start):
    """The top-level comma-separated arguments of the call whose '(' is at start."""
    depth, args, cur = 0, [], []
    for ch in text[start:]:
        if ch == "(":
            depth += 1
            if depth == 1:
                continue
        elif ch == ")":
            depth -= 1
            if depth == 0:
                args.append("".join(cur).strip())
                return args
        elif ch == "," and depth == 1:
            args.append("".join(cur).strip())
            cur = []
            continue
        cur.append(ch)
    raise AssertionError("unbalanced call")


def test_every_lds_copy_in_the_library_has_a_zero_immediate_offset():
    calls = 0
    for name in sorted(os.listdir(CSRC)):
        if not name.endswith((".hip", ".hpp")):
            continue
        text = open(os.path.join(CSRC, name)).read()
        for m in re.finditer(r"__builtin_amdgcn_global_load_lds\s*\(", text):
            args = _call_arguments(text, m.end() - 1)
            assert len(args) == 5, (name, args)
            assert args[3] == "0", f"{name}: global_load_lds with immediate offset {args[3]!r}"
            calls += 1
    assert calls >= 5


PROBE = r"""
#include <hip/hip_runtime.h>
#include <stdint.h>
typedef __attribute__((address_space(3))) void* lds_void;
template <int OFF>
__global__ void probe(const uint8_t* g, uint32_t* out) {
    __shared__ uint32_t stage[1024];
    __builtin_amdgcn_global_load_lds(g + 16 * threadIdx.x, (lds_void)stage, 16, OFF, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    out[threadIdx.x] = stage[threadIdx.x];
}
template __global__ void probe<4095>(const uint8_t*, uint32_t*);
template __global__ void probe<4096>(const uint8_t*, uint32_t*);
template __global__ void probe<8192>(const uint8_t*, uint32_t*);
"""


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not on PATH")
def test_the_compiler_wraps_an_immediate_offset_past_4095():
    with tempfile.TemporaryDirectory() as d:
        src, asm = os.path.join(d, "probe.hip"), os.path.join(d, "probe.s")
        open(src, "w").write(PROBE)
        subprocess.run(["hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
                        "-o", asm, src], check=True, capture_output=True, timeout=300)
        text = open(asm).read()
    encoded = {}
    for fn in re.split(r"\n(?=_Z\w*probe\w*:)", text)[1:]:
        off = int(re.search(r"_Z\w*probeILi(\d+)E", fn).group(1))
        ins = re.search(r"global_load_lds_dwordx4[^\n]*", fn).group(0)
        m = re.search(r"offset:(-?\d+)", ins)
        encoded[off] = int(m.group(1)) if m else 0
    assert encoded == {4095: 4095, 4096: -4096, 8192: 0}, encoded
