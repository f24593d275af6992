"""The built libraries' gfx950 code holds no packed FP32 arithmetic.

Packed FP32 instructions (v_pk_fma_f32, v_pk_mul_f32, v_pk_add_f32) are kept
out of every kernel: the build passes `-Xclang -target-feature -Xclang
-packed-fp32-ops`, and this test reads the device code the build produced to
hold it there. CPU only: a library's `.hip_fatbin` section holds one offload
bundle per object file; each is unbundled to its gfx950 code object and
disassembled with the ROCm LLVM tools, and every instruction is checked.
"""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LLVM = "/opt/rocm/llvm/bin"
LIBS = [os.path.join(ROOT, "charlotte_amd", n) for n in ("libcharlotte_hip_matmul.so", "libcharlotte_hip_harness.so")]
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
PACKED_FP32 = ("v_pk_fma_f32", "v_pk_mul_f32", "v_pk_add_f32")


def _tools():
    need = [shutil.which("objcopy"), os.path.join(LLVM, "clang-offload-bundler"), os.path.join(LLVM, "llvm-objdump")]
    if not all(t and os.path.exists(t) for t in need):
        pytest.skip("objcopy or the ROCm LLVM tools are absent")
    return need


def _disassembly(lib, tmp):
    objcopy, bundler, objdump = _tools()
    fat = os.path.join(tmp, "fat.bin")
    subprocess.run([objcopy, "-O", "binary", "--only-section=.hip_fatbin", lib, fat], check=True)
    data = open(fat, "rb").read()
    starts = []
    at = data.find(MAGIC)
    while at >= 0:
        starts.append(at)
        at = data.find(MAGIC, at + 1)
    assert starts, f"{lib}: no offload bundle"
    text = []
    for i, s in enumerate(starts):
        piece, code = os.path.join(tmp, f"b{i}.bin"), os.path.join(tmp, f"b{i}.co")
        open(piece, "wb").write(data[s : starts[i + 1] if i + 1 < len(starts) else len(data)])
        subprocess.run([bundler, "--unbundle", "--type=o", f"--input={piece}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={code}"], check=True)
        out = subprocess.run([objdump, "-d", "--mcpu=gfx950", code], check=True, capture_output=True, text=True)
        text.append(out.stdout)
    return "\n".join(text)


@pytest.mark.parametrize("lib", LIBS, ids=os.path.basename)
def test_no_packed_fp32_instructions(lib, tmp_path):
    if not os.path.exists(lib):
        pytest.skip(f"{os.path.basename(lib)} is not built")
    asm = _disassembly(lib, str(tmp_path))
    words = asm.split()
    assert sum(w.startswith("v_") for w in words) > 100, "too little code disassembled"
    found = {op: words.count(op) for op in PACKED_FP32 if op in words}
    assert not found, f"{os.path.basename(lib)}: packed FP32 instructions {found}"


def test_the_check_sees_a_packed_instruction(tmp_path):
    """The scan is not blind: a kernel built without the flag, from float2
    arithmetic, shows a packed FP32 instruction in the same disassembly path."""
    _tools()
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc absent")
    src = tmp_path / "probe.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "__global__ void probe(float2* a, const float2* b, float s) {\n"
        "  const int i = threadIdx.x; float2 x = a[i], y = b[i];\n"
        "  x.x = x.x * y.x + s; x.y = x.y * y.y + s; a[i] = x; }\n")
    lib = tmp_path / "libprobe.so"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-shared", "-fPIC", str(src), "-o", str(lib)], check=True,
                   capture_output=True)
    words = _disassembly(str(lib), str(tmp_path)).split()
    assert any(w in PACKED_FP32 for w in words)
