"""charlotte_amd — the quantized GGUF matrix product of plainsight-systems/charlotte
(Q4_0 and repacked Q6_K weights times f32 activations; decode GEMV and prefill
GEMM) as hand-written HIP for MI355X, behind the C ABI of
include/charlotte_hip_matmul.h. ``charlotte_amd.matmul`` is the operator
interface; ``charlotte_amd.harness`` the device plumbing tests and the
benchmark use; ``charlotte_amd.synthetic`` the seeded inputs of the
benchmark's configurations.
"""

__all__ = ["matmul", "harness", "synthetic"]
