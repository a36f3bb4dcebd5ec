"""raceline_amd: raceline's 4-bit group-quantized matmul path, MI355X-native.

The compute lives in libraceline_amd.so (hand-written HIP for gfx950, C ABI in
include/rlq.h). This package binds it (lib), wraps it for torch device tensors (ops,
moe) and generates the BASELINE configs' synthetic inputs (configs).
"""

__all__ = ["lib", "ops"]
