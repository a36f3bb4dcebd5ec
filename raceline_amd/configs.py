"""Shapes of the BASELINE configurations (4-bit affine, group 64, fp16 scales and biases).

(name, K, N) per projection. The 27B prefill config reuses the 27B decode shapes at M=2048.
"""

CFG1_SINGLE = [("linear", 4096, 4096)]                                   # M = 1, CPU reference case

CFG2_9B = [("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
           ("gate_up", 4096, 24576), ("down", 12288, 4096)]               # M in {1, 5}

# The same layer as the reference's engine runs it: q, k and v stacked into one matrix
# (the model file's attn.qkv with parts q, k, v; one linear over it, src/engine.mm:1163-1167).
CFG2_9B_STACKED = [("qkv", 4096, 4096 + 2 * 1024), ("o", 4096, 4096), ("gate_up", 4096, 24576),
                   ("down", 12288, 4096)]                                # M in {1, 5}

CFG3_27B = [("qkv", 5120, 5120 + 2 * 1024), ("o", 5120, 5120), ("gate_up", 5120, 34816),
            ("down", 17408, 5120)]                                        # M in {1, 8}

CFG4_PREFILL_M = 2048                                                     # 27B shapes, M = 2048

# MoE in the style of a 35B-A3B model: hidden 2048, 256 routed experts + 1 shared,
# expert gate_up K=2048 N=2*512, down K=512 N=2048, top-8 with renormalised weights.
MOE = dict(H=2048, I=512, E=256, topk=8, norm_topk=True, tokens=(1, 512))


def linear_bytes(M: int, K: int, N: int) -> int:
    """Algorithmic HBM bytes of one linear: codes + fp16 scale and bias + fp16 x + fp32 y."""
    return K * N // 2 + 4 * N * (K // 64) + 2 * M * K + 4 * M * N


def linear_flops(M: int, K: int, N: int) -> int:
    return 2 * M * N * K
