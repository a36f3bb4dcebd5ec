"""Seeded synthetic inputs of the BASELINE configs, generated on the device.

Weights are drawn from N(0, 0.02) and quantized to 4-bit affine groups of 64 the way
tools/quantize.py:258-264 restates MLX's round-to-nearest: per (row, group) lo = min,
step = max((hi - lo)/15, 1e-12); the scale and bias are stored in the 16-bit dtype and
the codes are computed from the stored values, q = clip(round((W - b)/s), 0, 15) (q = 0
where the stored scale is 0). Codes are packed 8 per uint32, element k in bits 4*(k%8).
Activations are fp16 N(0, 1), optionally with a fraction of entries scaled by 20.

This is the producer side of the layout (what tools/convert.py writes), on the GPU so
that the benchmark can build gigabytes of distinct weights in seconds.
"""

from __future__ import annotations

import torch

from .ops import GROUP, pack_affine


def pack_codes(q: torch.Tensor) -> torch.Tensor:
    """[N][K] codes 0..15 (any integer dtype) -> [N][K/8] int32 words (bit pattern of uint32)."""
    N, K = q.shape
    qi = q.to(torch.int64).view(N, K // 8, 8)
    shifts = torch.arange(0, 32, 4, device=q.device, dtype=torch.int64)
    words = (qi << shifts).sum(-1)                    # disjoint bits: sum == or
    words = torch.where(words >= 1 << 31, words - (1 << 32), words)
    return words.to(torch.int32).contiguous()


def quantize_affine(W: torch.Tensor, scale_dtype: torch.dtype = torch.float16):
    """[N][K] float weights -> MLX layout (codes int32 [N][K/8], scales, biases [N][K/64])."""
    W = W.to(torch.float32)
    N, K = W.shape
    g = W.view(N, K // GROUP, GROUP)
    lo = g.amin(-1)
    hi = g.amax(-1)
    step = torch.clamp((hi - lo) / 15.0, min=1e-12)
    s = step.to(scale_dtype)
    b = lo.to(scale_dtype)
    sf = s.float().unsqueeze(-1)
    bf = b.float().unsqueeze(-1)
    q = torch.clamp(torch.round((g - bf) / sf), 0, 15)
    q = torch.where(sf == 0, torch.zeros_like(q), q)
    return pack_codes(q.view(N, K)), s.contiguous(), b.contiguous()


def random_affine(N: int, K: int, seed: int, device, std: float = 0.02,
                  scale_dtype: torch.dtype = torch.float16, chunk_rows: int = 8192, packed: bool = True):
    """N(0, std) weights quantized per group, generated in row chunks to bound memory.
    Returns a PackedWeight, or the MLX-layout (w, s, b) tensors when packed is False."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    ws, ss, bs = [], [], []
    for r0 in range(0, N, chunk_rows):
        r = min(chunk_rows, N - r0)
        W = torch.randn((r, K), generator=gen, device=device, dtype=torch.float32) * std
        w, s, b = quantize_affine(W, scale_dtype)
        ws.append(w)
        ss.append(s)
        bs.append(b)
        del W
    mlx = (torch.cat(ws), torch.cat(ss), torch.cat(bs))
    if not packed:
        return mlx
    return pack_affine(*mlx)


def random_activations(M: int, K: int, seed: int, device, outliers: float = 0.0) -> torch.Tensor:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    x = torch.randn((M, K), generator=gen, device=device, dtype=torch.float32)
    if outliers > 0:
        mask = torch.rand((M, K), generator=gen, device=device) < outliers
        x = torch.where(mask, x * 20.0, x)
    return x.to(torch.float16).contiguous()
