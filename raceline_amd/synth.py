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


# ------------------------------------------------------------------ synthetic model files

def model_config(hidden: int, layers: int, intermediate: int, vocab: int, experts: int = 0, topk: int = 0,
                 moe_inter: int = 0) -> dict:
    """A model header's config in the reference's fields, with the attention geometry the
    engine requires (src/engine.mm:394-396: Dk = 128, head_dim = 256, 64 rotary dims, 4
    conv taps); the attention itself is not on this path."""
    c = dict(hidden_size=hidden, num_hidden_layers=layers, intermediate_size=intermediate, num_attention_heads=16,
             num_key_value_heads=4, head_dim=256, linear_num_value_heads=32, linear_num_key_heads=16,
             linear_key_head_dim=128, linear_value_head_dim=128, linear_conv_kernel_dim=4, vocab_size=vocab,
             rms_norm_eps=1e-6, full_attention_interval=4, rope_theta=1e7, partial_rotary_factor=0.25,
             eos_token_id=7)
    if experts:
        c.update(num_experts=experts, num_experts_per_tok=topk, moe_intermediate_size=moe_inter, norm_topk_prob=True)
    return c


def _bf16_values(x):
    import numpy as np

    return (np.ascontiguousarray(x, np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def _random_affine_host(rng, n: int, k: int):
    """Codes uniform in 0..15 with bf16 scales and biases (the .rlm affine format) drawn
    directly: the file's bytes are what matter to a timing, not where they came from."""
    import numpy as np

    raw = np.frombuffer(rng.bytes(n * k // 2), np.uint8).reshape(n, k // 2)    # two codes per random byte
    q = np.empty((n, k), np.uint8)
    q[:, 0::2] = raw & 15
    q[:, 1::2] = raw >> 4
    s = _bf16_values(rng.uniform(0.001, 0.005, (n, k // GROUP)))
    b = _bf16_values(-7.5 * s)
    return q, s, b


def write_mlp_model(path: str, layers: int, hidden: int, intermediate: int = 0, experts: int = 0, topk: int = 0,
                    moe_inter: int = 0, seed: int = 0) -> dict:
    """An affine .rlm file (bf16 scales and biases, tools/convert.py's format) holding only
    what rl_mlp reads: per layer the post-attention norm and either a dense MLP (mlp.gate_up
    with parts gate and up, mlp.down) or a mixture of experts (moe.router, half, E + 1 rows;
    moe.gate_up [(E+1) 2I][H] and moe.down [(E+1) H][I], tools/quantize.py:168-228). Every
    layer holds the same bytes (drawn once) in its own place in the file, so that the engine
    uploads distinct copies. Returns the config."""
    import numpy as np

    from . import rlm

    rng = np.random.default_rng(seed)
    cfg = model_config(hidden, layers, intermediate or moe_inter, 1024, experts, topk, moe_inter)
    post = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    if experts:
        E1 = experts + 1
        router = (rng.standard_normal((E1, hidden)) * 0.05).astype(np.float16)
        mats = {"moe.gate_up": (["experts"], rlm.pack_blocked([_random_affine_host(rng, E1 * 2 * moe_inter, hidden)])),
                "moe.down": (["experts"], rlm.pack_blocked([_random_affine_host(rng, E1 * hidden, moe_inter)]))}
    else:
        gate, up = _random_affine_host(rng, intermediate, hidden), _random_affine_host(rng, intermediate, hidden)
        mats = {"mlp.gate_up": (["gate", "up"], rlm.pack_blocked([gate, up])),
                "mlp.down": (["out"], rlm.pack_blocked([_random_affine_host(rng, hidden, intermediate)]))}
        del gate, up
    w = rlm.Writer(path)
    for i in range(layers):
        w.begin(f"layer.{i}")
        w.add_float(f"layers.{i}.post_norm", post)
        if experts:
            w.add_dense(f"layers.{i}.moe.router", router)
        for name, (parts, packed) in mats.items():
            w.add_blocked_packed(f"layers.{i}.{name}", parts, packed)
        w.end()
    w.finish(rlm.affine_meta(cfg))
    return cfg
