"""Seeded random shapes through the automatic kernel choice, against the oracle.

The other files pin fixed cases (the BASELINE configs, the reference's own cases, edge
shapes); these draw ragged M, K and N at random (fixed seeds, so a failure names its shape
and reproduces), with both scale types, the three native codebooks, decode sizes long
enough for the K split, and random MoE layers.
Same bars as the other files: max|y - ref| / rms(ref) <= 1e-3 and the reference's own
criterion (tests/test_linear.mm:178), both via oracle.check_close.
"""

import numpy as np
import pytest

import oracle as O
from tests.qdata import make_layer, make_x, to_dev, upload

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _shapes(seed, n, max_groups):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.choice([1, 2, 3, 5, 7, 8, 9, 16, 17, 63, 128, 129, 200]))
        K = 64 * int(rng.integers(1, max_groups + 1))
        N = int(rng.integers(1, 700))
        out.append((M, K, N))
    return out


def _sync():
    import torch

    torch.cuda.synchronize()


@pytest.mark.parametrize("M,K,N", _shapes(2026, 24, 72))
def test_affine_random_shapes(gpu, M, K, N):
    from raceline_amd import ops

    sd = "f16" if (31 * M + K + N) % 2 else "bf16"
    q, s, b = make_layer(M + 3 * K + 7 * N, N, K, sd)
    x = make_x(M * 7 + K + N, M, K, outliers=0.01)
    y = ops.linear(to_dev(x, gpu), upload(q, s, b, sd, gpu))
    _sync()
    O.check_close(y.cpu().numpy(), O.linear_affine_f64(x, q, s, b, sd), TOL, f"affine {sd} M={M} K={K} N={N}")


def _split_shapes(seed, n):
    """Decode sizes whose K the kernel splits across workgroups (K >= 17024, few tiles)."""
    rng = np.random.default_rng(seed)
    return [(int(rng.choice([1, 2, 5, 8])), 64 * int(rng.integers(266, 385)), int(rng.integers(1, 3000)))
            for _ in range(n)]


@pytest.mark.parametrize("M,K,N", _split_shapes(2029, 5))
def test_affine_random_split_decode(gpu, M, K, N):
    from raceline_amd import ops

    q, s, b = make_layer(M + K + N, N, K, "f16")
    x = make_x(K + N, M, K)
    y = ops.linear(to_dev(x, gpu), upload(q, s, b, "f16", gpu))
    _sync()
    O.check_close(y.cpu().numpy(), O.linear_affine_f64(x, q, s, b, "f16"), TOL, f"split decode M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N", _shapes(2027, 12, 72))
def test_native_random_shapes(gpu, M, K, N):
    import torch

    from raceline_amd import ops

    book = ("int15", "int16", "fp4")[(M + K + N) % 3]
    rng = np.random.default_rng(M * 5 + K + N)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s_row = rng.uniform(0.002, 0.02, size=N).astype(np.float32)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    w = torch.from_numpy(O.pack_nibbles_u32(q).view(np.int32)).to(gpu)
    nw = ops.pack_native(w, to_dev(s_row, gpu), book)
    y = ops.linear_native(to_dev(x, gpu), nw)
    _sync()
    O.check_close(y.cpu().numpy(), O.linear_native_f64(x, q, s_row, book), TOL,
                  f"native {book} M={M} K={K} N={N}")


def _moe_shapes(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(rng.choice([8, 16, 32, 64]))
        topk = int(rng.integers(1, min(8, E) + 1))
        T = int(rng.choice([1, 2, 3, 4, 5, 9, 16, 17, 40, 100]))
        H = 64 * int(rng.integers(1, 9))
        I = 64 * int(rng.integers(1, 9))
        out.append((T, E, topk, H, I))
    return out


@pytest.mark.parametrize("T,E,topk,H,I", _moe_shapes(2028, 10))
def test_moe_random_shapes(gpu, T, E, topk, H, I):
    from raceline_amd import ops
    from tests.qdata import upload_mlx

    rng = np.random.default_rng(T * 13 + E + H + I)
    Wg = rng.standard_normal(((E + 1) * 2 * I, H), dtype=np.float32) * np.float32(0.02)
    Wd = rng.standard_normal(((E + 1) * H, I), dtype=np.float32) * np.float32(0.02)
    gu, dn = O.quantize_affine_rtn(Wg, "f16"), O.quantize_affine_rtn(Wd, "f16")
    mw = ops.pack_moe(upload_mlx(*gu, "f16", gpu), upload_mlx(*dn, "f16", gpu), E, H, I)
    x = rng.standard_normal((T, H), dtype=np.float32).astype(np.float16)
    logits = rng.standard_normal((T, E + 1), dtype=np.float32)
    h0 = rng.standard_normal((T, H)).astype(np.float32)
    h = to_dev(h0, gpu)
    ops.moe(to_dev(x, gpu), to_dev(logits, gpu), mw, topk, h)
    _sync()
    ref, _, _ = O.moe_layer_f64(x, logits, gu, dn, E, topk, I, H)
    O.check_close(h.cpu().numpy().astype(np.float64) - h0, ref, TOL, f"moe T={T} E={E} topk={topk} H={H} I={I}")
