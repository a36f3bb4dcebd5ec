"""Seeded inputs built with the oracle's quantizer, and their upload to the GPU."""

import numpy as np

import oracle as O


def make_layer(seed, N, K, sd="f16", std=0.02):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(std)).astype(np.float32)
    return O.quantize_affine_rtn(W, sd)


def make_x(seed, M, K, outliers=0.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    if outliers:
        mask = rng.random((M, K)) < outliers
        x = np.where(mask, x * 20.0, x)
    return x.astype(np.float16)


def sample_cols(N, count=256, seed=0):
    """Output columns to check at full size: the first and last four and random ones
    (the sampling of tests/test_linear.mm:163-164)."""
    if N <= count:
        return np.arange(N)
    rng = np.random.default_rng(seed)
    mid = rng.choice(np.arange(4, N - 4), size=count - 8, replace=False)
    return np.unique(np.concatenate([np.arange(4), np.arange(N - 4, N), mid]))


def upload(q, s, b, sd, device):
    import torch

    from raceline_amd.ops import AffineWeight

    w = torch.from_numpy(O.pack_nibbles_u32(q).view(np.int32)).to(device)
    dt = torch.float16 if sd == "f16" else torch.bfloat16
    st = torch.from_numpy(s.view(np.int16)).to(device).view(dt)
    bt = torch.from_numpy(b.view(np.int16)).to(device).view(dt)
    return AffineWeight(w, st, bt)


def to_dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)
