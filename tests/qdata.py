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


def upload_mlx(q, s, b, sd, device):
    """Oracle codes and 16-bit scale bits -> MLX-layout device tensors (w, s, b)."""
    import torch

    w = torch.from_numpy(O.pack_nibbles_u32(q).view(np.int32)).to(device)
    dt = torch.float16 if sd == "f16" else torch.bfloat16
    st = torch.from_numpy(s.view(np.int16)).to(device).view(dt)
    bt = torch.from_numpy(b.view(np.int16)).to(device).view(dt)
    return w, st, bt


def upload(q, s, b, sd, device):
    """Oracle codes -> PackedWeight on the device (packed by the library's upload kernel)."""
    from raceline_amd import ops

    return ops.pack_affine(*upload_mlx(q, s, b, sd, device))


def packed_layout_np(q, s, b):
    """The packed device layout of include/rlq.h restated in numpy: codes then scale/bias quads.

    Tiles of 16 rows, groups padded to quads; per (tile t, group pair p) 64 lanes x 16 bytes,
    lane 16j + c holding words 8g + 4s + j of row 16t + c for (g, s) = (2p,0),(2p,1),(2p+1,0),(2p+1,1);
    then per (tile, quad q, row c) 16 bytes: s | b << 16 for groups 4q .. 4q+3."""
    N, K = q.shape
    G = K // 64
    G4 = (G + 3) // 4
    T = (N + 15) // 16
    qp = np.zeros((T * 16, G4 * 4 * 64), np.uint8)
    qp[:N, :K] = q
    words = O.pack_nibbles_u32(qp).reshape(T, 16, 2 * G4, 2, 2, 4)    # [t][c][p][g in pair][s][j]
    codes = words.transpose(0, 2, 5, 1, 3, 4).reshape(-1)               # [t][p][j][c][g in pair][s]
    sp = np.zeros((T * 16, G4 * 4), np.uint32)
    sp[:N, :G] = s.astype(np.uint32) | (b.astype(np.uint32) << 16)
    sb = sp.reshape(T, 16, G4, 4).transpose(0, 2, 1, 3).reshape(-1)     # [t][q][c][e]
    return np.concatenate([codes.view(np.uint8), sb.view(np.uint8)])


def to_dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)
