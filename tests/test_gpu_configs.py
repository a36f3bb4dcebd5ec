"""Parity at the BASELINE configurations' full shapes, through the automatic kernel choice.

Weights are drawn as the configs say (N(0, 0.02), 4-bit affine groups of 64, fp16 scales and
biases; raceline_amd.synth, on the device), activations fp16 N(0, 1) (the prefill config
with 1% of entries x20). The outputs are checked on sampled columns (the first and last four
and random ones, as tests/test_linear.mm:163-164 samples) against the fp64 dequant+matmul of
the stored codes, scales and biases (oracle.linear_affine_f64): max|err|/rms <= 1e-3 and the
reference test's rule max|err| < 2e-3 rms + 1e-4.
"""

import numpy as np
import pytest

import oracle as O
from raceline_amd import configs as C
from tests.qdata import sample_cols

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _host_rows(mlx, cols):
    import torch

    w, s, b = mlx
    idx = torch.as_tensor(cols, device=w.device)
    q = O.unpack_nibbles_u32(w.index_select(0, idx).cpu().numpy().view(np.uint32))
    sb = s.index_select(0, idx).cpu().view(torch.int16).numpy().view(np.uint16)
    bb = b.index_select(0, idx).cpu().view(torch.int16).numpy().view(np.uint16)
    return q, sb, bb


def _check_projection(gpu, name, K, N, Ms, seed, outliers=0.0):
    import torch

    from raceline_amd import ops, synth

    mlx = synth.random_affine(N, K, seed, gpu, packed=False)
    pw = ops.pack_affine(*mlx)
    cols = sample_cols(N, 256, seed=seed)
    q, s, b = _host_rows(mlx, cols)
    for M in Ms:
        x = synth.random_activations(M, K, seed + M, gpu, outliers=outliers)
        y = ops.linear(x, pw)
        torch.cuda.synchronize()
        ref = O.linear_affine_f64(x.cpu().numpy(), q, s, b, "f16")
        O.check_close(y.cpu().numpy()[:, cols], ref, TOL, f"{name} K={K} N={N} M={M}")


@pytest.mark.parametrize("name,K,N", C.CFG3_27B)
def test_27b_decode(gpu, name, K, N):
    """Config 3: the 27B layer's projections at M = 1 and 8 (the decode kernel)."""
    _check_projection(gpu, name, K, N, (1, 8), seed=300 + N % 97)


@pytest.mark.parametrize("name,K,N", C.CFG3_27B)
def test_27b_prefill(gpu, name, K, N):
    """Config 4: the same projections at M = 2048 with 1% outliers x20 (the prefill kernel;
    the down projection's K is split in two)."""
    _check_projection(gpu, name, K, N, (C.CFG4_PREFILL_M,), seed=400 + N % 89, outliers=0.01)


@pytest.mark.parametrize("name,K,N", C.CFG2_9B)
def test_9b_decode(gpu, name, K, N):
    """Config 2: the 9B layer's six projections at M = 1 and 5."""
    _check_projection(gpu, name, K, N, (1, 5), seed=200 + N % 83)


def test_cfg1_single_linear(gpu):
    """Config 1's shape (M = 1, K = N = 4096) on every output column."""
    import torch

    from raceline_amd import ops, synth

    K = N = 4096
    mlx = synth.random_affine(N, K, 0, gpu, packed=False)
    pw = ops.pack_affine(*mlx)
    q, s, b = _host_rows(mlx, np.arange(N))
    x = synth.random_activations(1, K, 1, gpu)
    y = ops.linear(x, pw)
    torch.cuda.synchronize()
    O.check_close(y.cpu().numpy(), O.linear_affine_f64(x.cpu().numpy(), q, s, b, "f16"), TOL, "cfg1")


@pytest.mark.parametrize("M", [1, 8])
def test_decode_beyond_24576_inputs(gpu, M):
    """A reduction longer than the decode kernel's 16 waves x 24 groups (K > 24576: an
    intermediate size above that in a down projection) still runs at decode sizes."""
    _check_projection(gpu, "long K", 26624, 512, (M,), seed=500)
