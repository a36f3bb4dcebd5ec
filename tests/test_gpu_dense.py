"""Parity of the HIP dense fp16 linear (the reference's linear_f16, kernels/linear.metal:
186-225) with the fp64 product of the same fp16 weights: max|y - ref| / rms(ref) <= 1e-3
(fp32 accumulation of exact fp16 products), via oracle.check_close; packing from the
blocked f16b file layout (tools/convert.py:218-226) is checked against numpy's restatement."""

import numpy as np
import pytest

import oracle as O
from tests.qdata import to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _blocked_f16(W):
    """numpy restatement of tools/convert.py:218-226: rows padded to 256, [blocks][K][256]."""
    n, k = W.shape
    n_pad = -(-n // 256) * 256
    full = np.zeros((n_pad, k), dtype=np.float16)
    full[:n] = W
    return np.ascontiguousarray(full.reshape(n_pad // 256, 256, k).transpose(0, 2, 1)), n_pad


@pytest.mark.parametrize("M,K,N", [(1, 2048, 257), (3, 10240, 512), (9, 512, 96), (512, 2048, 257), (40, 96, 33)])
def test_dense_parity(gpu, M, K, N):
    import torch

    from raceline_amd import ops

    rng = np.random.default_rng(M * 31 + K + N)
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float16)
    dw = ops.pack_f16(to_dev(W, gpu))
    y = ops.linear_f16(to_dev(x, gpu), dw)
    torch.cuda.synchronize()
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    O.check_close(y.cpu().numpy(), ref, TOL, f"f16 linear M={M} K={K} N={N}")
    # accumulate
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    h = to_dev(y0, gpu)
    ops.linear_f16(to_dev(x, gpu), dw, out=h, accum=True)
    torch.cuda.synchronize()
    O.check_close(h.cpu().numpy() - y0, ref, TOL, f"f16 linear accumulate M={M}")


def test_dense_blocked_parts(gpu):
    """A stacked tensor in the f16b layout: each part packed from its rows."""
    import torch

    from raceline_amd import ops

    rng = np.random.default_rng(5)
    K = 1024
    W = (rng.standard_normal((300, K)) * 0.05).astype(np.float16)
    w_blk, n_pad = _blocked_f16(W)
    x = rng.standard_normal((4, K)).astype(np.float16)
    for row0, rows in ((0, 200), (200, 100)):
        dw = ops.pack_f16_blocked(to_dev(w_blk, gpu), K, n_pad, row0, rows)
        y = ops.linear_f16(to_dev(x, gpu), dw)
        torch.cuda.synchronize()
        ref = x.astype(np.float64) @ W[row0:row0 + rows].astype(np.float64).T
        O.check_close(y.cpu().numpy(), ref, TOL, f"f16 blocked part {row0}")


def test_dense_reads_nothing_past_the_weight(gpu):
    """K = 10240 splits into 16 waves of 24 steps of which the last wave has only 20:
    its 4 steps past the range must read zeros, not the all-ones bytes (NaN as fp16) that
    follow the packed matrix in its buffer."""
    import torch

    from raceline_amd import ops

    rng = np.random.default_rng(12)
    M, K, N = 2, 10240, 40
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float16)
    dw = ops.pack_f16(to_dev(W, gpu))
    nbytes = dw.packed.numel()
    big = torch.full((nbytes + 16384,), 255, dtype=torch.uint8, device=gpu)
    big[:nbytes] = dw.packed
    y = ops.linear_f16(to_dev(x, gpu), ops.DenseWeight(big, K, N))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert np.isfinite(y).all(), "the dense kernel read past the packed weight"
    O.check_close(y, x.astype(np.float64) @ W.astype(np.float64).T, TOL, "f16 linear tail")
