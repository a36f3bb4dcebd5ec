"""Parity of the HIP native-format ("q4n") linear with the oracle.

The native format has one fp32 scale per output row and a 4-bit codebook value per
weight (tools/quantlib.py:23-28: int15, int16 = int15 + 0.5, fp4 e2m1); the column scale
is folded into the activations upstream (src/engine.mm:515-530), so these tests pass x
with it applied. Bar: max|y - ref| / rms(ref) <= 1e-3 against the fp64 product
(oracle.linear_native_f64), plus the reference test's own criterion (via
oracle.check_close); the codebook decode is checked exactly through a one-hot input.
"""

import numpy as np
import pytest

import oracle as O
from tests.qdata import sample_cols, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-3
BOOKS = ["int15", "int16", "fp4"]


def _upload(q, s_row, book, dev):
    import torch

    from raceline_amd import ops

    w = torch.from_numpy(O.pack_nibbles_u32(q).view(np.int32)).to(dev)
    return ops.pack_native(w, to_dev(s_row.astype(np.float32), dev), book)


def _run(dev, x, nw, kernel=0, accum_into=None):
    import torch

    from raceline_amd import ops

    out = None if accum_into is None else to_dev(accum_into.astype(np.float32), dev)
    y = ops.linear_native(to_dev(x, dev), nw, out=out, accum=accum_into is not None, kernel=kernel)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("book", BOOKS)
def test_codebook_decode_is_exact(gpu, book):
    """Every code of every row, read out by one-hot activations (x = e_k): y[k][n] is
    exactly s[n] * L[q[n][k]] (+ 0.5 s[n] for int16) in both kernels."""
    K, N = 64, 48
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    q[:, :16] = np.arange(16, dtype=np.uint8)[None, :]              # every code appears
    s_row = np.ones(N, np.float32)
    nw = _upload(q, s_row, book, gpu)
    x = np.eye(K, dtype=np.float16)
    levels = O.LEVELS[book]
    for kernel, rows in ((1, [0, 5, 17, 63]), (2, list(range(K)))):
        xs = x[rows]
        y = _run(gpu, xs, nw, kernel=kernel)
        ref = levels[q[:, rows].T] if book != "int16" else O.LEVELS["int15"][q[:, rows].T] + 0.5
        np.testing.assert_array_equal(y, ref.astype(np.float32), err_msg=f"{book} kernel {kernel}")


@pytest.mark.parametrize("book", BOOKS)
@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (3, 2560, 1000), (8, 12288, 512), (1, 17408, 640),
                                   (9, 512, 96), (130, 5120, 1024), (257, 1024, 300)])
def test_native_parity(gpu, book, M, K, N):
    rng = np.random.default_rng(M + K + N)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s_row = rng.uniform(0.002, 0.02, size=N).astype(np.float32)
    c_col = rng.uniform(0.5, 2.0, size=K).astype(np.float32)
    x = (rng.standard_normal((M, K), dtype=np.float32) * c_col[None, :]).astype(np.float16)  # column scale folded
    nw = _upload(q, s_row, book, gpu)
    y = _run(gpu, x, nw)
    O.check_close(y, O.linear_native_f64(x, q, s_row, book), TOL, f"native {book} M={M} K={K} N={N}")


@pytest.mark.parametrize("book", BOOKS)
def test_native_accumulates(gpu, book):
    rng = np.random.default_rng(77)
    for M, K, N in ((2, 1024, 256), (40, 1024, 256), (40, 8192, 512)):   # the last splits K
        q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
        s_row = rng.uniform(0.002, 0.02, size=N).astype(np.float32)
        x = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
        y0 = rng.standard_normal((M, N)).astype(np.float32)
        y = _run(gpu, x, _upload(q, s_row, book, gpu), accum_into=y0)
        O.check_close(y - y0, O.linear_native_f64(x, q, s_row, book), TOL, f"native accumulate {book} M={M}")


@pytest.mark.parametrize("book", BOOKS)
@pytest.mark.parametrize("M,K,N", O.REFERENCE_NATIVE_CASES)
def test_reference_native_cases(gpu, book, M, K, N):
    """The reference's native correctness cases (tests/test_linear.mm:447-450): drawn with
    its generator, stored in the blocked file layout, packed on the device."""
    from raceline_amd import ops

    q, s, x = O.reference_native_case(M, K, N)
    w_blk, s_pad, n_pad = O.pack_native_blocked(q, s)
    nw = ops.pack_native_blocked(to_dev(w_blk, gpu), to_dev(s_pad, gpu), K, n_pad, 0, N, book)
    y = _run(gpu, x, nw)
    cols = sample_cols(N, 256, seed=M)
    O.check_close(y[:, cols], O.linear_native_f64(x, q[cols], s[cols], book), TOL,
                  f"reference native case {book} M={M} K={K} N={N}")


def test_native_rows_do_not_depend_on_other_rows(gpu):
    rng = np.random.default_rng(91)
    K, N = 2048, 512
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s_row = rng.uniform(0.002, 0.02, size=N).astype(np.float32)
    x = rng.standard_normal((8, K), dtype=np.float32).astype(np.float16)
    nw = _upload(q, s_row, "int16", gpu)
    y_all = _run(gpu, x, nw, kernel=1)
    for m in (0, 5):
        np.testing.assert_array_equal(_run(gpu, x[m:m + 1], nw, kernel=1)[0], y_all[m])


@pytest.mark.parametrize("book", BOOKS)
def test_native_reads_nothing_past_the_weight(gpu, book):
    """As the affine test of the same name: codes past a wave's range read zeros, never the
    all-ones bytes that follow the packed codes in their buffer."""
    import torch

    from raceline_amd import ops

    rng = np.random.default_rng(5)
    M, K, N = 3, 17408, 40
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s_row = rng.uniform(0.002, 0.02, size=N).astype(np.float32)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    nw = _upload(q, s_row, book, gpu)
    nbytes = nw.packed.numel()
    big = torch.full((nbytes + 16384,), 255, dtype=torch.uint8, device=gpu)
    big[:nbytes] = nw.packed
    nw2 = ops.NativeWeight(big, nw.s_row, K, N, book)
    for kernel in (1, 2):
        y = _run(gpu, x, nw2, kernel=kernel)
        assert np.isfinite(y).all(), f"kernel {kernel} read past the packed codes"
        O.check_close(y, O.linear_native_f64(x, q, s_row, book), TOL, f"native tail {book} kernel {kernel}")


@pytest.mark.parametrize("book", ["int15", "fp4"])
@pytest.mark.parametrize("M,K,N", [(1, 4096, 1024), (5, 12288, 512), (64, 2048, 300)])
def test_raw_product(gpu, book, M, K, N):
    """rlq_linear_native_raw (linear_q4n_raw, kernels/linear.metal:226-252): the product
    without the row scale. It equals the scaled product with unit row scales bit for bit
    (the epilogue multiplies by 1), and the fp64 product x . L(q)^T."""
    import torch

    from raceline_amd import ops

    rng = np.random.default_rng(M + K)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    x = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    raw = ops.linear_native_raw(to_dev(x, gpu), _upload(q, rng.uniform(0.5, 2, N), book, gpu))
    unit = ops.linear_native(to_dev(x, gpu), _upload(q, np.ones(N, np.float32), book, gpu))
    torch.cuda.synchronize()
    assert torch.equal(raw, unit)
    O.check_close(raw.cpu().numpy(), O.linear_native_f64(x, q, np.ones(N), book), TOL, f"raw {book} M={M}")
