"""Parity of the HIP affine 4-bit linear (decode GEMV and prefill GEMM) with the oracle.

Bar: dequantized weights bit-exact; outputs max|y - ref| / rms(ref) <= 1e-3 against the
fp64 dequant+matmul (oracle.linear_affine_f64), and the reference test's own criterion
max|err| < 2e-3 * rms + 1e-4 (tests/test_linear.mm:178), both via oracle.check_close.
"""

import numpy as np
import pytest

import oracle as O
from tests.qdata import make_layer, make_x, packed_layout_np, sample_cols, to_dev, upload, upload_mlx

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _run(gpu, x_np, wt, kernel=0, accum_into=None):
    import torch

    from raceline_amd import ops

    x = to_dev(x_np, gpu)
    out = None if accum_into is None else to_dev(accum_into.astype(np.float32), gpu)
    y = ops.linear(x, wt, out=out, accum=accum_into is not None, kernel=kernel)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("sd", ["f16", "bf16"])
def test_dequant_bit_exact(gpu, sd):
    import torch

    from raceline_amd import ops

    rng = np.random.default_rng(100)
    N, K = 300, 512
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    # scales over the whole finite range of the format, subnormals and both signs included
    s = rng.integers(0, 1 << 16, size=(N, K // 64), dtype=np.uint32).astype(np.uint16)
    b = rng.integers(0, 1 << 16, size=(N, K // 64), dtype=np.uint32).astype(np.uint16)
    if sd == "f16":
        s &= np.uint16(0x7BFF) | np.uint16(0x8000)     # keep exponents finite
        b &= np.uint16(0x7BFF) | np.uint16(0x8000)
    else:
        s &= np.uint16(0x7F7F) | np.uint16(0x8000)
        b &= np.uint16(0x7F7F) | np.uint16(0x8000)
    wt = upload(q, s, b, sd, gpu)
    got = ops.dequant(wt)
    torch.cuda.synchronize()
    with np.errstate(over="ignore", invalid="ignore"):
        ref = O.dequant_affine(q, s, b, sd)
    g = got.cpu().numpy()
    same = (g.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(g) & np.isnan(ref))
    assert same.all(), f"{(~same).sum()} dequantized weights differ"


GEMV_CASES = [  # (M, K, N); the decode kernel takes M <= 8
    (1, 256, 32), (1, 4096, 4096), (5, 2560, 9216), (3, 9216, 2560), (2, 2560, 1000),
    (8, 512, 2048), (8, 1024, 300), (7, 640, 96), (1, 17408, 640), (4, 64, 33), (1, 12288, 4096),
    (5, 4096, 6144),  # the 9B layer's stacked q/k/v
    (1, 64, 16), (3, 320, 40), (8, 576, 17),  # one group; odd group counts
    # several tokens over 12, 16 and 24 groups per wave (activation rows staged 8 groups at
    # a time; the last wave's range ends inside its second chunk or holds one group of it)
    (6, 13312, 200), (2, 8256, 64), (8, 17408, 48),
]


@pytest.mark.parametrize("M,K,N", GEMV_CASES)
def test_gemv_parity(gpu, M, K, N):
    sd = "f16" if (M + K + N) % 2 else "bf16"
    q, s, b = make_layer(M * 1000 + N, N, K, sd)
    x = make_x(K + M, M, K)
    y = _run(gpu, x, upload(q, s, b, sd, gpu), kernel=1)
    ref = O.linear_affine_f64(x, q, s, b, sd)
    O.check_close(y[:, :N], ref, TOL, f"gemv M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N", [(1, 1024, 512), (7, 4096, 1024), (8, 512, 96)])
def test_gemv_accumulates(gpu, M, K, N):
    q, s, b = make_layer(7, N, K)
    x = make_x(8, M, K)
    y0 = np.random.default_rng(9).standard_normal((M, N)).astype(np.float32)
    y = _run(gpu, x, upload(q, s, b, "f16", gpu), kernel=1, accum_into=y0)
    ref = O.linear_affine_f64(x, q, s, b) + y0.astype(np.float64)
    O.check_close(y, ref, TOL, "gemv accum")


GEMM_CASES = [(9, 512, 96), (16, 1024, 300), (32, 2048, 1024), (33, 256, 64), (130, 5120, 1024),
              (512, 2048, 1024), (70, 9216, 2560), (256, 1024, 300), (40, 2560, 1000),
              # an odd number of groups (the last pair half empty), a single group, ragged M and N
              (129, 320, 17), (64, 64, 48), (200, 576, 272), (300, 192, 513),
              # a long K with an odd number of groups
              (100, 4160, 1000)]


@pytest.mark.parametrize("M,K,N", GEMM_CASES)
def test_gemm_parity(gpu, M, K, N):
    sd = "f16" if (M + N) % 2 else "bf16"
    q, s, b = make_layer(M * 7 + N, N, K, sd)
    x = make_x(M + K, M, K, outliers=0.01)
    y = _run(gpu, x, upload(q, s, b, sd, gpu), kernel=2)
    ref = O.linear_affine_f64(x, q, s, b, sd)
    O.check_close(y, ref, TOL, f"gemm M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N", [(200, 1024, 384), (150, 8192, 1024)])   # the second splits K
def test_gemm_accumulates(gpu, M, K, N):
    q, s, b = make_layer(1, N, K)
    x = make_x(2, M, K)
    y0 = np.random.default_rng(3).standard_normal((M, N)).astype(np.float32)
    y = _run(gpu, x, upload(q, s, b, "f16", gpu), kernel=2, accum_into=y0)
    O.check_close(y, O.linear_affine_f64(x, q, s, b) + y0, TOL, "gemm accum")


@pytest.mark.parametrize("K", [4096, 9216, 17408])   # two tiles per workgroup; 12 and 24 groups per wave
def test_rows_do_not_depend_on_other_rows(gpu, K):
    """A token's result is bit-identical whatever rows share the call (the reference's
    determinism rule, kernels/linear.metal:264-266): one row alone vs. inside M = 8."""
    M, N = 8, 1024
    q, s, b = make_layer(11, N, K)
    x = make_x(12, M, K)
    wt = upload(q, s, b, "f16", gpu)
    y_all = _run(gpu, x, wt, kernel=1)
    for m in (0, 3, 7):
        y_one = _run(gpu, x[m:m + 1], wt, kernel=1)
        np.testing.assert_array_equal(y_one[0], y_all[m])


@pytest.mark.parametrize("K,N,sd", [(1024, 65552, "bf16"), (512, 65536 + 160, "f16")])
def test_one_token_two_tiles_per_workgroup(gpu, K, N, sd):
    """One token on a weight of 4096 tiles or more runs two tiles per workgroup (an odd tile
    count leaves the last workgroup one tile): the row is within the bar of the fp64 product,
    bit-identical to the same row inside a 2-row call (one tile per workgroup), and ACCUM
    adds to y."""
    q, s, b = make_layer(K + 5, N, K, sd)
    x = make_x(K + 6, 2, K)
    wt = upload(q, s, b, sd, gpu)
    y1 = _run(gpu, x[:1], wt, kernel=1)
    y2 = _run(gpu, x, wt, kernel=1)
    np.testing.assert_array_equal(y1[0], y2[0])
    cols = sample_cols(N, seed=K)
    O.check_close(y1[:, cols], O.linear_affine_f64(x[:1], q[cols], s[cols], b[cols], sd), TOL, f"K={K} N={N}")
    y0 = np.random.default_rng(K + 1).standard_normal((1, N)).astype(np.float32)
    ya = _run(gpu, x[:1], wt, kernel=1, accum_into=y0)
    np.testing.assert_array_equal(ya, y0 + y1)


@pytest.mark.parametrize("K,N", [(2048, 640), (8192, 1024)])   # the second splits K
def test_gemm_rows_do_not_depend_on_other_rows(gpu, K, N):
    """The prefill kernel keeps the same rule: rows 50..119 alone (M = 70) give the same
    bits as inside M = 200, wherever the 128-row tiles fall (the split of K depends on the
    shape of the weight only)."""
    M = 200
    q, s, b = make_layer(15, N, K)
    x = make_x(16, M, K)
    wt = upload(q, s, b, "f16", gpu)
    y_all = _run(gpu, x, wt, kernel=2)
    y_sub = _run(gpu, x[50:120], wt, kernel=2)
    np.testing.assert_array_equal(y_sub, y_all[50:120])


# Weights whose K the prefill kernel splits over 2 workgroups per output tile (from the
# weight's shape: at most 32 feature blocks, 64 group pairs or more, rounds at 16 token
# blocks 1.25 times fuller split): an odd number of groups (K = 8256: splits of 33 and 32
# group pairs, the last pair half empty), bf16 biases, ragged M and N, the 27B down shape.
SPLIT_GEMM_CASES = [(150, 8192, 1024, "f16"), (300, 8256, 1000, "f16"), (257, 9216, 600, "bf16"),
                    (130, 17408, 5120, "f16")]


@pytest.mark.parametrize("M,K,N,sd", SPLIT_GEMM_CASES)
def test_gemm_split_k(gpu, M, K, N, sd):
    """The last split to arrive adds the partials in split order: the result matches the
    oracle, with ACCUM too, and a repeat call gives the same bits (the counters are left
    zero)."""
    q, s, b = make_layer(M + K + N, N, K, sd)
    x = make_x(M + 5, M, K, outliers=0.01)
    wt = upload(q, s, b, sd, gpu)
    cols = sample_cols(N, 384, seed=K)
    ref = O.linear_affine_f64(x, q[cols], s[cols], b[cols], sd)
    y = _run(gpu, x, wt, kernel=2)
    O.check_close(y[:, cols], ref, TOL, f"split gemm M={M} K={K} N={N}")
    np.testing.assert_array_equal(_run(gpu, x, wt, kernel=2), y)
    y0 = np.random.default_rng(M).standard_normal((M, N)).astype(np.float32)
    ya = _run(gpu, x, wt, kernel=2, accum_into=y0)
    O.check_close(ya[:, cols], ref + y0[:, cols], TOL, f"split gemm accum M={M} K={K} N={N}")


def test_gemm_split_k_row_chunks(gpu):
    """A split weight whose output tiles outnumber the workspace's 1024 counters launches in
    chunks of rows: at the 27B down shape (K = 17408, N = 5120: 20 feature blocks, split in 2)
    a launch takes 51 token blocks, 6528 rows. Rows on both sides of the chunk boundary give
    the bits they give in a call of their own, which matches the oracle."""
    import torch

    from raceline_amd import ops, synth

    K, N = 17408, 5120
    M = 6528 + 300
    mlx = synth.random_affine(N, K, 91, gpu, packed=False)
    pw = ops.pack_affine(*mlx)
    x = synth.random_activations(M, K, 92, gpu, outliers=0.01)
    y = ops.linear(x, pw, kernel=2)
    r0, r1 = 6400, 6700
    y_sub = ops.linear(x[r0:r1].contiguous(), pw, kernel=2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y_sub.cpu().numpy(), y[r0:r1].cpu().numpy())
    cols = sample_cols(N, 128, seed=93)
    w, sc, bi = mlx
    idx = torch.as_tensor(cols, device=gpu)
    q = O.unpack_nibbles_u32(w.index_select(0, idx).cpu().numpy().view(np.uint32))
    sb = sc.index_select(0, idx).cpu().view(torch.int16).numpy().view(np.uint16)
    bb = bi.index_select(0, idx).cpu().view(torch.int16).numpy().view(np.uint16)
    ref = O.linear_affine_f64(x[r0:r1].cpu().numpy(), q, sb, bb, "f16")
    O.check_close(y_sub.cpu().numpy()[:, cols], ref, TOL, "split gemm across a row chunk boundary")


@pytest.mark.parametrize("K,N", [(17024, 512), (17472, 40), (17408, 1000)])   # K split in 7; 266 and 273 groups; ragged N
def test_split_k_decode_between_other_calls(gpu, K, N):
    """Weights whose K the decode kernel splits across workgroups (few tiles, long K) keep
    their arrival counters in the workspace's first bytes and leave them zero: a split call,
    a prefill call that fills the same workspace with its own data, a split call of other
    rows, and a split call with ACCUM all match the oracle; one row alone gives the same
    bits as inside M = 8."""
    q, s, b = make_layer(21 + K, N, K)
    wt = upload(q, s, b, "f16", gpu)
    x8 = make_x(22, 8, K)
    ref8 = O.linear_affine_f64(x8, q, s, b)
    y8 = _run(gpu, x8, wt, kernel=1)
    O.check_close(y8, ref8, TOL, f"split gemv M=8 K={K} N={N}")
    xg = make_x(23, 64, K)
    O.check_close(_run(gpu, xg, wt, kernel=2), O.linear_affine_f64(xg, q, s, b), TOL, "gemm on the same workspace")
    for m in (0, 5, 7):
        np.testing.assert_array_equal(_run(gpu, x8[m:m + 1], wt, kernel=1)[0], y8[m])
    y0 = np.random.default_rng(24).standard_normal((3, N)).astype(np.float32)
    y = _run(gpu, x8[:3], wt, kernel=1, accum_into=y0)
    O.check_close(y, ref8[:3] + y0, TOL, "split gemv accum")


def test_repeat_calls_reuse_workspace(gpu):
    """Repeated calls give identical results (no state carried between calls)."""
    M, K, N = 1, 4096, 1024
    q, s, b = make_layer(13, N, K)
    x = make_x(14, M, K)
    wt = upload(q, s, b, "f16", gpu)
    first = _run(gpu, x, wt, kernel=1)
    for _ in range(3):
        np.testing.assert_array_equal(_run(gpu, x, wt, kernel=1), first)


@pytest.mark.parametrize("M,K,N", [(1, 17408, 1000), (8, 17408, 1000), (150, 8192, 1024)])   # decode split in 7; prefill in 2
def test_split_k_replays_in_a_graph(gpu, M, K, N):
    """A call whose K is split across workgroups, captured in a graph, gives the eager call's
    bits on every replay, with eager work on the same output and workspace between the
    replays: every call leaves its arrival counters zero, so replays need no reset."""
    import torch

    from raceline_amd import ops, synth

    pw = ops.pack_affine(*synth.random_affine(N, K, 31 + M, gpu, packed=False))
    x = synth.random_activations(M, K, 32 + M, gpu, outliers=0.01)
    want = ops.linear(x, pw)                       # eager; also sizes the workspace
    out = torch.empty(M, N, dtype=torch.float32, device=gpu)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.linear(x, pw, out=out)
    for _ in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        assert torch.equal(ops.linear(x, pw), want)   # an eager split call between replays


@pytest.mark.parametrize("sd", ["f16", "bf16"])
def test_repack_blocked_round_trip(gpu, sd):
    """.rlm blocked q4a tensor (tools/convert.py:92-117) -> MLX layout, per stacked part."""
    import torch

    from raceline_amd import ops

    K = 256
    parts = [make_layer(20 + i, rows, K, sd) for i, rows in enumerate((200, 300))]
    w, s, b, n_pad, offs = O.pack_blocked(parts)
    wb, sb, bb = to_dev(w, gpu), to_dev(s.view(np.int16), gpu), to_dev(b.view(np.int16), gpu)
    dt = torch.float16 if sd == "f16" else torch.bfloat16
    for (off, rows), (q, s_p, b_p) in zip(offs, parts):
        wt, st, bt = ops.repack_blocked(wb, sb, bb, K, n_pad, off, rows, scale_dtype=dt)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(wt.cpu().numpy().view(np.uint32), O.pack_nibbles_u32(q))
        np.testing.assert_array_equal(st.cpu().view(torch.int16).numpy().view(np.uint16), s_p)
        np.testing.assert_array_equal(bt.cpu().view(torch.int16).numpy().view(np.uint16), b_p)


@pytest.mark.parametrize("sd", ["f16", "bf16"])
def test_packed_layout(gpu, sd):
    """The upload packers (from the MLX layout and from the blocked file layout) both
    produce exactly the layout include/rlq.h documents."""
    import torch

    from raceline_amd import ops

    K = 320
    parts = [make_layer(40 + i, rows, K, sd) for i, rows in enumerate((70, 33))]
    for q, s_p, b_p in parts:
        pw = upload(q, s_p, b_p, sd, gpu)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(pw.packed.cpu().numpy(), packed_layout_np(q, s_p, b_p))
    w, s, b, n_pad, offs = O.pack_blocked(parts)
    wb, sb, bb = to_dev(w, gpu), to_dev(s.view(np.int16), gpu), to_dev(b.view(np.int16), gpu)
    dt = torch.float16 if sd == "f16" else torch.bfloat16
    for (off, rows), (q, s_p, b_p) in zip(offs, parts):
        pw = ops.pack_blocked(wb, sb, bb, K, n_pad, off, rows, scale_dtype=dt)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(pw.packed.cpu().numpy(), packed_layout_np(q, s_p, b_p))


def test_blocked_file_tensor_end_to_end(gpu):
    """A stacked q/k/v tensor in the .rlm blocked layout with bf16 scales (what
    tools/convert.py writes): pack each part on the device and run the decode kernel."""
    import torch

    from raceline_amd import ops

    K = 1024
    parts = [make_layer(50 + i, rows, K, "bf16") for i, rows in enumerate((512, 128, 128))]
    w, s, b, n_pad, offs = O.pack_blocked(parts)
    wb, sb, bb = to_dev(w, gpu), to_dev(s.view(np.int16), gpu), to_dev(b.view(np.int16), gpu)
    x = make_x(51, 3, K)
    for (off, rows), (q, s_p, b_p) in zip(offs, parts):
        pw = ops.pack_blocked(wb, sb, bb, K, n_pad, off, rows, scale_dtype=torch.bfloat16)
        y = _run(gpu, x, pw, kernel=1)
        O.check_close(y, O.linear_affine_f64(x, q, s_p, b_p, "bf16"), TOL, f"blocked part at {off}")


def test_group_sums(gpu):
    import torch

    from raceline_amd import ops

    x = make_x(30, 5, 1024)
    got = ops.group_sums(to_dev(x, gpu))
    torch.cuda.synchronize()
    # sequential fp32 sum, as kernels/linear.metal:42-44
    ref = np.zeros((5, 16), np.float32)
    for m in range(5):
        for g in range(16):
            acc = np.float32(0)
            for v in x[m, 64 * g:64 * g + 64]:
                acc = np.float32(acc + np.float32(v))
            ref[m, g] = acc
    np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_stream_read_probe(gpu):
    """rlq_stream_read (the bench's read-rate probe) streams a buffer, ragged sizes included,
    without writing its output for ordinary data, and refuses misaligned arguments."""
    import torch

    from raceline_amd import lib, ops

    buf = torch.arange(1 << 20, dtype=torch.int32, device=gpu)
    out = torch.full((1,), -2.0, dtype=torch.float32, device=gpu)
    for nbytes in (0, 16, 4096 + 48, buf.numel() * 4):
        assert lib.call("rlq_stream_read", buf.data_ptr(), nbytes, out.data_ptr(), ops._stream()) == 0
    torch.cuda.synchronize()
    assert out.item() == -2.0
    with pytest.raises(lib.RlqError):
        lib.call("rlq_stream_read", buf.data_ptr() + 4, 64, out.data_ptr(), ops._stream())
    with pytest.raises(lib.RlqError):
        lib.call("rlq_stream_read", buf.data_ptr(), 40, out.data_ptr(), ops._stream())


@pytest.mark.parametrize("M,K,N", O.REFERENCE_TEST_CASES)
def test_reference_correctness_cases(gpu, M, K, N):
    """The reference's own correctness cases (tests/test_linear.mm:440-446): layers drawn
    with its generator (bf16 scales, blocked file layout), checked on sampled columns
    against the fp64 dequant+matmul, through both weight producers."""
    import torch

    from raceline_amd import ops

    q, s, b, x = O.reference_test_case(M, K, N)
    cols = sample_cols(N, 256, seed=M)
    ref = O.linear_affine_f64(x, q, s, b, "bf16", cols=cols)
    w_blk, s_blk, b_blk, n_pad, offs = O.pack_blocked([(q, s, b)])
    pw_blk = ops.pack_blocked(to_dev(w_blk, gpu), to_dev(s_blk.view(np.int16), gpu), to_dev(b_blk.view(np.int16), gpu),
                              K, n_pad, 0, N, scale_dtype=torch.bfloat16)
    pw_mlx = upload(q, s, b, "bf16", gpu)
    for name, pw in (("blocked", pw_blk), ("mlx", pw_mlx)):
        y = _run(gpu, x, pw)
        O.check_close(y[:, cols], ref, TOL, f"reference case M={M} K={K} N={N} via {name}")


@pytest.mark.parametrize("M,K,N", [(1, 17408, 40), (5, 17408, 40), (1, 640, 48), (3, 2560, 33),
                                   (1, 17472, 40), (8, 17472, 40)])   # K split in 7, the last split short
def test_gemv_reads_nothing_past_the_weight(gpu, M, K, N):
    """A wave's last groups past K (K not a multiple of its group range) must read zeros,
    not whatever follows the packed weight in memory: the weight sits at the head of a
    buffer whose tail is all-ones bits (NaN as fp16 scales). A load past the range that
    escaped the descriptor's range check would turn a zero product into NaN."""
    import torch

    from raceline_amd import ops

    q, s, b = make_layer(17 + K, N, K, "f16")
    x = make_x(3, M, K)
    pw = upload(q, s, b, "f16", gpu)
    nbytes = pw.packed.numel()
    big = torch.full((nbytes + 16384,), 255, dtype=torch.uint8, device=gpu)
    big[:nbytes] = pw.packed
    y = _run(gpu, x, ops.PackedWeight(big, K, N, torch.float16), kernel=1)
    assert np.isfinite(y).all(), "the decode kernel read past the packed weight"
    O.check_close(y, O.linear_affine_f64(x, q, s, b, "f16"), TOL, f"gemv tail M={M} K={K} N={N}")
