"""Precision of the affine path whatever the activations' scale, and the in-kernel dequant.

- Activations far from N(0, 1): rows scaled by 1e-2, 1e-3 and 1e-4 (many entries then fp16
  subnormals), and rows that mix 1e-4 entries with O(1) ones, through the decode GEMV, the
  prefill GEMM and the affine MoE kernels, against the fp64 dequant+matmul at the same bar
  as every other parity test (max|err|/rms <= 1e-3 and tests/test_linear.mm:178's rule).
  The reference hands its fp16 activations to the matrix unit unchanged
  (kernels/linear.metal:67,86-88), so its accuracy does not depend on their scale.
- One-hot activations (x = e_k): every output is one dequantized weight,
  y[m][n] = fp32(s) * q + fp32(b) (kernels/linear.metal:3-4), which both hot kernels must
  give bit for bit: this pins the codes' conversion and the scale/bias epilogue inside the
  kernels that run the model, not only the checking kernel rlq_dequant_affine.
"""

import numpy as np
import pytest

import oracle as O
from tests.qdata import make_layer, to_dev, upload, upload_mlx

pytestmark = pytest.mark.gpu
TOL = 1e-3
SCALES = [1e-2, 1e-3, 1e-4]


def _linear(gpu, x_np, wt, kernel):
    import torch

    from raceline_amd import ops

    y = ops.linear(to_dev(x_np, gpu), wt, kernel=kernel)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def scaled_x(seed, M, K, scale):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((M, K)) * scale).astype(np.float16)


def mixed_x(seed, M, K):
    """Rows of 1e-4-scale entries with a few O(1) ones, and rows whose groups alternate
    between the two scales."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)) * 1e-4
    big = rng.random((M, K)) < 0.02
    x = np.where(big, rng.standard_normal((M, K)), x)
    for m in range(1, M, 2):
        g = np.arange(K) // 64
        x[m] = np.where(g % 2 == 0, rng.standard_normal(K), rng.standard_normal(K) * 1e-4)
    return x.astype(np.float16)


GEMV_SHAPES = [(1, 4096, 512), (5, 4096, 512), (8, 12288, 256), (1, 17408, 128), (3, 9216, 96)]
GEMM_SHAPES = [(64, 4096, 512), (200, 2048, 384), (150, 8192, 1024)]   # the last splits K


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("M,K,N", GEMV_SHAPES)
def test_gemv_small_activations(gpu, M, K, N, scale):
    sd = "f16" if M % 2 else "bf16"
    q, s, b = make_layer(M + K + N, N, K, sd)
    x = scaled_x(K + M, M, K, scale)
    y = _linear(gpu, x, upload(q, s, b, sd, gpu), kernel=1)
    O.check_close(y, O.linear_affine_f64(x, q, s, b, sd), TOL, f"gemv M={M} K={K} x*{scale:g}")


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("M,K,N", GEMM_SHAPES)
def test_gemm_small_activations(gpu, M, K, N, scale):
    sd = "f16" if M % 2 else "bf16"
    q, s, b = make_layer(M + K + N, N, K, sd)
    x = scaled_x(K + M, M, K, scale)
    y = _linear(gpu, x, upload(q, s, b, sd, gpu), kernel=2)
    O.check_close(y, O.linear_affine_f64(x, q, s, b, sd), TOL, f"gemm M={M} K={K} x*{scale:g}")


@pytest.mark.parametrize("kernel,M", [(1, 1), (1, 6), (2, 96)])
def test_mixed_scale_rows(gpu, kernel, M):
    K, N = 4096, 512
    q, s, b = make_layer(60 + M, N, K)
    x = mixed_x(61 + M, M, K)
    y = _linear(gpu, x, upload(q, s, b, "f16", gpu), kernel=kernel)
    ref = O.linear_affine_f64(x, q, s, b)
    for m in range(M):   # each row on its own: the bar holds per token, not only on the batch's rms
        O.check_close(y[m:m + 1], ref[m:m + 1], TOL, f"mixed-scale row {m} (kernel {kernel})")


def test_gemm_extreme_rows(gpu):
    """Rows at the ends of the fp16 range go through the prefill kernel's prescale: entries
    near 60000, a row of subnormals only, an all-zero row."""
    M, K, N = 16, 1024, 256
    q, s, b = make_layer(70, N, K)
    rng = np.random.default_rng(71)
    x = rng.standard_normal((M, K))
    x[0] = np.clip(x[0] * 5e3, -6e4, 6e4)          # finite in fp16 (max 65504)
    x[0, 5] = 60000.0
    x[1] = rng.integers(-1023, 1024, size=K) * 2.0 ** -24   # fp16 subnormals only
    x[2] = 0.0
    x[3] *= 1e-5
    x = x.astype(np.float16)
    y = _linear(gpu, x, upload(q, s, b, "f16", gpu), kernel=2)
    ref = O.linear_affine_f64(x, q, s, b)
    assert (y[2] == 0).all()
    for m in (0, 1, 3, 4):
        O.check_close(y[m:m + 1], ref[m:m + 1], TOL, f"extreme row {m}")


@pytest.mark.parametrize("sd", ["f16", "bf16"])
@pytest.mark.parametrize("kernel,M,K,N", [(1, 1, 4096, 256), (1, 8, 4096, 256), (1, 5, 17408, 48),
                                          (2, 40, 2048, 272), (2, 33, 8256, 1024)])
def test_one_hot_rows_give_dequantized_weights(gpu, sd, kernel, M, K, N):
    """x = e_k: y[m][n] must equal fp32(s[n][k/64]) * q[n][k] + fp32(b[n][k/64]) exactly,
    the affine dequant of kernels/linear.metal:3-4 (rounded once, as
    oracle.dequant_affine), through the decode kernel (kernel 1) and the prefill kernel
    (kernel 2, K split in two on the last shape). Scales and biases follow the reference
    test's generator (s in [0.001, 0.012], b = -7.5 s + U(-0.01, 0.01), rounded to the
    16-bit format), with a quarter of the biases replaced by values below 2^-14; codes are
    uniform."""
    rng = np.random.default_rng(80 + M + K)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    sf = rng.uniform(0.001, 0.012, size=(N, K // 64)).astype(np.float32)
    bf = (-7.5 * sf + rng.uniform(-0.01, 0.01, size=sf.shape)).astype(np.float32)
    # a quarter of the biases below fp16's normal range (2^-14), where a conversion of a bf16
    # bias to fp16 would round
    tiny = rng.random(sf.shape) < 0.25
    bf = np.where(tiny, rng.uniform(-2.0 ** -15, 2.0 ** -15, size=sf.shape), bf).astype(np.float32)
    s, b = O.scale_from_f32(sf, sd), O.scale_from_f32(bf, sd)
    ks = rng.choice(K, size=M, replace=False)
    ks[0] = K - 1                                    # the last input of the last group
    if M > 1:
        ks[1] = 64 * (K // 128) + 1                  # an odd element mid-row
    x = np.zeros((M, K), np.float16)
    x[np.arange(M), ks] = 1.0
    y = _linear(gpu, x, upload(q, s, b, sd, gpu), kernel=kernel)
    W = O.dequant_affine(q, s, b, sd)
    ref = W[:, ks].T.astype(np.float32)
    diff = y.view(np.uint32) != ref.view(np.uint32)
    assert not diff.any(), (f"{diff.sum()} outputs differ from the dequantized weight; first at "
                            f"{np.argwhere(diff)[0]}: {y[diff][0]!r} vs {ref[diff][0]!r}")


# ------------------------------------------------------------------ MoE (affine experts)

def _moe_weights(seed, E, H, I, dev):
    from raceline_amd import ops

    rng = np.random.default_rng(seed)
    Wg = (rng.standard_normal(((E + 1) * 2 * I, H), dtype=np.float32) * np.float32(0.02))
    Wd = (rng.standard_normal(((E + 1) * H, I), dtype=np.float32) * np.float32(0.02))
    gu, dn = O.quantize_affine_rtn(Wg, "f16"), O.quantize_affine_rtn(Wd, "f16")
    return gu, dn, ops.pack_moe(upload_mlx(*gu, "f16", dev), upload_mlx(*dn, "f16", dev), E, H, I)


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("T", [1, 3, 40, 80])   # one-token launch, per-tile kernel, staged kernel
def test_moe_small_activations(gpu, T, scale):
    """gate/up + SwiGLU and down with small inputs: act against the fp64 value (half an
    ulp of the fp16 output, a subnormal step included, plus 1e-4 rms), and the down
    product, fed act rows scaled the same way, within 1e-3."""
    import torch

    from raceline_amd import ops

    E, H, I, topk = 16, 1024, 256, 4
    gu, dn, mw = _moe_weights(90 + T, E, H, I, gpu)
    rng = np.random.default_rng(91 + T)
    x = (rng.standard_normal((T, H)) * scale).astype(np.float16)
    logits = rng.standard_normal((T, E + 1)).astype(np.float32)
    r = ops.moe_route(to_dev(logits, gpu), E, topk)
    act = ops.moe_gate_up(to_dev(x, gpu), mw, r)
    torch.cuda.synchronize()
    sel, inv = r.sel.cpu().numpy(), r.inv.cpu().numpy()
    act_g = act.cpu().numpy().astype(np.float64)
    S = topk + 1
    act_ref = np.zeros_like(act_g)
    for a in range(T * S):
        e, row, t = sel[a], inv[a], a // S
        g = O.linear_affine_f64(x[t:t + 1], *(v[O.expert_rows(e, 2 * I)] for v in gu))
        act_ref[row] = O.silu(g[0, :I]) * g[0, I:]
    rms = float(np.sqrt(np.mean(act_ref ** 2)))
    bound = 2.0 ** -10 * np.abs(act_ref) + 2.0 ** -24 + 1e-4 * rms
    bad = np.abs(act_g - act_ref) > bound
    assert not bad.any(), f"act x*{scale:g}: {bad.sum()} values off; worst {np.abs(act_g - act_ref).max():.3e}"
    # the down product on act rows of the same scale (SwiGLU of x*scale would be ~scale^2)
    a_in = (rng.standard_normal(act_g.shape) * scale).astype(np.float16)
    y = ops.moe_down(to_dev(a_in, gpu), mw, r)
    torch.cuda.synchronize()
    y_g = y.cpu().numpy()
    y_ref = np.zeros(y_g.shape)
    for a in range(T * S):
        e, row = sel[a], inv[a]
        y_ref[row] = O.linear_affine_f64(a_in[row:row + 1], *(v[O.expert_rows(e, H)] for v in dn))[0]
    O.check_close(y_g, y_ref, TOL, f"moe down x*{scale:g} T={T}")


@pytest.mark.parametrize("T", [1, 4, 40, 96])
def test_moe_layer_small_activations(gpu, T):
    """The whole layer (rlq_moe) at x * 0.1 against oracle.moe_layer_f64. (Smaller inputs
    put the SwiGLU outputs, which the reference stores as fp16, among fp16 subnormals,
    whose spacing is then a few thousandths of their size: a single rounding flip between
    the fp32 and the fp64 computation moves the layer's output by more than the 1e-3 bar.
    The gate/up and down products themselves are checked down to 1e-4 above.)"""
    import torch

    from raceline_amd import ops

    E, H, I, topk = 16, 1024, 256, 4
    gu, dn, mw = _moe_weights(95 + T, E, H, I, gpu)
    rng = np.random.default_rng(96 + T)
    x = (rng.standard_normal((T, H)) * 0.1).astype(np.float16)
    logits = rng.standard_normal((T, E + 1)).astype(np.float32)
    h = torch.zeros((T, H), dtype=torch.float32, device=gpu)
    ops.moe(to_dev(x, gpu), to_dev(logits, gpu), mw, topk, h)
    torch.cuda.synchronize()
    ref, _, _ = O.moe_layer_f64(x, logits, gu, dn, E, topk, I, H)
    O.check_close(h.cpu().numpy().astype(np.float64), ref, TOL, f"moe layer x*0.1 T={T}")
