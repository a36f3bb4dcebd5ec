"""CPU restatement of the engine steps on the quantized matmul path. TEST INFRASTRUCTURE:
only tests/, __graft_entry__.smoke() and bench.py's CPU baseline may use it, as the checker.

- rms_norm_f16: kernels/ops.metal:74-112 (rms_norm_rows): xn = half(x * inv * w),
  inv = 1/sqrt(mean(x^2) + eps); for native files w is the norm weight times the column
  scales of the matrix it feeds (src/engine.mm:517-530).
- mlp_dense_f64: Engine::encode_mlp (src/engine.mm:943-958): gate_up, SwiGLU
  (ops.metal:446-455, act = half(silu(g) * u * cs)), down added into h.
- head_f64: the final norm and lm_head (engine.mm:1634-1638).
- top_k: rl_top_k (src/capi.mm:74-101): the k largest in descending order, equal values
  by index, NaN left out.

PINNED_BY (checked in tests/test_oracle_engine.py):
- rms_norm_f16: a constant row c gives w / sqrt(1 + eps / c^2) rounded to half; the
  result does not change when the row is scaled (eps = 0); it equals the textbook
  x / rms(x) * w computed by numpy's own norm.
- mlp_dense_f64: with one-hot activations through identity-like weights the SwiGLU of
  known gate and up values comes out; it is linear in h's residual part (h + MLP(h) minus
  h is what the down product adds).
- top_k: against a brute-force stable sort; all-NaN input gives nothing; k > n gives n.
"""

from __future__ import annotations

import numpy as np

from .moe import silu


def rms_norm_f16(h, w, eps: float) -> np.ndarray:
    """half(h[r] * 1/sqrt(mean(h[r]^2) + eps) * w), computed in float64 and rounded once."""
    h = np.asarray(h, np.float64)
    inv = 1.0 / np.sqrt(np.mean(h * h, axis=-1, keepdims=True) + eps)
    return (h * inv * np.asarray(w, np.float64)).astype(np.float16)


def mlp_dense_f64(h, norm_w, eps, linear_gu, linear_dn, I: int, cs=None) -> np.ndarray:
    """h + down(SwiGLU(gate_up(rms_norm(h)))); linear_gu and linear_dn map fp16 rows to the
    float64 product (the oracle's linear for the matrix's format)."""
    xn = rms_norm_f16(h, norm_w, eps)
    g = linear_gu(xn)
    v = silu(g[:, :I]) * g[:, I:2 * I]
    if cs is not None:
        v = v * np.asarray(cs, np.float64)[None, :I]
    act = v.astype(np.float16)
    return np.asarray(h, np.float64) + linear_dn(act)


def top_k(x, k: int):
    """(ids, vals) of the k largest non-NaN entries, descending, ties by index."""
    x = np.asarray(x, np.float32)
    idx = np.nonzero(~np.isnan(x))[0]
    order = idx[np.lexsort((idx, -x[idx].astype(np.float64)))]
    order = order[:max(0, min(k, len(order)))]
    return order.astype(np.int32), x[order]
