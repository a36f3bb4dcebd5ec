"""Oracle for raceline's 4-bit quantized linear layer: packing, dequant, matmul.

TEST INFRASTRUCTURE ONLY. A numpy restatement of the reference's closed forms,
used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker. The product path (raceline_amd, HIP) never imports it.

Every function cites the reference file:line it restates (paths are relative
to the reference repository root). How each one is pinned is listed in
``PINNED_BY`` at the bottom; the tests in tests/test_oracle_*.py carry it out.
"""

from __future__ import annotations

import numpy as np

GROUP = 64     # quantization group along K (kernels/linear.metal:3; tools/convert.py:33)
BLOCK = 256    # output rows per block of the blocked file layout (tools/convert.py:32)

__all__ = [
    "GROUP", "BLOCK", "LEVELS",
    "f32_to_bf16_bits", "bf16_bits_to_f32", "to_bf16_exact", "f32_to_f16_bits", "f16_bits_to_f32",
    "scale_to_f32", "scale_from_f32",
    "unpack_nibbles_u32", "pack_nibbles_u32",
    "pack_blocked", "unpack_blocked", "pack_native_blocked", "unpack_native_blocked",
    "quantize_affine_rtn", "dequant_affine", "dequant_native",
    "group_sums", "linear_affine_f64", "linear_affine_factored_f64", "linear_affine_cpu_f32",
    "linear_native_f64", "check_close", "rel_err",
    "XorShift64", "reference_test_case", "REFERENCE_TEST_CASES", "reference_native_case",
    "REFERENCE_NATIVE_CASES",
]


# ------------------------------------------------------------------ number formats

def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even.

    tests/test_linear.mm:29-33: ``(u + 0x7FFF + ((u >> 16) & 1)) >> 16``.
    NaN inputs are not handled (the reference does not handle them either)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_bits_to_f32(h) -> np.ndarray:
    """bfloat16 bits -> float32, exact widening (tools/convert.py:63-65; tests/test_linear.mm:34-37)."""
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_bf16_exact(x, what: str = "value") -> np.ndarray:
    """float32 -> bfloat16 bits, refusing values that bfloat16 cannot hold exactly.

    tools/convert.py:73-79 (the converter carries MLX's bf16 scales over losslessly)."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    if (bits & 0xFFFF).any():
        raise ValueError(f"{what}: values are not exactly representable in bfloat16")
    return (bits >> 16).astype(np.uint16)


def f32_to_f16_bits(x) -> np.ndarray:
    """float32 -> IEEE binary16 bits, round to nearest even (numpy's conversion)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(h) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def scale_to_f32(bits, scale_dtype: str) -> np.ndarray:
    """Stored 16-bit scale/bias bits -> float32 (exact). scale_dtype is "f16" or "bf16"."""
    if scale_dtype == "f16":
        return f16_bits_to_f32(bits)
    if scale_dtype == "bf16":
        return bf16_bits_to_f32(bits)
    raise ValueError(scale_dtype)


def scale_from_f32(x, scale_dtype: str) -> np.ndarray:
    """float32 -> stored 16-bit bits of the given dtype, round to nearest even."""
    if scale_dtype == "f16":
        return f32_to_f16_bits(x)
    if scale_dtype == "bf16":
        return f32_to_bf16_bits(x)
    raise ValueError(scale_dtype)


# ------------------------------------------------------------------ nibble layouts

def unpack_nibbles_u32(w_u32) -> np.ndarray:
    """MLX packing: [N, K/8] uint32 -> [N, K] uint8; element i sits in bits 4i..4i+3.

    tools/convert.py:82-89 (little-endian bytes; the even element is the low nibble)."""
    w = np.ascontiguousarray(w_u32, dtype=np.uint32)
    n = w.shape[0]
    b = w.view(np.uint8).reshape(n, -1)
    out = np.empty((n, b.shape[1] * 2), dtype=np.uint8)
    out[:, 0::2] = b & 0x0F
    out[:, 1::2] = b >> 4
    return out


def pack_nibbles_u32(q) -> np.ndarray:
    """Inverse of unpack_nibbles_u32: [N, K] codes (0..15) -> [N, K/8] uint32."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    n, k = q.shape
    if k % 8:
        raise ValueError("K must be a multiple of 8")
    if (q > 15).any():
        raise ValueError("codes must be 0..15")
    b = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return np.ascontiguousarray(b).view(np.uint32).reshape(n, k // 8)


def pack_blocked(parts):
    """Blocked q4a layout of the .rlm file (tools/convert.py:92-117).

    parts: list of (q [N,K] uint8, s bits [N,G] uint16, b bits [N,G] uint16), already in the
    16-bit storage dtype. Returns (w bytes [blocks][K][128], s [blocks][G][256],
    b [blocks][G][256], n_pad, [(row offset, rows) per part]). Padding rows are zero
    (q = s = b = 0) as in convert.py:101-103."""
    k = parts[0][0].shape[1]
    g = k // GROUP
    offsets, n = [], 0
    for q, _, _ in parts:
        offsets.append((n, q.shape[0]))
        n += q.shape[0]
    n_pad = -(-n // BLOCK) * BLOCK
    q_all = np.zeros((n_pad, k), dtype=np.uint8)
    s_all = np.zeros((n_pad, g), dtype=np.uint16)
    b_all = np.zeros((n_pad, g), dtype=np.uint16)
    for (off, rows), (q, s, b) in zip(offsets, parts):
        q_all[off:off + rows] = q
        s_all[off:off + rows] = s
        b_all[off:off + rows] = b
    blocks = n_pad // BLOCK
    qb = q_all.reshape(blocks, BLOCK, k).transpose(0, 2, 1)                 # [blocks][K][256]
    w = (qb[:, :, 0::2] | (qb[:, :, 1::2] << 4)).astype(np.uint8)           # even row in the low nibble
    s_out = np.ascontiguousarray(s_all.reshape(blocks, BLOCK, g).transpose(0, 2, 1))
    b_out = np.ascontiguousarray(b_all.reshape(blocks, BLOCK, g).transpose(0, 2, 1))
    return np.ascontiguousarray(w), s_out, b_out, n_pad, offsets


def unpack_blocked(w, s, b, n: int, k: int):
    """Blocked q4a -> (q [n,K] uint8, s bits [n,G], b bits [n,G]); the inverse of pack_blocked.

    Decoding as tools/rlmfile.py:65-75 does for the native kind."""
    g = k // GROUP
    w = np.asarray(w, dtype=np.uint8)
    blocks = w.size // (k * (BLOCK // 2))
    wb = w.reshape(blocks, k, BLOCK // 2)
    codes = np.empty((blocks, k, BLOCK), dtype=np.uint8)
    codes[:, :, 0::2] = wb & 15
    codes[:, :, 1::2] = wb >> 4
    q = codes.transpose(0, 2, 1).reshape(blocks * BLOCK, k)[:n]
    s_rows = np.asarray(s, dtype=np.uint16).reshape(blocks, g, BLOCK).transpose(0, 2, 1).reshape(-1, g)[:n]
    b_rows = np.asarray(b, dtype=np.uint16).reshape(blocks, g, BLOCK).transpose(0, 2, 1).reshape(-1, g)[:n]
    return np.ascontiguousarray(q), np.ascontiguousarray(s_rows), np.ascontiguousarray(b_rows)


def pack_native_blocked(codes, s_row):
    """Blocked q4n layout (tools/convert.py:197-216): codes [N,K] -> w bytes [blocks][K][128],
    row scales padded with 0 to n_pad (float32)."""
    codes = np.asarray(codes, dtype=np.uint8)
    n, k = codes.shape
    n_pad = -(-n // BLOCK) * BLOCK
    q = np.zeros((n_pad, k), dtype=np.uint8)
    q[:n] = codes
    blocks = n_pad // BLOCK
    qb = q.reshape(blocks, BLOCK, k).transpose(0, 2, 1)
    w = np.ascontiguousarray((qb[:, :, 0::2] | (qb[:, :, 1::2] << 4)).astype(np.uint8))
    s_pad = np.zeros(n_pad, dtype=np.float32)
    s_pad[:n] = s_row
    return w, s_pad, n_pad


def unpack_native_blocked(w, n: int, k: int):
    """Blocked q4n codes -> [n, K] codes (tools/rlmfile.py:65-75)."""
    w = np.asarray(w, dtype=np.uint8)
    blocks = w.size // (k * (BLOCK // 2))
    wb = w.reshape(blocks, k, BLOCK // 2)
    codes = np.empty((blocks, k, BLOCK), dtype=np.uint8)
    codes[:, :, 0::2] = wb & 15
    codes[:, :, 1::2] = wb >> 4
    return np.ascontiguousarray(codes.transpose(0, 2, 1).reshape(blocks * BLOCK, k)[:n])


# ------------------------------------------------------------------ quantizer

def quantize_affine_rtn(W, scale_dtype: str = "f16"):
    """Affine 4-bit round-to-nearest per (row, group of 64 along K).

    The BASELINE configs fix this quantizer; it follows MLX's affine RTN as the
    reference restates it (tools/quantize.py:258-264, tools/quant_study.py:146-153):
    lo = min, step = max((hi - lo)/15, tiny); scale and bias are stored in the
    16-bit dtype; the codes are computed from the *stored* values,
    q = clip(rint((W - bias)/scale), 0, 15), and q = 0 where the scale rounded to 0.

    Returns (q [N,K] uint8, s bits [N,G] uint16, b bits [N,G] uint16)."""
    W = np.asarray(W, dtype=np.float32)
    n, k = W.shape
    if k % GROUP:
        raise ValueError("K must be a multiple of 64")
    g = W.reshape(n, k // GROUP, GROUP)
    lo = g.min(axis=-1)
    hi = g.max(axis=-1)
    step = np.maximum((hi - lo) / np.float32(15), np.float32(1e-12)).astype(np.float32)
    s_bits = scale_from_f32(step, scale_dtype)
    b_bits = scale_from_f32(lo, scale_dtype)
    s = scale_to_f32(s_bits, scale_dtype)[..., None]
    b = scale_to_f32(b_bits, scale_dtype)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint((g - b) / s)
    q = np.where(s == 0, 0, np.clip(q, 0, 15))
    return q.astype(np.uint8).reshape(n, k), s_bits, b_bits


# ------------------------------------------------------------------ dequant

def dequant_affine(q, s_bits, b_bits, scale_dtype: str = "f16") -> np.ndarray:
    """W[n][k] = fp32(s[n][g]) * q[n][k] + fp32(b[n][g]), g = k // 64, in float32.

    kernels/linear.metal:3-4; src/model_file.h:42; tests/test_linear.mm:166-169. The
    product of a 16-bit float and a 4-bit integer is exact in float32, so the one
    rounding is the addition and the result is the float32 rounding of the exact value."""
    q = np.asarray(q, dtype=np.uint8)
    n, k = q.shape
    s = scale_to_f32(s_bits, scale_dtype)
    b = scale_to_f32(b_bits, scale_dtype)
    qg = q.reshape(n, k // GROUP, GROUP).astype(np.float32)
    W = qg * s[..., None] + b[..., None]
    return W.reshape(n, k).astype(np.float32)


LEVELS = {
    # tools/quantlib.py:23-28 (also tests/test_linear.mm:239-244)
    "fp4": np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float32),
    "int15": np.array([0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1], dtype=np.float32),
    "int16": np.array([.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, 7.5, -7.5, -6.5, -5.5, -4.5, -3.5, -2.5, -1.5, -.5],
                      dtype=np.float32),
}


def dequant_native(codes, s_row, c_col, book: str) -> np.ndarray:
    """W = L[q] * s[n] * c[k] (tools/quantlib.py:62-64)."""
    L = LEVELS[book]
    return (L[np.asarray(codes)] * np.asarray(s_row, np.float32)[:, None] * np.asarray(c_col, np.float32)[None, :]
            ).astype(np.float32)


# ------------------------------------------------------------------ matmul

def group_sums(x) -> np.ndarray:
    """gsum[m][g] = sum_{k<64} x[m][64g+k], accumulated in float64 here.

    kernels/linear.metal:34-45 (the reference sums sequentially in float32; the
    fp64 sum is the exact value both orders approximate)."""
    x = np.asarray(x)
    m, k = x.shape
    return x.astype(np.float64).reshape(m, k // GROUP, GROUP).sum(-1)


def linear_affine_f64(x, q, s_bits, b_bits, scale_dtype: str = "f16", cols=None) -> np.ndarray:
    """y[m][n] = sum_k x[m][k] * W[n][k] in float64 with the affine dequant of
    kernels/linear.metal:3 (the double-precision loop of tests/test_linear.mm:162-176).

    cols: optional array of output columns to evaluate (the reference test samples
    columns the same way). Returns [M, len(cols)] or [M, N]."""
    q = np.asarray(q)
    s_bits = np.asarray(s_bits)
    b_bits = np.asarray(b_bits)
    if cols is not None:
        q, s_bits, b_bits = q[cols], s_bits[cols], b_bits[cols]
    n, k = q.shape
    s = scale_to_f32(s_bits, scale_dtype).astype(np.float64)
    b = scale_to_f32(b_bits, scale_dtype).astype(np.float64)
    W = (q.reshape(n, k // GROUP, GROUP).astype(np.float64) * s[..., None] + b[..., None]).reshape(n, k)
    return np.asarray(x, dtype=np.float64) @ W.T


def linear_affine_factored_f64(x, q, s_bits, b_bits, scale_dtype: str = "f16") -> np.ndarray:
    """The same product in the form the reference kernel evaluates it
    (kernels/linear.metal:5-9,85-101): sum_g s[n][g] * (x_g . q_g) + b[n][g] * gsum[m][g]."""
    x = np.asarray(x, dtype=np.float64)
    q = np.asarray(q)
    n, k = q.shape
    G = k // GROUP
    s = scale_to_f32(s_bits, scale_dtype).astype(np.float64)
    b = scale_to_f32(b_bits, scale_dtype).astype(np.float64)
    part = np.einsum("mgk,ngk->mng", x.reshape(-1, G, GROUP), q.reshape(n, G, GROUP).astype(np.float64))
    return (part * s[None]).sum(-1) + group_sums(x) @ b.T


def linear_affine_cpu_f32(x, w_u32, s_bits, b_bits, scale_dtype: str = "f16"):
    """The reference-style CPU path (numpy dequant + float32 matmul): unpack
    (tools/convert.py:82-89), W = s*q + b per group (kernels/linear.metal:4), y = x @ W^T.

    This is the CPU baseline bench.py times; returns (y float32, W float32)."""
    q = unpack_nibbles_u32(w_u32)
    W = dequant_affine(q, s_bits, b_bits, scale_dtype)
    y = np.asarray(x, dtype=np.float32) @ W.T
    return y, W


def linear_native_f64(x, codes, s_row, book: str, c_col=None) -> np.ndarray:
    """Native 4-bit product C = s[n] * (x' . L(q)^T), x' = x * c (column scale folded upstream).

    kernels/linear.metal:118-184 (HALF_STEP for int16 is the same product with L[q] = q' + 0.5)."""
    x = np.asarray(x, dtype=np.float64)
    if c_col is not None:
        x = x * np.asarray(c_col, np.float64)[None, :]
    L = LEVELS[book].astype(np.float64)
    return (x @ L[np.asarray(codes)].T) * np.asarray(s_row, np.float64)[None, :]


# ------------------------------------------------------------------ tolerance

def rel_err(got, ref) -> float:
    """max |got - ref| / rms(ref): the error measure the parity bar (1e-3) is stated in.

    Normalising by the rms of the reference, rather than element by element, keeps the
    measure meaningful for outputs near zero; it is twice as strict as the reference
    test's own bar max|err| < 2e-3 * rms + 1e-4 (tests/test_linear.mm:178)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = float(np.sqrt(np.mean(ref * ref)))
    if rms == 0.0:
        return float(np.abs(got - ref).max(initial=0.0))
    return float(np.abs(got - ref).max(initial=0.0) / rms)


def check_close(got, ref, tol: float = 1e-3, what: str = "output"):
    """Assert the parity bar; also the reference test's own (tests/test_linear.mm:178)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    e = rel_err(got, ref)
    if not np.isfinite(got).all():
        raise AssertionError(f"{what}: non-finite values")
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    max_abs = float(np.abs(got - ref).max(initial=0.0))
    if e > tol or max_abs >= 2e-3 * rms + 1e-4:
        raise AssertionError(f"{what}: max|err|/rms = {e:.3e} (tol {tol:g}), max|err| = {max_abs:.3e}, rms = {rms:.3e}")
    return e


# ------------------------------------------------------------------ the reference test's generator

class XorShift64:
    """The generator of tests/test_linear.mm:27-39 (xorshift64, seed 0x9e3779b97f4a7c15).

    Restated so the reference's known-answer cases (shapes at :440-451) can be rebuilt
    exactly: codes = rnd() & 15, scales U(0.001, 0.012) -> bf16 RNE, bias = -7.5 s +
    U(-0.01, 0.01) -> bf16, A = fp16 U(-2, 2)."""

    MASK = (1 << 64) - 1

    def __init__(self, seed: int = 0x9E3779B97F4A7C15):
        self.state = seed & self.MASK

    def next(self) -> int:
        s = self.state
        s ^= (s << 13) & self.MASK
        s ^= s >> 7
        s ^= (s << 17) & self.MASK
        self.state = s
        return s

    def uniform(self, lo: float, hi: float) -> np.float32:
        # float(lo + (hi - lo) * (float)((rnd() >> 11) * 2^-53)), all in float32 but the product in double
        u = float(np.float32((self.next() >> 11) * (1.0 / 9007199254740992.0)))
        return np.float32(np.float32(lo) + np.float32(np.float32(hi) - np.float32(lo)) * np.float32(u))

    def codes(self, count: int) -> np.ndarray:
        return np.array([self.next() & 15 for _ in range(count)], dtype=np.uint8)

    # xorshift64 is linear over GF(2): one step is a 64x64 bit matrix T, so the state L steps
    # ahead is T^L applied to the current one. stream() computes L outputs serially, then
    # every later block of L as T^L of the previous block, with T^L applied through eight
    # byte-indexed tables (out = XOR_p table[p][byte p of the state]).
    _BLOCK = 1 << 16
    _tables = None

    @staticmethod
    def _step(s: int) -> int:
        m = XorShift64.MASK
        s ^= (s << 13) & m
        s ^= s >> 7
        s ^= (s << 17) & m
        return s

    @classmethod
    def _jump_tables(cls) -> np.ndarray:
        if cls._tables is None:
            def apply(cols, v):
                r = 0
                for i in range(64):
                    if (v >> i) & 1:
                        r ^= cols[i]
                return r
            cols = [cls._step(1 << c) for c in range(64)]                 # columns of T
            for _ in range(cls._BLOCK.bit_length() - 1):                  # T^(2^k), k -> log2(BLOCK)
                cols = [apply(cols, cols[c]) for c in range(64)]
            t = np.zeros((8, 256), dtype=np.uint64)
            for p in range(8):
                for v in range(256):
                    t[p, v] = np.uint64(apply(cols[8 * p:8 * p + 8] + [0] * 56, v))
            cls._tables = t
        return cls._tables

    def stream(self, count: int) -> np.ndarray:
        """The next `count` outputs as uint64, identical to `count` calls of next()."""
        L = self._BLOCK
        first = min(count, L)
        out = np.empty(count, dtype=np.uint64)
        for i in range(first):
            out[i] = self.next()
        if count > L:
            t = self._jump_tables()
            for b0 in range(L, count, L):
                prev = out[b0 - L:b0]
                nxt = t[0][(prev & np.uint64(0xFF)).astype(np.intp)]
                for p in range(1, 8):
                    nxt = nxt ^ t[p][((prev >> np.uint64(8 * p)) & np.uint64(0xFF)).astype(np.intp)]
                n = min(L, count - b0)
                out[b0:b0 + n] = nxt[:n]
            self.state = int(out[-1])
        return out

    @staticmethod
    def uniform_of(r: np.ndarray, lo: float, hi: float) -> np.ndarray:
        """uniform(lo, hi) of tests/test_linear.mm:39 for each output r (vectorised):
        lo + (hi - lo) * float((r >> 11) * 2^-53), the last two operations in float32."""
        u = ((np.asarray(r, dtype=np.uint64) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0))
        return np.float32(lo) + (np.float32(hi) - np.float32(lo)) * u.astype(np.float32)


def reference_test_case(M: int, K: int, N: int, gen: XorShift64 | None = None):
    """The inputs of one correctness case of tests/test_linear.mm (check(), :149-185), drawn
    as make_layer(keep_ref) (:68-89) and make_input (:141-147) draw them:
    codes rnd() & 15 row-major [N][K]; per (row, group) s = bf16(U(0.001, 0.012)) then
    b = bf16(-7.5 s + U(-0.01, 0.01)); activations fp16(U(-2, 2)) [M][K].
    Each case starts from the test's seed. (The reference's compiler may contract
    -7.5*s + u into one fused multiply-add; that can move a bias by one bf16 step, which
    does not matter here because parity is computed from the stored values.)
    Returns (q uint8 [N][K], s, b uint16 bf16 bits [N][K/64], x float16 [M][K])."""
    gen = gen or XorShift64()
    G = K // GROUP
    q = (gen.stream(N * K) & np.uint64(15)).astype(np.uint8).reshape(N, K)
    r = gen.stream(2 * N * G)
    sv = XorShift64.uniform_of(r[0::2], 0.001, 0.012)
    s = f32_to_bf16_bits(sv)
    bv = np.float32(-7.5) * sv + XorShift64.uniform_of(r[1::2], -0.01, 0.01)
    b = f32_to_bf16_bits(bv.astype(np.float32))
    x = XorShift64.uniform_of(gen.stream(M * K), -2.0, 2.0).astype(np.float16).reshape(M, K)
    return q, s.reshape(N, G), b.reshape(N, G), x


def reference_native_case(M: int, K: int, N: int, gen: XorShift64 | None = None):
    """The inputs of one native-format case of tests/test_linear.mm (check_native, :316-350),
    drawn as make_native(keep_ref) (:252-266) and make_input (:141-147) draw them: row
    scales U(0.002, 0.02) for each of the N rows, then codes rnd() & 15 row-major [N][K],
    then activations fp16(U(-2, 2)) [M][K]. Returns (codes uint8 [N][K], s float32 [N],
    x float16 [M][K])."""
    gen = gen or XorShift64()
    s = XorShift64.uniform_of(gen.stream(N), 0.002, 0.02).astype(np.float32)
    q = (gen.stream(N * K) & np.uint64(15)).astype(np.uint8).reshape(N, K)
    x = XorShift64.uniform_of(gen.stream(M * K), -2.0, 2.0).astype(np.float16).reshape(M, K)
    return q, s, x


# The native cases of tests/test_linear.mm:447-450 (each for every codebook) as (M, K, N).
REFERENCE_NATIVE_CASES = [(1, 2560, 9216), (40, 2560, 1000), (70, 9216, 2560)]

# The correctness cases of tests/test_linear.mm:440-446 as (M, K, N).
REFERENCE_TEST_CASES = [(1, 2560, 9216), (5, 2560, 9216), (40, 2560, 9216), (70, 2560, 9216),
                        (3, 9216, 2560), (2, 2560, 1000), (130, 5120, 1024)]


PINNED_BY = {
    "f32_to_bf16_bits": "torch's bfloat16 conversion (independent RNE implementation); exact cases",
    "bf16_bits_to_f32": "round trip with f32_to_bf16_bits on every bf16 pattern",
    "to_bf16_exact": "accepts widened bf16, rejects a value with low bits set",
    "unpack_nibbles_u32": "known answer 0x76543210 -> 0..7; brute-force bit extraction",
    "pack_nibbles_u32": "round trip with unpack_nibbles_u32",
    "pack_blocked": "per-element packer restated from tests/test_linear.mm:73-85; padding rows zero",
    "unpack_blocked": "round trip with pack_blocked",
    "quantize_affine_rtn": "codes in range; |W - deq| <= step/2 + rounding; constant group -> q=0",
    "dequant_affine": "equals float32 rounding of the exact float64 value; s=1,b=0 -> q",
    "group_sums": "math.fsum per group",
    "linear_affine_f64": "s=1,b=0 integer GEMM exact vs int64 arithmetic; factored form agrees",
    "linear_native_f64": "codebook identities (int15 two's complement, int16 = int15 + 0.5, fp4 e2m1 decode)",
}
