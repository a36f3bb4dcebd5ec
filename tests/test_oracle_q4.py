"""Pins the CPU oracle (oracle/q4.py) against independent statements of the reference's
formats and arithmetic: library conversions, per-element packers restated from the
reference's own test, exact integer arithmetic, and closed forms. No GPU needed."""

import math

import numpy as np
import pytest

import oracle as O


# ------------------------------------------------------------------ 16-bit float formats

def test_bf16_rne_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
                        np.array([0.0, -0.0, 1.0, -1.0, 3.0e38, 1e-40, 65504.0, np.inf, -np.inf], np.float32)])
    # values exactly half-way between two bf16 numbers exercise the tie-to-even rule
    ties = (np.arange(1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties]).astype(np.float32)
    ours = O.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)


def test_bf16_round_trip_every_pattern():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = O.bf16_bits_to_f32(bits)
    keep = ~np.isnan(f)
    np.testing.assert_array_equal(O.f32_to_bf16_bits(f[keep]), bits[keep])


def test_to_bf16_exact():
    ok = O.bf16_bits_to_f32(np.array([0x3F80, 0xBC23, 0x0001], np.uint16))
    np.testing.assert_array_equal(O.to_bf16_exact(ok), [0x3F80, 0xBC23, 0x0001])
    with pytest.raises(ValueError):
        O.to_bf16_exact(np.array([1.0000001], np.float32))


def test_f16_round_trip_every_pattern():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = O.f16_bits_to_f32(bits)
    keep = ~np.isnan(f)
    np.testing.assert_array_equal(O.f32_to_f16_bits(f[keep]), bits[keep])


# ------------------------------------------------------------------ nibble layouts

def test_unpack_nibbles_known_answer():
    w = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    np.testing.assert_array_equal(O.unpack_nibbles_u32(w), [list(range(16))])


def test_unpack_nibbles_brute_force():
    rng = np.random.default_rng(2)
    w = rng.integers(0, 1 << 32, size=(7, 5), dtype=np.uint64).astype(np.uint32)
    q = O.unpack_nibbles_u32(w)
    for n in range(7):
        for i in range(40):
            assert q[n, i] == (int(w[n, i // 8]) >> (4 * (i % 8))) & 15


def test_pack_nibbles_round_trip():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, size=(33, 128), dtype=np.uint8)
    np.testing.assert_array_equal(O.unpack_nibbles_u32(O.pack_nibbles_u32(q)), q)
    with pytest.raises(ValueError):
        O.pack_nibbles_u32(np.full((1, 8), 16, np.uint8))


def _blocked_by_element(q, s, b):
    """Per-element packer following tests/test_linear.mm:73-85 (and the bf16 s/b placement
    of :81-85): an independent statement of the blocked layout of tools/convert.py:92-117."""
    N, K = q.shape
    G = K // 64
    nb = (N + 255) // 256
    w = np.zeros(nb * K * 128, np.uint8)
    so = np.zeros(nb * G * 256, np.uint16)
    bo = np.zeros(nb * G * 256, np.uint16)
    for n in range(N):
        blk, col = n // 256, n % 256
        for k in range(K):
            byte = (blk * K + k) * 128 + col // 2
            w[byte] |= (q[n, k] << 4) if (col & 1) else q[n, k]
        for g in range(G):
            o = (blk * G + g) * 256 + col
            so[o] = s[n, g]
            bo[o] = b[n, g]
    return w, so, bo


def test_pack_blocked_matches_reference_test_packer():
    rng = np.random.default_rng(4)
    K = 128
    parts = []
    for rows in (200, 70):      # two parts, 270 rows: not a multiple of the block
        q = rng.integers(0, 16, size=(rows, K), dtype=np.uint8)
        s = rng.integers(0, 1 << 16, size=(rows, K // 64), dtype=np.uint32).astype(np.uint16)
        b = rng.integers(0, 1 << 16, size=(rows, K // 64), dtype=np.uint32).astype(np.uint16)
        parts.append((q, s, b))
    w, s, b, n_pad, offs = O.pack_blocked(parts)
    assert n_pad == 512 and offs == [(0, 200), (200, 70)]
    q_all = np.concatenate([p[0] for p in parts])
    s_all = np.concatenate([p[1] for p in parts])
    b_all = np.concatenate([p[2] for p in parts])
    w_ref, s_ref, b_ref = _blocked_by_element(q_all, s_all, b_all)
    np.testing.assert_array_equal(w.reshape(-1), w_ref)
    np.testing.assert_array_equal(s.reshape(-1), s_ref)
    np.testing.assert_array_equal(b.reshape(-1), b_ref)
    # round trip and zero padding
    q2, s2, b2 = O.unpack_blocked(w, s, b, n_pad, K)
    np.testing.assert_array_equal(q2[:270], q_all)
    assert not q2[270:].any() and not s2[270:].any() and not b2[270:].any()
    np.testing.assert_array_equal(s2[:270], s_all)
    np.testing.assert_array_equal(b2[:270], b_all)


def test_native_blocked_round_trip():
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 16, size=(300, 64), dtype=np.uint8)
    s = rng.random(300).astype(np.float32)
    w, s_pad, n_pad = O.pack_native_blocked(codes, s)
    assert n_pad == 512 and not s_pad[300:].any()
    np.testing.assert_array_equal(O.unpack_native_blocked(w, 300, 64), codes)
    zeros = np.zeros(300, np.uint16)
    w_a, _, _, _, _ = O.pack_blocked([(codes, np.zeros((300, 1), np.uint16), np.zeros((300, 1), np.uint16))])
    np.testing.assert_array_equal(w, w_a)   # both kinds share the blocked nibble layout
    del zeros


# ------------------------------------------------------------------ quantizer and dequant

@pytest.mark.parametrize("sd", ["f16", "bf16"])
def test_quantizer_invariants(sd):
    rng = np.random.default_rng(6)
    W = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    W[3, :64] = 0.25                      # constant group: step = tiny, bias = the value
    q, s, b = O.quantize_affine_rtn(W, sd)
    assert q.dtype == np.uint8 and q.max() <= 15
    deq = O.dequant_affine(q, s, b, sd)
    sf = O.scale_to_f32(s, sd)
    bf = O.scale_to_f32(b, sd)
    # within half a step of the stored grid (plus the rounding of the stored scale and bias)
    step = np.repeat(sf, 64, axis=1)
    ok = np.abs(deq - W) <= 0.5 * step + 2e-3 * np.abs(W) + np.repeat(np.abs(bf), 64, axis=1) * 2e-3 + 1e-6
    ok[3, :64] = True
    assert ok.all()
    assert (q[3, :64] == 0).all() and np.allclose(deq[3, :64], 0.25, rtol=1e-2)
    # the group minimum maps to code 0 (bias = stored lo)
    g = W.reshape(64, -1, 64)
    arg = g.argmin(-1)
    qg = q.reshape(64, -1, 64)
    assert (np.take_along_axis(qg, arg[..., None], -1) <= 1).all()


@pytest.mark.parametrize("sd", ["f16", "bf16"])
def test_dequant_is_single_rounding_of_exact_value(sd):
    rng = np.random.default_rng(7)
    q = rng.integers(0, 16, size=(40, 256), dtype=np.uint8)
    s = O.scale_from_f32(rng.uniform(1e-7, 5.0, size=(40, 4)).astype(np.float32) *
                         rng.choice([-1, 1], size=(40, 4)).astype(np.float32), sd)
    b = O.scale_from_f32(rng.standard_normal((40, 4)).astype(np.float32), sd)
    got = O.dequant_affine(q, s, b, sd)
    exact = (q.reshape(40, 4, 64).astype(np.float64) * O.scale_to_f32(s, sd).astype(np.float64)[..., None]
             + O.scale_to_f32(b, sd).astype(np.float64)[..., None]).reshape(40, 256)
    np.testing.assert_array_equal(got, exact.astype(np.float32))
    # s = 1, b = 0 gives the codes themselves
    one = O.scale_from_f32(np.ones((40, 4), np.float32), sd)
    zero = np.zeros((40, 4), np.uint16)
    np.testing.assert_array_equal(O.dequant_affine(q, one, zero, sd), q.astype(np.float32))


def test_group_sums_fsum():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 192)).astype(np.float16)
    gs = O.group_sums(x)
    for m in range(3):
        for g in range(3):
            assert gs[m, g] == math.fsum(float(v) for v in x[m, 64 * g:64 * g + 64])


# ------------------------------------------------------------------ matmul

def test_linear_integer_case_is_exact():
    """s = 1, b = 0 and small-integer activations: the product is an integer GEMM."""
    rng = np.random.default_rng(9)
    q = rng.integers(0, 16, size=(37, 192), dtype=np.uint8)
    x = rng.integers(-8, 9, size=(5, 192)).astype(np.float16)
    s = O.f32_to_f16_bits(np.ones((37, 3), np.float32))
    b = np.zeros((37, 3), np.uint16)
    y = O.linear_affine_f64(x, q, s, b)
    ref = x.astype(np.int64) @ q.astype(np.int64).T
    np.testing.assert_array_equal(y, ref.astype(np.float64))


@pytest.mark.parametrize("sd", ["f16", "bf16"])
def test_linear_factored_form_agrees(sd):
    rng = np.random.default_rng(10)
    W = (rng.standard_normal((96, 320)) * 0.02).astype(np.float32)
    q, s, b = O.quantize_affine_rtn(W, sd)
    x = rng.standard_normal((4, 320)).astype(np.float16)
    y1 = O.linear_affine_f64(x, q, s, b, sd)
    y2 = O.linear_affine_factored_f64(x, q, s, b, sd)
    np.testing.assert_allclose(y1, y2, rtol=1e-12, atol=1e-12)
    cols = np.array([0, 5, 95])
    np.testing.assert_allclose(O.linear_affine_f64(x, q, s, b, sd, cols=cols), y1[:, cols], rtol=0, atol=0)
    # the reference-style CPU path (numpy dequant + fp32 matmul) is within the parity bar
    y3, _ = O.linear_affine_cpu_f32(x, O.pack_nibbles_u32(q), s, b, sd)
    assert O.rel_err(y3, y1) < 1e-5


def test_linear_sign_and_index_mistakes_are_caught():
    """A plausible slip (biases of the wrong group, swapped nibble order) breaks the check."""
    rng = np.random.default_rng(11)
    W = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    q, s, b = O.quantize_affine_rtn(W)
    x = rng.standard_normal((2, 256)).astype(np.float16)
    y = O.linear_affine_f64(x, q, s, b)
    b_shift = np.roll(b, 1, axis=1)
    assert O.rel_err(O.linear_affine_f64(x, q, s, b_shift), y) > 1e-2
    q_swap = q.copy()
    q_swap[:, 0::2], q_swap[:, 1::2] = q[:, 1::2], q[:, 0::2]
    assert O.rel_err(O.linear_affine_f64(x, q_swap, s, b), y) > 1e-2
    with pytest.raises(AssertionError):
        O.check_close(O.linear_affine_f64(x, q_swap, s, b), y)


def test_native_codebooks():
    L = O.LEVELS
    codes = np.arange(16)
    twos = np.where(codes < 8, codes, codes - 16)
    np.testing.assert_array_equal(L["int15"], twos)            # two's-complement nibble
    np.testing.assert_array_equal(L["int16"], twos + 0.5)      # plus one half
    # fp4 e2m1: sign bit 3, exponent bits 2..1, mantissa bit 0
    s_, e_, m_ = codes >> 3, (codes >> 1) & 3, codes & 1
    mag = np.where(e_ == 0, 0.5 * m_, 2.0 ** (e_ - 1) * (1 + 0.5 * m_))
    np.testing.assert_array_equal(np.abs(L["fp4"]), mag)
    assert (np.signbit(L["fp4"]) == (s_ == 1)).all()
    rng = np.random.default_rng(12)
    c = rng.integers(0, 16, size=(8, 64))
    x = rng.standard_normal((3, 64)).astype(np.float16)
    sr = rng.random(8).astype(np.float32)
    y = O.linear_native_f64(x, c, sr, "int16")
    np.testing.assert_allclose(y, (x.astype(np.float64) @ (twos[c] + 0.5).T) * sr, rtol=1e-12)


def test_xorshift_generator_properties():
    g = O.XorShift64()
    vals = [g.next() for _ in range(1000)]
    assert len(set(vals)) == 1000 and all(0 < v < (1 << 64) for v in vals)
    u = [float(g.uniform(0.001, 0.012)) for _ in range(1000)]
    assert min(u) >= 0.001 and max(u) < 0.012


def test_xorshift_stream_equals_serial_steps():
    """The block-jump stream (T^L by byte tables) against plain serial xorshift64 steps,
    across several block boundaries; the state continues identically afterwards."""
    a, b = O.XorShift64(), O.XorShift64()
    fast = a.stream(3 * a._BLOCK + 123)
    slow = np.array([b.next() for _ in range(len(fast))], dtype=np.uint64)
    np.testing.assert_array_equal(fast, slow)
    assert a.state == b.state and a.next() == b.next()
    # vectorised uniform == the scalar one on the same outputs
    c, d = O.XorShift64(7), O.XorShift64(7)
    r = c.stream(64)
    assert [float(v) for v in O.XorShift64.uniform_of(r, -2.0, 2.0)] == [float(d.uniform(-2.0, 2.0)) for _ in range(64)]


def test_reference_test_case_draws():
    """Inputs of the reference's correctness cases have the distribution its test states
    (tests/test_linear.mm:80-88,145): codes 0..15, s in [0.001, 0.012), b = -7.5 s +
    U(-0.01, 0.01), x = fp16 U(-2, 2); the first codes are the generator's first outputs."""
    q, s, b, x = O.reference_test_case(3, 256, 512)
    g = O.XorShift64()
    assert [int(v) for v in q[0, :16]] == [g.next() & 15 for _ in range(16)]
    sf, bf = O.bf16_bits_to_f32(s), O.bf16_bits_to_f32(b)
    assert q.max() <= 15 and sf.min() >= 0.00099 and sf.max() <= 0.012 + 2.0 ** -14   # one bf16 step
    assert np.all(np.abs(bf + 7.5 * sf) <= 0.0101 + 0.01 * np.abs(bf))
    assert x.dtype == np.float16 and np.abs(x).max() <= 2.0 and x.shape == (3, 256)


def test_reference_native_case_draws():
    """Native cases draw the row scales first (tests/test_linear.mm:260), then the codes."""
    q, s, x = O.reference_native_case(2, 128, 40)
    g = O.XorShift64()
    first_s = [float(g.uniform(0.002, 0.02)) for _ in range(40)]
    assert [float(v) for v in s] == first_s
    assert [int(v) for v in q[0, :8]] == [g.next() & 15 for _ in range(8)]
    assert x.shape == (2, 128) and s.min() >= 0.002 and s.max() < 0.02
