"""Pins the MoE oracle (oracle/moe.py) with special cases and permutation invariants."""

import numpy as np

import oracle as O


def test_route_equal_logits_picks_lowest_experts():
    E, K = 32, 4
    logits = np.zeros((2, E + 1), np.float32)
    sel, w = O.moe_route(logits, E, K, norm_topk=True)
    S = K + 1
    np.testing.assert_array_equal(sel[:K], np.arange(K))
    np.testing.assert_allclose(w[:K], 1.0 / K)
    assert sel[K] == E and abs(w[K] - 0.5) < 1e-15           # sigmoid(0)
    _, w2 = O.moe_route(logits, E, K, norm_topk=False)
    np.testing.assert_allclose(w2[:K], 1.0 / E)                # softmax over all experts
    assert sel.shape == (2 * S,)


def test_route_matches_brute_force_argmax():
    rng = np.random.default_rng(20)
    E, K, T = 256, 8, 40
    logits = rng.standard_normal((T, E + 1)).astype(np.float32)
    logits[0, 7] = logits[0, 3] = logits[0].max() + 1.0      # a tie: the lower expert first
    sel, w = O.moe_route(logits, E, K)
    S = K + 1
    for t in range(T):
        v = list(logits[t, :E])
        picked = []
        for _ in range(K):   # repeated argmax, ties to the lower index (kernels/moe.metal:75-91)
            best = max(range(E), key=lambda e: (v[e], -e))
            picked.append(best)
            v[best] = -np.inf
        assert list(sel[t * S:t * S + K]) == picked
        ex = np.exp(logits[t, picked].astype(np.float64) - logits[t, :E].max())
        np.testing.assert_allclose(w[t * S:t * S + K], ex / ex.sum(), rtol=1e-12)
        assert abs(w[t * S:t * S + K].sum() - 1.0) < 1e-12
    assert list(sel[0:2]) == [3, 7]


def test_items_cover_every_row_once():
    rng = np.random.default_rng(21)
    E, K, T, TM = 64, 8, 100, 16
    sel, _ = O.moe_route(rng.standard_normal((T, E + 1)).astype(np.float32), E, K)
    counts, off, items = O.moe_items(sel, E, TM)
    assert counts.sum() == T * (K + 1) and counts[E] == T
    covered = np.zeros(T * (K + 1), int)
    for e, r0, rows, _ in items:
        assert 1 <= rows <= TM and off[e] <= r0 and r0 + rows <= off[e + 1]
        covered[r0:r0 + rows] += 1
    assert (covered == 1).all()
    assert len(items) <= T * (K + 1) // TM + E + 1


def test_swiglu_half():
    gu = np.array([[0.0, 1.0, 2.0, 3.0], [-1.0, 0.5, 10.0, -2.0]])
    a = O.swiglu_f16(gu, 2)
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    ref = np.array([[silu(0.0) * 2.0, silu(1.0) * 3.0], [silu(-1.0) * 10.0, silu(0.5) * -2.0]])
    np.testing.assert_array_equal(a, ref.astype(np.float16))


def test_moe_layer_linearity_in_h0_and_weights():
    rng = np.random.default_rng(22)
    E, K, I, H, T = 8, 2, 64, 128, 3
    Wg = (rng.standard_normal(((E + 1) * 2 * I, H)) * 0.02).astype(np.float32)
    Wd = (rng.standard_normal(((E + 1) * H, I)) * 0.02).astype(np.float32)
    gu = O.quantize_affine_rtn(Wg)
    dn = O.quantize_affine_rtn(Wd)
    x = rng.standard_normal((T, H)).astype(np.float16)
    logits = rng.standard_normal((T, E + 1)).astype(np.float32)
    h, sel, w = O.moe_layer_f64(x, logits, gu, dn, E, K, I, H)
    h0 = rng.standard_normal((T, H))
    h2, _, _ = O.moe_layer_f64(x, logits, gu, dn, E, K, I, H, h0=h0)
    np.testing.assert_allclose(h2 - h0, h, rtol=1e-12, atol=1e-12)
    # the layer is the weighted sum of the expert outputs: rebuild one token directly
    S = K + 1
    t = 1
    acc = np.zeros(H)
    for s in range(S):
        e = sel[t * S + s]
        Wge = O.dequant_affine(*gu)[e * 2 * I:(e + 1) * 2 * I].astype(np.float64)
        Wde = O.dequant_affine(*dn)[e * H:(e + 1) * H].astype(np.float64)
        g = x[t].astype(np.float64) @ Wge.T
        a = (g[:I] / (1 + np.exp(-g[:I])) * g[I:]).astype(np.float16).astype(np.float64)
        acc += w[t * S + s] * (a @ Wde.T)
    np.testing.assert_allclose(h[t], acc, rtol=1e-9, atol=1e-12)


def test_given_activations_replace_the_swiglu():
    """acts: the layer's own half activations (in token, slot order) give its result bit for
    bit, and a changed activation moves h by exactly w * (delta a) . W_down of that slot."""
    rng = np.random.default_rng(24)
    E, K, I, H, T = 8, 2, 64, 128, 2
    gu = O.quantize_affine_rtn((rng.standard_normal(((E + 1) * 2 * I, H)) * 0.02).astype(np.float32))
    dn = O.quantize_affine_rtn((rng.standard_normal(((E + 1) * H, I)) * 0.02).astype(np.float32))
    x = rng.standard_normal((T, H)).astype(np.float16)
    logits = rng.standard_normal((T, E + 1)).astype(np.float32)
    h, sel, w = O.moe_layer_f64(x, logits, gu, dn, E, K, I, H)
    S = K + 1
    acts = np.zeros((T * S, I), np.float16)
    for a in range(T * S):
        e = int(sel[a])
        Wge = O.dequant_affine(*gu)[e * 2 * I:(e + 1) * 2 * I].astype(np.float64)
        acts[a] = O.swiglu_f16(x[a // S:a // S + 1].astype(np.float64) @ Wge.T, I)[0]
    h2, _, _ = O.moe_layer_f64(x, logits, gu, dn, E, K, I, H, acts=acts)
    np.testing.assert_array_equal(h2, h)
    bumped = acts.copy()
    bumped[S + 1, 5] = np.float16(float(bumped[S + 1, 5]) + 0.25)
    h3, _, _ = O.moe_layer_f64(x, logits, gu, dn, E, K, I, H, acts=bumped)
    e = int(sel[S + 1])
    Wde = O.dequant_affine(*dn)[e * H:(e + 1) * H].astype(np.float64)
    delta = float(bumped[S + 1, 5]) - float(acts[S + 1, 5])
    np.testing.assert_allclose(h3[1] - h[1], w[S + 1] * delta * Wde[:, 5], rtol=1e-9, atol=1e-15)
    np.testing.assert_array_equal(h3[0], h[0])


def _native_stack(rng, n_slots, Ne, K):
    codes = rng.integers(0, 16, size=(n_slots * Ne, K), dtype=np.uint8)
    s_row = rng.uniform(0.01, 0.03, size=n_slots * Ne).astype(np.float32)
    return codes, s_row


def test_native_expert_product_follows_the_slot_table():
    """Moving the experts to other slots and the table with them leaves every product
    unchanged (a kernel that indexed by expert instead of slot would not); with the
    identity table an item's rows are the plain native product of its expert's rows."""
    rng = np.random.default_rng(3)
    E, Ne, K, T, topk = 6, 32, 128, 5, 2
    codes, s_row = _native_stack(rng, E + 1, Ne, K)
    x = rng.standard_normal((T, K)).astype(np.float16)
    sel, _ = O.moe_route(rng.standard_normal((T, E + 1)).astype(np.float32), E, topk)
    _, off, items = O.moe_items(sel, E, 16)
    S = topk + 1
    # the sorted rows' tokens: rows of an expert in token order
    tok = np.zeros(T * S, dtype=np.int64)
    for e in range(E + 1):
        tok[off[e]:off[e + 1]] = np.flatnonzero(sel == e) // S
    ident = np.arange(E + 1)
    C = O.moe_linear_native_f64(x, items, len(items), ident, codes, s_row, Ne, "int15", tok=tok, n_rows=T * S)
    for e, r0, rows, _ in items:
        ref = O.linear_native_f64(x[tok[r0:r0 + rows]], codes[e * Ne:(e + 1) * Ne], s_row[e * Ne:(e + 1) * Ne], "int15")
        np.testing.assert_allclose(C[r0:r0 + rows], ref, rtol=1e-12, atol=1e-12)
    perm = rng.permutation(E + 3)[:E + 1]          # slots in a larger cache, some left empty
    codes2 = np.zeros(((E + 3) * Ne, K), dtype=np.uint8)
    s2 = np.zeros((E + 3) * Ne, dtype=np.float32)
    for e in range(E + 1):
        codes2[perm[e] * Ne:(perm[e] + 1) * Ne] = codes[e * Ne:(e + 1) * Ne]
        s2[perm[e] * Ne:(perm[e] + 1) * Ne] = s_row[e * Ne:(e + 1) * Ne]
    C2 = O.moe_linear_native_f64(x, items, len(items), perm, codes2, s2, Ne, "int15", tok=tok, n_rows=T * S)
    np.testing.assert_array_equal(C2, C)


def test_native_layer_token_loop_equals_sorted_pipeline():
    """The token-by-token native layer equals the reference's sorted pipeline (route,
    items, gathered gate_up product, SwiGLU with the column scale, down product over
    sorted rows, combine in slot order), both in float64 with act stored as half."""
    rng = np.random.default_rng(4)
    E, H, I, T, topk = 5, 64, 64, 7, 2
    S = topk + 1
    gq, gs = _native_stack(rng, E + 1, 2 * I, H)
    dq, ds = _native_stack(rng, E + 1, H, I)
    cs = rng.uniform(0.5, 1.5, size=I).astype(np.float32)
    slots = np.arange(E + 1)[::-1].copy()          # expert e stored in slot E - e
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
    logits = rng.standard_normal((T, E + 1)).astype(np.float32)
    h, sel, w = O.moe_layer_native_f64(x, logits, (gq, gs), (dq, ds), cs, slots, E, topk, I, H, "fp4")
    _, off, items = O.moe_items(sel, E, 16)
    tok = np.zeros(T * S, dtype=np.int64)
    inv = np.zeros(T * S, dtype=np.int64)
    for e in range(E + 1):
        a_e = np.flatnonzero(sel == e)
        tok[off[e]:off[e + 1]] = a_e // S
        inv[a_e] = np.arange(off[e], off[e + 1])
    gu = O.moe_linear_native_f64(x, items, len(items), slots, gq, gs, 2 * I, "fp4", tok=tok, n_rows=T * S)
    act = O.swiglu_f16(gu, I, cs)
    y = O.moe_linear_native_f64(act, items, len(items), slots, dq, ds, H, "fp4", n_rows=T * S)
    h2 = np.zeros((T, H))
    for t in range(T):
        for j in range(S):
            h2[t] += w[t * S + j] * y[inv[t * S + j]]
    np.testing.assert_allclose(h2, h, rtol=1e-9, atol=1e-12)
