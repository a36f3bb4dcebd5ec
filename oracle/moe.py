"""Oracle for the mixture-of-experts part of the path: routing, gather, SwiGLU, combine.

TEST INFRASTRUCTURE ONLY (see oracle/q4.py). Restated from kernels/moe.metal and
kernels/ops.metal:446-455 of the reference. The grouped expert matmuls come in two
forms: the affine product of oracle/q4.py, which is what the BASELINE MoE config asks
for, and the native q4n product with the slot table of linear_q4n_moe
(kernels/linear.metal:254-308; the reference's own MoE files are native).
"""

from __future__ import annotations

import numpy as np

from .q4 import GROUP, LEVELS, linear_affine_f64, linear_native_f64, scale_to_f32

__all__ = ["moe_route", "moe_items", "silu", "swiglu_f16", "moe_layer_f64", "expert_rows",
           "moe_linear_native_f64", "moe_layer_native_f64"]


def moe_route(logits, E: int, topk: int, norm_topk: bool = True):
    """Top-k routing per token (kernels/moe.metal:40-106).

    logits: [T][>= E+1] float32; column E is the shared expert's gate logit.
    Slots 0..topk-1 hold the chosen experts in falling order of logit (equal
    logits: the lower expert first, :75-91); weights are exp(l - max) over the
    softmax denominator of all E logits, or renormalised over the chosen ones when
    norm_topk (:92-102). Slot topk is the shared expert (number E) with weight
    sigmoid(logit[E]) (:103-104).

    One deliberate difference: when a row has fewer than topk finite logits, the reference's
    rounds go on picking the lowest-numbered expert whose value is -inf (:75-91), which can
    be an expert already chosen (chosen ones are set to -inf), so it repeats experts. This
    restatement, like the HIP kernels, takes distinct experts (the remaining ones in index
    order): the sort's per-token ranking needs distinct experts. The weights of those slots
    are exp(-inf) = 0 in both, so h is the same; sel, tok and items differ.

    Returns (sel [T*S] int, w [T*S] float64), S = topk + 1, in (token, slot) order."""
    L = np.asarray(logits, dtype=np.float32)
    T = L.shape[0]
    S = topk + 1
    sel = np.empty(T * S, dtype=np.int64)
    w = np.empty(T * S, dtype=np.float64)
    for t in range(T):
        v = L[t, :E].astype(np.float64)
        m = v.max()
        z = np.exp(v - m).sum()
        # stable sort on (-logit): equal logits keep the lower index first
        order = np.argsort(-L[t, :E], kind="stable")[:topk]
        ex = np.exp(v[order] - m)
        denom = ex.sum() if norm_topk else z
        sel[t * S:t * S + topk] = order
        w[t * S:t * S + topk] = ex / denom
        sel[t * S + topk] = E
        w[t * S + topk] = 1.0 / (1.0 + np.exp(-np.float64(L[t, E])))
    return sel, w


def moe_items(sel, E: int, TM: int):
    """Counting sort of the assignments by expert and the grouped matmuls' work list
    (kernels/moe.metal:109-139).

    Returns (counts [E+1], offsets [E+2], items [n_items][4] = (expert, first sorted
    row, rows <= TM, 0)). Rows inside an expert's range may come in any order (the
    reference places them with atomics, :133-139); a valid placement is any tok/inv
    pair consistent with these offsets."""
    sel = np.asarray(sel)
    counts = np.bincount(sel, minlength=E + 1)[:E + 1]
    off = np.zeros(E + 2, dtype=np.int64)
    off[1:] = np.cumsum(counts)
    items = []
    for e in range(E + 1):
        c = int(counts[e])
        for r in range(0, c, TM):
            items.append((e, int(off[e]) + r, min(TM, c - r), 0))
    return counts, off, np.array(items, dtype=np.int64).reshape(-1, 4)


def silu(v):
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def swiglu_f16(gu, I: int, cs=None):
    """act[r][i] = half(silu(gu[r][i]) * gu[r][I + i] * cs[i]) (kernels/ops.metal:446-455).

    cs is the down projection's column scale; affine (q4a) matrices bind ones
    (src/engine.mm:937-940)."""
    gu = np.asarray(gu, dtype=np.float64)
    a = silu(gu[:, :I]) * gu[:, I:2 * I]
    if cs is not None:
        a = a * np.asarray(cs, np.float64)[None, :]
    return a.astype(np.float16)


def expert_rows(e: int, rows_per_expert: int):
    """Rows of expert e in a stacked tensor (tools/quantize.py:168-228: gate_up holds
    expert e's gate rows then its up rows at [e*2I, (e+1)*2I); down holds [e*H, (e+1)*H))."""
    return slice(e * rows_per_expert, (e + 1) * rows_per_expert)


def moe_layer_f64(x, logits, gu, dn, E: int, topk: int, I: int, H: int, norm_topk: bool = True,
                  scale_dtype: str = "f16", h0=None, act_f16: bool = True, acts=None):
    """The whole MoE MLP of src/engine.mm:965-1059 on the CPU, float64 throughout
    except the SwiGLU output, which the reference stores as half (ops.metal:454).

    x: [T][H] fp16 (the normed rows); logits [T][E+1] float32;
    gu = (q [(E+1)*2I][H], s, b), dn = (q [(E+1)*H][I], s, b) with 16-bit scale bits.
    acts: optional fp16 activations [T*S][I] in (token, slot) order used in place of the
    SwiGLU of the gate/up product (a test passes the kernel's own, so that the check of the
    down product and the combine does not depend on where a half rounds).
    Returns (h [T][H] float64 = h0 + sum over slots of w * expert(x), sel, w)."""
    x = np.asarray(x)
    T = x.shape[0]
    S = topk + 1
    sel, w = moe_route(logits, E, topk, norm_topk)
    h = np.zeros((T, H), dtype=np.float64) if h0 is None else np.asarray(h0, np.float64).copy()
    qg, sg, bg = gu
    qd, sd, bd = dn
    for t in range(T):
        for s in range(S):
            e = int(sel[t * S + s])
            rg = expert_rows(e, 2 * I)
            rd = expert_rows(e, H)
            if acts is not None:
                a = np.asarray(acts[t * S + s:t * S + s + 1], np.float16)
            else:
                g = linear_affine_f64(x[t:t + 1].astype(np.float64), qg[rg], sg[rg], bg[rg], scale_dtype)
                a = swiglu_f16(g, I) if act_f16 else (silu(g[:, :I]) * g[:, I:])
            y = linear_affine_f64(np.asarray(a, np.float64), qd[rd], sd[rd], bd[rd], scale_dtype)
            h[t] += w[t * S + s] * y[0]
    return h, sel, w


# ------------------------------------------------------------------ native experts

def moe_linear_native_f64(a, items, n_items: int, slots, codes, s_row, Ne: int, book: str, tok=None, n_rows=None):
    """linear_q4n_moe (kernels/linear.metal:254-308) in float64: for work item i < n_items,
    (e, r0, rows) = items[i], slot = slots[e],

        C[r0+j][n] = s[slot*Ne + n] * (A[src(r0+j)] . L(q[slot*Ne + n])^T),  j < rows, n < Ne,

    src(r) = tok[r] when tok is given (the gather of moe.metal:143-155, a holds the tokens),
    else r. codes [n_slots*Ne][K] (0..15), s_row [n_slots*Ne]. Rows no item covers stay 0;
    a slot outside [0, n_slots) gives zero rows. Returns C [n_rows][Ne] float64."""
    a = np.asarray(a, dtype=np.float64)
    codes = np.asarray(codes)
    s_row = np.asarray(s_row, np.float64)
    n_slots = codes.shape[0] // Ne
    L = LEVELS[book].astype(np.float64)
    if n_rows is None:
        n_rows = int(max((int(it[1]) + int(it[2]) for it in np.asarray(items)[:n_items]), default=0))
    C = np.zeros((n_rows, Ne), dtype=np.float64)
    for e, r0, rows, _ in np.asarray(items)[:n_items]:
        slot = int(slots[int(e)])
        if not 0 <= slot < n_slots:
            continue
        W = L[codes[slot * Ne:(slot + 1) * Ne]]                     # [Ne][K]
        src = [int(tok[r]) if tok is not None else r for r in range(int(r0), int(r0) + int(rows))]
        C[int(r0):int(r0) + int(rows)] = (a[src] @ W.T) * s_row[slot * Ne:(slot + 1) * Ne][None, :]
    return C


def moe_layer_native_f64(x, logits, gu, dn, cs, slots, E: int, topk: int, I: int, H: int, book: str,
                         norm_topk: bool = True, h0=None, acts=None):
    """The native MoE MLP of src/engine.mm:965-1059 (route, gather, linear_q4n_moe,
    swiglu with the down matrix's column scale, linear_q4n_moe, combine), token by token
    in float64 except the SwiGLU output, stored as half (ops.metal:454).

    x: [T][H] fp16 (already times gate_up's column scale, as the reference folds it);
    gu = (codes [n_slots*2I][H], s [n_slots*2I]): gate rows then up rows per slot;
    dn = (codes [n_slots*H][I], s [n_slots*H]); cs [I] or None; slots [E+1]; acts as in
    moe_layer_f64. Returns (h [T][H] float64, sel, w)."""
    x = np.asarray(x)
    T = x.shape[0]
    S = topk + 1
    sel, w = moe_route(logits, E, topk, norm_topk)
    h = np.zeros((T, H), dtype=np.float64) if h0 is None else np.asarray(h0, np.float64).copy()
    (qg, sg), (qd, sd) = gu, dn
    for t in range(T):
        for j in range(S):
            slot = int(slots[int(sel[t * S + j])])
            if acts is not None:
                a = np.asarray(acts[t * S + j:t * S + j + 1], np.float16)
            else:
                g = linear_native_f64(x[t:t + 1], qg[expert_rows(slot, 2 * I)], sg[expert_rows(slot, 2 * I)], book)
                a = swiglu_f16(g, I, cs)
            y = linear_native_f64(a, qd[expert_rows(slot, H)], sd[expert_rows(slot, H)], book)
            h[t] += w[t * S + j] * y[0]
    return h, sel, w
