"""Parity of the native-format expert path (linear_q4n_moe, kernels/linear.metal:254-308,
with the SwiGLU of kernels/ops.metal:446-455 between the two products) with the oracle
(oracle/moe.py: moe_linear_native_f64, moe_layer_native_f64).

- One kind of experts: every covered row against the float64 product, max|err|/rms <= 1e-3,
  with the experts stored in a larger slot table in shuffled order.
- The whole native MoE MLP against the float64 layer, max|err|/rms <= 1e-3 (act rounded to
  half as the reference stores it), and a token's result bit-identical whatever other
  tokens share the call (kernels/moe.metal:9-12).
"""

import numpy as np
import pytest

import oracle as O
from tests.qdata import to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _sync():
    import torch

    torch.cuda.synchronize()


def make_stack(rng, n_slots, Ne, K, book):
    codes = rng.integers(0, 16, size=(n_slots * Ne, K), dtype=np.uint8)
    top = 6.0 if book == "fp4" else 8.0
    s_row = (rng.uniform(0.5, 1.5, size=n_slots * Ne) * 0.02 / top).astype(np.float32)
    return codes, s_row


def upload_stack(codes, s_row, Ne, book, dev):
    from raceline_amd import ops

    return ops.pack_moe_native(to_dev(O.pack_nibbles_u32(codes).view(np.int32), dev), to_dev(s_row, dev), Ne, book)


def shuffled_slots(rng, E, extra):
    """Experts 0..E stored at distinct slots of an (E + 1 + extra)-slot cache."""
    return rng.permutation(E + 1 + extra)[:E + 1].astype(np.int32)


def place(codes, s_row, slots, Ne, n_slots):
    """The stack with expert e moved to slot slots[e] (other slots hold noise)."""
    rng = np.random.default_rng(99)
    c2 = rng.integers(0, 16, size=(n_slots * Ne, codes.shape[1]), dtype=np.uint8)
    s2 = rng.uniform(0.001, 0.002, size=n_slots * Ne).astype(np.float32)
    for e, sl in enumerate(slots):
        c2[sl * Ne:(sl + 1) * Ne] = codes[e * Ne:(e + 1) * Ne]
        s2[sl * Ne:(sl + 1) * Ne] = s_row[e * Ne:(e + 1) * Ne]
    return c2, s2


@pytest.mark.parametrize("book", ["int15", "fp4"])
@pytest.mark.parametrize("gather,K,Ne,T", [(True, 512, 256, 11), (False, 256, 512, 11), (True, 4096, 64, 11),
                                          (False, 9216, 48, 11), (False, 512, 256, 20), (False, 2048, 64, 20)])
def test_native_expert_linear(gpu, book, gather, K, Ne, T):
    """(the last two: sorted rows in bulk, the staged kernel; K = 2048 sums in sub-parts)"""
    from raceline_amd import ops

    rng = np.random.default_rng(K + Ne + T + (7 if gather else 0))
    E, topk = 16, 4
    S = topk + 1
    codes, s_row = make_stack(rng, E + 1, Ne, K, book)
    slots = shuffled_slots(rng, E, 3)
    c2, s2 = place(codes, s_row, slots, Ne, E + 4)
    st = upload_stack(c2, s2, Ne, book, gpu)
    logits = rng.standard_normal((T, E + 1), dtype=np.float32)
    r = ops.moe_route(to_dev(logits, gpu), E, topk)
    a = rng.standard_normal((T if gather else T * S, K)).astype(np.float16)
    c = ops.moe_linear_native(to_dev(a, gpu), st, to_dev(slots, gpu), r, gather)
    _sync()
    n = int(r.n_items.cpu()[0])
    items = r.items.cpu().numpy()
    ref = O.moe_linear_native_f64(a, items, n, slots, c2, s2, Ne, book,
                                  tok=r.tok.cpu().numpy() if gather else None, n_rows=T * S)
    O.check_close(c.cpu().numpy().astype(np.float64), ref, TOL, f"native experts {book} K={K} Ne={Ne}")


def test_native_slot_outside_the_table_gives_zero_rows(gpu):
    from raceline_amd import ops

    rng = np.random.default_rng(5)
    E, T, topk, K, Ne = 8, 6, 2, 256, 64
    codes, s_row = make_stack(rng, E + 1, Ne, K, "int15")
    st = upload_stack(codes, s_row, Ne, "int15", gpu)
    slots = np.arange(E + 1, dtype=np.int32)
    slots[E] = E + 1          # the shared expert points past the table
    slots[2] = -1
    logits = rng.standard_normal((T, E + 1), dtype=np.float32)
    r = ops.moe_route(to_dev(logits, gpu), E, topk)
    a = rng.standard_normal((T, K)).astype(np.float16)
    c = ops.moe_linear_native(to_dev(a, gpu), st, to_dev(slots, gpu), r, True)
    _sync()
    sel = r.sel.cpu().numpy()
    inv = r.inv.cpu().numpy()
    got = c.cpu().numpy()
    for asg in range(T * (topk + 1)):
        if sel[asg] in (2, E):
            assert not got[inv[asg]].any()
        else:
            assert np.abs(got[inv[asg]]).max() > 0


def test_native_int16_is_refused(gpu):
    from raceline_amd import lib, ops

    rng = np.random.default_rng(6)
    codes, s_row = make_stack(rng, 3, 32, 128, "int15")
    st = upload_stack(codes, s_row, 32, "int16", gpu)
    r = ops.moe_route(to_dev(rng.standard_normal((2, 3), dtype=np.float32), gpu), 2, 1)
    with pytest.raises(lib.RlqError, match="half step"):
        ops.moe_linear_native(to_dev(rng.standard_normal((2, 128)).astype(np.float16), gpu), st,
                              to_dev(np.arange(3, dtype=np.int32), gpu), r, True)


@pytest.mark.parametrize("book", ["int15", "fp4"])
@pytest.mark.parametrize("T,E,topk,H,I", [(1, 16, 4, 256, 128), (6, 64, 8, 512, 256), (40, 32, 4, 256, 512),
                                           (20, 16, 4, 256, 2048)])
def test_native_layer_matches_oracle(gpu, book, T, E, topk, H, I):
    """(T = 20 and 40: the down product of the batch runs on the staged kernel, the token
    alone on the per-tile or the down + combine kernel: the bits must agree)"""
    import torch

    from raceline_amd import ops

    rng = np.random.default_rng(T * 13 + E + H)
    gq, gs = make_stack(rng, E + 1, 2 * I, H, book)
    dq, ds = make_stack(rng, E + 1, H, I, book)
    slots = shuffled_slots(rng, E, 2)
    gq2, gs2 = place(gq, gs, slots, 2 * I, E + 3)
    dq2, ds2 = place(dq, ds, slots, H, E + 3)
    gu = upload_stack(gq2, gs2, 2 * I, book, gpu)
    dn = upload_stack(dq2, ds2, H, book, gpu)
    cs = rng.uniform(0.5, 1.5, size=I).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float16)
    logits = rng.standard_normal((T, E + 1), dtype=np.float32)
    h0 = rng.standard_normal((T, H)).astype(np.float32)
    h = to_dev(h0, gpu)
    sl = to_dev(slots, gpu)
    ops.moe_native(to_dev(x, gpu), to_dev(logits, gpu), gu, dn, sl, topk, h, cs=to_dev(cs, gpu))
    _sync()
    ref, _, _ = O.moe_layer_native_f64(x, logits, (gq2, gs2), (dq2, ds2), cs, slots, E, topk, I, H, book)
    O.check_close(h.cpu().numpy().astype(np.float64) - h0, ref, TOL, f"native MoE layer {book} T={T} E={E}")
    # a token alone gives the bits it gets inside the batch
    h1 = to_dev(h0[:1], gpu)
    ops.moe_native(to_dev(x[:1], gpu), to_dev(logits[:1], gpu), gu, dn, sl, topk, h1, cs=to_dev(cs, gpu))
    _sync()
    assert torch.equal(h1, h[:1])


@pytest.mark.parametrize("book", ["int15", "fp4"])
@pytest.mark.parametrize("H,I,T,bad", [(512, 256, 9, False), (4096, 64, 9, False), (2048, 128, 12, False),
                                       (512, 256, 3, False), (1024, 192, 10, True), (512, 128, 2, True)])
def test_native_gate_up_fused_equals_two_launches(gpu, book, H, I, T, bad):
    """rlq_moe_gate_up_native gives the bits of the gate/up product followed by the SwiGLU,
    with and without a column scale, at 8 and 16 groups per wave and ragged I. bad: two
    experts' slots point outside the table (zero rows before the SwiGLU)."""
    import torch

    from raceline_amd import ops

    rng = np.random.default_rng(H + I + T)
    E, topk = 16, 4
    codes, s_row = make_stack(rng, E + 1, 2 * I, H, book)
    slots = shuffled_slots(rng, E, 1)
    c2, s2 = place(codes, s_row, slots, 2 * I, E + 2)
    if bad:
        slots[3], slots[E] = -1, E + 2
    st = upload_stack(c2, s2, 2 * I, book, gpu)
    r = ops.moe_route(to_dev(rng.standard_normal((T, E + 1), dtype=np.float32), gpu), E, topk)
    x = to_dev(rng.standard_normal((T, H)).astype(np.float16), gpu)
    sl = to_dev(slots, gpu)
    for cs in (None, to_dev(rng.uniform(0.5, 1.5, size=I).astype(np.float32), gpu)):
        fused = ops.moe_gate_up_native(x, st, sl, r, cs)
        two = ops.moe_swiglu(ops.moe_linear_native(x, st, sl, r, True), I, cs)
        _sync()
        assert torch.equal(fused, two)


@pytest.mark.parametrize("T", [1, 3, 4, 5, 40])
def test_native_one_call_equals_steps(gpu, T):
    """rlq_moe_native (down and combine in one launch up to four tokens) gives the bits of
    the step-by-step entry points."""
    import torch

    from raceline_amd import ops

    rng = np.random.default_rng(T + 70)
    E, topk, H, I = 32, 8, 512, 512
    gq, gs = make_stack(rng, E + 2, 2 * I, H, "fp4")
    dq, ds = make_stack(rng, E + 2, H, I, "fp4")
    gu = upload_stack(gq, gs, 2 * I, "fp4", gpu)
    dn = upload_stack(dq, ds, H, "fp4", gpu)
    slots = to_dev(shuffled_slots(rng, E, 1), gpu)
    cs = to_dev(rng.uniform(0.5, 1.5, size=I).astype(np.float32), gpu)
    x = to_dev(rng.standard_normal((T, H)).astype(np.float16), gpu)
    logits = to_dev(rng.standard_normal((T, E + 1), dtype=np.float32), gpu)
    h0 = rng.standard_normal((T, H)).astype(np.float32)
    h1, h2 = to_dev(h0, gpu), to_dev(h0, gpu)
    ops.moe_native(x, logits, gu, dn, slots, topk, h1, cs=cs)
    ops.moe_native(x, logits, gu, dn, slots, topk, h2, cs=cs, one_call=False)
    _sync()
    assert torch.equal(h1, h2)
