"""Parity of the HIP mixture-of-experts path with the oracle (oracle/moe.py).

- Routing: the selected experts are exact (fp32 comparisons, ties to the lower expert);
  the weights are within 1e-6 relative (the GPU sums the softmax denominator in fp32);
  the sort and the work list equal the oracle's counting sort with rows in token order.
- gate/up + SwiGLU: act = half(silu(g) * u) against the fp64 value, element-wise
  |err| <= 2^-10 |ref| + 1e-4 rms(ref): the half output rounds each value by up to half
  an ulp (<= 2^-11 of itself), and the fp32 products feeding it are far more accurate.
- down: against the fp64 product of the GPU's own act, max|err| / rms <= 1e-3.
- The whole layer: against oracle.moe_layer_f64 (fp64, act rounded to half as the
  reference stores it), max|err| / rms <= 1e-3; a token's result is bit-identical
  whatever other tokens share the call (kernels/moe.metal:9-12).
"""

import numpy as np
import pytest

import oracle as O
from tests.qdata import to_dev, upload_mlx

pytestmark = pytest.mark.gpu
TOL = 1e-3


def check_half_output(got, ref, what):
    """got: a half-rounded result; ref: the exact value (see the module docstring)."""
    rms = float(np.sqrt(np.mean(ref ** 2)))
    bound = 2.0 ** -10 * np.abs(ref) + 1e-4 * rms
    bad = np.abs(got - ref) > bound
    assert not bad.any(), f"{what}: {bad.sum()} values outside one half ulp; worst err {np.abs(got - ref).max():.3e}"


def make_moe(seed, E, H, I, sd="f16"):
    rng = np.random.default_rng(seed)
    Wg = (rng.standard_normal(((E + 1) * 2 * I, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    Wd = (rng.standard_normal(((E + 1) * H, I), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    return O.quantize_affine_rtn(Wg, sd), O.quantize_affine_rtn(Wd, sd)


def upload_moe(gu, dn, E, H, I, sd, dev):
    from raceline_amd import ops

    return ops.pack_moe(upload_mlx(*gu, sd, dev), upload_mlx(*dn, sd, dev), E, H, I)


def make_inputs(seed, T, E, H):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H), dtype=np.float32).astype(np.float16)
    logits = rng.standard_normal((T, E + 1), dtype=np.float32)
    return x, logits


def _sync():
    import torch

    torch.cuda.synchronize()


@pytest.mark.parametrize("T,E,topk,norm", [(1, 16, 4, True), (7, 16, 4, False), (40, 64, 8, True),
                                           (300, 256, 8, True), (1, 256, 8, True), (2000, 8, 2, True),
                                           (16, 256, 8, True), (17, 64, 8, False), (16, 700, 16, False),
                                           (4000, 64, 8, True)])
def test_route(gpu, T, E, topk, norm):
    from raceline_amd import ops

    rng = np.random.default_rng(T * 7 + E)
    logits = rng.standard_normal((T, E + 1), dtype=np.float32)
    if T > 1:
        logits[1, 5] = logits[1, 2] = logits[1, :E].max() + 0.5     # a tie: the lower expert first
    r = ops.moe_route(to_dev(logits, gpu), E, topk, norm)
    _sync()
    sel_ref, w_ref = O.moe_route(logits, E, topk, norm)
    np.testing.assert_array_equal(r.sel.cpu().numpy(), sel_ref)
    np.testing.assert_allclose(r.w.cpu().numpy(), w_ref, rtol=1e-6, atol=1e-7)
    S = topk + 1
    counts, off, items = O.moe_items(sel_ref, E, 16)
    n = int(r.n_items.cpu()[0])
    assert n == len(items)
    np.testing.assert_array_equal(r.items.cpu().numpy()[:n], items)
    tok, inv = r.tok.cpu().numpy(), r.inv.cpu().numpy()
    # every assignment's row holds its token, rows are grouped by expert in token order
    a = np.arange(T * S)
    np.testing.assert_array_equal(tok[inv], a // S)
    for e in range(E + 1):
        rows = tok[off[e]:off[e + 1]]
        assert (np.diff(rows) > 0).all()
        np.testing.assert_array_equal(np.sort(inv[sel_ref == e]), np.arange(off[e], off[e + 1]))


@pytest.mark.parametrize("T,E,topk,norm", [(1, 256, 8, True), (3, 256, 8, False), (33, 64, 8, True),
                                           (20, 16, 16, True), (5, 700, 16, True)])
def test_route_many_ties(gpu, T, E, topk, norm):
    """Logits that tie a lot: small integers, one row all equal, one row with only three
    finite logits (the rest -inf, so the picks run into the -inf ties). The chosen experts
    follow the stable order: equal logits by expert number."""
    from raceline_amd import ops

    rng = np.random.default_rng(T * 11 + E)
    logits = rng.integers(-2, 3, size=(T, E + 1)).astype(np.float32)
    logits[0, :E] = 0.5
    if T > 1:
        logits[1, :E] = -np.inf
        logits[1, [E - 1, E // 2, 3]] = [1.0, 1.0, -1.0]
    r = ops.moe_route(to_dev(logits, gpu), E, topk, norm)
    _sync()
    sel_ref, w_ref = O.moe_route(logits, E, topk, norm)
    np.testing.assert_array_equal(r.sel.cpu().numpy(), sel_ref)
    np.testing.assert_allclose(r.w.cpu().numpy(), w_ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("sd", ["f16", "bf16"])
def test_gate_up_swiglu_and_down(gpu, sd):
    from raceline_amd import ops

    E, H, I, T, topk = 16, 256, 128, 9, 4
    gu, dn = make_moe(31, E, H, I, sd)
    mw = upload_moe(gu, dn, E, H, I, sd, gpu)
    x, logits = make_inputs(32, T, E, H)
    r = ops.moe_route(to_dev(logits, gpu), E, topk)
    act = ops.moe_gate_up(to_dev(x, gpu), mw, r)
    y = ops.moe_down(act, mw, r)
    _sync()
    sel, tok, inv = r.sel.cpu().numpy(), r.tok.cpu().numpy(), r.inv.cpu().numpy()
    act_g = act.cpu().numpy().astype(np.float64)
    y_g = y.cpu().numpy()
    S = topk + 1
    act_ref = np.zeros_like(act_g)
    y_ref = np.zeros(y_g.shape)
    for a in range(T * S):
        e, row, t = sel[a], inv[a], a // S
        assert tok[row] == t
        g = O.linear_affine_f64(x[t:t + 1], *(v[O.expert_rows(e, 2 * I)] for v in gu), sd)
        act_ref[row] = O.silu(g[0, :I]) * g[0, I:]
        y_ref[row] = O.linear_affine_f64(act_g[row:row + 1], *(v[O.expert_rows(e, H)] for v in dn), sd)[0]
    check_half_output(act_g, act_ref, f"moe act ({sd})")
    O.check_close(y_g, y_ref, TOL, f"moe down ({sd})")


@pytest.mark.parametrize("T,E,topk,H,I", [(1, 16, 4, 256, 128), (33, 32, 4, 512, 256), (5, 256, 8, 2048, 512),
                                           (4, 64, 8, 512, 512), (2, 16, 4, 256, 1024),
                                           (70, 32, 4, 512, 256), (130, 16, 4, 320, 192)])
def test_layer_matches_oracle(gpu, T, E, topk, H, I):
    import torch

    from raceline_amd import ops

    gu, dn = make_moe(40 + T, E, H, I)
    mw = upload_moe(gu, dn, E, H, I, "f16", gpu)
    x, logits = make_inputs(41 + T, T, E, H)
    h0 = np.random.default_rng(42).standard_normal((T, H)).astype(np.float32)
    h = to_dev(h0, gpu)
    ops.moe(to_dev(x, gpu), to_dev(logits, gpu), mw, topk, h)
    _sync()
    ref, _, _ = O.moe_layer_f64(x, logits, gu, dn, E, topk, I, H)
    O.check_close(h.cpu().numpy().astype(np.float64) - h0, ref, TOL, f"moe layer T={T} E={E}")
    # the step-by-step entry points give the same bits as the one-call layer
    r = ops.moe_route(to_dev(logits, gpu), E, topk)
    h2 = to_dev(h0, gpu)
    ops.moe_combine(ops.moe_down(ops.moe_gate_up(to_dev(x, gpu), mw, r), mw, r), r, h2)
    _sync()
    assert torch.equal(h, h2)


def test_layer_full_size_batch_invariance(gpu):
    """BASELINE MoE config at T=512 (H=2048, E=256+1, I=512, top-8): tokens 100..163 run
    alone give the same bits as inside the 512-token call; a sample of tokens matches the
    oracle, computed expert by expert for those tokens only."""
    import torch

    from raceline_amd import ops, synth

    E, H, I, topk, T = 256, 2048, 512, 8, 512
    dev = gpu
    gu_t = synth.random_affine((E + 1) * 2 * I, H, 71, dev, packed=False)
    dn_t = synth.random_affine((E + 1) * H, I, 72, dev, packed=False)
    mw = ops.pack_moe(gu_t, dn_t, E, H, I)
    x = synth.random_activations(T, H, 73, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(74)
    logits = torch.randn((T, E + 1), generator=g, device=dev, dtype=torch.float32)
    h = torch.zeros((T, H), dtype=torch.float32, device=dev)
    ops.moe(x, logits, mw, topk, h)
    h_sub = torch.zeros((64, H), dtype=torch.float32, device=dev)
    ops.moe(x[100:164].contiguous(), logits[100:164].contiguous(), mw, topk, h_sub)
    # one token alone (routing inside the gate/up launch, down and combine in one) and three
    h_one = torch.zeros((1, H), dtype=torch.float32, device=dev)
    ops.moe(x[163:164].contiguous(), logits[163:164].contiguous(), mw, topk, h_one)
    h_three = torch.zeros((3, H), dtype=torch.float32, device=dev)
    ops.moe(x[254:257].contiguous(), logits[254:257].contiguous(), mw, topk, h_three)
    _sync()
    assert torch.equal(h_sub, h[100:164])
    assert torch.equal(h_one, h[163:164])
    assert torch.equal(h_three, h[254:257])

    # oracle on sampled tokens
    def host(t3):
        w, s, b = t3
        return (w.cpu().numpy().view(np.uint32), s.cpu().view(torch.int16).numpy().view(np.uint16),
                b.cpu().view(torch.int16).numpy().view(np.uint16))
    wg, sg, bg = host(gu_t)
    wd, sd_, bd = host(dn_t)
    xs, ls = x.cpu().numpy(), logits.cpu().numpy()
    toks = [0, 1, 255, 511, 100, 163]
    sel, w = O.moe_route(ls[toks], E, topk)
    S = topk + 1
    ref = np.zeros((len(toks), H))
    for i, t in enumerate(toks):
        for s in range(S):
            e = int(sel[i * S + s])
            rg, rd = O.expert_rows(e, 2 * I), O.expert_rows(e, H)
            gq = O.linear_affine_f64(xs[t:t + 1], O.unpack_nibbles_u32(wg[rg]), sg[rg], bg[rg])
            a = O.swiglu_f16(gq, I)
            ref[i] += w[i * S + s] * O.linear_affine_f64(a.astype(np.float64), O.unpack_nibbles_u32(wd[rd]), sd_[rd],
                                                         bd[rd])[0]
    O.check_close(h.cpu().numpy()[toks].astype(np.float64), ref, TOL, "moe full-size sampled tokens")


@pytest.mark.parametrize("E,H,I", [(64, 2048, 512), (16, 1024, 1536), (16, 1536, 1024), (16, 4096, 256),
                                   (32, 576, 320)])
def test_token_result_same_across_kernel_choice(gpu, E, H, I):
    """Calls of fewer than 8 tokens run the per-tile expert kernel, larger ones the kernel
    that stages each item's rows in LDS; a token's result must not depend on which one
    ran or on how many tokens share an expert: tokens 3..7 alone (per-tile) and the first
    40 give the same bits as inside a 100-token call.
    The shapes cover K (H for gate/up, I for down) where the staged kernel's waves take
    one (512, 1024, 4096) and two (1536, 2048) of the per-tile kernel's group ranges, and
    odd group counts (576 = 9 groups, 320 = 5)."""
    import torch

    from raceline_amd import ops

    topk = 8
    gu, dn = make_moe(90, E, H, I)
    mw = upload_moe(gu, dn, E, H, I, "f16", gpu)
    x, logits = make_inputs(91, 100, E, H)
    h = torch.zeros((100, H), dtype=torch.float32, device=gpu)
    ops.moe(to_dev(x, gpu), to_dev(logits, gpu), mw, topk, h)
    h40 = torch.zeros((40, H), dtype=torch.float32, device=gpu)
    ops.moe(to_dev(x[:40].copy(), gpu), to_dev(logits[:40].copy(), gpu), mw, topk, h40)
    h5 = torch.zeros((5, H), dtype=torch.float32, device=gpu)
    ops.moe(to_dev(x[3:8].copy(), gpu), to_dev(logits[3:8].copy(), gpu), mw, topk, h5)
    # up to 4 tokens also fold the combine into the down launch; one token also routes in
    # the gate/up launch
    h3 = torch.zeros((3, H), dtype=torch.float32, device=gpu)
    ops.moe(to_dev(x[3:6].copy(), gpu), to_dev(logits[3:6].copy(), gpu), mw, topk, h3)
    h1 = torch.zeros((1, H), dtype=torch.float32, device=gpu)
    ops.moe(to_dev(x[7:8].copy(), gpu), to_dev(logits[7:8].copy(), gpu), mw, topk, h1)
    _sync()
    assert torch.equal(h40, h[:40])
    assert torch.equal(h5, h[3:8])
    assert torch.equal(h3, h[3:6])
    assert torch.equal(h1, h[7:8])
    ref, _, _ = O.moe_layer_f64(x[3:8], logits[3:8], gu, dn, E, topk, I, H)
    O.check_close(h5.cpu().numpy().astype(np.float64), ref, TOL, "moe per-tile vs staged")


@pytest.mark.parametrize("T", [1, 3, 70])
def test_layer_replays_in_a_graph(gpu, T):
    """rlq_moe captured in a graph gives the eager call's bits on every replay, with eager
    calls on the same workspace between the replays: one token (the routing inside the
    gate/up launch), three (the down product and the combine in one launch) and a batch
    (top-k, sort, staged experts, combine)."""
    import torch

    from raceline_amd import ops

    E, topk, H, I = 32, 4, 512, 256
    gu, dn = make_moe(50 + T, E, H, I)
    mw = upload_moe(gu, dn, E, H, I, "f16", gpu)
    x, logits = make_inputs(51 + T, T, E, H)
    xd, ld = to_dev(x, gpu), to_dev(logits, gpu)
    h0 = to_dev(np.random.default_rng(52).standard_normal((T, H)).astype(np.float32), gpu)
    ws = torch.empty(ops.moe_workspace_bytes(T, E, topk, H, I), dtype=torch.uint8, device=gpu)
    want = ops.moe(xd, ld, mw, topk, h0.clone(), workspace=ws)
    h = h0.clone()
    _sync()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.moe(xd, ld, mw, topk, h, workspace=ws)
    for _ in range(4):
        h.copy_(h0)
        g.replay()
        _sync()
        assert torch.equal(h, want)
        assert torch.equal(ops.moe(xd, ld, mw, topk, h0.clone(), workspace=ws), want)


def test_combine_one_and_four_wide_paths_agree(gpu):
    """The combine takes four floats per thread when rows and pointers allow 16-byte accesses
    and one otherwise; both follow the same per-element order, so they give the same bits,
    and both match h + sum_s w_s y_s in float64."""
    import torch

    from raceline_amd import ops

    T, E, topk, H = 37, 16, 4, 192
    S = topk + 1
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((T, E + 1), dtype=np.float32)
    r = ops.moe_route(to_dev(logits, gpu), E, topk)
    y = rng.standard_normal((T * S, H + 1)).astype(np.float32)
    h0 = rng.standard_normal((T, H)).astype(np.float32)
    y_odd = to_dev(y, gpu)[:, :H]                      # row stride H + 1: one float per thread
    y_even = to_dev(np.ascontiguousarray(y[:, :H]), gpu)
    h1, h4 = to_dev(h0, gpu), to_dev(h0, gpu)
    ops.moe_combine(y_odd, r, h1)
    ops.moe_combine(y_even, r, h4)
    _sync()
    assert torch.equal(h1, h4)
    inv, w = r.inv.cpu().numpy(), r.w.cpu().numpy().astype(np.float64)
    ref = h0.astype(np.float64).copy()
    for t in range(T):
        for s in range(S):
            ref[t] += w[t * S + s] * y[inv[t * S + s], :H].astype(np.float64)
    O.check_close(h4.cpu().numpy(), ref, TOL, "moe combine")
