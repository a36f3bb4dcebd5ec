"""The engine layer on the GPU (include/rl_engine.h) over .rlm files written with the product
writer, against the oracle:

- rl_linear on every tensor kind (q4a with bf16 scales, q4n int15 and fp4, f16b) and on the
  parts of stacked tensors, with and without ACCUM (Engine::encode_linear,
  src/engine.mm:832-906): max|err|/rms <= 1e-3 of the fp64 product.
- rl_norm (rms_norm_rows, kernels/ops.metal:74-112, with the native column-scale fold of
  engine.mm:517-530): each half within one fp16 ulp of the fp64 value rounded once.
- rl_mlp, dense (encode_mlp, engine.mm:943-958) and mixture of experts (encode_moe,
  :965-1059; native and affine stacks): the MLP's contribution within 1e-3; a token's
  result is the same bits whatever other tokens share the call, within one kernel family
  (the decode kernel up to 8 rows, the prefill kernel above; the MoE kernels throughout).
  At the other model sizes the contribution is held to 1e-3 once the oracle's down product
  takes the GPU's own half activations, and to a looser bound against the oracle's own.
- Chunking (ops.metal:60-72): a row from an 8-row call (decode kernel) and from a 9-row
  call (prefill kernel) agree within a stated bound, for rl_linear and rl_mlp.
- rl_head and the draft head (engine.mm:1425-1458,1634-1638): logits within 1e-3; the draft
  logits are exactly the main and tail slices of the full head's; rl_top_k_device and
  rl_argmax give rl_top_k's ids and values exactly.
"""

import ctypes

import numpy as np
import pytest

import oracle as O
import oracle.engine as OE
from raceline_amd import lib
from raceline_amd.model import Engine, top_k
from tests import model_files as MF
from tests.qdata import to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-3
BOOKS = [None, "int15", "fp4"]


def _sync():
    import torch

    torch.cuda.synchronize()


def _x(seed, rows, k, scale=1.0):
    return (np.random.default_rng(seed).standard_normal((rows, k)) * scale).astype(np.float16)


def _col_scale(m, name):
    return m.native[name][2] if name in m.native else None


@pytest.mark.parametrize("book", BOOKS)
def test_linear_every_kind_and_part(gpu, tmp_path, book):
    m = MF.write_dense_model(str(tmp_path / "m.rlm"), seed=10, native_book=book)
    with Engine(m.path, max_chunk=64) as e:
        assert e.vocab == 1000 and e.hidden_size == 256 and e.logits_stride == 1024
        for rows in (1, 5, 40):                               # decode kernel, and prefill at 40
            x = _x(rows, rows, 256)
            xd = to_dev(x, gpu)
            for name, part, r in (("layers.0.attn.qkv", None, (0, 1024)), ("layers.0.attn.qkv", "k", (512, 768)),
                                  ("layers.1.attn.qkv", "v", (768, 1024)), ("layers.1.mlp.gate_up", "up", (512, 1024)),
                                  ("lm_head", None, (0, 1000)), ("extra.dense", None, (0, 300))):
                y = e.linear(name, xd, part=part, n=r[1] - r[0])
                _sync()
                ref = MF.linear_f64(m, name, x, rows=r)
                O.check_close(y.cpu().numpy(), ref, TOL, f"{name}[{part}] rows={rows} book={book}")
            act = _x(rows + 50, rows, 512, 0.1)
            h0 = np.random.default_rng(rows).standard_normal((rows, 256)).astype(np.float32)
            h = to_dev(h0, gpu)
            e.linear("layers.1.mlp.down", to_dev(act, gpu), out=h, accum=True)
            _sync()
            ref = h0 + MF.linear_f64(m, "layers.1.mlp.down", act)
            O.check_close(h.cpu().numpy(), ref, TOL, f"down accum rows={rows} book={book}")


def _check_half(got, ref, what):
    ref = np.asarray(ref, np.float64)
    bound = 2.0 ** -10 * np.abs(ref) + 2.0 ** -24
    bad = np.abs(np.asarray(got, np.float64) - ref) > bound
    assert not bad.any(), f"{what}: {bad.sum()} halves off by more than one ulp"


@pytest.mark.parametrize("book", BOOKS)
def test_norm(gpu, tmp_path, book):
    m = MF.write_dense_model(str(tmp_path / "m.rlm"), seed=11, native_book=book)
    eps = m.cfg["rms_norm_eps"]
    h0 = (np.random.default_rng(12).standard_normal((9, 256)) * 3.0).astype(np.float32)
    with Engine(m.path, max_chunk=16) as e:
        for which, layer, fname, consumer in ((0, 1, "layers.1.in_norm", "layers.1.attn.qkv"),
                                              (1, 0, "layers.0.post_norm", "layers.0.mlp.gate_up"),
                                              (2, 0, "final_norm", "lm_head")):
            xn = e.norm(which, layer, to_dev(h0, gpu))
            _sync()
            w = m.floats[fname].astype(np.float64)
            c = _col_scale(m, consumer)
            if c is not None:
                w = (m.floats[fname] * c[:256]).astype(np.float32).astype(np.float64)   # folded in fp32, as the engine does
            ref = np.asarray(h0, np.float64) / np.sqrt(np.mean(np.asarray(h0, np.float64) ** 2, 1, keepdims=True) + eps) * w
            _check_half(xn.cpu().numpy(), ref, f"norm {which} book={book}")
            one = e.norm(which, layer, to_dev(h0[4:5].copy(), gpu))
            _sync()
            np.testing.assert_array_equal(one.cpu().numpy()[0], xn.cpu().numpy()[4])


def _mlp_ref(m, layer, h0):
    I = m.cfg["intermediate_size"]
    gu, dn = f"layers.{layer}.mlp.gate_up", f"layers.{layer}.mlp.down"
    w = m.floats[f"layers.{layer}.post_norm"]
    cg = _col_scale(m, gu)
    if cg is not None:
        w = (w * cg).astype(np.float32)
    return OE.mlp_dense_f64(h0, w, m.cfg["rms_norm_eps"], lambda xn: MF.linear_f64(m, gu, xn),
                            lambda a: MF.linear_f64(m, dn, a), I, cs=_col_scale(m, dn))


@pytest.mark.parametrize("book", BOOKS)
def test_dense_mlp(gpu, tmp_path, book):
    import torch

    m = MF.write_dense_model(str(tmp_path / "m.rlm"), seed=13, native_book=book)
    with Engine(m.path, max_chunk=64) as e:
        for T in (1, 6, 40):
            h0 = np.random.default_rng(T).standard_normal((T, 256)).astype(np.float32)
            h = to_dev(h0, gpu)
            e.mlp(1, h)
            _sync()
            ref = _mlp_ref(m, 1, h0)
            O.check_close(h.cpu().numpy().astype(np.float64) - h0, ref - h0, TOL, f"dense MLP T={T} book={book}")
            # a token's result does not depend on the other tokens of the call, within one kernel
            # family: up to 8 rows (decode kernel) one row alone; above 8 (prefill kernel) a sub-batch
            if T > 1:
                lo = 0 if T <= 8 else T - 12
                sub = to_dev(h0[lo:T].copy() if T > 8 else h0[T - 1:T].copy(), gpu)
                e.mlp(1, sub)
                _sync()
                assert torch.equal(sub, h[lo:T] if T > 8 else h[T - 1:T])


@pytest.mark.parametrize("hidden,inter", [(256, 512), (4096, 1024), (320, 768)])
def test_dense_mlp_same_bits_as_its_steps(gpu, tmp_path, hidden, inter):
    """rl_mlp on an affine dense MLP at decode sizes fuses the SwiGLU into the gate/up launch;
    its result must be the bits of the steps run one by one: rl_norm, rl_linear on gate_up,
    the SwiGLU kernel (rlq_moe_swiglu), rl_linear on down with ACCUM."""
    import torch

    from raceline_amd import ops

    m = MF.write_dense_model(str(tmp_path / "m.rlm"), seed=hidden + inter, hidden=hidden, intermediate=inter,
                             layers=2)
    with Engine(m.path, max_chunk=16) as e:
        for T in (1, 3, 8, 9):
            h0 = np.random.default_rng(T + hidden).standard_normal((T, hidden)).astype(np.float32)
            h = to_dev(h0, gpu)
            e.mlp(1, h)
            hs = to_dev(h0, gpu)
            xn = e.norm(1, 1, hs)
            g = e.linear("layers.1.mlp.gate_up", xn, n=2 * inter)
            act = torch.empty((T, inter), dtype=torch.float16, device=gpu)
            ops.lib.call("rlq_moe_swiglu", g.data_ptr(), g.stride(0), T, inter, None, act.data_ptr(), act.stride(0),
                         ops._stream())
            e.linear("layers.1.mlp.down", act, out=hs, accum=True)
            _sync()
            assert torch.equal(h, hs), f"T={T} H={hidden} I={inter}"


def _moe_ref(m, layer, h0):
    cfg = m.cfg
    E, topk, I, H = cfg["num_experts"], cfg["num_experts_per_tok"], cfg["moe_intermediate_size"], cfg["hidden_size"]
    gu, dn = f"layers.{layer}.moe.gate_up", f"layers.{layer}.moe.down"
    w = m.floats[f"layers.{layer}.post_norm"]
    cg = _col_scale(m, gu)
    if cg is not None:
        w = (w * cg).astype(np.float32)
    xn = OE.rms_norm_f16(h0, w, cfg["rms_norm_eps"])
    logits = (xn.astype(np.float64) @ m.dense[f"layers.{layer}.moe.router"].astype(np.float64).T).astype(np.float32)
    srt = np.sort(logits[:, :E], axis=1)[:, ::-1]
    assert (srt[:, topk - 1] - srt[:, topk] > 1e-4).all(), "routing margin too small for a stable comparison"
    if m.book:
        (qg, sg, _, _), (qd, sd, cd, _) = m.native[gu], m.native[dn]
        ref, _, _ = O.moe_layer_native_f64(xn, logits, (qg, sg), (qd, sd), cd, np.arange(E + 1), E, topk, I, H, m.book,
                                           h0=h0)
    else:
        ref, _, _ = O.moe_layer_f64(xn, logits, m.affine[gu][:3], m.affine[dn][:3], E, topk, I, H, scale_dtype="bf16",
                                    h0=h0)
    return ref


@pytest.mark.parametrize("book", BOOKS)
def test_moe_mlp(gpu, tmp_path, book):
    import torch

    m = MF.write_moe_model(str(tmp_path / "moe.rlm"), seed=14, native_book=book)
    with Engine(m.path, max_chunk=64) as e:
        for T in (1, 3, 24):
            h0 = np.random.default_rng(100 + T).standard_normal((T, 256)).astype(np.float32)
            h = to_dev(h0, gpu)
            e.mlp(0, h)
            _sync()
            ref = _moe_ref(m, 0, h0)
            O.check_close(h.cpu().numpy().astype(np.float64) - h0, ref - h0, TOL, f"MoE T={T} book={book}")
            if T > 1:
                one = to_dev(h0[1:2].copy(), gpu)
                e.mlp(0, one)
                _sync()
                assert torch.equal(one[0], h[1])
        # every expert is resident: no expert cache, as the reference reports without one
        assert e.expert_cache() is None and e.expert_cache_size() is None
        hits, loads = ctypes.c_ulonglong(7), ctypes.c_ulonglong(7)
        assert lib.load().rl_expert_cache(e._e, ctypes.byref(hits), ctypes.byref(loads)) == 0
        assert hits.value == 0 and loads.value == 0


@pytest.mark.parametrize("book", [None, "int15"])
@pytest.mark.parametrize("hidden", [1024, 2048])
def test_moe_mlp_one_token_norm_and_router_in_one_launch(gpu, tmp_path, book, hidden):
    """At one token of a MoE layer whose router K takes 4 waves or more, rl_mlp runs the
    post-attention norm and the router product in one launch: the token's result is within
    the bar of the oracle and bit-identical to the same token inside a 3-token call (the
    norm and the router as separate launches; the experts read the normed row the fused
    launch leaves, so equal bits also pin that row)."""
    import torch

    m = MF.write_moe_model(str(tmp_path / "moe.rlm"), seed=hidden + 3, native_book=book, hidden=hidden, experts=32,
                           topk=4, moe_inter=256)
    with Engine(m.path, max_chunk=16) as e:
        h0 = np.random.default_rng(hidden).standard_normal((3, hidden)).astype(np.float32)
        h3 = to_dev(h0, gpu)
        e.mlp(0, h3)
        h1 = to_dev(h0[1:2].copy(), gpu)
        e.mlp(0, h1)
        _sync()
        assert torch.equal(h1[0], h3[1])
        ref = _moe_ref(m, 0, h0[1:2])
        O.check_close(h1.cpu().numpy().astype(np.float64) - h0[1:2], ref - h0[1:2], TOL, f"MoE T=1 H={hidden}")


def _check_layer(got, ref, what):
    """A layer's contribution through fp16 activations, against the fp64 reference that
    rounds the same activations: where the kernel's fp32 value and the fp64 one fall on
    either side of a rounding point, the two activations are one half ulp apart, which
    moves every output of that token's row. So the bulk is held tight (rms error <= 2e-4
    of the rms) and isolated rows may carry such a step (max <= 3e-3 of the rms); measured
    at these sizes: bulk <= 9.3e-5, single-activation rows up to 1.8e-3, other rows exact
    or near 3e-5."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    rms = float(np.sqrt(np.mean(ref ** 2)))
    err = got - ref
    bulk = float(np.sqrt(np.mean(err ** 2))) / rms
    worst = float(np.abs(err).max()) / rms
    assert bulk <= 2e-4 and worst <= 3e-3, f"{what}: rms err/rms = {bulk:.3e}, max err/rms = {worst:.3e}"


@pytest.mark.parametrize("book", [None, "int15"])
@pytest.mark.parametrize("hidden,inter,vocab", [(320, 768, 700), (512, 256, 1300)])
def test_dense_layer_and_head_other_sizes(gpu, tmp_path, book, hidden, inter, vocab):
    """Model sizes the other tests do not use: a hidden size of 5 groups (320) or 8 (512),
    intermediate sizes of 768 and 256, and vocabularies that are not a multiple of the
    256-row block (the head's padding rows). rl_mlp at decode and prefill row counts and
    rl_head against the fp64 reference: the head within 1e-3 (one product), the MLP by
    _check_layer (its contribution passes through fp16 activations)."""
    m = MF.write_dense_model(str(tmp_path / "m.rlm"), seed=hidden + inter, native_book=book, hidden=hidden,
                             intermediate=inter, vocab=vocab, layers=1)
    with Engine(m.path, max_chunk=64) as e:
        assert e.vocab == vocab and e.hidden_size == hidden
        for T in (1, 7, 33):
            h0 = np.random.default_rng(T + hidden).standard_normal((T, hidden)).astype(np.float32)
            h = to_dev(h0, gpu)
            e.mlp(0, h)
            _sync()
            ref = _mlp_ref(m, 0, h0)
            _check_layer(h.cpu().numpy().astype(np.float64) - h0, ref - h0, f"dense MLP T={T} H={hidden} I={inter} "
                         f"book={book}")
        h0 = np.random.default_rng(vocab).standard_normal((3, hidden)).astype(np.float32)
        logits = e.head(to_dev(h0, gpu))
        _sync()
        w = m.floats["final_norm"]
        c = _col_scale(m, "lm_head")
        if c is not None:
            w = (w * c).astype(np.float32)
        ref = MF.linear_f64(m, "lm_head", OE.rms_norm_f16(h0, w, m.cfg["rms_norm_eps"]))
        got = logits.cpu().numpy()
        O.check_close(got[:, :vocab], ref, TOL, f"head vocab={vocab} H={hidden} book={book}")
        assert (got[:, vocab:] == 0).all()                     # padding rows of the head


@pytest.mark.parametrize("book", [None, "fp4"])
def test_moe_layer_other_sizes(gpu, tmp_path, book):
    """A mixture of experts of other sizes (H = 512, 32 experts + shared, top-3, I = 384; the
    reader takes expert counts that are multiples of 32, as src/model_file.mm:75 does)
    through rl_mlp at one token, a few, and a batch on the staged kernels, checked by
    _check_layer."""
    m = MF.write_moe_model(str(tmp_path / "moe.rlm"), seed=21, native_book=book, hidden=512, experts=32, topk=3,
                           moe_inter=384)
    with Engine(m.path, max_chunk=64) as e:
        for T in (1, 5, 40):
            h0 = np.random.default_rng(300 + T).standard_normal((T, 512)).astype(np.float32)
            h = to_dev(h0, gpu)
            e.mlp(0, h)
            _sync()
            ref = _moe_ref(m, 0, h0)
            _check_layer(h.cpu().numpy().astype(np.float64) - h0, ref - h0, f"MoE T={T} book={book}")


def _dense_from_gpu_acts(e, m, layer, h0, gpu):
    """The dense MLP's contribution computed by the oracle's down product from the GPU's own
    half activations. rl_norm, rl_linear on the gate/up matrix and the SwiGLU kernel are the
    steps rl_mlp runs (the same kernels on the same rows, so the same bits)."""
    from raceline_amd import ops

    I = m.cfg["intermediate_size"]
    xn = e.norm(1, layer, to_dev(h0, gpu))
    g = e.linear(f"layers.{layer}.mlp.gate_up", xn, n=2 * I)
    cs = _col_scale(m, f"layers.{layer}.mlp.down")
    act = ops.moe_swiglu(g, I, None if cs is None else to_dev(cs, gpu))
    _sync()
    return MF.linear_f64(m, f"layers.{layer}.mlp.down", act.cpu().numpy())


def _moe_from_gpu_acts(e, m, layer, h0, gpu):
    """The MoE MLP by the oracle (routing, down products, combine) from the GPU's normed rows,
    router logits and half activations, taken by the step entry points that rlq_moe and
    rlq_moe_native equal bit for bit (the gate/up product with the SwiGLU fused)."""
    import torch

    from raceline_amd import ops
    from tests.qdata import upload_mlx

    cfg = m.cfg
    E, topk, I, H = cfg["num_experts"], cfg["num_experts_per_tok"], cfg["moe_intermediate_size"], cfg["hidden_size"]
    gu, dn = f"layers.{layer}.moe.gate_up", f"layers.{layer}.moe.down"
    xn = e.norm(1, layer, to_dev(h0, gpu))
    logits = e.linear(f"layers.{layer}.moe.router", xn, n=E + 1)
    r = ops.moe_route(logits, E, topk)
    if m.book:
        qg, sg, _, _ = m.native[gu]
        stack = ops.pack_moe_native(to_dev(O.pack_nibbles_u32(qg).view(np.int32), gpu), to_dev(sg, gpu), 2 * I, m.book)
        slots = torch.arange(E + 1, dtype=torch.int32, device=gpu)
        act = ops.moe_gate_up_native(xn, stack, slots, r, to_dev(m.native[dn][2], gpu))
    else:
        mw = ops.pack_moe(upload_mlx(*m.affine[gu][:3], "bf16", gpu), upload_mlx(*m.affine[dn][:3], "bf16", gpu),
                          E, H, I)
        act = ops.moe_gate_up(xn, mw, r)
    acts = act[r.inv.long()]                      # (token, slot) order
    _sync()
    xn_h, lg, acts_h = xn.cpu().numpy(), logits.cpu().numpy(), acts.cpu().numpy()
    if m.book:
        (qg, sg, _, _), (qd, sd, cd, _) = m.native[gu], m.native[dn]
        ref, _, _ = O.moe_layer_native_f64(xn_h, lg, (qg, sg), (qd, sd), cd, np.arange(E + 1), E, topk, I, H, m.book,
                                           h0=h0, acts=acts_h)
    else:
        ref, _, _ = O.moe_layer_f64(xn_h, lg, m.affine[gu][:3], m.affine[dn][:3], E, topk, I, H, scale_dtype="bf16",
                                    h0=h0, acts=acts_h)
    return ref


@pytest.mark.parametrize("book", [None, "int15"])
@pytest.mark.parametrize("hidden,inter", [(320, 768), (512, 256)])
def test_dense_mlp_other_sizes_from_the_gpus_activations(gpu, tmp_path, book, hidden, inter):
    """rl_mlp at the other sizes, held to 1e-3 of the fp64 product once the oracle's down
    product takes the GPU's own half activations (where a half rounds is then the same on
    both sides; the gate/up product and the SwiGLU are checked by the other tests)."""
    m = MF.write_dense_model(str(tmp_path / "m.rlm"), seed=hidden + inter + 1, native_book=book, hidden=hidden,
                             intermediate=inter, vocab=700, layers=1)
    with Engine(m.path, max_chunk=64) as e:
        for T in (1, 7, 33):
            h0 = np.random.default_rng(T + hidden + 1).standard_normal((T, hidden)).astype(np.float32)
            h = to_dev(h0, gpu)
            e.mlp(0, h)
            _sync()
            ref = _dense_from_gpu_acts(e, m, 0, h0, gpu)
            O.check_close(h.cpu().numpy().astype(np.float64) - h0, ref, TOL,
                          f"dense MLP T={T} H={hidden} I={inter} book={book}")


@pytest.mark.parametrize("book", [None, "fp4", "int15"])
def test_moe_other_sizes_from_the_gpus_activations(gpu, tmp_path, book):
    """rl_mlp over a mixture of experts of other sizes (H = 512, 32 experts + shared, top-3,
    I = 384), held to 1e-3 of the oracle fed the GPU's own activations."""
    m = MF.write_moe_model(str(tmp_path / "moe.rlm"), seed=22, native_book=book, hidden=512, experts=32, topk=3,
                           moe_inter=384)
    with Engine(m.path, max_chunk=64) as e:
        for T in (1, 5, 40):
            h0 = np.random.default_rng(310 + T).standard_normal((T, 512)).astype(np.float32)
            h = to_dev(h0, gpu)
            e.mlp(0, h)
            _sync()
            ref = _moe_from_gpu_acts(e, m, 0, h0, gpu)
            O.check_close(h.cpu().numpy().astype(np.float64) - h0, ref - h0, TOL, f"MoE T={T} book={book}")


CHUNK_LINEAR_BOUND = 5e-5     # max |row from 8 rows - row from 9 rows| / rms
CHUNK_MLP_BULK, CHUNK_MLP_MAX = 2e-4, 3e-3


@pytest.mark.parametrize("book", BOOKS)
def test_rows_agree_between_decode_and_prefill_chunks(gpu, tmp_path, book):
    """The reference gives a token the same bits however a prompt is chunked
    (kernels/ops.metal:60-72). Here a call of up to 8 rows runs the decode kernel and a longer
    one the prefill kernel, which sum in different orders, so a row from an 8-row call and
    from a 9-row call are held to a bound instead: rl_linear within CHUNK_LINEAR_BOUND of the
    output's rms; rl_mlp, whose products pass through half activations that may round
    either way, within CHUNK_MLP_BULK (rms) and CHUNK_MLP_MAX (max) of its contribution's rms."""
    m = MF.write_dense_model(str(tmp_path / "m.rlm"), seed=40, native_book=book)
    rng = np.random.default_rng(41)
    with Engine(m.path, max_chunk=64) as e:
        x = to_dev(rng.standard_normal((9, 512)).astype(np.float16), gpu)
        for name, k, n in (("layers.0.attn.qkv", 256, 1024), ("layers.1.mlp.gate_up", 256, 1024),
                           ("layers.0.mlp.down", 512, 256), ("lm_head", 256, 1000)):
            y8 = e.linear(name, x[:8, :k].contiguous(), n=n)
            y9 = e.linear(name, x[:9, :k].contiguous(), n=n)
            _sync()
            a, b = y8.cpu().numpy().astype(np.float64), y9.cpu().numpy()[:8].astype(np.float64)
            rms = float(np.sqrt(np.mean(b ** 2)))
            d = float(np.abs(a - b).max()) / rms
            print(f"[chunk] {name} book={book}: max|y(8 rows) - y(9 rows)|/rms = {d:.2e}")
            assert d <= CHUNK_LINEAR_BOUND, f"{name}: {d:.3e}"
        h0 = rng.standard_normal((9, 256)).astype(np.float32)
        h8, h9 = to_dev(h0[:8].copy(), gpu), to_dev(h0.copy(), gpu)
        e.mlp(1, h8)
        e.mlp(1, h9)
        _sync()
        a = h8.cpu().numpy().astype(np.float64) - h0[:8]
        b = h9.cpu().numpy()[:8].astype(np.float64) - h0[:8]
        rms = float(np.sqrt(np.mean(b ** 2)))
        bulk, worst = float(np.sqrt(np.mean((a - b) ** 2))) / rms, float(np.abs(a - b).max()) / rms
        print(f"[chunk] rl_mlp book={book}: rms {bulk:.2e}, max {worst:.2e} of the contribution's rms")
        assert bulk <= CHUNK_MLP_BULK and worst <= CHUNK_MLP_MAX, f"rl_mlp: {bulk:.3e} {worst:.3e}"


@pytest.mark.parametrize("book", BOOKS)
def test_head_draft_vocab_and_top_k(gpu, tmp_path, book):
    import torch

    m = MF.write_dense_model(str(tmp_path / "m.rlm"), seed=15, native_book=book)
    h0 = np.random.default_rng(16).standard_normal((4, 256)).astype(np.float32)
    with Engine(m.path, max_chunk=16) as e:
        logits = e.head(to_dev(h0, gpu))
        _sync()
        w = m.floats["final_norm"]
        c = _col_scale(m, "lm_head")
        if c is not None:
            w = (w * c).astype(np.float32)
        xn = OE.rms_norm_f16(h0, w, m.cfg["rms_norm_eps"])
        ref = MF.linear_f64(m, "lm_head", xn)
        got = logits.cpu().numpy()
        O.check_close(got[:, :1000], ref, TOL, f"head book={book}")
        assert (got[:, 1000:] == 0).all()                     # padding rows of the head
        # top-k of the vocabulary on the device, and rl_argmax, against rl_top_k
        for k in (1, 8, 256):
            ids, vals = e.top_k_device(logits[0, :1000].contiguous(), k)
            rid, rvals = top_k(got[0, :1000], k)
            assert ids == list(rid) and np.array_equal(np.float32(vals), rvals)
        assert e.argmax() == int(np.argmax(got[0, :1000]))
        # the draft vocabulary: the main rows, then the tail rows (native heads only)
        e.set_draft_vocab(300)
        e.set_draft_tail(800)
        assert e.draft_main == 512
        assert e.draft_tail == (768 if book else -1)
        d = e.draft_head(to_dev(h0[2].copy(), gpu))
        _sync()
        full = e.head(to_dev(h0[2:3].copy(), gpu))[0]
        _sync()
        want = torch.cat([full[:512], full[768:]]) if book else full[:512]
        assert e.draft_vocab == want.numel()
        assert torch.equal(d, want)
        e.set_draft_vocab(0)
        e.set_draft_tail(-1)
        assert e.draft_main == 1024 and e.draft_tail == -1 and e.draft_vocab == 1024


def test_device_top_k_ties_nan_and_infinities(gpu, tmp_path):
    m = MF.write_dense_model(str(tmp_path / "m.rlm"), seed=17, layers=1)
    rng = np.random.default_rng(18)
    with Engine(m.path, max_chunk=16) as e:
        for n in (5, 3000, 16000):
            x = rng.integers(-30, 30, n).astype(np.float32)
            x[rng.random(n) < 0.1] = np.nan
            x[rng.random(n) < 0.02] = -np.inf
            x[rng.random(n) < 0.01] = np.inf
            for k in (1, 7, 64, 256):
                ids, vals = e.top_k_device(to_dev(x, gpu), k)
                rid, rvals = top_k(x, k)
                assert ids == list(rid), f"n={n} k={k}"
                np.testing.assert_array_equal(np.float32(vals), rvals)
