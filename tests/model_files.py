"""Small synthetic .rlm model files for the reader and engine tests, written with the
product writer (raceline_amd.rlm), with the host arrays kept for the oracle.

The configs satisfy the geometry the engine checks (src/engine.mm:394-396: Dk = 128,
head_dim = 256, 64 rotary dimensions, 4 conv taps); the files hold only what the matmul
path reads: the MLP (dense or mixture of experts), the norms, the output head, and a few
extra tensors of every kind.
"""

from __future__ import annotations

import numpy as np

import oracle as O
from raceline_amd import rlm


def config(hidden=256, layers=2, intermediate=512, vocab=1000, experts=0, topk=0, moe_inter=0):
    c = dict(hidden_size=hidden, num_hidden_layers=layers, intermediate_size=intermediate, num_attention_heads=8,
             num_key_value_heads=2, head_dim=256, linear_num_value_heads=16, linear_num_key_heads=8,
             linear_key_head_dim=128, linear_value_head_dim=128, linear_conv_kernel_dim=4, vocab_size=vocab,
             rms_norm_eps=1e-6, full_attention_interval=4, rope_theta=1e7, partial_rotary_factor=0.25,
             eos_token_id=7)
    if experts:
        c.update(num_experts=experts, num_experts_per_tok=topk, moe_intermediate_size=moe_inter, norm_topk_prob=True)
    return c


def affine_bf16(rng, n, k, std=0.02):
    """An affine matrix with bf16 scales and biases (what tools/convert.py stores):
    (q, s float32 bf16 values, b float32 bf16 values, s bits, b bits)."""
    W = (rng.standard_normal((n, k)) * std).astype(np.float32)
    q, sb, bb = O.quantize_affine_rtn(W, "bf16")
    return q, O.bf16_bits_to_f32(sb), O.bf16_bits_to_f32(bb), sb, bb


def native(rng, n, k, book):
    codes = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    s = (rng.uniform(0.5, 1.5, n) * 0.01).astype(np.float32)
    c = rng.uniform(0.5, 2.0, k).astype(np.float32)
    return codes, s, c


class Model:
    """What a test needs to recompute the file's tensors: name -> arrays."""

    def __init__(self, path, cfg, native_book=None):
        self.path, self.cfg, self.book = path, cfg, native_book
        self.affine, self.native, self.dense, self.floats = {}, {}, {}, {}


def write_dense_model(path, seed=0, native_book=None, hidden=256, intermediate=512, vocab=1000, layers=2,
                      head_rows=None):
    """A dense-MLP model: per layer in_norm, post_norm, attn.qkv (parts q, k, v), mlp.gate_up
    (parts gate, up), mlp.down; final_norm, lm_head, a token table and a half matrix.
    Affine (bf16 scales) unless native_book names a codebook."""
    rng = np.random.default_rng(seed)
    cfg = config(hidden, layers, intermediate, vocab)
    m = Model(path, cfg, native_book)
    w = rlm.Writer(path)

    def matrix(name, parts, k):
        if native_book:
            n = sum(r for _, r in parts)
            codes, s, c = native(rng, n, k, native_book)
            w.add_native(name, parts, codes, s, c, native_book)
            m.native[name] = (codes, s, c, dict(parts))
        else:
            arrs = [(pn, affine_bf16(rng, r, k)) for pn, r in parts]
            w.add_blocked(name, [(pn, a[:3]) for pn, a in arrs])
            q = np.concatenate([a[0] for _, a in arrs])
            sb = np.concatenate([a[3] for _, a in arrs])
            bb = np.concatenate([a[4] for _, a in arrs])
            m.affine[name] = (q, sb, bb, dict(parts))

    def floats(name, arr):
        w.add_float(name, arr)
        m.floats[name] = np.asarray(arr, np.float32)

    w.begin("embed")
    eq = rng.integers(0, 16, size=(vocab, hidden), dtype=np.uint8)
    if native_book:
        w.add_native_rows("embed", eq, np.ones(vocab, np.float32), np.ones(hidden, np.float32), native_book)
    else:
        es = np.full((vocab, hidden // 64), 0.0078125, np.float32)
        w.add_rows("embed", eq, es, -8 * es)
    w.end()
    for i in range(layers):
        w.begin(f"layer.{i}")
        floats(f"layers.{i}.in_norm", rng.uniform(0.5, 1.5, hidden))
        floats(f"layers.{i}.post_norm", rng.uniform(0.5, 1.5, hidden))
        matrix(f"layers.{i}.attn.qkv", [("q", 512), ("k", 256), ("v", 256)], hidden)
        matrix(f"layers.{i}.mlp.gate_up", [("gate", intermediate), ("up", intermediate)], hidden)
        matrix(f"layers.{i}.mlp.down", [("out", hidden)], intermediate)
        w.end()
    w.begin("head")
    floats("final_norm", rng.uniform(0.5, 1.5, hidden))
    matrix("lm_head", [("out", head_rows or vocab)], hidden)
    dense = (rng.standard_normal((300, hidden)) * 0.05).astype(np.float16)
    w.add_dense("extra.dense", dense)
    m.dense["extra.dense"] = dense
    w.end()
    w.finish(rlm.native_meta(cfg, native_book) if native_book else rlm.affine_meta(cfg))
    return m


def write_moe_model(path, seed=0, native_book=None, hidden=256, experts=32, topk=4, moe_inter=128, layers=1,
                    vocab=512):
    """A mixture-of-experts model: per layer post_norm, moe.router (half, E+1 rows, the last
    the shared expert's gate), moe.gate_up [(E+1) 2I][H] and moe.down [(E+1) H][I] (the
    stacks of tools/quantize.py:168-228, in an experts section of their own), final norm
    and head. Native (the reference's MoE files) or affine with bf16 scales."""
    rng = np.random.default_rng(seed)
    cfg = config(hidden, layers, moe_inter, vocab, experts, topk, moe_inter)
    m = Model(path, cfg, native_book)
    w = rlm.Writer(path)
    E1 = experts + 1
    for i in range(layers):
        w.begin(f"layer.{i}")
        post = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
        w.add_float(f"layers.{i}.post_norm", post)
        m.floats[f"layers.{i}.post_norm"] = post
        router = (rng.standard_normal((E1, hidden)) * 0.1).astype(np.float16)
        w.add_dense(f"layers.{i}.moe.router", router)
        m.dense[f"layers.{i}.moe.router"] = router
        w.end()
        w.begin(f"experts.{i}")
        for name, n, k in (("moe.gate_up", E1 * 2 * moe_inter, hidden), ("moe.down", E1 * hidden, moe_inter)):
            full = f"layers.{i}.{name}"
            if native_book:
                codes, s, c = native(rng, n, k, native_book)
                w.add_native(full, [("experts", n)], codes, s, c, native_book)
                m.native[full] = (codes, s, c, {"experts": (0, n)})
            else:
                q, sf, bf, sb, bb = affine_bf16(rng, n, k)
                w.add_blocked(full, [("experts", (q, sf, bf))])
                m.affine[full] = (q, sb, bb, {"experts": (0, n)})
        w.end()
    w.begin("head")
    fin = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    w.add_float("final_norm", fin)
    m.floats["final_norm"] = fin
    if native_book:
        codes, s, c = native(rng, vocab, hidden, native_book)
        w.add_native("lm_head", [("out", vocab)], codes, s, c, native_book)
        m.native["lm_head"] = (codes, s, c, {"out": (0, vocab)})
    else:
        q, sf, bf, sb, bb = affine_bf16(rng, vocab, hidden)
        w.add_blocked("lm_head", [("out", (q, sf, bf))])
        m.affine["lm_head"] = (q, sb, bb, {"out": (0, vocab)})
    w.end()
    w.finish(rlm.native_meta(cfg, native_book) if native_book else rlm.affine_meta(cfg))
    return m


def _bf16_values(x):
    """float32 values that bfloat16 holds exactly (the low 16 bits cleared)."""
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def write_head_model(path, hidden, vocab, native_book=None, seed=0, mtp=False):
    """Only what the output head reads, at a real vocabulary: one layer of norms, final_norm
    and lm_head [vocab][hidden]. The head is drawn directly as codes (uniform 0..15) with
    bf16 scales and biases (affine) or row and column scales (native), not quantized from
    floats, so that a 248,320-row head is written in seconds. mtp (native files) adds the
    MTP head's mtp.fc [hidden][2 hidden] and mtp.norm, which make the engine norm a draft
    row with mtp.norm (src/engine.mm:398,534)."""
    rng = np.random.default_rng(seed)
    cfg = config(hidden, 1, 512, vocab)
    m = Model(path, cfg, native_book)
    w = rlm.Writer(path)
    w.begin("layer.0")
    for name in ("layers.0.in_norm", "layers.0.post_norm"):
        arr = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
        w.add_float(name, arr)
        m.floats[name] = arr
    w.end()
    w.begin("head")
    fin = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    w.add_float("final_norm", fin)
    m.floats["final_norm"] = fin
    q = rng.integers(0, 16, size=(vocab, hidden), dtype=np.uint8)
    if native_book:
        s = rng.uniform(0.002, 0.02, vocab).astype(np.float32)
        c = rng.uniform(0.5, 2.0, hidden).astype(np.float32)
        w.add_native("lm_head", [("out", vocab)], q, s, c, native_book)
        m.native["lm_head"] = (q, s, c, {"out": (0, vocab)})
    else:
        G = hidden // 64
        sf = _bf16_values(rng.uniform(0.001, 0.006, (vocab, G)))
        bf = _bf16_values(-7.5 * sf + rng.uniform(-0.002, 0.002, (vocab, G)))
        w.add_blocked("lm_head", [("out", (q, sf, bf))])
        m.affine["lm_head"] = (q, O.f32_to_bf16_bits(sf), O.f32_to_bf16_bits(bf), {"out": (0, vocab)})
    if mtp:
        assert native_book, "the reference's MTP head is in native files"
        codes, s, c = native(rng, hidden, 2 * hidden, native_book)
        w.add_native("mtp.fc", [("out", hidden)], codes, s, c, native_book)
        m.native["mtp.fc"] = (codes, s, c, {"out": (0, hidden)})
        mn = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
        w.add_float("mtp.norm", mn)
        m.floats["mtp.norm"] = mn
    w.end()
    w.finish(rlm.native_meta(cfg, native_book) if native_book else rlm.affine_meta(cfg))
    return m


def linear_f64(m: Model, name: str, x, rows=None):
    """The oracle's product of the model's tensor `name` (rows [r0, r1) if given) with x
    (fp16 rows; for native tensors x already carries the column scale)."""
    r0, r1 = rows if rows else (0, None)
    if name in m.affine:
        q, sb, bb, _ = m.affine[name]
        return O.linear_affine_f64(x, q[r0:r1], sb[r0:r1], bb[r0:r1], "bf16")
    if name in m.native:
        codes, s, c, _ = m.native[name]
        return O.linear_native_f64(x, codes[r0:r1], s[r0:r1], m.book)
    if name in m.dense:
        return np.asarray(x, np.float64) @ m.dense[name][r0:r1].astype(np.float64).T
    raise KeyError(name)
