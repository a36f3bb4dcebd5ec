"""The call sequence of the writer's golden file.

One small model file that uses every tensor kind of the .rlm format and an embedded file:
affine blocked matrices with parts (q4a), a native blocked matrix with parts (q4n), a dense
half matrix (f16b), affine and native row tables (q4a_rows, q4n_rows), float vectors and
matrices (f32), and the files section. The inputs are drawn from a seeded numpy generator,
so the same calls on any writer with tools/convert.py's interface give the same file.

make_writer_golden.py runs this sequence on tools/convert.py's Writer (the reference) in
the build container and records the file's length and sha256 in writer_golden.json;
tests/test_rlm.py runs it on raceline_amd.rlm.Writer and compares.
"""

from __future__ import annotations

import numpy as np

SEED = 20261202
FILES = {"tokenizer.json": b'{"model": {"type": "BPE", "vocab": {"a": 0, "b": 1}}}\n',
         "chat_template.jinja": b"{% for m in messages %}{{ m.content }}{% endfor %}\n"}


def _bf16_values(x):
    """float32 values that bfloat16 holds exactly (the low 16 bits cleared)."""
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def _affine(rng, n, k):
    q = rng.integers(0, 16, (n, k), dtype=np.uint8)
    s = _bf16_values(rng.uniform(0.001, 0.01, (n, k // 64)))
    b = _bf16_values(rng.uniform(-0.08, -0.01, (n, k // 64)))
    return q, s, b


def meta():
    return dict(format="raceline", version=1, arch="qwen3_5",
                config=dict(hidden_size=192, num_hidden_layers=1, vocab_size=300, intermediate_size=320),
                quant=dict(bits=4, group=64, block=256, mode="affine", scale_dtype="bf16"))


def write(w, add_files):
    """Runs the sequence on writer w; add_files(w) embeds FILES in a section of its own
    (tools/convert.py's Writer.add_files takes a directory, this repository's add_file the
    bytes, so the caller supplies it)."""
    rng = np.random.default_rng(SEED)
    k = 192
    w.begin("embed")
    w.add_rows("embed_tokens", *_affine(rng, 300, k))
    codes = rng.integers(0, 16, (40, 128), dtype=np.uint8)
    w.add_native_rows("embed_images", codes, rng.uniform(0.5, 2.0, 40).astype(np.float32),
                      rng.uniform(0.5, 2.0, 128).astype(np.float32), "int15")
    w.end()
    w.begin("layer.0")
    w.add_float("layers.0.in_norm", rng.standard_normal(k).astype(np.float32))
    w.add_float("layers.0.lin.conv", rng.standard_normal((72, 4)).astype(np.float32))
    w.add_blocked("layers.0.attn.qkv", [("q", _affine(rng, 130, k)), ("k", _affine(rng, 64, k)),
                                        ("v", _affine(rng, 64, k))])
    w.add_blocked("layers.0.mlp.gate_up", [("gate", _affine(rng, 320, k)), ("up", _affine(rng, 320, k))])
    w.add_blocked("layers.0.mlp.down", [("out", _affine(rng, k, 320))])
    w.add_dense("layers.0.moe.router", rng.standard_normal((9, k)).astype(np.float16))
    w.end()
    w.begin("head")
    codes = rng.integers(0, 16, (300, k), dtype=np.uint8)
    w.add_native("lm_head", [("main", 280), ("extra", 20)], codes, rng.uniform(0.002, 0.02, 300).astype(np.float32),
                 rng.uniform(0.5, 2.0, k).astype(np.float32), "fp4")
    w.add_float("final_norm", np.ones(k, np.float32))
    w.end()
    add_files(w)
    w.finish(meta())
