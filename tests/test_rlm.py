"""The .rlm writer (raceline_amd/rlm.py) and the library's reader (csrc/model_file.cpp),
without a GPU: the writer's bytes against the reference writer's (a golden sha256 made
from tools/convert.py), layout replay (the writer's placement recomputed by Layout, the
property tests/test_runtime.py:296-323 checks for tools/convert.py), the blocked packing against
the oracle's restatement of tools/convert.py:92-117, the reader's tables against what the
writer recorded, the reader's fatal cases (src/model_file.mm:44-167), rl_open's checks that
run before any device work (src/engine.mm:394-396,516), rl_top_k's order
(src/capi.mm:74-101) and the fp32 -> bf16 conversions (tools/convert.py:73-79,
tests/test_linear.mm:29-37)."""

import json
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

import oracle as O
import oracle.engine as OE
from raceline_amd import lib, rlm
from raceline_amd.model import ModelFile, top_k
from tests import model_files as MF
from tests.golden import writer_case as WC

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _golden_files(w):
    w.begin("files")
    for name, data in WC.FILES.items():
        w.add_file(name, data)
    w.end()


def test_writer_matches_the_reference_writer(tmp_path):
    """rlm.Writer writes, byte for byte, the file tools/convert.py's Writer writes for the same
    calls: every tensor kind, parts, an embedded file section and the header (the length and
    sha256 that tests/golden/make_writer_golden.py recorded from the reference's writer)."""
    import hashlib

    golden = json.load(open(os.path.join(ROOT, "tests", "golden", "writer_golden.json")))
    path = str(tmp_path / "golden.rlm")
    WC.write(rlm.Writer(path), _golden_files)
    data = open(path, "rb").read()
    assert len(data) == golden["bytes"]
    assert hashlib.sha256(data).hexdigest() == golden["sha256"]


def test_layout_counts_what_the_writer_writes(tmp_path):
    """Layout, given a Writer's sequence of calls (native matrices by their sizes only),
    arrives at the Writer's section and tensor tables and its final offset, which is the
    length of the finished file's body."""
    rng = np.random.default_rng(23)
    k = 256
    gate, up = MF.affine_bf16(rng, 200, k), MF.affine_bf16(rng, 56, k)
    rows_q = MF.affine_bf16(rng, 90, 128)
    lm = MF.native(rng, 520, k, "int15")
    tok = MF.native(rng, 33, 64, "fp4")
    wr, lay = rlm.Writer(str(tmp_path / "w.rlm")), rlm.Layout()
    for o in (wr, lay):
        o.begin("tables")
        o.add_rows("tok_affine", *rows_q[:3])
        if o is wr:
            o.add_native_rows("tok_native", *tok, "fp4")
        else:
            o.add_native_rows_layout("tok_native", 33, 64, "fp4")
        o.end()
        for i in range(2):
            o.begin(f"blk.{i}")
            o.add_blocked(f"blk.{i}.ffn", [("gate", gate[:3]), ("up", up[:3])])
            o.add_float(f"blk.{i}.scale", np.full((3, 5), i, np.float32))
            o.add_dense(f"blk.{i}.gate", np.zeros((260, 64), np.float16))
            o.end()
        o.begin("out")
        if o is wr:
            o.add_native("head", [("a", 500), ("b", 20)], *lm, "int15")
        else:
            o.add_native_layout("head", [("a", 500), ("b", 20)], k, "int15")
        o.end()
    assert wr.tensors == lay.tensors
    assert wr.sections == lay.sections
    assert wr.f.tell() == lay.pos
    wr.finish({})
    assert os.path.getsize(str(tmp_path / "w.rlm")) == lay.pos


def test_blocked_packing_matches_the_oracle():
    """The writer's q4a blocks equal the oracle's restatement of tools/convert.py:92-117."""
    rng = np.random.default_rng(1)
    parts = [MF.affine_bf16(rng, rows, 192) for rows in (200, 77, 300)]
    w, s, b, n_pad, spans = rlm.pack_blocked([p[:3] for p in parts])
    ow, os_, ob, on_pad, ospans = O.pack_blocked([(p[0], p[3], p[4]) for p in parts])
    assert n_pad == on_pad == 768
    assert [tuple(x) for x in spans] == [tuple(x) for x in ospans]
    np.testing.assert_array_equal(w, ow)
    np.testing.assert_array_equal(s, os_)
    np.testing.assert_array_equal(b, ob)
    # and back: the oracle's decoder of the blocked layout returns the codes and scales
    q, sb, bb = O.unpack_blocked(w, s, b, n_pad, 192)
    np.testing.assert_array_equal(q[:577], np.concatenate([p[0] for p in parts]))


def test_reader_tables_match_the_writer(tmp_path):
    path = str(tmp_path / "dense.rlm")
    m = MF.write_dense_model(path, seed=3)
    header = _header(path)
    with ModelFile(path) as f:
        assert f.config("hidden_size") == 256 and f.config("vocab_size") == 1000
        assert f.config("num_hidden_layers") == 2 and f.config("intermediate_size") == 512
        assert f.config("block") == 256 and f.config("group") == 64 and f.config("native") == 0
        assert f.config("eos_token_id") == 7 and f.config("num_experts") == 0
        assert f.config("sections") == len(header["sections"]) and f.config("no such key") == -1
        for i, sec in enumerate(header["sections"]):
            assert f.section(i) == (sec["offset"], sec["nbytes"])
            assert sec["offset"] % rlm.PAGE == 0
        for name, t in header["tensors"].items():
            got = f.tensor(name)
            assert got["kind"] == t["kind"] and got["section"] == t["section"]
            if t["kind"] == "f32":
                assert got["w"] == t["offset"] and got["n"] == int(np.prod(t["shape"]))
                continue
            assert (got["k"], got["n"]) == (t["k"], t["n"])
            assert got["w"] == t["w"]
            for fld in ("s", "b", "c"):
                if fld in t:
                    assert got[fld] == t[fld]
            assert got["n_pad"] == t.get("n_pad", t["n"])
            for pn, p in t.get("parts", {}).items():
                assert f.part(name, pn) == (p["offset"], p["n"])
    # the bytes at the offsets are what was written
    raw = np.fromfile(path, np.uint8)
    q, sb, bb, _ = m.affine["layers.1.mlp.down"]
    t = header["tensors"]["layers.1.mlp.down"]
    wb, s_blk, b_blk, n_pad, _ = rlm.pack_blocked([(q, O.bf16_bits_to_f32(sb), O.bf16_bits_to_f32(bb))])
    np.testing.assert_array_equal(raw[t["w"]:t["w"] + wb.size], wb.reshape(-1))
    np.testing.assert_array_equal(raw[t["s"]:t["s"] + 2 * s_blk.size].view(np.uint16), s_blk.reshape(-1))


def test_native_and_moe_files_read(tmp_path):
    for book in ("int15", "fp4"):
        path = str(tmp_path / f"moe_{book}.rlm")
        m = MF.write_moe_model(path, seed=4, native_book=book)
        with ModelFile(path) as f:
            assert f.config("native") == 1 and f.config("num_experts") == 32
            assert f.config("num_experts_per_tok") == 4 and f.config("moe_intermediate_size") == 128
            t = f.tensor("layers.0.moe.gate_up")
            assert t["kind"] == "q4n" and t["n"] == 33 * 256 and t["k"] == 256
            assert t["c"] == t["s"] + 4 * t["n_pad"] + (-(4 * t["n_pad"]) % rlm.ALIGN)
            r = f.tensor("layers.0.moe.router")
            assert r["kind"] == "f16b" and r["n"] == 33 and r["n_pad"] == 256
            assert f.part("layers.0.moe.router", "out") == (0, 33)
        assert m.native["lm_head"][0].shape == (512, 256)


def _header(path):
    with open(path, "rb") as fh:
        assert fh.read(4) == b"RLM1"
        _, n = struct.unpack("<IQ", fh.read(12))
        return json.loads(fh.read(n))


def _rewrite(path, out, hdr=None, patch=None):
    """A copy of a model file with its header replaced (and raw bytes patched)."""
    data = bytearray(open(path, "rb").read())
    if hdr is not None:
        body = json.dumps(hdr, separators=(",", ":")).encode()
        data[4:16] = struct.pack("<IQ", 1, len(body))
        data[16:16 + len(body)] = body
    if patch:
        for off, b in patch:
            data[off:off + len(b)] = b
    open(out, "wb").write(bytes(data))
    return str(out)


def _fails(path, match):
    with pytest.raises(lib.RlqError, match=match):
        ModelFile(path)


def test_reader_fatal_cases(tmp_path):
    good = str(tmp_path / "good.rlm")
    MF.write_dense_model(good, seed=5, layers=1)
    h = _header(good)
    _fails(str(tmp_path / "missing.rlm"), "cannot open")
    _fails(_rewrite(good, tmp_path / "magic.rlm", patch=[(0, b"RLMX")]), "is not a raceline model file")
    open(tmp_path / "short.rlm", "wb").write(b"RLM1")
    _fails(str(tmp_path / "short.rlm"), "is not a raceline model file")
    _fails(_rewrite(good, tmp_path / "hdrlen.rlm", patch=[(8, struct.pack("<Q", 1 << 40))]), "runs past the end")
    _fails(_rewrite(good, tmp_path / "json.rlm", patch=[(16, b"[")]), "not valid JSON")
    bad = json.loads(json.dumps(h))
    del bad["config"]["hidden_size"]
    _fails(_rewrite(good, tmp_path / "cfg.rlm", bad), "missing integer 'hidden_size'")
    bad = json.loads(json.dumps(h))
    bad["config"].update(num_experts=40, num_experts_per_tok=4, moe_intermediate_size=64)
    _fails(_rewrite(good, tmp_path / "moe.rlm", bad), "unsupported mixture of experts: 40 experts")
    bad = json.loads(json.dumps(h))
    bad["quant"]["rotation"] = {"kind": "givens", "block": 64}
    _fails(_rewrite(good, tmp_path / "rot.rlm", bad), "unsupported rotation")
    bad = json.loads(json.dumps(h))
    bad["sections"][-1]["nbytes"] += 1 << 30
    _fails(_rewrite(good, tmp_path / "sec.rlm", bad), "section 'head' runs past the end of the file")
    bad = json.loads(json.dumps(h))
    bad["tensors"]["lm_head"]["w"] = os.path.getsize(good) - 100
    _fails(_rewrite(good, tmp_path / "tensor.rlm", bad), "tensor 'lm_head' reaches past the end")
    bad = json.loads(json.dumps(h))
    bad["tensors"]["lm_head"]["section"] = 99
    _fails(_rewrite(good, tmp_path / "tsec.rlm", bad), "names section 99")
    bad = json.loads(json.dumps(h))
    del bad["quant"]["group"]
    _fails(_rewrite(good, tmp_path / "group.rlm", bad), "missing integer 'group'")
    # float tensor shapes: whole numbers within int range, whose byte count cannot wrap
    f32 = next(n for n, t in h["tensors"].items() if t["kind"] == "f32")
    for i, shape in enumerate(([1 << 31], [2.5], [1 << 20, 1 << 20, 1 << 20, 1 << 10], [-3])):
        bad = json.loads(json.dumps(h))
        bad["tensors"][f32]["shape"] = shape
        _fails(_rewrite(good, tmp_path / f"shape{i}.rlm", bad), f"tensor '{f32}' has a bad shape")
    bad = json.loads(json.dumps(h))
    bad["config"]["hidden_size"] = 1 << 40
    _fails(_rewrite(good, tmp_path / "bigint.rlm", bad), "integer 'hidden_size' is out of range")
    with ModelFile(good) as f:
        with pytest.raises(lib.RlqError, match="model has no tensor 'layers.9.mlp.down'"):
            f.tensor("layers.9.mlp.down")
        with pytest.raises(lib.RlqError, match="quantized tensor has no part 'z'"):
            f.part("layers.0.attn.qkv", "z")


def test_reader_errors_are_fatal_by_default(tmp_path):
    bad = tmp_path / "bad.rlm"
    bad.write_bytes(b"NOPE" + bytes(64))
    code = ("import ctypes, sys; sys.path.insert(0, %r); from raceline_amd import lib; "
            "L = ctypes.CDLL(lib.library_path()); L.rlm_open(%r); print('not reached')") % (ROOT, str(bad).encode())
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1
    assert f"raceline: fatal: {bad} is not a raceline model file" in r.stderr
    assert "not reached" not in r.stdout


def test_rl_open_checks_before_device_work(tmp_path):
    """rl_open refuses an unsupported geometry and a native codebook this build lacks before
    it touches the GPU (src/engine.mm:394-396, :516)."""
    good = str(tmp_path / "good.rlm")
    MF.write_dense_model(good, seed=6, layers=1)
    h = _header(good)
    L = lib.load()
    L.rlq_set_fatal(0)
    bad = json.loads(json.dumps(h))
    bad["config"]["head_dim"] = 128
    assert not L.rl_open(_rewrite(good, tmp_path / "geo.rlm", bad).encode(), 1024, 16)
    assert "unsupported model geometry" in L.rlq_last_error().decode()
    bad = json.loads(json.dumps(h))
    bad["quant"] = {"mode": "native", "bits": 4, "book": "int16", "block": 256}
    assert not L.rl_open(_rewrite(good, tmp_path / "book.rlm", bad).encode(), 1024, 16)
    assert "codebook 'int16' is not supported by this build" in L.rlq_last_error().decode()
    assert not L.rl_open(good.encode(), 1024, 0)
    assert "max_chunk=0" in L.rlq_last_error().decode()


@pytest.mark.parametrize("seed", range(4))
def test_top_k_order(seed):
    """rl_top_k: descending, ties to the lower index, NaN skipped, -inf kept; k > n gives n."""
    rng = np.random.default_rng(seed)
    n = 5000
    x = rng.integers(-20, 20, n).astype(np.float32)      # many ties
    x[rng.random(n) < 0.05] = np.nan
    x[rng.random(n) < 0.02] = -np.inf
    x[7] = np.inf
    x[rng.random(n) < 0.01] = -0.0
    for k in (1, 5, 64, 256, n + 10):
        ids, vals = top_k(x, k)
        rid, rvals = OE.top_k(x, k)
        np.testing.assert_array_equal(ids, rid)
        np.testing.assert_array_equal(vals.view(np.uint32), rvals.view(np.uint32))
    ids, _ = top_k(np.full(10, np.nan, np.float32), 3)
    assert len(ids) == 0


def test_bf16_conversions():
    import torch

    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 10000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -3e-39, 3.4e38], np.float32)]).astype(np.float32)
    # halfway cases: the dropped half exactly 0x8000, both parities of the kept bit
    halves = (np.arange(1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, halves])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(rlm.bf16_rne(x), want)
    assert np.isnan(O.bf16_bits_to_f32(rlm.bf16_rne(np.array([np.nan], np.float32))))
    exact = O.bf16_bits_to_f32(want[np.isfinite(x)])
    np.testing.assert_array_equal(rlm.to_bf16(exact), want[np.isfinite(x)])
    with pytest.raises(ValueError, match="not exactly representable"):
        rlm.to_bf16(np.array([1.0 + 2 ** -10], np.float32), "scales")
