"""Writer of .rlm model files, the format the engine's reader (csrc/model_file.cpp) maps.

The reference writes this format with tools/convert.py (affine files, :128-296) and
tools/quantize.py (native files); this module produces the same bytes from numpy arrays:

  file    = "RLM1" | u32 version (1) | u64 header length | JSON header | sections
  header  = {..meta.., "sections": [{name, offset, nbytes}], "tensors": {name: {...}},
             "files": {...}}, written compactly at the end into the first 64 pages
  section = page-aligned (16384) run of 128-byte-aligned blobs

Tensor kinds (the table entries' fields are absolute file offsets):
  q4a       affine 4-bit, blocked: w bytes [n_pad/256][K][128] (row 2j in the low nibble,
            tools/convert.py:92-117), s and b bf16 bits [n_pad/256][K/64][256]; parts
  q4n       native 4-bit, blocked codes as q4a, s fp32 [n_pad] (padding rows 0), c fp32 [K]
  q4a_rows  affine row-major (token tables): w [n][K/2], s, b bf16 [n][K/64]
  q4n_rows  native row-major: w [n][K/2], s fp32 [n], c fp32 [K]
  f16b      half [n_pad/256][K][256], rows padded with zeros; one part "out"
  f32       float32 vector or matrix, with its shape

`Layout` computes where a Writer would put everything without writing: replaying a
conversion's calls on it rebuilds the tensor table of a file whose header was never
written (what tools/quantize.py --resume relies on).
"""

from __future__ import annotations

import json
import struct

import numpy as np

PAGE = 16384        # section alignment (tools/convert.py:30)
ALIGN = 128         # blob alignment (:31)
BLOCK = 256         # rows per block of the blocked layouts (:32)
GROUP = 64          # affine quantization group (:33)
MAGIC = b"RLM1"
VERSION = 1
HEADER_PAGES = 64   # room reserved for the header before the first section


# ------------------------------------------------------------------ number formats

def to_bf16(x, what: str = "values") -> np.ndarray:
    """float32 -> bfloat16 bits, which must be exact: the affine scales and biases of an MLX
    checkpoint are bfloat16 values read as float32 (tools/convert.py:73-79). Raises
    ValueError when any value would round."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    if np.any(bits & np.uint32(0xFFFF)):
        raise ValueError(f"{what}: not exactly representable in bfloat16")
    return (bits >> np.uint32(16)).astype(np.uint16)


def bf16_rne(x) -> np.ndarray:
    """float32 -> bfloat16 bits rounded to nearest, ties to even (the rounding
    tests/test_linear.mm:29-37 uses for scales it draws). NaN stays a quiet NaN."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (bits >> np.uint64(16)) & np.uint64(1)
    rounded = ((bits + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, ((bits >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16), rounded)


def unpack_nibbles(w_u32) -> np.ndarray:
    """MLX codes [N][K/8] uint32 (element i in bits 4i..4i+3, little endian) -> [N][K] uint8."""
    w = np.ascontiguousarray(w_u32, dtype=np.uint32)
    by = w.view(np.uint8).reshape(w.shape[0], -1)
    return np.stack([by & 0x0F, by >> 4], axis=-1).reshape(w.shape[0], -1)


def _blocked_nibbles(q: np.ndarray) -> np.ndarray:
    """[n_pad][K] codes -> [n_pad/256][K][128] bytes: byte j of input k holds rows 2j (low
    nibble) and 2j+1 (high nibble) of the block."""
    n_pad, k = q.shape
    per_block = q.reshape(n_pad // BLOCK, BLOCK // 2, 2, k)          # [b][j][row parity][k]
    packed = per_block[:, :, 0, :] | (per_block[:, :, 1, :] << 4)    # [b][j][k]
    return np.ascontiguousarray(packed.transpose(0, 2, 1).astype(np.uint8))


def _block_columns(m: np.ndarray) -> np.ndarray:
    """[n_pad][C] per-row values -> [n_pad/256][C][256] (a block's rows become columns)."""
    n_pad, c = m.shape
    return np.ascontiguousarray(m.reshape(n_pad // BLOCK, BLOCK, c).transpose(0, 2, 1))


def _rows_pad(n: int) -> int:
    return -(-n // BLOCK) * BLOCK


def pack_blocked(parts):
    """Affine matrices sharing K, stacked in order: parts = [(q [N][K] uint8, s [N][K/64],
    b [N][K/64])] with s and b float32 bfloat16 values. Returns (w, s_bits, b_bits, n_pad,
    [(first row, rows)])."""
    k = parts[0][0].shape[1]
    rows = [p[0].shape[0] for p in parts]
    n = sum(rows)
    n_pad = _rows_pad(n)
    q = np.zeros((n_pad, k), np.uint8)
    s = np.zeros((n_pad, k // GROUP), np.uint16)
    b = np.zeros((n_pad, k // GROUP), np.uint16)
    spans, r0 = [], 0
    for (qp, sp, bp), r in zip(parts, rows):
        q[r0:r0 + r] = qp
        s[r0:r0 + r] = to_bf16(sp, "scales")
        b[r0:r0 + r] = to_bf16(bp, "biases")
        spans.append((r0, r))
        r0 += r
    return _blocked_nibbles(q), _block_columns(s), _block_columns(b), n_pad, spans


def pack_rows(q, s, b):
    """Row-major affine matrix (token tables): two codes per byte, even one low."""
    q = np.asarray(q, np.uint8)
    return (np.ascontiguousarray(q[:, 0::2] | (q[:, 1::2] << 4)), to_bf16(s, "scales"), to_bf16(b, "biases"))


# ------------------------------------------------------------------ placement

class _Placement:
    """The section and tensor tables and where each blob goes, shared by Writer (which
    writes the bytes) and Layout (which only counts them): subclasses define _pad(align) ->
    the aligned position, and _emit(array or byte count)."""

    def _init_tables(self):
        self.tensors, self.sections, self.files = {}, [], {}
        self._sec = None

    def blob(self, arr) -> int:
        off = self._pad(ALIGN)
        self._emit(arr)
        return off

    def begin(self, name: str):
        self._sec = {"name": name, "offset": self._pad(PAGE)}

    def end(self):
        stop = self._pad(PAGE)
        self._sec["nbytes"] = stop - self._sec["offset"]
        self.sections.append(self._sec)
        self._sec = None

    def _section(self) -> int:
        return len(self.sections)

    @staticmethod
    def _parts(named_rows):
        out, r0 = {}, 0
        for pn, r in named_rows:
            out[pn] = {"offset": r0, "n": r}
            r0 += r
        return out

    def add_float(self, name, arr):
        a = np.ascontiguousarray(arr, dtype=np.float32)
        self.tensors[name] = {"kind": "f32", "section": self._section(), "shape": list(a.shape), "offset": self.blob(a)}

    def add_blocked(self, name, named_parts):
        """Affine matrices stacked as one q4a tensor: named_parts = [(part name, (q, s, b))]."""
        self.add_blocked_packed(name, [pn for pn, _ in named_parts], pack_blocked([p for _, p in named_parts]))

    def add_blocked_packed(self, name, part_names, packed):
        """A q4a tensor from what pack_blocked returned, (w, s, b, n_pad, spans), with the
        parts' names: the same entry and bytes as add_blocked, without packing again (a
        tensor written to several places or files is packed once)."""
        w, s, b, n_pad, spans = packed
        entry = {"kind": "q4a", "section": self._section(), "k": int(w.shape[1]), "n": sum(r for _, r in spans),
                 "n_pad": n_pad}
        entry["w"] = self.blob(w)
        entry["s"] = self.blob(s)
        entry["b"] = self.blob(b)
        entry["parts"] = {pn: {"offset": o, "n": r} for pn, (o, r) in zip(part_names, spans)}
        self.tensors[name] = entry

    def add_native(self, name, named_parts, codes, s, c, book):
        """A native matrix [N][K]: codes (one per weight, 0..15), row scales s [N] and column
        scales c [K]; rows padded to a block with scale 0. named_parts = [(name, rows)]."""
        codes = np.asarray(codes, np.uint8)
        n, k = codes.shape
        n_pad = _rows_pad(n)
        q = np.zeros((n_pad, k), np.uint8)
        q[:n] = codes
        s_pad = np.zeros(n_pad, np.float32)
        s_pad[:n] = s
        entry = {"kind": "q4n", "section": self._section(), "book": book, "k": k, "n": n, "n_pad": n_pad}
        entry["w"] = self.blob(_blocked_nibbles(q))
        entry["s"] = self.blob(s_pad)
        entry["c"] = self.blob(np.asarray(c, np.float32))
        entry["parts"] = self._parts(named_parts)
        self.tensors[name] = entry

    def add_native_layout(self, name, named_parts, k, book):
        """The table entry add_native would make, its blobs only reserved."""
        n = sum(r for _, r in named_parts)
        n_pad = _rows_pad(n)
        entry = {"kind": "q4n", "section": self._section(), "book": book, "k": k, "n": n, "n_pad": n_pad}
        entry["w"] = self.blob(n_pad * k // 2)
        entry["s"] = self.blob(4 * n_pad)
        entry["c"] = self.blob(4 * k)
        entry["parts"] = self._parts(named_parts)
        self.tensors[name] = entry

    def add_dense(self, name, W):
        """Half-precision matrix [N][K] (the MoE router), blocked, rows padded with zeros."""
        W = np.asarray(W)
        n, k = W.shape
        n_pad = _rows_pad(n)
        full = np.zeros((n_pad, k), np.float16)
        full[:n] = W
        entry = {"kind": "f16b", "section": self._section(), "k": k, "n": n, "n_pad": n_pad}
        entry["w"] = self.blob(_block_columns(full))
        entry["parts"] = {"out": {"offset": 0, "n": n}}
        self.tensors[name] = entry

    def add_native_rows(self, name, codes, s, c, book):
        """Row-major native matrix (token tables)."""
        codes = np.asarray(codes, np.uint8)
        entry = {"kind": "q4n_rows", "section": self._section(), "book": book, "k": codes.shape[1], "n": codes.shape[0]}
        entry["w"] = self.blob(np.ascontiguousarray(codes[:, 0::2] | (codes[:, 1::2] << 4)))
        entry["s"] = self.blob(np.asarray(s, np.float32))
        entry["c"] = self.blob(np.asarray(c, np.float32))
        self.tensors[name] = entry

    def add_native_rows_layout(self, name, n, k, book):
        entry = {"kind": "q4n_rows", "section": self._section(), "book": book, "k": k, "n": n}
        entry["w"] = self.blob(n * k // 2)
        entry["s"] = self.blob(4 * n)
        entry["c"] = self.blob(4 * k)
        self.tensors[name] = entry

    def add_rows(self, name, q, s, b):
        """Row-major affine matrix (token tables)."""
        w, s16, b16 = pack_rows(q, s, b)
        entry = {"kind": "q4a_rows", "section": self._section(), "k": int(np.asarray(q).shape[1]),
                 "n": int(np.asarray(q).shape[0])}
        entry["w"] = self.blob(w)
        entry["s"] = self.blob(s16)
        entry["b"] = self.blob(b16)
        self.tensors[name] = entry

    def add_file(self, name: str, data: bytes):
        """An embedded file (tokenizer, chat template), in the current section."""
        arr = np.frombuffer(data, np.uint8)
        self.files[name] = {"offset": self.blob(arr), "nbytes": int(arr.size)}


class Writer(_Placement):
    """Writes a .rlm file: begin(section) ... add_*() ... end(), then finish(meta)."""

    def __init__(self, path: str):
        self.f = open(path, "wb")
        self.header_room = HEADER_PAGES * PAGE
        self.f.write(bytes(self.header_room))
        self._init_tables()

    def _pad(self, align: int) -> int:
        pos = self.f.tell()
        gap = -pos % align
        if gap:
            self.f.write(bytes(gap))
        return pos + gap

    def _emit(self, arr):
        if isinstance(arr, (int, np.integer)):        # a reserved blob: zeros
            self.f.write(bytes(int(arr)))
        else:
            self.f.write(np.ascontiguousarray(arr).tobytes())

    def finish(self, meta: dict):
        hdr = json.dumps(dict(meta, sections=self.sections, tensors=self.tensors, files=self.files),
                         separators=(",", ":")).encode()
        if 16 + len(hdr) > self.header_room:
            raise ValueError(f"the {16 + len(hdr)}-byte header is larger than the {self.header_room} bytes kept "
                             f"for it at the start of the file")
        self.f.seek(0)
        self.f.write(MAGIC + struct.pack("<IQ", VERSION, len(hdr)) + hdr)
        self.f.close()


class Layout(_Placement):
    """The placement a Writer makes for the same calls, counted only: no bytes are written."""

    def __init__(self):
        self.header_room = HEADER_PAGES * PAGE
        self.pos = self.header_room
        self._init_tables()

    def _pad(self, align: int) -> int:
        self.pos += -self.pos % align
        return self.pos

    def _emit(self, arr):
        self.pos += int(arr) if isinstance(arr, (int, np.integer)) else np.asarray(arr).nbytes


def affine_meta(config: dict, scale_dtype: str = "bf16") -> dict:
    """The header fields of an affine file (tools/convert.py:291-292)."""
    return dict(format="raceline", version=VERSION, arch="qwen3_5", config=config,
                quant=dict(bits=4, group=GROUP, block=BLOCK, mode="affine", scale_dtype=scale_dtype))


def native_meta(config: dict, book: str) -> dict:
    """The header fields of a native file (tools/quantize.py:705-709 writes version 2, quant
    mode "native" with its codebook)."""
    return dict(format="raceline", version=2, arch="qwen3_5", config=config,
                quant=dict(mode="native", bits=4, book=book, block=BLOCK))
