"""Python side of the engine layer (include/rl_engine.h), in the manner of the reference's
ctypes binding (raceline/engine.py:67-125): the .rlm reader and the engine steps over torch
device tensors. Every computation runs in libraceline_amd.so.
"""

from __future__ import annotations

import ctypes
import functools

import torch

from . import lib

KINDS = {1: "q4a", 2: "q4n", 3: "q4a_rows", 4: "q4n_rows", 5: "f16b", 6: "f32"}


class TensorInfo(ctypes.Structure):
    """rlm_tensor_info of include/rl_engine.h."""
    _fields_ = [("kind", ctypes.c_int), ("section", ctypes.c_int), ("k", ctypes.c_int), ("n", ctypes.c_int),
                ("n_pad", ctypes.c_int), ("n_parts", ctypes.c_int), ("w", ctypes.c_uint64), ("s", ctypes.c_uint64),
                ("b", ctypes.c_uint64), ("c", ctypes.c_uint64)]


def _error(what: str) -> lib.RlqError:
    return lib.RlqError(f"{what}: {lib.load().rlq_last_error().decode(errors='replace')}")


def _check(rc: int, what: str):
    if rc != 0:
        raise _error(what)


class ModelFile:
    """A .rlm file through the library's reader (no GPU work)."""

    def __init__(self, path: str):
        L = lib.load()
        L.rlq_set_fatal(0)
        self._h = L.rlm_open(path.encode())
        if not self._h:
            raise _error(f"rlm_open({path})")

    def close(self):
        if self._h:
            lib.load().rlm_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def config(self, key: str) -> int:
        return int(lib.load().rlm_config_int(self._h, key.encode()))

    def tensor(self, name: str) -> dict:
        info = TensorInfo()
        _check(lib.load().rlm_tensor(self._h, name.encode(), ctypes.byref(info)), f"rlm_tensor({name})")
        d = {f: getattr(info, f) for f, _ in TensorInfo._fields_}
        d["kind"] = KINDS[d["kind"]]
        return d

    def part(self, name: str, part: str):
        off, rows = ctypes.c_int(), ctypes.c_int()
        _check(lib.load().rlm_tensor_part(self._h, name.encode(), part.encode(), ctypes.byref(off), ctypes.byref(rows)),
               f"rlm_tensor_part({name}, {part})")
        return off.value, rows.value

    def section(self, i: int):
        off, n = ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib.load().rlm_section(self._h, i, ctypes.byref(off), ctypes.byref(n)), f"rlm_section({i})")
        return off.value, n.value


@functools.lru_cache(maxsize=1)
def _hip():
    h = ctypes.CDLL("libamdhip64.so")
    h.hipMemcpy.restype = ctypes.c_int
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return h


def copy_from_device_ptr(ptr: int, shape, dtype=torch.float32, device="cuda") -> torch.Tensor:
    """A torch copy of device memory the engine owns (its logits)."""
    out = torch.empty(shape, dtype=dtype, device=device)
    torch.cuda.current_stream().synchronize()
    rc = _hip().hipMemcpy(out.data_ptr(), ptr, out.numel() * out.element_size(), 3)   # device to device
    if rc != 0:
        raise RuntimeError(f"hipMemcpy failed ({rc})")
    return out


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class Engine:
    """rl_open / rl_close and the engine steps (include/rl_engine.h)."""

    def __init__(self, path: str, max_ctx: int = 4096, max_chunk: int = 64):
        L = lib.load()
        L.rlq_set_fatal(0)
        self._e = L.rl_open(path.encode(), max_ctx, max_chunk)
        if not self._e:
            raise _error(f"rl_open({path})")
        self.max_chunk = max_chunk

    def close(self):
        if self._e:
            lib.load().rl_close(self._e)
            self._e = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def vocab(self) -> int:
        return int(lib.load().rl_vocab(self._e))

    @property
    def hidden_size(self) -> int:
        return int(lib.load().rl_hidden_size(self._e))

    @property
    def logits_stride(self) -> int:
        return int(lib.load().rl_logits_stride(self._e))

    def linear(self, name: str, x: torch.Tensor, out: torch.Tensor | None = None, accum: bool = False,
               part: str | None = None, n: int | None = None) -> torch.Tensor:
        """out (+)= x W^T for the model's tensor `name` (or one part); x fp16 [rows][>= k]."""
        rows = x.shape[0]
        if out is None:
            out = torch.zeros((rows, n), dtype=torch.float32, device=x.device)
        _check(lib.load().rl_linear(self._e, name.encode(), part.encode() if part else None, x.data_ptr(), x.stride(0),
                                    rows, out.data_ptr(), out.stride(0), 1 if accum else 0, _stream()),
               f"rl_linear({name})")
        return out

    def norm(self, which: int, layer: int, h: torch.Tensor) -> torch.Tensor:
        xn = torch.empty((h.shape[0], self.hidden_size), dtype=torch.float16, device=h.device)
        _check(lib.load().rl_norm(self._e, which, layer, h.data_ptr(), h.stride(0), h.shape[0], xn.data_ptr(),
                                  xn.stride(0), _stream()), "rl_norm")
        return xn

    def mlp(self, layer: int, h: torch.Tensor) -> torch.Tensor:
        _check(lib.load().rl_mlp(self._e, layer, h.data_ptr(), h.stride(0), h.shape[0], _stream()), "rl_mlp")
        return h

    def head(self, h: torch.Tensor) -> torch.Tensor:
        """Logits of the rows of h: [rows][logits_stride] (a copy of the engine's)."""
        ptr = lib.load().rl_head(self._e, h.data_ptr(), h.stride(0), h.shape[0], _stream())
        if not ptr:
            raise _error("rl_head")
        return copy_from_device_ptr(ptr, (h.shape[0], self.logits_stride), device=h.device)

    def set_draft_vocab(self, rows: int):
        lib.load().rl_set_draft_vocab(self._e, rows)

    def set_draft_tail(self, first: int):
        lib.load().rl_set_draft_tail(self._e, first)

    @property
    def draft_main(self) -> int:
        return int(lib.load().rl_draft_main(self._e))

    @property
    def draft_tail(self) -> int:
        return int(lib.load().rl_draft_tail(self._e))

    @property
    def draft_vocab(self) -> int:
        return int(lib.load().rl_draft_vocab(self._e))

    def expert_cache(self):
        """(slots, hits, loads) of the expert cache, or None when every expert is in memory
        (raceline/engine.py:262-267); this engine keeps them all in HBM."""
        hits, loads = ctypes.c_ulonglong(), ctypes.c_ulonglong()
        slots = lib.load().rl_expert_cache(self._e, ctypes.byref(hits), ctypes.byref(loads))
        return (slots, hits.value, loads.value) if slots else None

    def expert_cache_size(self):
        """(GB the cache holds, share of the experts that fit in it), or None when every
        expert is in memory (raceline/engine.py:269-276)."""
        slots = lib.load().rl_expert_cache(self._e, None, None)
        if not slots:
            return None
        n, size = ctypes.c_int(), ctypes.c_ulonglong()
        lib.load().rl_expert_cache_size(self._e, ctypes.byref(n), ctypes.byref(size))
        return slots * size.value / 1e9, slots / max(1, n.value)

    def draft_head(self, h_row: torch.Tensor) -> torch.Tensor:
        ptr = lib.load().rl_draft_head(self._e, h_row.data_ptr(), _stream())
        if not ptr:
            raise _error("rl_draft_head")
        return copy_from_device_ptr(ptr, (self.draft_vocab,), device=h_row.device)

    def top_k_device(self, logits: torch.Tensor, k: int):
        ids = (ctypes.c_int32 * max(k, 1))()
        vals = (ctypes.c_float * max(k, 1))()
        got = lib.load().rl_top_k_device(self._e, logits.data_ptr(), logits.numel(), k, ids, vals, _stream())
        if got < 0:
            raise _error("rl_top_k_device")
        return list(ids[:got]), list(vals[:got])

    def argmax(self) -> int:
        return int(lib.load().rl_argmax(self._e))


def top_k(logits, k: int):
    """rl_top_k on host floats (a numpy array or a CPU tensor)."""
    import numpy as np

    x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
    ids = np.zeros(max(k, 1), np.int32)
    vals = np.zeros(max(k, 1), np.float32)
    got = lib.load().rl_top_k(x.ctypes.data, x.size, k, ids.ctypes.data, vals.ctypes.data)
    return ids[:got], vals[:got]
