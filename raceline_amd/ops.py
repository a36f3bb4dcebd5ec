"""Torch-facing host layer over the C ABI: the quantized linear of raceline's engine.

Mirrors what Engine::encode_linear does for one QTensor (src/engine.mm:832-906): pick
the kernel for the row count, bind the activations, the packed weight and the output,
and run it with ACCUM for the residual writers. Tensors are torch CUDA tensors (HBM
plumbing only); every computation runs in libraceline_amd.so.

Weights arrive in one of the reference's layouts (the MLX u32 layout of the BASELINE
configs and tools/convert.py:82-89, or the blocked q4a layout of .rlm files,
tools/convert.py:92-117) and are packed once, on the device, into the layout the kernels
stream (see include/rlq.h); the dequantized value of every weight is unchanged.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass, field

import torch

from . import lib

GROUP = 64
F16, BF16 = 0, 1
KERNEL_AUTO, KERNEL_GEMV, KERNEL_GEMM = 0, 1, 2
GEMV_MAX_M = 8


def _ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def scale_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return F16
    if dtype == torch.bfloat16:
        return BF16
    raise ValueError(f"scales must be float16 or bfloat16, not {dtype}")


def packed_bytes(K: int, N: int) -> int:
    return int(lib.load().rlq_packed_affine_bytes(K, N))


@dataclass
class PackedWeight:
    """A 4-bit affine matrix [N][K] in the packed device layout, with the dtype of its
    16-bit scales and biases. Like the reference's QTensor (src/model_file.h:44-55) it
    may name the row ranges of stacked parts."""
    packed: torch.Tensor            # uint8, rlq_packed_affine_bytes(K, N) bytes
    K: int
    N: int
    scale_dtype: torch.dtype = torch.float16
    parts: dict = field(default_factory=dict)

    def __post_init__(self):
        if self.packed.dtype != torch.uint8 or not self.packed.is_contiguous():
            raise TypeError("packed weight must be a contiguous uint8 tensor")
        if self.packed.numel() < packed_bytes(self.K, self.N):
            raise ValueError("packed buffer is smaller than the layout needs")

    @property
    def code(self) -> int:
        return scale_code(self.scale_dtype)


def _check_mlx(w: torch.Tensor, s: torch.Tensor, b: torch.Tensor):
    if w.dtype not in (torch.int32, torch.uint32) or w.dim() != 2:
        raise TypeError("codes must be 32-bit words [N][K/8]")
    N, K8 = w.shape
    if s.shape != (N, K8 * 8 // GROUP) or b.shape != s.shape:
        raise ValueError(f"scales/biases {tuple(s.shape)} do not match codes {tuple(w.shape)}")
    if s.dtype != b.dtype:
        raise TypeError("scales and biases must share a dtype")
    for t in (w, s, b):
        if not t.is_contiguous():
            raise ValueError("weight tensors must be contiguous")
    return N, K8 * 8


def pack_affine(w: torch.Tensor, s: torch.Tensor, b: torch.Tensor, stream=None) -> PackedWeight:
    """MLX layout (codes [N][K/8] 32-bit words, scales and biases [N][K/64]) -> PackedWeight."""
    N, K = _check_mlx(w, s, b)
    out = torch.empty(packed_bytes(K, N), dtype=torch.uint8, device=w.device)
    lib.call("rlq_pack_affine", _ptr(w), _ptr(s), _ptr(b), K, N, _ptr(out), _stream(stream))
    return PackedWeight(out, K, N, s.dtype)


def pack_blocked(w_blk: torch.Tensor, s_blk: torch.Tensor, b_blk: torch.Tensor, K: int, n_pad: int, row0: int,
                 rows: int, scale_dtype: torch.dtype = torch.bfloat16, stream=None) -> PackedWeight:
    """Rows [row0, row0 + rows) of a blocked q4a tensor of a .rlm file (already in device
    memory) -> PackedWeight."""
    out = torch.empty(packed_bytes(K, rows), dtype=torch.uint8, device=w_blk.device)
    lib.call("rlq_pack_affine_blocked", _ptr(w_blk), _ptr(s_blk), _ptr(b_blk), K, n_pad, row0, rows, _ptr(out),
             _stream(stream))
    return PackedWeight(out, K, rows, scale_dtype)


def repack_blocked(w_blk: torch.Tensor, s_blk: torch.Tensor, b_blk: torch.Tensor, K: int, n_pad: int,
                   row0: int, rows: int, scale_dtype: torch.dtype = torch.bfloat16, stream=None):
    """Blocked q4a rows -> MLX layout tensors (w int32 [rows][K/8], s, b [rows][K/64])."""
    dev = w_blk.device
    w = torch.empty((rows, K // 8), dtype=torch.int32, device=dev)
    s = torch.empty((rows, K // GROUP), dtype=scale_dtype, device=dev)
    b = torch.empty((rows, K // GROUP), dtype=scale_dtype, device=dev)
    lib.call("rlq_repack_blocked", _ptr(w_blk), _ptr(s_blk), _ptr(b_blk), K, n_pad, row0, rows, _ptr(w), _ptr(s),
             _ptr(b), _stream(stream))
    return w, s, b


BOOKS = {"int15": 1, "int16": 2, "fp4": 3}   # native codebooks (include/rlq.h RLQ_BOOK_*)


@dataclass
class NativeWeight:
    """A native 4-bit matrix [N][K]: codebook codes in the packed tile layout (no
    scale/bias section) and one fp32 scale per row. The column scale belongs to the
    producer of the activations (it is folded into x before the product)."""
    packed: torch.Tensor     # uint8, rlq_packed_codes_bytes(K, N)
    s_row: torch.Tensor      # float32 [N]
    K: int
    N: int
    book: str

    @property
    def code(self) -> int:
        return BOOKS[self.book]


def _native_rows(s_row, N, book):
    if book not in BOOKS:
        raise ValueError(f"unknown codebook {book!r}")
    if s_row.dtype != torch.float32 or s_row.dim() != 1 or s_row.numel() < N or not s_row.is_contiguous():
        raise ValueError("s_row must be a contiguous float32 vector of >= N row scales")


def pack_native(w: torch.Tensor, s_row: torch.Tensor, book: str, stream=None) -> NativeWeight:
    """Row-major codes (32-bit words [N][K/8], element k at bits 4*(k%8)) -> NativeWeight."""
    if w.dtype not in (torch.int32, torch.uint32) or w.dim() != 2 or not w.is_contiguous():
        raise TypeError("codes must be contiguous 32-bit words [N][K/8]")
    N, K = w.shape[0], w.shape[1] * 8
    _native_rows(s_row, N, book)
    out = torch.empty(int(lib.load().rlq_packed_codes_bytes(K, N)), dtype=torch.uint8, device=w.device)
    lib.call("rlq_pack_codes", _ptr(w), K, N, _ptr(out), _stream(stream))
    return NativeWeight(out, s_row[:N], K, N, book)


def pack_native_blocked(w_blk: torch.Tensor, s_pad: torch.Tensor, K: int, n_pad: int, row0: int, rows: int, book: str,
                        stream=None) -> NativeWeight:
    """Rows [row0, row0 + rows) of a blocked q4n tensor (with its padded row scales) -> NativeWeight."""
    _native_rows(s_pad, row0 + rows, book)
    out = torch.empty(int(lib.load().rlq_packed_codes_bytes(K, rows)), dtype=torch.uint8, device=w_blk.device)
    lib.call("rlq_pack_native_blocked", _ptr(w_blk), K, n_pad, row0, rows, _ptr(out), _stream(stream))
    return NativeWeight(out, s_pad[row0:row0 + rows].contiguous(), K, rows, book)


def linear_native(x: torch.Tensor, nw: NativeWeight, out: torch.Tensor | None = None, accum: bool = False,
                  kernel: int = KERNEL_AUTO, stream=None) -> torch.Tensor:
    """out[m][n] (+)= s[n] * sum_k x[m][k] * L[q[n][k]] for fp16 x (column scale already applied)."""
    if x.dtype != torch.float16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a row-major float16 matrix")
    M, K, N = x.shape[0], nw.K, nw.N
    if x.shape[1] < K:
        raise ValueError(f"x has {x.shape[1]} columns, the weight needs {K}")
    if out is None:
        if accum:
            raise ValueError("accum needs an output to add into")
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    if out.dtype != torch.float32 or out.stride(1) != 1 or out.shape[0] < M or out.shape[1] < N:
        raise ValueError("out must be a row-major float32 [M][>=N] matrix")
    nbytes = workspace_bytes(M, K, N)
    ws = _WS.get(x.device, nbytes)
    lib.call("rlq_linear_native_kernel", kernel, _ptr(x), x.stride(0), M, K, N, _ptr(nw.packed), _ptr(nw.s_row),
             nw.code, _ptr(out), out.stride(0), 1 if accum else 0, _ptr(ws), 0 if ws is None else ws.numel(),
             _stream(stream))
    return out


def linear_native_raw(x: torch.Tensor, nw: NativeWeight, out: torch.Tensor | None = None,
                      kernel_stream=None) -> torch.Tensor:
    """out[m][n] = sum_k x[m][k] * L[q[n][k]]: the native product without the row scale
    (rlq_linear_native_raw; int15 and fp4 only)."""
    if x.dtype != torch.float16 or x.dim() != 2 or x.stride(1) != 1 or x.shape[1] < nw.K:
        raise ValueError("x must be a row-major float16 [M][>= K] matrix")
    M, K, N = x.shape[0], nw.K, nw.N
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    ws = _WS.get(x.device, workspace_bytes(M, K, N))
    lib.call("rlq_linear_native_raw", _ptr(x), x.stride(0), M, K, N, _ptr(nw.packed), nw.code, _ptr(out),
             out.stride(0), _ptr(ws), 0 if ws is None else ws.numel(), _stream(kernel_stream))
    return out


@dataclass
class DenseWeight:
    """A half-precision matrix [N][K] in MFMA operand order (rlq_pack_f16)."""
    packed: torch.Tensor
    K: int
    N: int


def pack_f16(w: torch.Tensor, stream=None) -> DenseWeight:
    if w.dtype != torch.float16 or w.dim() != 2 or not w.is_contiguous():
        raise TypeError("w must be a contiguous float16 [N][K] matrix")
    N, K = w.shape
    out = torch.empty(int(lib.load().rlq_packed_f16_bytes(K, N)), dtype=torch.uint8, device=w.device)
    lib.call("rlq_pack_f16", _ptr(w), K, N, _ptr(out), _stream(stream))
    return DenseWeight(out, K, N)


def pack_f16_blocked(w_blk: torch.Tensor, K: int, n_pad: int, row0: int, rows: int, stream=None) -> DenseWeight:
    out = torch.empty(int(lib.load().rlq_packed_f16_bytes(K, rows)), dtype=torch.uint8, device=w_blk.device)
    lib.call("rlq_pack_f16_blocked", _ptr(w_blk), K, n_pad, row0, rows, _ptr(out), _stream(stream))
    return DenseWeight(out, K, rows)


def linear_f16(x: torch.Tensor, dw: DenseWeight, out: torch.Tensor | None = None, accum: bool = False,
               stream=None) -> torch.Tensor:
    if x.dtype != torch.float16 or x.dim() != 2 or x.stride(1) != 1 or x.shape[1] < dw.K:
        raise ValueError("x must be a row-major float16 [M][>= K] matrix")
    M = x.shape[0]
    if out is None:
        if accum:
            raise ValueError("accum needs an output to add into")
        out = torch.empty((M, dw.N), dtype=torch.float32, device=x.device)
    lib.call("rlq_linear_f16", _ptr(x), x.stride(0), M, dw.K, dw.N, _ptr(dw.packed), _ptr(out), out.stride(0),
             1 if accum else 0, _stream(stream))
    return out


class _Workspaces:
    """One scratch buffer per device, grown on demand, zero-filled when allocated (the
    decode kernel keeps its split counters at the start of the linear workspace and leaves
    them zero after every call; nothing else is kept between calls). Calls that use it
    must not overlap on two streams of one device."""

    def __init__(self):
        self._bufs = {}
        self._lock = threading.Lock()

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        key = device.index if device.index is not None else torch.cuda.current_device()
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf


_WS = _Workspaces()


def workspace_bytes(M: int, K: int, N: int) -> int:
    return int(lib.load().rlq_linear_workspace_bytes(M, K, N))


def linear(x: torch.Tensor, pw: PackedWeight, out: torch.Tensor | None = None, accum: bool = False,
           kernel: int = KERNEL_AUTO, stream=None) -> torch.Tensor:
    """out[m][n] (+)= sum_k x[m][k] * W[n][k] for fp16 x [M][>=K] (row stride x.stride(0))."""
    if x.dtype != torch.float16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a row-major float16 matrix")
    M, K, N = x.shape[0], pw.K, pw.N
    if x.shape[1] < K:
        raise ValueError(f"x has {x.shape[1]} columns, the weight needs {K}")
    if out is None:
        if accum:
            raise ValueError("accum needs an output to add into")
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    if out.dtype != torch.float32 or out.stride(1) != 1 or out.shape[0] < M or out.shape[1] < N:
        raise ValueError("out must be a row-major float32 [M][>=N] matrix")
    nbytes = workspace_bytes(M, K, N)
    ws = _WS.get(x.device, nbytes)
    lib.call("rlq_linear_affine_kernel", kernel, _ptr(x), x.stride(0), M, K, N, _ptr(pw.packed), pw.code,
             _ptr(out), out.stride(0), 1 if accum else 0, _ptr(ws), 0 if ws is None else ws.numel(),
             _stream(stream))
    return out


def group_sums(x: torch.Tensor, K: int | None = None, stream=None) -> torch.Tensor:
    K = x.shape[1] if K is None else K
    out = torch.empty((x.shape[0], K // GROUP), dtype=torch.float32, device=x.device)
    lib.call("rlq_group_sums", _ptr(x), x.stride(0), x.shape[0], K, _ptr(out), _stream(stream))
    return out


def dequant(pw: PackedWeight, stream=None) -> torch.Tensor:
    out = torch.empty((pw.N, pw.K), dtype=torch.float32, device=pw.packed.device)
    lib.call("rlq_dequant_affine", _ptr(pw.packed), pw.code, pw.K, pw.N, _ptr(out), _stream(stream))
    return out


# ------------------------------------------------------------------ mixture of experts

@dataclass
class MoeWeights:
    """The expert stacks of one MoE MLP (E routed experts + the shared one, number E):
    gate_up packed with gate/up rows interleaved per tile (K = H, N = (E+1)*2I) and down
    packed plainly (K = I, N = (E+1)*H)."""
    gate_up: PackedWeight
    down: PackedWeight
    E: int
    H: int
    I: int


def pack_moe(gu: tuple, dn: tuple, E: int, H: int, I: int, stream=None) -> MoeWeights:
    """MLX-layout stacks -> MoeWeights. gu = (w [(E+1)*2I][H/8], s, b [(E+1)*2I][H/64]);
    dn = (w [(E+1)*H][I/8], s, b [(E+1)*H][I/64])."""
    gw, gs, gb = gu
    N, K = _check_mlx(gw, gs, gb)
    if (N, K) != ((E + 1) * 2 * I, H):
        raise ValueError(f"gate/up stack is [{N}][{K}], expected [{(E + 1) * 2 * I}][{H}]")
    out = torch.empty(packed_bytes(H, N), dtype=torch.uint8, device=gw.device)
    lib.call("rlq_pack_moe_gate_up", _ptr(gw), _ptr(gs), _ptr(gb), H, E + 1, I, _ptr(out), _stream(stream))
    g = PackedWeight(out, H, N, gs.dtype)
    d = pack_affine(*dn, stream=stream)
    if (d.N, d.K) != ((E + 1) * H, I):
        raise ValueError(f"down stack is [{d.N}][{d.K}], expected [{(E + 1) * H}][{I}]")
    return MoeWeights(g, d, E, H, I)


@dataclass
class MoeRouting:
    sel: torch.Tensor       # int32 [T*S]
    w: torch.Tensor         # float32 [T*S]
    tok: torch.Tensor       # int32 [T*S]: token of each sorted row
    inv: torch.Tensor       # int32 [T*S]: sorted row of each assignment
    items: torch.Tensor     # int32 [max_items][4]
    n_items: torch.Tensor   # int32 [1]
    T: int
    topk: int


def moe_route(logits: torch.Tensor, E: int, topk: int, norm_topk: bool = True, stream=None) -> MoeRouting:
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1 or logits.shape[1] < E + 1:
        raise ValueError("logits must be a row-major float32 [T][>= E+1] matrix")
    T = logits.shape[0]
    A = T * (topk + 1)
    dev = logits.device
    mi = int(lib.load().rlq_moe_max_items(T, E, topk))
    r = MoeRouting(torch.empty(A, dtype=torch.int32, device=dev), torch.empty(A, dtype=torch.float32, device=dev),
                   torch.empty(A, dtype=torch.int32, device=dev), torch.empty(A, dtype=torch.int32, device=dev),
                   torch.empty((max(mi, 1), 4), dtype=torch.int32, device=dev),
                   torch.empty(1, dtype=torch.int32, device=dev), T, topk)
    lib.call("rlq_moe_route", _ptr(logits), logits.stride(0), T, E, topk, 1 if norm_topk else 0, _ptr(r.sel), _ptr(r.w),
             _ptr(r.tok), _ptr(r.inv), _ptr(r.items), _ptr(r.n_items), _stream(stream))
    return r


def moe_gate_up(x: torch.Tensor, mw: MoeWeights, r: MoeRouting, stream=None) -> torch.Tensor:
    """act fp16 [T*S][I]: SwiGLU of the routed rows' gate/up products (sorted row order)."""
    if x.dtype != torch.float16 or x.dim() != 2 or x.stride(1) != 1 or x.shape[1] < mw.H:
        raise ValueError("x must be a row-major float16 [T][>= H] matrix")
    act = torch.empty((r.T * (r.topk + 1), mw.I), dtype=torch.float16, device=x.device)
    lib.call("rlq_moe_gate_up", _ptr(x), x.stride(0), r.T, mw.H, mw.I, mw.E, r.topk, _ptr(mw.gate_up.packed),
             mw.gate_up.code, _ptr(r.tok), _ptr(r.items), _ptr(r.n_items), _ptr(act), act.stride(0), _stream(stream))
    return act


def moe_down(act: torch.Tensor, mw: MoeWeights, r: MoeRouting, stream=None) -> torch.Tensor:
    y = torch.empty((r.T * (r.topk + 1), mw.H), dtype=torch.float32, device=act.device)
    lib.call("rlq_moe_down", _ptr(act), act.stride(0), r.T, mw.H, mw.I, mw.E, r.topk, _ptr(mw.down.packed),
             mw.down.code, _ptr(r.items), _ptr(r.n_items), _ptr(y), y.stride(0), _stream(stream))
    return y


def moe_combine(y: torch.Tensor, r: MoeRouting, h: torch.Tensor, stream=None) -> torch.Tensor:
    lib.call("rlq_moe_combine", _ptr(y), y.stride(0), _ptr(r.inv), _ptr(r.w), r.T, r.topk, h.shape[1], _ptr(h),
             h.stride(0), _stream(stream))
    return h


def moe_workspace_bytes(T: int, E: int, topk: int, H: int, I: int) -> int:
    return int(lib.load().rlq_moe_workspace_bytes(T, E, topk, H, I))


def moe(x: torch.Tensor, logits: torch.Tensor, mw: MoeWeights, topk: int, h: torch.Tensor, norm_topk: bool = True,
        workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """h[t] += the MoE MLP of x[t] (route, gate/up + SwiGLU, down, combine), in one call."""
    T = x.shape[0]
    if h.dtype != torch.float32 or h.stride(1) != 1 or h.shape[0] < T or h.shape[1] < mw.H:
        raise ValueError("h must be a row-major float32 [T][>= H] matrix")
    nbytes = moe_workspace_bytes(T, mw.E, topk, mw.H, mw.I)
    ws = workspace if workspace is not None else torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    lib.call("rlq_moe", _ptr(x), x.stride(0), _ptr(logits), logits.stride(0), T, mw.E, topk, 1 if norm_topk else 0,
             mw.H, mw.I, _ptr(mw.gate_up.packed), _ptr(mw.down.packed), mw.gate_up.code, _ptr(h), h.stride(0), _ptr(ws),
             ws.numel(), _stream(stream))
    return h


# ------------------------------------------------------------------ native experts

@dataclass
class MoeNativeStack:
    """One kind of expert matrices (gate_up or down) in the native format: n_slots slots of
    Ne rows each (the stacked tensor, slot = expert, or an expert cache), codes in the tile
    layout and one fp32 scale per row (kernels/linear.metal:254-308)."""
    packed: torch.Tensor     # uint8, rlq_packed_codes_bytes(K, n_slots * Ne)
    s_row: torch.Tensor      # float32 [n_slots * Ne]
    K: int
    Ne: int
    n_slots: int
    book: str

    @property
    def code(self) -> int:
        return BOOKS[self.book]


def pack_moe_native(w: torch.Tensor, s_row: torch.Tensor, Ne: int, book: str, stream=None) -> MoeNativeStack:
    """Row-major codes of the stacked tensor (32-bit words [n_slots*Ne][K/8]) -> MoeNativeStack."""
    nw = pack_native(w, s_row, book, stream=stream)
    if nw.N % Ne:
        raise ValueError(f"{nw.N} rows is not a whole number of {Ne}-row slots")
    return MoeNativeStack(nw.packed, nw.s_row, nw.K, Ne, nw.N // Ne, book)


def moe_linear_native(a: torch.Tensor, st: MoeNativeStack, slots: torch.Tensor, r: MoeRouting, gather: bool,
                      out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """c fp32 [T*S][Ne]: each sorted row times its expert's slot (rlq_moe_linear_native);
    gather: a holds the T tokens and row r reads token tok[r], else a holds sorted rows."""
    if a.dtype != torch.float16 or a.dim() != 2 or a.stride(1) != 1 or a.shape[1] < st.K:
        raise ValueError("a must be a row-major float16 matrix of >= K columns")
    if slots.dtype != torch.int32 or not slots.is_contiguous():
        raise ValueError("slots must be a contiguous int32 vector [E+1]")
    A = r.T * (r.topk + 1)
    if out is None:
        out = torch.empty((A, st.Ne), dtype=torch.float32, device=a.device)
    lib.call("rlq_moe_linear_native", _ptr(a), a.stride(0), a.shape[0], _ptr(r.tok) if gather else 0, st.K, st.Ne,
             _ptr(st.packed), _ptr(st.s_row), _ptr(slots), st.n_slots, st.code, _ptr(r.items), _ptr(r.n_items),
             r.items.shape[0], _ptr(out), out.stride(0), _stream(stream))
    return out


def moe_swiglu(gu: torch.Tensor, I: int, cs: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """act fp16 [A][I] = half(silu(g) * u * cs) (rlq_moe_swiglu)."""
    if gu.dtype != torch.float32 or gu.dim() != 2 or gu.stride(1) != 1:
        raise ValueError("gu must be a row-major float32 matrix")
    if cs is not None and (cs.dtype != torch.float32 or not cs.is_contiguous() or cs.numel() < I):
        raise ValueError("cs must be a contiguous float32 vector of >= I column scales")
    act = torch.empty((gu.shape[0], I), dtype=torch.float16, device=gu.device)
    lib.call("rlq_moe_swiglu", _ptr(gu), gu.stride(0), gu.shape[0], I, _ptr(cs) if cs is not None else 0, _ptr(act),
             act.stride(0), _stream(stream))
    return act


def moe_gate_up_native(x: torch.Tensor, gu: MoeNativeStack, slots: torch.Tensor, r: MoeRouting,
                       cs: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """act fp16 [T*S][I]: the gathered gate/up product and the SwiGLU in one launch
    (rlq_moe_gate_up_native; the bits of moe_linear_native + moe_swiglu)."""
    if x.dtype != torch.float16 or x.dim() != 2 or x.stride(1) != 1 or x.shape[1] < gu.K:
        raise ValueError("x must be a row-major float16 [T][>= H] matrix")
    if cs is not None and (cs.dtype != torch.float32 or not cs.is_contiguous() or cs.numel() < gu.Ne // 2):
        raise ValueError("cs must be a contiguous float32 vector of >= I column scales")
    I = gu.Ne // 2
    act = torch.empty((r.T * (r.topk + 1), I), dtype=torch.float16, device=x.device)
    lib.call("rlq_moe_gate_up_native", _ptr(x), x.stride(0), x.shape[0], _ptr(r.tok), gu.K, I, _ptr(gu.packed),
             _ptr(gu.s_row), _ptr(slots), gu.n_slots, gu.code, _ptr(r.items), _ptr(r.n_items), r.items.shape[0],
             _ptr(cs) if cs is not None else 0, _ptr(act), act.stride(0), _stream(stream))
    return act


def moe_native(x: torch.Tensor, logits: torch.Tensor, gu: MoeNativeStack, dn: MoeNativeStack, slots: torch.Tensor,
               topk: int, h: torch.Tensor, cs: torch.Tensor | None = None, norm_topk: bool = True,
               fused: bool = True, one_call: bool = True, workspace: torch.Tensor | None = None,
               stream=None) -> torch.Tensor:
    """The native MoE MLP in the reference's order (src/engine.mm:965-1059): route, gate_up
    product with the gather fused, SwiGLU with the down matrix's column scale cs (folded
    into the gate_up launch when fused), down product, combine into h. x is already times
    gate_up's column scale. one_call: rlq_moe_native (the same bits as the steps)."""
    E = slots.numel() - 1
    if gu.Ne % 2 or dn.K != gu.Ne // 2 or dn.Ne != gu.K:
        raise ValueError("gate_up [2I][H] and down [H][I] stacks do not match")
    if gu.book != dn.book:
        raise ValueError("gate_up and down stacks use different codebooks")
    if one_call:
        T, H, I = x.shape[0], gu.K, gu.Ne // 2
        if x.dtype != torch.float16 or x.dim() != 2 or x.stride(1) != 1 or x.shape[1] < H:
            raise ValueError("x must be a row-major float16 [T][>= H] matrix")
        if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
            raise ValueError("logits must be a row-major float32 matrix")
        if slots.dtype != torch.int32 or not slots.is_contiguous():
            raise ValueError("slots must be a contiguous int32 vector [E+1]")
        nbytes = moe_workspace_bytes(T, E, topk, H, I)
        if workspace is None:
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        lib.call("rlq_moe_native", _ptr(x), x.stride(0), _ptr(logits), logits.stride(0), T, E, topk,
                 1 if norm_topk else 0, H, I, _ptr(gu.packed), _ptr(gu.s_row), _ptr(dn.packed), _ptr(dn.s_row),
                 _ptr(slots), gu.n_slots, gu.code, _ptr(cs) if cs is not None else 0, _ptr(h), h.stride(0),
                 _ptr(workspace), workspace.numel(), _stream(stream))
        return h
    r = moe_route(logits, E, topk, norm_topk, stream=stream)
    if fused:
        act = moe_gate_up_native(x, gu, slots, r, cs, stream=stream)
    else:
        act = moe_swiglu(moe_linear_native(x, gu, slots, r, True, stream=stream), gu.Ne // 2, cs, stream=stream)
    y = moe_linear_native(act, dn, slots, r, False, stream=stream)
    return moe_combine(y, r, h, stream=stream)
