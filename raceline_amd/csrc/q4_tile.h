// The packed 4-bit affine weight layout and the MFMA tile arithmetic shared by the dense
// decode kernel (linear.hip) and the grouped expert kernels (moe.hip).
//
// Packed device layout (made once at upload, from the MLX layout or the .rlm blocked
// layout; see include/rlq.h), for tiles t of 16 output rows, G = K/64 groups padded to
// G4 = ceil(G/4) quads, and group pairs p (groups 2p, 2p+1):
//   codes: 1024 bytes per (t, p) at ((t*2*G4 + p) * 64 + l) * 16: lane l = 16j + c holds
//          words (8g + 4s + j of row 16t + c) for (g, s) = (2p,0), (2p,1), (2p+1,0), (2p+1,1)
//          (tools/convert.py:82-89 nibble order);
//   scale/bias: after the codes, 16 bytes per (t, quad q, row c) at ((t*G4 + q)*16 + c)*16:
//          s | b << 16 for groups 4q .. 4q+3;
// rows beyond N and groups beyond G zero. One 16-byte load per lane brings a lane its
// operands for two groups, and a wave's loads for consecutive group pairs are
// consecutive kilobytes: a plain stream for the memory system. A stack of matrices whose
// row counts are multiples of 16 (the experts of a MoE layer) packs as one matrix, and
// matrix e starts at tile e * rows / 16.
//
// Matrix cores: v_mfma_f32_16x16x32_f16 (wave64), A = activations (rows = tokens), B =
// codes (cols = output features):
//   A (16 x 32): lane l holds row l%16, k = 8*(l/16) .. +7
//   B (32 x 16): lane l holds col l%16, k = 8*(l/16) .. +7
//   D (16 x 16): lane l holds col l%16, rows 4*(l/16) .. +3
// One group of 64 inputs is two MFMA steps s = 0, 1 (k = 64g + 32s .. +31); lane (c, j) =
// (l%16, l/16) feeds uint32 word 8g + 4s + j of row c (k = 64g + 32s + 8j .. +7).
//
// Operand trick: a uint32 of eight codes becomes four fp16 pairs with seven ops,
//   d0 = u & 0x000F000F -> (q0, q4)          d1 = (u>>4) & 0x000F000F -> (q1, q5)
//   d2 = (u>>8) & 0x000F000F -> (q2, q6)     d3 = (u>>12) & 0x000F000F -> (q3, q7)
// each half being the subnormal code * 2^-24, exact. The activation operand carries the
// same element order, (x0, x4, x1, x5, x2, x6, x3, x7): a permutation of the fp16 values
// the caller passed, with nothing rounded, so one MFMA step sums x_e * q_e * 2^-24 over
// the eight elements for activations of any magnitude. The f16 MFMA of gfx950 sums
// products of subnormal operands with about five bits less precision than normal ones
// (measured: 4e-6 of a group's rms against 1e-7, at every activation scale from 3e-5 to
// 300; the loss is relative, not a floor), so only the codes take this fast path: the
// group sums come from a second MFMA against a constant operand of ones, which lands them
// in the accumulator layout. Per group, acc += (s * 2^24) * part + b * gsum in fp32 (both
// rescalings exact). An MFMA output row depends only on its own operand row, so a token's
// result does not depend on which other tokens share the tile.
// (The prefill GEMM uses a cheaper five-op form of the codes, with the odd codes at 16 times
// the scale, behind an exact per-row power-of-two prescale of the activations: gemm.hip.)
#pragma once

#include "rlq_common.h"

namespace rlq {

constexpr int kGroup = 64;
constexpr int kBufFlags = 0x00020000;             // buffer descriptor word 3 for raw 32-bit accesses
constexpr int kNonTemporal = 2;                   // buffer load cache policy: stream, do not keep
constexpr uint32_t kFarOffset = 0x7FFFFFF0u;      // a buffer offset past every range: reads zero
constexpr float kTwo24 = 16777216.0f;             // undoes the 2^-24 of subnormal code operands

__host__ __device__ inline int tiles_of(int N) { return (N + 15) / 16; }
__host__ __device__ inline int quads_of(int K) { return (K / kGroup + 3) / 4; }
inline size_t packed_code_bytes(int K, int N) { return (size_t)tiles_of(N) * quads_of(K) * 2048; }
inline size_t packed_bytes(int K, int N) { return (size_t)tiles_of(N) * quads_of(K) * 2304; }

// Row order of a packed MoE gate/up stack: the source stack holds, per expert, I gate rows
// then I up rows ([E][2I][K], tools/quantize.py:168-228); packed tile j of an expert holds
// gate rows 8j .. 8j+7 then up rows 8j .. 8j+7, so one 16-row tile yields both halves of
// SwiGLU for 8 features. Returns the source row of packed row n (I % 8 == 0).
__host__ __device__ inline int gate_up_source_row(int n, int I) {
  const int e = n / (2 * I), r = n - e * 2 * I, j = r >> 4, c = r & 15;
  return e * 2 * I + (c < 8 ? 8 * j + c : I + 8 * j + (c - 8));
}

// eight codes (element e at bits 4e) -> (q0, q4, q1, q5, q2, q6, q3, q7) * 2^-24, fp16 subnormals
__device__ __forceinline__ half8 nib8_to_half8_sub(uint32_t u) {
  u32x4 d;
  d[0] = u & 0x000F000Fu;
  d[1] = (u >> 4) & 0x000F000Fu;
  d[2] = (u >> 8) & 0x000F000Fu;
  // the top nibble of each 16-bit half: one packed 16-bit shift clears the rest (six ops
  // in all instead of seven; the same bits)
  d[3] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, u) >> (u16x2){12, 12});
  return __builtin_bit_cast(half8, d);
}

// The five-op form for the prefill GEMM: (q0, q4, 16 q1, 16 q5, q2, q6, 16 q3, 16 q7) * 2^-24,
// for activations in the matching order with the odd ones divided by 16 (gemm.hip prescales
// each row by a power of two first, so that the division rounds nothing that matters).
__device__ __forceinline__ half8 nib8_to_half8_oddx16(uint32_t u) {
  const uint32_t t = u >> 8;
  u32x4 d;
  d[0] = u & 0x000F000Fu;
  d[1] = u & 0x00F000F0u;
  d[2] = t & 0x000F000Fu;
  d[3] = t & 0x00F000F0u;
  return __builtin_bit_cast(half8, d);
}

// eight consecutive activations -> operand order (x0, x4, x1, x5, x2, x6, x3, x7): a
// permutation of the halves, exact
__device__ __forceinline__ u32x4 prep_x8(u32x4 p) {
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(p[2], p[0], 0x05040100u);  // (x0, x4)
  r[1] = __builtin_amdgcn_perm(p[2], p[0], 0x07060302u);  // (x1, x5)
  r[2] = __builtin_amdgcn_perm(p[3], p[1], 0x05040100u);  // (x2, x6)
  r[3] = __builtin_amdgcn_perm(p[3], p[1], 0x07060302u);  // (x3, x7)
  return r;
}

// SwiGLU's gate activation, silu(v) = v / (1 + e^-v) (kernels/ops.metal:446-455); one
// definition for every kernel that applies it, so that they give the same bits
__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// half(silu(g) * u) with the product rounded to fp32 and then to fp16, as the SwiGLU kernel
// over fp32 gate/up rows computes it (moe_swiglu_kernel). The barrier keeps the compiler
// from fusing the multiply into the conversion (v_fma_mix rounds once, which can differ in
// the last bit), so a kernel with the SwiGLU fused gives that kernel's bits.
__device__ __forceinline__ _Float16 swiglu_half(float g, float u) {
  float p = silu(g) * u;
  asm volatile("" : "+v"(p));
  return static_cast<_Float16>(p);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, kBufFlags);
}

// acc + float(s16) * p with the 16-bit float taken from the low or high half of a packed pair
template <int SD, int HI>
__device__ __forceinline__ float fma_scale(uint32_t pr, float p, float acc) {
  if constexpr (SD == 0) {
    const _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)(HI ? (pr >> 16) : (pr & 0xFFFFu)));
    return __builtin_fmaf(static_cast<float>(v), p, acc);
  } else {
    const float v = __uint_as_float(HI ? (pr & 0xFFFF0000u) : (pr << 16));
    return __builtin_fmaf(v, p, acc);
  }
}

// Descriptors over one wave's part of one 16-row tile: groups [wg0, wg0 + GPW) of tile t.
// Loads past the wave's part (padding groups, the next wave's range) return zeros; a wave
// whose range starts past the tile's groups gets empty descriptors.
struct WaveTile {
  __amdgpu_buffer_rsrc_t rw, rs;
};

__device__ __forceinline__ WaveTile wave_tile(const u32x4 *codes, const u32x4 *sb, int t, int G4, int wg0, int gpw) {
  const int wq1 = max(wg0, min(4 * G4, wg0 + gpw));
  WaveTile w;
  w.rw = make_rsrc(codes + ((size_t)t * 2 * G4 + wg0 / 2) * 64, (uint32_t)(wq1 - wg0) / 2u * 1024u);
  w.rs = make_rsrc(sb + ((size_t)t * G4 + wg0 / 4) * 16, (uint32_t)(wq1 - wg0) / 4u * 256u);
  return w;
}

// Every code load of the wave's part and (affine) every scale/bias load, issued at once
// (non-temporal). The whole offset goes in the vector offset operand: only that part
// (with the instruction's immediate) is range-checked against the descriptor; the scalar
// offset operand is not, so loads past the wave's part would read whatever follows.
template <int GPW, int BOOK = kAffine>
__device__ __forceinline__ void issue_tile_loads(const WaveTile &w, int lane, u32x4 (&wq)[GPW / 2],
                                                 u32x4 (&sq)[GPW / 4]) {
#pragma unroll
  for (int pp = 0; pp < GPW / 2; ++pp)
    wq[pp] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(w.rw, 16u * lane + (uint32_t)pp * 1024u, 0,
                                                                             kNonTemporal));
  if constexpr (BOOK == kAffine) {
#pragma unroll
    for (int qq = 0; qq < GPW / 4; ++qq)
      sq[qq] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             w.rs, 16u * (lane & 15) + (uint32_t)qq * 256u, 0, kNonTemporal));
  }
}

// Activations -> operand order: the permuted order of prep_x8 for the affine and integer
// books (whose code conversions, nib8_to_half8_sub and native8_operand, give that order),
// the element order for fp4.
template <int BOOK>
__device__ __forceinline__ u32x4 prep_act(u32x4 v) {
  if constexpr (BOOK == kFp4) return v;
  else return prep_x8(v);
}

// One group of a native-book tile: the products chain straight into the accumulator (no
// per-group scale); kInt16 also chains the activation sums (for its +0.5 levels).
template <int GPW, int BOOK>
__device__ __forceinline__ void native_step(f32x4 &acc, f32x4 &asum, const half8 (&af)[2], const u32x4 (&wq)[GPW / 2],
                                            int jg) {
  const half8 ones = __builtin_bit_cast(half8, u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], native8_operand<BOOK>(wq[jg >> 1][2 * (jg & 1) + s]), acc, 0,
                                                 0, 0);
    if constexpr (BOOK == kInt16) asum = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], ones, asum, 0, 0, 0);
  }
}


// The activation sums of one group for 16 token rows, as two products with a constant
// operand of ones (lane (c16, j4) gets rows 4 j4 + v). Every tile of the same rows needs
// the same sums: a caller that forms them once and hands them to group_step_gs gets the
// bits group_step gets.
__device__ __forceinline__ f32x4 group_sums(const half8 (&af)[2]) {
  const half8 ones = __builtin_bit_cast(half8, u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});
  f32x4 gsv = {};
#pragma unroll
  for (int s = 0; s < 2; ++s) gsv = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], ones, gsv, 0, 0, 0);
  return gsv;
}

// One group jg of the wave's part with the group's activation sums given: acc[r] +=
// s * (x . q) + b * gsv[r] for the first NACC accumulator rows.
template <int GPW, int SD, int NACC>
__device__ __forceinline__ void group_step_gs(f32x4 &acc, const half8 (&af)[2], const f32x4 &gsv,
                                              const u32x4 (&wq)[GPW / 2], const u32x4 (&sq)[GPW / 4], int jg) {
  f32x4 p = {};
#pragma unroll
  for (int s = 0; s < 2; ++s)
    p = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], nib8_to_half8_sub(wq[jg >> 1][2 * (jg & 1) + s]), p, 0, 0, 0);
  const uint32_t pr = sq[jg >> 2][jg & 3];
  const float sc = fma_scale<SD, 0>(pr, kTwo24, 0.0f);   // s * 2^24, exact: undoes the codes' 2^-24
#pragma unroll
  for (int r = 0; r < NACC; ++r) acc[r] = fma_scale<SD, 1>(pr, gsv[r], __builtin_fmaf(sc, p[r], acc[r]));
}

// group_step_gs with the group's two B operands already converted (bq[s] =
// nib8_to_half8_sub of word 2 (jg & 1) + s of wq[jg >> 1]): the same operations, for a
// caller that multiplies the same codes into several blocks of rows.
template <int GPW, int SD, int NACC>
__device__ __forceinline__ void group_step_gs_b(f32x4 &acc, const half8 (&af)[2], const f32x4 &gsv,
                                                const half8 (&bq)[2], const u32x4 (&sq)[GPW / 4], int jg) {
  f32x4 p = {};
#pragma unroll
  for (int s = 0; s < 2; ++s) p = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], bq[s], p, 0, 0, 0);
  const uint32_t pr = sq[jg >> 2][jg & 3];
  const float sc = fma_scale<SD, 0>(pr, kTwo24, 0.0f);   // s * 2^24, exact: undoes the codes' 2^-24
#pragma unroll
  for (int r = 0; r < NACC; ++r) acc[r] = fma_scale<SD, 1>(pr, gsv[r], __builtin_fmaf(sc, p[r], acc[r]));
}

// One group jg of the wave's part: acc[r] += s * (x . q) + b * gsum for the first NACC
// accumulator rows (NACC = 1 when only token row 0 is live).
template <int GPW, int SD, int NACC>
__device__ __forceinline__ void group_step(f32x4 &acc, const half8 (&af)[2], const u32x4 (&wq)[GPW / 2],
                                           const u32x4 (&sq)[GPW / 4], int jg) {
  group_step_gs<GPW, SD, NACC>(acc, af, group_sums(af), wq, sq, jg);
}

// The per-group step of any book: affine (group_step, scales applied per group) or native.
template <int GPW, int SD, int NACC, int BOOK>
__device__ __forceinline__ void book_step(f32x4 &acc, f32x4 &asum, const half8 (&af)[2], const u32x4 (&wq)[GPW / 2],
                                          const u32x4 (&sq)[GPW / 4], int jg) {
  if constexpr (BOOK == kAffine) group_step<GPW, SD, NACC>(acc, af, wq, sq, jg);
  else native_step<GPW, BOOK>(acc, asum, af, wq, jg);
}

// The wave's part of a 16-row weight tile times up to 16 token rows whose activations
// are read straight from memory (L2-resident), two groups ahead, and put in operand order
// in registers. rx covers the activations; lane (c16, j4) reads its row at byte offset
// xoff (row start + wave's first element + 16 * j4); lanes of rows that do not exist pass
// live = false and read zeros. wn = real groups of the wave's part.
// For native books the returned total already includes 0.5 * asum (kInt16); the row
// scale is the caller's.
// NACC: accumulator rows formed (1 when only token row 0 exists; its value is the same).
// PRE (affine): gs0 holds the group sums of token row 0 for the wave's groups, formed
// beforehand (row0_group_sums: the same two MFMAs, so the same bits), in place of forming
// them here; only row 0's results are then valid (NACC = 1).
template <int GPW, int SD, int BOOK = kAffine, int NACC = 4, bool PRE = false>
__device__ __forceinline__ f32x4 tile_dot_rows(const WaveTile &w, __amdgpu_buffer_rsrc_t rx, uint32_t xoff, bool live,
                                               int wn, int lane, const float *gs0 = nullptr) {
  u32x4 wq[GPW / 2], sq[GPW / 4];
  auto ldx = [&](int jg, int s) -> u32x4 {
    const bool ok = live && jg < wn;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                         rx, ok ? xoff + (uint32_t)(jg * kGroup + 32 * s) * 2u : kFarOffset, 0, 0));
  };
  u32x4 ax[3][2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int s = 0; s < 2; ++s) ax[d][s] = ldx(d, s);
  issue_tile_loads<GPW, BOOK>(w, lane, wq, sq);
  __builtin_amdgcn_sched_barrier(0);   // every weight load is in flight before the first multiply
  f32x4 acc = {}, asum = {};
#pragma unroll
  for (int jg = 0; jg < GPW; ++jg) {
    if (jg + 2 < GPW) {
#pragma unroll
      for (int s = 0; s < 2; ++s) ax[(jg + 2) % 3][s] = ldx(jg + 2, s);
    }
    const half8 af[2] = {__builtin_bit_cast(half8, prep_act<BOOK>(ax[jg % 3][0])),
                         __builtin_bit_cast(half8, prep_act<BOOK>(ax[jg % 3][1]))};
    if constexpr (BOOK == kAffine) {
      if constexpr (PRE) {
        const float g = jg < wn ? gs0[jg] : 0.0f;   // past the range: the zero sum of zero operands
        group_step_gs<GPW, SD, NACC>(acc, af, f32x4{g, g, g, g}, wq, sq, jg);
      } else {
        group_step<GPW, SD, NACC>(acc, af, wq, sq, jg);
      }
    } else {
      book_step<GPW, SD, NACC, BOOK>(acc, asum, af, wq, sq, jg);
    }
    // The group's epilogue happens here, not after the last group: without this the
    // compiler sinks every group's scale/bias FMAs below the last MFMA and keeps all
    // the partial products alive (register spills).
    asm volatile("" : "+v"(acc));
  }
  if constexpr (BOOK == kInt16) {
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(0.5f, asum[v], acc[v]);
  }
  return acc;
}

// The group sums of token row 0 for groups [0, wn) of a wave's part, as tile_dot_rows forms
// them (the same operands and the same two MFMAs against ones), written to out[jg] by lane
// 0. rx and xoff as for tile_dot_rows, with lane (c16, j4) live only for c16 = 0.
template <int GPW>
__device__ __forceinline__ void row0_group_sums(__amdgpu_buffer_rsrc_t rx, uint32_t xoff, int wn, int lane,
                                                float *out) {
  const bool live = (lane & 15) == 0;
  constexpr int C = GPW < 8 ? GPW : 8;   // groups loaded at once (2 C operands in registers)
#pragma unroll
  for (int c0 = 0; c0 < GPW; c0 += C) {
    u32x4 ax[C][2];
#pragma unroll
    for (int j = 0; j < C; ++j)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        ax[j][s] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rx, live && c0 + j < wn ? xoff + (uint32_t)((c0 + j) * kGroup + 32 * s) * 2u : kFarOffset, 0,
                       0));
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const half8 af[2] = {__builtin_bit_cast(half8, prep_x8(ax[j][0])), __builtin_bit_cast(half8, prep_x8(ax[j][1]))};
      const f32x4 gsv = group_sums(af);
      if (lane == 0 && c0 + j < wn) out[c0 + j] = gsv[0];
    }
  }
}

// tile_dot_rows for two tiles at once (the same groups of two weight tiles, w0 and w1, one
// activation stream): every activation operand is loaded once and multiplied into both
// tiles, and the activation-only terms (affine group sums, kInt16 activation sums) are
// formed once. Each tile's products and sums are the ones tile_dot_rows forms, in the
// same order, so acc0 and acc1 hold its bits.
template <int GPW, int SD, int BOOK = kAffine>
__device__ __forceinline__ void tile_dot_rows2(const WaveTile &w0, const WaveTile &w1, __amdgpu_buffer_rsrc_t rx,
                                               uint32_t xoff, bool live, int wn, int lane, f32x4 &acc0, f32x4 &acc1) {
  u32x4 wq0[GPW / 2], sq0[GPW / 4], wq1[GPW / 2], sq1[GPW / 4];
  auto ldx = [&](int jg, int s) -> u32x4 {
    const bool ok = live && jg < wn;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                         rx, ok ? xoff + (uint32_t)(jg * kGroup + 32 * s) * 2u : kFarOffset, 0, 0));
  };
  u32x4 ax[3][2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int s = 0; s < 2; ++s) ax[d][s] = ldx(d, s);
  issue_tile_loads<GPW, BOOK>(w0, lane, wq0, sq0);
  issue_tile_loads<GPW, BOOK>(w1, lane, wq1, sq1);
  __builtin_amdgcn_sched_barrier(0);   // every weight load is in flight before the first multiply
  const half8 ones = __builtin_bit_cast(half8, u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});
  f32x4 asum = {};
  acc0 = f32x4{};
  acc1 = f32x4{};
#pragma unroll
  for (int jg = 0; jg < GPW; ++jg) {
    if (jg + 2 < GPW) {
#pragma unroll
      for (int s = 0; s < 2; ++s) ax[(jg + 2) % 3][s] = ldx(jg + 2, s);
    }
    const half8 af[2] = {__builtin_bit_cast(half8, prep_act<BOOK>(ax[jg % 3][0])),
                         __builtin_bit_cast(half8, prep_act<BOOK>(ax[jg % 3][1]))};
    if constexpr (BOOK == kAffine) {
      const f32x4 gsv = group_sums(af);
      group_step_gs<GPW, SD, 4>(acc0, af, gsv, wq0, sq0, jg);
      group_step_gs<GPW, SD, 4>(acc1, af, gsv, wq1, sq1, jg);
    } else {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], native8_operand<BOOK>(wq0[jg >> 1][2 * (jg & 1) + s]),
                                                      acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], native8_operand<BOOK>(wq1[jg >> 1][2 * (jg & 1) + s]),
                                                      acc1, 0, 0, 0);
        if constexpr (BOOK == kInt16) asum = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], ones, asum, 0, 0, 0);
      }
    }
    asm volatile("" : "+v"(acc0), "+v"(acc1));   // each group's epilogue stays with its group
  }
  if constexpr (BOOK == kInt16) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc0[v] = __builtin_fmaf(0.5f, asum[v], acc0[v]);
      acc1[v] = __builtin_fmaf(0.5f, asum[v], acc1[v]);
    }
  }
}

// LDS bytes of one staged activation row of an 8-group wave range: its 64 chunks of 16
// bytes, chunk c of row r at position c ^ (r & 15), so the 16 rows a wave reads at once
// (the same chunk of each) fall in different banks without padding.
constexpr int kStagedXRow = 8 * kGroup * 2;
__device__ __forceinline__ int staged_pos(int c, int r) { return c ^ (r & 15); }

// s_waitcnt immediate that waits until at most n vector memory operations are outstanding
// (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt at their no-wait maximum).
constexpr int waitcnt_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

// The wave's part of two tiles at once (the same groups of two weight tiles, w0 and w1, one
// activation stream): every activation operand is read once and multiplied into both
// tiles, and the activation-only terms (affine group sums, kInt16 activation sums) are
// formed once; each tile's products and sums are the ones tile_dot_rows forms, in the same
// order, so acc0 and acc1 hold its bits. The activations are staged in LDS first: one
// LDS-DMA per token row (stage_rows: the row's part of the wave's range, with no registers
// or ALU work), issued before the weight loads, so the activations and the weights are in
// flight together and the groups then read their operands from LDS instead of waiting on
// L2 reads. xs: the wave's M * kStagedXRow bytes; xstride: bytes between token rows in
// memory. Rows >= M and groups >= wn use zero operands, as tile_dot_rows's zero reads give.
// GPW = 8 only (a row's part is one 1024-byte LDS-DMA).
template <int GPW, int SD, int BOOK = kAffine>
__device__ __forceinline__ void tile_dot_rows2_staged(const WaveTile &w0, const WaveTile &w1,
                                                      __amdgpu_buffer_rsrc_t rx, uint32_t xstride, int M,
                                                      unsigned char *xs, int wn, int lane, f32x4 &acc0,
                                                      f32x4 &acc1) {
  static_assert(GPW == 8, "one 1024-byte LDS-DMA per activation row");
  u32x4 wq0[GPW / 2], sq0[GPW / 4], wq1[GPW / 2], sq1[GPW / 4];
  stage_rows(rx, [=](int r) { return (uint32_t)r * xstride; }, M, 0, xs, lane);
  __builtin_amdgcn_sched_barrier(0);   // the activations are requested first: they complete first
  issue_tile_loads<GPW, BOOK>(w0, lane, wq0, sq0);
  issue_tile_loads<GPW, BOOK>(w1, lane, wq1, sq1);
  // the activation DMAs have landed once at most the weight loads are outstanding
  constexpr int kWeightLoads = 2 * (GPW / 2 + (BOOK == kAffine ? GPW / 4 : 0));
  __builtin_amdgcn_s_waitcnt(waitcnt_vmcnt(kWeightLoads));
  __builtin_amdgcn_sched_barrier(0);
  const bool live = (lane & 15) < M;
  const int row = live ? lane & 15 : 0;
  // chunk 8 jg + 4 s + j4 of the lane's row: the swizzle only moves it inside its 256-byte
  // block, so four per-lane bases (jg odd or even, s) and a constant offset reach every one
  const unsigned char *xq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) xq[q] = xs + row * kStagedXRow + 16 * staged_pos(8 * (q >> 1) + 4 * (q & 1) + (lane >> 4), row);
  auto ldx = [&](int jg, int s) -> u32x4 {
    const u32x4 v = *reinterpret_cast<const u32x4 *>(xq[2 * (jg & 1) + s] + 256 * (jg >> 1));
    return live && jg < wn ? v : u32x4{};
  };
  const half8 ones = __builtin_bit_cast(half8, u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});
  f32x4 asum = {};
  acc0 = f32x4{};
  acc1 = f32x4{};
  u32x4 ax[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s) ax[0][s] = ldx(0, s);
#pragma unroll
  for (int jg = 0; jg < GPW; ++jg) {
    if (jg + 1 < GPW) {
#pragma unroll
      for (int s = 0; s < 2; ++s) ax[(jg + 1) & 1][s] = ldx(jg + 1, s);
    }
    const half8 af[2] = {__builtin_bit_cast(half8, prep_act<BOOK>(ax[jg & 1][0])),
                         __builtin_bit_cast(half8, prep_act<BOOK>(ax[jg & 1][1]))};
    if constexpr (BOOK == kAffine) {
      const f32x4 gsv = group_sums(af);
      group_step_gs<GPW, SD, 4>(acc0, af, gsv, wq0, sq0, jg);
      group_step_gs<GPW, SD, 4>(acc1, af, gsv, wq1, sq1, jg);
    } else {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], native8_operand<BOOK>(wq0[jg >> 1][2 * (jg & 1) + s]),
                                                      acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], native8_operand<BOOK>(wq1[jg >> 1][2 * (jg & 1) + s]),
                                                      acc1, 0, 0, 0);
        if constexpr (BOOK == kInt16) asum = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], ones, asum, 0, 0, 0);
      }
    }
    asm volatile("" : "+v"(acc0), "+v"(acc1));   // each group's epilogue stays with its group
  }
  if constexpr (BOOK == kInt16) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc0[v] = __builtin_fmaf(0.5f, asum[v], acc0[v]);
      acc1[v] = __builtin_fmaf(0.5f, asum[v], acc1[v]);
    }
  }
}

// Requests chunk `chunk` (groups 8 chunk .. 8 chunk + 7 of the wave's range) of M token
// rows into LDS: row r's 1024 bytes, from byte offset row_off(r) (uniform) of rx, land at
// xs + r * kStagedXRow in staged_pos order (one LDS-DMA per row, no registers or ALU work:
// lane l fills position l, so it brings source chunk staged_pos(l, r)); bytes past rx's
// range read as zero.
template <typename RowOff>
__device__ __forceinline__ void stage_rows(__amdgpu_buffer_rsrc_t rx, RowOff row_off, int M, int chunk,
                                           unsigned char *xs, int lane) {
  for (int r = 0; r < M; ++r)   // uniform
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rx, (__attribute__((address_space(3))) void *)(xs + r * kStagedXRow), 16,
        row_off(r) + (uint32_t)chunk * 8u * kGroup * 2u + 16u * (uint32_t)staged_pos(lane, r), 0, 0, 0);
}

// tile_dot_rows with the activations staged in LDS by DMA (stage_rows), 8 groups at a
// time, for any wave range (the down projections' 12, 16 or 24 groups do not fit LDS whole
// for every row). Chunk 0 is requested before the weight loads, so it arrives with them
// (or, staged0, the caller requested it earlier, before any other vector memory load of
// the wave still in flight); each later chunk replaces the previous one in the wave's
// M * kStagedXRow bytes at xs once its groups are done. Row r comes from byte offset
// row_off(r) of rx. Rows >= M and groups >= wn use zero operands, as tile_dot_rows's zero
// reads give, so the result holds its bits.
template <int GPW, int SD, int BOOK = kAffine, typename RowOff>
__device__ __forceinline__ f32x4 tile_dot_rows_staged(const WaveTile &w, __amdgpu_buffer_rsrc_t rx, RowOff row_off,
                                                      int M, unsigned char *xs, int wn, int lane,
                                                      bool staged0 = false) {
  static_assert(GPW % 4 == 0, "chunks of 8 groups, the last possibly 4");
  u32x4 wq[GPW / 2], sq[GPW / 4];
  auto stage = [&](int chunk) { stage_rows(rx, row_off, M, chunk, xs, lane); };
  if (!staged0) stage(0);
  __builtin_amdgcn_sched_barrier(0);   // chunk 0 is requested first: it completes first
  issue_tile_loads<GPW, BOOK>(w, lane, wq, sq);
  constexpr int kWeightLoads = GPW / 2 + (BOOK == kAffine ? GPW / 4 : 0);
  __builtin_amdgcn_s_waitcnt(waitcnt_vmcnt(kWeightLoads));   // chunk 0 has landed
  __builtin_amdgcn_sched_barrier(0);
  const bool live = (lane & 15) < M;
  const int row = live ? lane & 15 : 0;
  // chunk 8 (jg % 8) + 4 s + j4 of the lane's row, reached as in tile_dot_rows2_staged
  const unsigned char *xq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) xq[q] = xs + row * kStagedXRow + 16 * staged_pos(8 * (q >> 1) + 4 * (q & 1) + (lane >> 4), row);
  auto ldx = [&](int jg, int s) -> u32x4 {
    const u32x4 v = *reinterpret_cast<const u32x4 *>(xq[2 * (jg & 1) + s] + 256 * ((jg & 7) >> 1));
    return live && jg < wn ? v : u32x4{};
  };
  f32x4 acc = {}, asum = {};
  u32x4 ax[2][2];
#pragma unroll
  for (int jg = 0; jg < GPW; ++jg) {
    if ((jg & 7) == 0) {
      if (jg > 0) {
        // the previous chunk's operands are in registers (its reads have returned); bring
        // the next chunk into the same bytes and wait for it
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt, expcnt: no wait
        __builtin_amdgcn_sched_barrier(0);
        stage(jg / 8);
        __builtin_amdgcn_s_waitcnt(waitcnt_vmcnt(0));
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) ax[jg & 1][s] = ldx(jg, s);
    }
    if (((jg + 1) & 7) != 0 && jg + 1 < GPW) {
#pragma unroll
      for (int s = 0; s < 2; ++s) ax[(jg + 1) & 1][s] = ldx(jg + 1, s);
    }
    const half8 af[2] = {__builtin_bit_cast(half8, prep_act<BOOK>(ax[jg & 1][0])),
                         __builtin_bit_cast(half8, prep_act<BOOK>(ax[jg & 1][1]))};
    book_step<GPW, SD, 4, BOOK>(acc, asum, af, wq, sq, jg);
    asm volatile("" : "+v"(acc));   // each group's epilogue stays with its group
  }
  if constexpr (BOOK == kInt16) {
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(0.5f, asum[v], acc[v]);
  }
  return acc;
}

// The wave's part of a 16-row affine weight tile (its loads already issued into wq, sq)
// times 16 token rows staged in LDS in operand order, with their group sums formed
// beforehand (group_sums): xs points at row 0's element 64 * wg0 (the wave's first group),
// rows rstride halves apart; gs at the sums of group wg0, 16 floats (row order) per group.
// Lane (c16, j4) reads row c16. The part is summed as SUB consecutive sub-parts of GPW / SUB
// groups, each in its own accumulator (acc[s], from zero), which is how a kernel with
// GPW / SUB groups per wave sums the same groups.
// BOOK: kAffine, or a native book (int15, fp4), whose products chain in the MFMA over each
// sub-part (no per-group scale or group sums; gs unused), as tile_dot_rows chains them.
// FULL: the caller guarantees wn == GPW (every group of the range is real), and the loop runs
// with no per-group branch: straight-line code, without the register moves that the
// branches' merge points cost (about 4 per group), with the same products in the same order.
template <int GPW, int SD, int SUB, int BOOK = kAffine, bool FULL = false>
__device__ __forceinline__ void tile_dot_lds(const u32x4 (&wq)[GPW / 2], const u32x4 (&sq)[GPW / 4],
                                             const _Float16 *xs, const float *gs, int rstride, int wn, int lane,
                                             f32x4 (&acc)[SUB]) {
  const _Float16 *xa = xs + (lane & 15) * rstride + 8 * (lane >> 4);
  const float *ga = gs + 4 * (lane >> 4);
#pragma unroll
  for (int s = 0; s < SUB; ++s) acc[s] = f32x4{};
#pragma unroll
  for (int jg = 0; jg < GPW; ++jg) {
    if (FULL || jg < wn) {   // uniform: the groups past the wave's range add nothing
      constexpr int per = GPW / SUB;
      half8 af[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) af[s] = *reinterpret_cast<const half8 *>(xa + jg * kGroup + 32 * s);
      if constexpr (BOOK == kAffine) {
        const f32x4 gsv = *reinterpret_cast<const f32x4 *>(ga + 16 * jg);
        group_step_gs<GPW, SD, 4>(acc[jg / per], af, gsv, wq, sq, jg);
      } else {
#pragma unroll
        for (int s = 0; s < 2; ++s)
          acc[jg / per] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              af[s], native8_operand<BOOK>(wq[jg >> 1][2 * (jg & 1) + s]), acc[jg / per], 0, 0, 0);
      }
      asm volatile("" : "+v"(acc[jg / per]));
    }
  }
}

// Waves 1.. of the workgroup hand their partials to wave 0, which adds them in wave order
// (a fixed order: the result depends only on the number of waves). red: (waves-1)*64
// f32x4 of LDS. Returns the total in wave 0 (other waves' return value is unspecified).
__device__ __forceinline__ f32x4 reduce_waves(f32x4 acc, f32x4 *red, int wave, int waves, int lane) {
  if (wave > 0) red[(wave - 1) * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0) {
    for (int w = 1; w < waves; ++w) {
      const f32x4 o = red[(w - 1) * 64 + lane];
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] += o[v];
    }
  }
  return acc;
}

}  // namespace rlq
