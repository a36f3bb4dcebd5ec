// Affine 4-bit group-quantized linear layer on gfx950: the packed device layout and its
// upload kernels, the decode GEMV, the prefill GEMM, group sums and a dequantizing check.
//
//   y[m][n] = sum_k x[m][k] * W[n][k],   W[n][k] = s[n][g] * q[n][k] + b[n][g],  g = k / 64
//
// evaluated, like the reference kernel (kernels/linear.metal:5-9,85-101), as
//   y[m][n] = sum_g ( s[n][g] * (x_g . q_g)[m][n] + b[n][g] * gsum[m][g] )
// so the weights are never dequantized in software: the integer codes go to the
// matrix cores as exact fp16 values and the scale and bias are applied per group
// to the fp32 partial product.
//
// The packed layout, the MFMA operand layout and the operand trick are described in
// q4_tile.h.
#include "gemm.h"
#include "linear.h"
#include "q4_tile.h"
#include "../../include/rlq.h"

#include <algorithm>

namespace rlq {

constexpr int kMaxTiles = 32768;                                   // N <= 16 * kMaxTiles

// ================================================================== packing (upload)

// MLX layout (codes uint32 [N][K/8], scales and biases [N][G]) -> packed. One thread per
// 16-byte piece of codes (tile t, pair p, lane l); threads of lane < 16 of even pairs
// also write the scale/bias quad of their row.
__global__ void pack_mlx_kernel(const uint32_t *w, const uint16_t *s, const uint16_t *b, int K, int N, int il,
                                u32x4 *codes, u32x4 *sb) {
  const int G = K / kGroup, G4 = quads_of(K), GP = 2 * G4;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;   // ((t * GP + p) * 64 + l)
  if (i >= (size_t)tiles_of(N) * GP * 64) return;
  const int l = (int)(i & 63);
  const size_t tp = i >> 6;
  const int t = (int)(tp / GP), p = (int)(tp - (size_t)t * GP);
  const int c = l & 15, j = l >> 4, n = 16 * t + c;
  const int src = il ? gate_up_source_row(n, il) : n;   // il: the gate/up interleave of a MoE stack
  u32x4 v = {};
  if (n < N) {
    const uint32_t *row = w + (size_t)src * (K / 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int g = 2 * p + (e >> 1), sx = e & 1;
      v[e] = g < G ? row[8 * g + 4 * sx + j] : 0u;
    }
  }
  codes[i] = v;
  if (sb != nullptr && j == 0 && (p & 1) == 0) {   // sb == nullptr: a codes-only (native) matrix
    const int q = p >> 1;
    u32x4 e4 = {};
    if (n < N) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int g = 4 * q + e;
        e4[e] = g < G ? ((uint32_t)s[(size_t)src * G + g] | ((uint32_t)b[(size_t)src * G + g] << 16)) : 0u;
      }
    }
    sb[((size_t)t * G4 + q) * 16 + c] = e4;
  }
}

// Blocked q4a file layout (tools/convert.py:92-117) rows [row0, row0 + rows) -> packed.
// The file stores, per block of 256 rows and input index k, 128 bytes with row 2i in the
// low and row 2i+1 in the high nibble of byte i.
__global__ void pack_blocked_kernel(const uint8_t *w_blk, const uint16_t *s_blk, const uint16_t *b_blk, int K,
                                    int row0, int rows, u32x4 *codes, u32x4 *sb) {
  const int G = K / kGroup, G4 = quads_of(K), GP = 2 * G4;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)tiles_of(rows) * GP * 64) return;
  const int l = (int)(i & 63);
  const size_t tp = i >> 6;
  const int t = (int)(tp / GP), p = (int)(tp - (size_t)t * GP);
  const int c = l & 15, j = l >> 4, r = 16 * t + c;
  u32x4 v = {};
  const int n = row0 + r, blk = n >> 8, cb = n & 255;
  if (r < rows) {
    const int shift = (cb & 1) ? 4 : 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int g = 2 * p + (e >> 1), sx = e & 1;
      uint32_t u = 0;
      if (g < G) {
        const uint8_t *src = w_blk + ((size_t)blk * K + 64 * g + 32 * sx + 8 * j) * 128 + (cb >> 1);
#pragma unroll
        for (int k = 0; k < 8; ++k) u |= ((uint32_t)(src[(size_t)k * 128] >> shift) & 15u) << (4 * k);
      }
      v[e] = u;
    }
  }
  codes[i] = v;
  if (sb != nullptr && j == 0 && (p & 1) == 0) {   // sb == nullptr: a codes-only (native) matrix
    const int q = p >> 1;
    u32x4 e4 = {};
    if (r < rows) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int g = 4 * q + e;
        const size_t o = ((size_t)blk * G + g) * 256 + cb;
        e4[e] = g < G ? ((uint32_t)s_blk[o] | ((uint32_t)b_blk[o] << 16)) : 0u;
      }
    }
    sb[((size_t)t * G4 + q) * 16 + c] = e4;
  }
}

// Blocked file layout -> MLX layout (the interchange format), rows [row0, row0 + rows).
__global__ void repack_w_kernel(const uint8_t *w_blk, int K, int row0, int rows, uint32_t *w) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int words = K / 8;
  if (i >= (size_t)rows * words) return;
  const int r = (int)(i / words), c = (int)(i - (size_t)r * words);
  const int n = row0 + r, blk = n >> 8, cb = n & 255;
  uint32_t u = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint8_t byte = w_blk[((size_t)blk * K + 8 * c + e) * 128 + (cb >> 1)];
    const uint32_t q = (cb & 1) ? (byte >> 4) : (byte & 15u);
    u |= q << (4 * e);
  }
  w[i] = u;
}

__global__ void repack_sb_kernel(const uint16_t *s_blk, const uint16_t *b_blk, int G, int row0, int rows, uint16_t *s,
                                 uint16_t *b) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)rows * G) return;
  const int r = (int)(i / G), g = (int)(i - (size_t)r * G);
  const int n = row0 + r, blk = n >> 8, cb = n & 255;
  const size_t src = ((size_t)blk * G + g) * 256 + cb;
  s[i] = s_blk[src];
  b[i] = b_blk[src];
}

// ================================================================== dequant (checking)

template <int SD>
__global__ void dequant_kernel(const u32x4 *codes, const u32x4 *sb, int K, int N, float *out) {
  const int G = K / kGroup, G4 = quads_of(K), GP = 2 * G4;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)tiles_of(N) * GP * 64) return;
  const int l = (int)(i & 63);
  const size_t tp = i >> 6;
  const int t = (int)(tp / GP), p = (int)(tp - (size_t)t * GP);
  const int c = l & 15, j = l >> 4, n = 16 * t + c;
  if (n >= N) return;
  const u32x4 v = codes[i];
  const u32x4 q4 = sb[((size_t)t * G4 + (p >> 1)) * 16 + c];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int g = 2 * p + (e >> 1), sx = e & 1;
    if (g >= G) continue;
    const uint32_t pr = q4[2 * (p & 1) + (e >> 1)];
    const float sc = scale_f32<SD>((uint16_t)(pr & 0xFFFF));
    const float bi = scale_f32<SD>((uint16_t)(pr >> 16));
    float *o = out + (size_t)n * K + 64 * g + 32 * sx + 8 * j;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = __fmaf_rn(sc, (float)((v[e] >> (4 * k)) & 15u), bi);
  }
}

// ================================================================== decode GEMV (M <= 8)
//
// Grid: one workgroup per tile of 16 output features; W = ceil(groups / GPW) waves (at
// most 16; GPW in {8, 12, 16, 24} groups per wave, a function of K only) split the K groups into
// consecutive ranges, and their partial sums meet in LDS in wave order. No split of K
// across workgroups: every output is written by the workgroup that owns it, and the
// order of every sum depends only on K, never on M or on timing, so a token's result is
// the same whatever other tokens share the call.
//
// Each wave is single-shot, like a streaming copy: it issues every load of its range at
// once (the codes as one 16-byte load per lane per group pair: a contiguous kilobyte per
// wave instruction; the scale/bias quads; the activations), then multiplies and exits.
// Latency is hidden by the many short-lived waves the hardware keeps in flight, not by a
// software pipeline. Loads go through buffer descriptors whose range check returns zero
// past the end of a wave's range, so the code is straight-line. Codes and scales are read
// non-temporally (they are used once).
//
// One token (M = 1): each wave stages its activation range in LDS, in operand order.
// Several tokens: each wave has its token rows brought into LDS by DMA (8 groups at a
// time for ranges longer than 8 groups; L2-resident, shared by every workgroup) and
// reorders each operand in registers as it reads it. Either way the group sums come from
// an MFMA against a constant operand, which lands them in the accumulator layout, and
// every weight load of a wave is issued before its first multiply.
//
// The operand trick and the MFMA group sums are described in q4_tile.h.
//
// Split of K across workgroups (split_of): a weight with few tiles and a long K (the
// down projections: 320 tiles of 272 groups at 27B) leaves most CUs one workgroup or
// none, and its loads cannot fill the chip. There, the grid is (tiles, S): workgroup
// (t, s) takes groups [s * gsplit, (s + 1) * gsplit) of tile t, stores its partial sums
// in the workspace as agent-scope atomic stores, waits for them to complete and adds one
// to the tile's counter (an agent-scope atomic); the workgroup that brings the counter to
// S reads the S partials back (agent-scope atomic loads, issued after its increment
// returned), adds them in split order 0, 1, ... from zero, writes y and sets the counter
// back to zero. No workgroup waits for another. The split depends on K and N only, so a
// token's result is the same whatever other tokens share the call.
constexpr int kGemvMaxM = 8;
struct GemvArgs {
  const _Float16 *x;
  const u32x4 *codes;
  const u32x4 *sb;      // affine: scale/bias quads
  const float *srow;    // native books: the scale of each output row
  float *y;
  int x_stride, M, K, N, y_stride;
  int split, gsplit;    // K split: S workgroups per tile, gsplit groups each (S = 1: none)
  float *part;          // S > 1: partial sums [S][M][N]
  int *cnt;             // S > 1: arrivals per tile (zero between calls)
  // SWIGLU kernels: tile t (gate rows) pairs with tile t + up_off (the matching up rows),
  // and act[m][n] = half(silu(gate) * up) replaces y
  int up_off, act_stride;
  _Float16 *act;
};

// The workspace's first kGemvCountBytes hold the split counters (zero before the first
// call; every call leaves them zero); the partials and the prefill kernel's data follow.
constexpr size_t kGemvCountBytes = 4096;
static_assert(kGemvCountBytes == kGemmMaxCounters * sizeof(int), "the prefill split shares the counters");
// S for a weight: 7 where the tiles are few (7 tiles <= 2240 workgroups) and each split
// keeps at least 38 groups, else 1. The hand-over costs a few microseconds of latency at
// the end (partials out, the count, partials back), which pays where K is long: measured
// on the 27B down (K = 17408, N = 5120) at M = 1, 16.2 -> 13.3 us with 4 splits; on the 9B
// down (K = 12288, N = 4096) a split in 2 lost (7.5 -> 8.9 us). 7 rather than 4: at
// M = 8 a split of the 27B down stages 40 groups of 8 rows (40 KB of LDS), so four
// two-tile workgroups share a CU and its 1120 workgroups take 1.09 rounds of the chip,
// against 1.25 for 640 workgroups of 68 groups (70 KB, two per CU): 27B layer at M = 8
// 65.2 -> 62.2 us, M = 1 unchanged.
constexpr int kSplit = 7;
static int split_of(int K, int N) {
  const int G = K / kGroup, tiles = tiles_of(N);
  return (long long)tiles * kSplit <= 2240 && G / kSplit >= 38 ? kSplit : 1;
}
static int gsplit_of(int K, int S) { return ((K / kGroup + S - 1) / S + 3) / 4 * 4; }

// Groups per wave: the smallest of 8, 12, 16, 24 that needs at most 16 waves. Smaller
// ranges put more waves (and more loads) in flight per tile; below 8 the per-wave setup
// and the cross-wave reduction cost more than they hide (measured on the 9B and 27B
// projections at M = 1, 5, 8).
static int gemv_gpw(int K) {
  const int g = 4 * quads_of(K);
  return g <= 8 * 16 ? 8 : g <= 12 * 16 ? 12 : g <= 16 * 16 ? 16 : 24;
}
static int gemv_waves(int K) { const int g = gemv_gpw(K); return (4 * quads_of(K) + g - 1) / g; }
// the K a workgroup covers: all of K, or one split's groups
static int gemv_k_per_wg(int K, int N) {
  const int S = split_of(K, N);
  return S == 1 ? K : gsplit_of(K, S) * kGroup;
}
// The automatic choice takes the decode kernel for M <= 8 when its 16 waves cover K
// (K <= 24576); longer reductions at decode sizes go to the prefill kernel, which takes
// any K.
static bool decode_fits(int M, int K, int N) { return M <= kGemvMaxM && gemv_waves(gemv_k_per_wg(K, N)) <= 16; }

// M = 1: the cross-wave reduction [waves-1][64][4] floats, then each wave's staged
// activations [gpw * 64] halves. M > 1: each wave's staged rows, M * kStagedXRow bytes
// (its partial takes their place for the reduction).
static size_t gemv_lds_bytes(int M, int waves, int gpw) {
  if (M > 1) return (size_t)waves * M * kStagedXRow;
  return (size_t)(waves - 1) * 64 * 16 + (size_t)waves * gpw * kGroup * 2;
}

// The end of a split workgroup (see split_of), in the wave holding its NT tiles' sums
// (tiles t0 .. t0 + NT - 1, arrivals counted on counter c): stores the partials, counts
// the arrival and returns false, except in the tile's last workgroup, where acc[h] becomes
// the sum of the S partials in split order and true is returned.
template <int NT>
__device__ __forceinline__ bool split_arrive(const GemvArgs &a, int c, int t0, f32x4 (&acc)[NT], int lane) {
  const int M = a.M, c16 = lane & 15, j4 = lane >> 4;
  float *part = a.part + (size_t)blockIdx.y * M * a.N;
#pragma unroll
  for (int h = 0; h < NT; ++h) {
    const int n = 16 * (t0 + h) + c16;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * j4 + v;
      if (n < a.N && m < M)
        __hip_atomic_store(part + (size_t)m * a.N + n, acc[h][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);                // the partials are stored before the count
  int old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(a.cnt + c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);    // lane 0's: every lane is active again here
  if (old != kSplit - 1) return false;          // uniform: the tile's last workgroup goes on
  // every partial is requested before the first is added (one wait for all of them); the
  // lanes past M or N read a stored partial (their row and column clamped) and drop it
  float p[kSplit][NT][4];
#pragma unroll
  for (int q = 0; q < kSplit; ++q)
#pragma unroll
    for (int h = 0; h < NT; ++h) {
      const int n = min(16 * (t0 + h) + c16, a.N - 1);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = min(4 * j4 + v, M - 1);
        p[q][h][v] = __hip_atomic_load(a.part + ((size_t)q * M + m) * a.N + n, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
      }
    }
#pragma unroll
  for (int h = 0; h < NT; ++h)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float sum = 0.0f;
#pragma unroll
      for (int q = 0; q < kSplit; ++q) sum += p[q][h][v];
      acc[h][v] = sum;
    }
  if (lane == 0) __hip_atomic_store(a.cnt + c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// MAXM: 1 (single-token decode: one activation row, one live accumulator) or 8.
// BOOK: kAffine (per-group scale and bias) or a native codebook (one scale per row).
template <int MAXM, int GPW, int SD, bool ACC, int BOOK>
__global__ __launch_bounds__(1024) void gemv_q4a_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int waves = blockDim.x >> 6;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: scalar control flow
  const int c16 = lane & 15, j4 = lane >> 4;
  const int G = a.K / kGroup, G4 = quads_of(a.K);
  const int t = blockIdx.x;
  const int n = 16 * t + c16;
  const int M = a.M;
  f32x4 *red = reinterpret_cast<f32x4 *>(lds);                              // [waves-1][64]

  // this wave's groups [wg0, wg0 + GPW) of tile t within its split's [g_lo, g_hi); wn of
  // them are real (the loads stop at the split's end, rounded up to a quad)
  const int g_lo = blockIdx.y * a.gsplit, g_hi = min(G, g_lo + a.gsplit);
  const int wg0 = g_lo + wave * GPW;
  const int wn = max(0, min(g_hi, wg0 + GPW) - wg0);
  const WaveTile wt = wave_tile(a.codes, a.sb, t, G4, wg0, wn > 0 ? min(GPW, (wn + 3) / 4 * 4) : 0);
  const uint32_t xrange = wn > 0 ? (uint32_t)((M - 1) * a.x_stride + wn * kGroup) * 2u : 0u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (size_t)min(wg0, G) * kGroup, xrange);

  f32x4 acc = {}, asum = {};
  if constexpr (MAXM == 1) {
    // One token: the wave's activation row is loaded first (the loads complete in issue
    // order, so waiting for it does not wait for the weights), then every weight load is
    // issued; the row is staged in LDS in operand order while the weights are in flight.
    // Every lane reads row 0's operand: MFMA rows are independent and only row 0 of the
    // result is kept, so no zero rows are needed.
    constexpr int XCH = GPW * 8;                 // chunks of 8 activations in the wave's range
    constexpr int XPER = (XCH + 63) / 64;
    _Float16 *xs = reinterpret_cast<_Float16 *>(lds + (size_t)(waves - 1) * 64 * 16) + (size_t)wave * GPW * kGroup;
    u32x4 xr[XPER], wq[GPW / 2], sq[GPW / 4];
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
      const int chunk = lane + 64 * i;
      const bool in_range = chunk < XCH && (chunk >> 3) < wn;
      xr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, in_range ? 16u * chunk : kFarOffset, 0, 0));
    }
    issue_tile_loads<GPW, BOOK>(wt, lane, wq, sq);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
      const int chunk = lane + 64 * i;
      if (chunk < XCH) *reinterpret_cast<u32x4 *>(xs + 8 * chunk) = prep_act<BOOK>(xr[i]);
    }
    // other lanes of this wave read what was just written: keep the LDS reads after the writes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const _Float16 *xa = xs + 8 * j4;
    half8 an[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) an[s] = *reinterpret_cast<const half8 *>(xa + 32 * s);
#pragma unroll
    for (int jg = 0; jg < GPW; ++jg) {
      const half8 af[2] = {an[0], an[1]};
      if (jg + 1 < GPW) {
#pragma unroll
        for (int s = 0; s < 2; ++s) an[s] = *reinterpret_cast<const half8 *>(xa + (jg + 1) * kGroup + 32 * s);
      }
      book_step<GPW, SD, 1, BOOK>(acc, asum, af, wq, sq, jg);
      // Up to 12 groups per wave, a token's groups overlap in registers (measured 0.4-0.5 us
      // faster per 9B layer); larger ranges go one group at a time (bounded registers).
      if constexpr (GPW >= 16) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (BOOK == kInt16) acc[0] = __builtin_fmaf(0.5f, asum[0], acc[0]);
  } else {
    // Several tokens: the wave's rows are staged in LDS 8 groups at a time (its
    // M * kStagedXRow bytes at wave * M * kStagedXRow); lane (c16, j4) multiplies token
    // row c16, rows >= M are zeros.
    unsigned char *xs = lds + (size_t)wave * M * kStagedXRow;
    const uint32_t xstride = (uint32_t)a.x_stride * 2u;
    acc = tile_dot_rows_staged<GPW, SD, BOOK>(wt, rx, [=](int r) { return (uint32_t)r * xstride; }, M, xs, wn, lane);
    // the partials meet in wave order, as in reduce_waves, each in its wave's staging bytes
    if (wave > 0) reinterpret_cast<f32x4 *>(xs)[lane] = acc;
    __syncthreads();
    if (wave == 0)
      for (int w = 1; w < waves; ++w) {
        const f32x4 o = reinterpret_cast<const f32x4 *>(lds + (size_t)w * M * kStagedXRow)[lane];
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] += o[v];
      }
  }

  // lane (c16, j4) holds token rows 4 j4 .. 4 j4 + 3 of output n
  if constexpr (MAXM == 1) acc = reduce_waves(acc, red, wave, waves, lane);
  if (a.split > 1) {
    if (wave != 0) return;
    f32x4 accs[1] = {acc};
    if (!split_arrive<1>(a, t, t, accs, lane)) return;
    acc = accs[0];
  }
  if (wave == 0 && n < a.N && 4 * j4 < M) {
    const float rs = BOOK == kAffine || !a.srow ? 1.0f : a.srow[n];   // no row scales: the raw product
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * j4 + v;
      if (m < M) {
        float *dst = a.y + (size_t)m * a.y_stride + n;
        const float val = BOOK == kAffine ? acc[v] : rs * acc[v];
        *dst = ACC ? *dst + val : val;
      }
    }
  }
}

// Several tokens, two adjacent tiles per workgroup (t0 = 2 * block, t1 = t0 + 1): each wave
// reads its activation operands once for both tiles (tile_dot_rows2_staged). At M > 1 the
// activations are a wave's largest stream (a group's operands are M * 128 bytes against
// the 576 bytes of one tile's codes and scales, and they come from L2 once per tile), so
// pairing halves it; and they are staged in LDS by DMA together with the weight loads, so
// no group waits on an L2 read. Taken where a wave holds 8 groups: two tiles' loads then
// fit the registers one tile of 16 groups takes. Each tile's sums are the one-tile
// kernel's, in the same order, so the results do not depend on the pairing.
// SWIGLU (affine, no K split): the workgroup's tiles are gate tile t0 = block and up tile
// t1 = t0 + up_off, and it writes act = half(silu(gate) * up) for its 16 features instead
// of y (the gate/up product of a dense MLP with the SwiGLU fused; each tile's sums are the
// same, so act has the bits of the linear followed by moe_swiglu_kernel).
template <int GPW, int SD, bool ACC, int BOOK, bool SWIGLU = false>
__global__ __launch_bounds__(1024) void gemv_q4a_pair_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, j4 = lane >> 4;
  const int G = a.K / kGroup, G4 = quads_of(a.K);
  const int tiles = tiles_of(a.N);
  const int t0 = SWIGLU ? (int)blockIdx.x : 2 * blockIdx.x, t1 = SWIGLU ? t0 + a.up_off : t0 + 1;
  const int M = a.M;

  const int g_lo = blockIdx.y * a.gsplit, g_hi = min(G, g_lo + a.gsplit);   // the split's groups
  const int wg0 = g_lo + wave * GPW;
  const int wn = max(0, min(g_hi, wg0 + GPW) - wg0);
  const int wl = wn > 0 ? min(GPW, (wn + 3) / 4 * 4) : 0;                   // loads stop at the split's end
  const WaveTile w0 = wave_tile(a.codes, a.sb, t0, G4, wg0, wl);
  const WaveTile w1 = wave_tile(a.codes, a.sb, min(t1, tiles - 1), G4, wg0, t1 < tiles ? wl : 0);
  const uint32_t xrange = wn > 0 ? (uint32_t)((M - 1) * a.x_stride + wn * kGroup) * 2u : 0u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (size_t)min(wg0, G) * kGroup, xrange);
  // LDS: wave w's staged activation rows at w * M * kStagedXRow; once the wave is done with
  // them, its two partials (2 x 64 f32x4 <= 2 rows) take their place
  unsigned char *xs = lds + (size_t)wave * M * kStagedXRow;
  f32x4 acc0, acc1;
  tile_dot_rows2_staged<GPW, SD, BOOK>(w0, w1, rx, (uint32_t)a.x_stride * 2u, M, xs, wn, lane, acc0, acc1);

  // the waves' partials meet in wave order, as in reduce_waves
  if (wave > 0) {
    reinterpret_cast<f32x4 *>(xs)[lane] = acc0;
    reinterpret_cast<f32x4 *>(xs)[64 + lane] = acc1;
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < waves; ++w) {
    const f32x4 *red = reinterpret_cast<const f32x4 *>(lds + (size_t)w * M * kStagedXRow);
    const f32x4 o0 = red[lane], o1 = red[64 + lane];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc0[v] += o0[v];
      acc1[v] += o1[v];
    }
  }
  if constexpr (SWIGLU) {
    const int n = 16 * t0 + c16;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * j4 + v;
      if (m < M) a.act[(size_t)m * a.act_stride + n] = swiglu_half(acc0[v], acc1[v]);
    }
    return;
  }
  if (a.split > 1) {
    f32x4 accs[2] = {acc0, acc1};
    if (!split_arrive<2>(a, blockIdx.x, t0, accs, lane)) return;
    acc0 = accs[0];
    acc1 = accs[1];
  }
  if (4 * j4 >= M) return;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int n = 16 * (t0 + h) + c16;
    if (n >= a.N) continue;
    const float rs = BOOK == kAffine || !a.srow ? 1.0f : a.srow[n];   // no row scales: the raw product
    const f32x4 &acc = h ? acc1 : acc0;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * j4 + v;
      if (m < M) {
        float *dst = a.y + (size_t)m * a.y_stride + n;
        const float val = BOOK == kAffine ? acc[v] : rs * acc[v];
        *dst = ACC ? *dst + val : val;
      }
    }
  }
}

// One token, two adjacent tiles per workgroup (t0 = 2 * block, t1 = t0 + 1; affine, no K
// split): each wave stages its activation range once, issues both tiles' weight loads at
// once, and forms each group's sums once for both tiles. A weight of many tiles then takes
// half as many workgroups, each with twice the loads in flight. Each tile's products, sums
// and cross-wave order are gemv_q4a_kernel<1>'s, so the bits are the same.
// Held to 80 VGPRs (six waves per SIMD): three 8-wave workgroups then share a CU, 768 at
// once on the chip.
// SWIGLU: as gemv_q4a_pair_kernel's (gate tile t0 = block, up tile t0 + up_off, act out).
template <int GPW, int SD, bool ACC, bool SWIGLU = false>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(6))) void gemv_q4a_m1_pair_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, j4 = lane >> 4;
  const int G = a.K / kGroup, G4 = quads_of(a.K);
  const int tiles = tiles_of(a.N);
  const int t0 = SWIGLU ? (int)blockIdx.x : 2 * blockIdx.x, t1 = SWIGLU ? t0 + a.up_off : t0 + 1;
  f32x4 *red0 = reinterpret_cast<f32x4 *>(lds), *red1 = red0 + (size_t)(waves - 1) * 64;   // [waves-1][64] each

  const int wg0 = wave * GPW;
  const int wn = max(0, min(G, wg0 + GPW) - wg0);
  const int wl = wn > 0 ? min(GPW, (wn + 3) / 4 * 4) : 0;
  const WaveTile w0 = wave_tile(a.codes, a.sb, t0, G4, wg0, wl);
  const WaveTile w1 = wave_tile(a.codes, a.sb, min(t1, tiles - 1), G4, wg0, t1 < tiles ? wl : 0);
  const uint32_t xrange = wn > 0 ? (uint32_t)(wn * kGroup) * 2u : 0u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (size_t)min(wg0, G) * kGroup, xrange);

  // as gemv_q4a_kernel<1>: the activation row first, then every weight load, the row staged
  // in LDS in operand order while the weights are in flight
  constexpr int XCH = GPW * 8;
  constexpr int XPER = (XCH + 63) / 64;
  _Float16 *xs = reinterpret_cast<_Float16 *>(lds + (size_t)2 * (waves - 1) * 64 * 16) + (size_t)wave * GPW * kGroup;
  u32x4 xr[XPER], wq0[GPW / 2], sq0[GPW / 4], wq1[GPW / 2], sq1[GPW / 4];
#pragma unroll
  for (int i = 0; i < XPER; ++i) {
    const int chunk = lane + 64 * i;
    const bool in_range = chunk < XCH && (chunk >> 3) < wn;
    xr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, in_range ? 16u * chunk : kFarOffset, 0, 0));
  }
  issue_tile_loads<GPW, kAffine>(w0, lane, wq0, sq0);
  issue_tile_loads<GPW, kAffine>(w1, lane, wq1, sq1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < XPER; ++i) {
    const int chunk = lane + 64 * i;
    if (chunk < XCH) *reinterpret_cast<u32x4 *>(xs + 8 * chunk) = prep_x8(xr[i]);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const _Float16 *xa = xs + 8 * j4;
  half8 an[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) an[s] = *reinterpret_cast<const half8 *>(xa + 32 * s);
  f32x4 acc0 = {}, acc1 = {};
#pragma unroll
  for (int jg = 0; jg < GPW; ++jg) {
    const half8 af[2] = {an[0], an[1]};
    if (jg + 1 < GPW) {
#pragma unroll
      for (int s = 0; s < 2; ++s) an[s] = *reinterpret_cast<const half8 *>(xa + (jg + 1) * kGroup + 32 * s);
    }
    const f32x4 gsv = group_sums(af);
    group_step_gs<GPW, SD, 1>(acc0, af, gsv, wq0, sq0, jg);
    group_step_gs<GPW, SD, 1>(acc1, af, gsv, wq1, sq1, jg);
  }

  // the waves' partials meet in wave order, as in reduce_waves
  if (wave > 0) {
    red0[(wave - 1) * 64 + lane] = acc0;
    red1[(wave - 1) * 64 + lane] = acc1;
  }
  __syncthreads();
  if (wave != 0 || j4 != 0) return;
  for (int w = 1; w < waves; ++w) {
    const f32x4 o0 = red0[(w - 1) * 64 + lane], o1 = red1[(w - 1) * 64 + lane];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc0[v] += o0[v];
      acc1[v] += o1[v];
    }
  }
  if constexpr (SWIGLU) {
    a.act[16 * t0 + c16] = swiglu_half(acc0[0], acc1[0]);
    return;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int n = 16 * (t0 + h) + c16;
    if (n < a.N) {
      float *dst = a.y + n;
      const float val = h ? acc1[0] : acc0[0];
      *dst = ACC ? *dst + val : val;
    }
  }
}

// the partials of a split weight (the counters sit in the workspace's first kGemvCountBytes)
static size_t gemv_workspace(int M, int K, int N) {
  const int S = split_of(K, N);
  return S == 1 ? 0 : (size_t)S * std::min(M, kGemvMaxM) * N * 4;
}

// PAIR: the two-tile kernel (M > 1 only).
template <int MAXM, int GPW, int SD, bool ACC, int BOOK, bool PAIR>
static int launch_gemv_inst(dim3 grid, int threads, size_t lds, hipStream_t st, const GemvArgs &a) {
  static LdsOptIn lds_opt;  // per instance and device, before its first launch there
  if constexpr (PAIR) {
    if (int rc = allow_large_lds(reinterpret_cast<const void *>(&gemv_q4a_pair_kernel<GPW, SD, ACC, BOOK>), lds_opt))
      return rc;
    gemv_q4a_pair_kernel<GPW, SD, ACC, BOOK><<<grid, threads, lds, st>>>(a);
  } else {
    if (int rc = allow_large_lds(reinterpret_cast<const void *>(&gemv_q4a_kernel<MAXM, GPW, SD, ACC, BOOK>), lds_opt))
      return rc;
    gemv_q4a_kernel<MAXM, GPW, SD, ACC, BOOK><<<grid, threads, lds, st>>>(a);
  }
  return 0;
}

template <int MAXM, int GPW, int BOOK, bool PAIR>
static int launch_gemv_acc(int sd, int accum, dim3 grid, int threads, size_t lds, hipStream_t st, const GemvArgs &a) {
  if constexpr (BOOK == kAffine) {
    if (sd == RLQ_BF16)
      return accum ? launch_gemv_inst<MAXM, GPW, 1, true, BOOK, PAIR>(grid, threads, lds, st, a)
                   : launch_gemv_inst<MAXM, GPW, 1, false, BOOK, PAIR>(grid, threads, lds, st, a);
  }
  return accum ? launch_gemv_inst<MAXM, GPW, 0, true, BOOK, PAIR>(grid, threads, lds, st, a)
               : launch_gemv_inst<MAXM, GPW, 0, false, BOOK, PAIR>(grid, threads, lds, st, a);
}

template <int MAXM, int GPW, bool PAIR = false>
static int launch_gemv(int book, int sd, int accum, dim3 grid, int threads, size_t lds, hipStream_t st,
                       const GemvArgs &a) {
  switch (book) {
    case kInt15: return launch_gemv_acc<MAXM, GPW, kInt15, PAIR>(sd, accum, grid, threads, lds, st, a);
    case kInt16: return launch_gemv_acc<MAXM, GPW, kInt16, PAIR>(sd, accum, grid, threads, lds, st, a);
    case kFp4: return launch_gemv_acc<MAXM, GPW, kFp4, PAIR>(sd, accum, grid, threads, lds, st, a);
    default: return launch_gemv_acc<MAXM, GPW, kAffine, PAIR>(sd, accum, grid, threads, lds, st, a);
  }
}

// book: kAffine (packed holds codes then scale/bias quads; sd their dtype) or a native
// codebook (packed holds codes only; srow the row scales).
// M > 1 with 8 groups per wave: two tiles per workgroup (each activation operand read once
// for both) unless the grid is small (under 1024 tile splits) and the staged rows take at
// most 48 KB, where one tile per workgroup puts twice the workgroups to work (three share
// a CU): 9B layer at M = 5 37.6 -> 36.5 us; at the 27B qkv and o (80 KB of rows at M = 8)
// the pairs stay faster. Both kernels give the same bits.
static bool pair_tiles(int M, int K, int N) {
  const int S = split_of(K, N);
  return (long long)tiles_of(N) * S >= 1024 || (long long)M * (S == 1 ? K : gsplit_of(K, S) * kGroup) > 24576;
}

// One token on a weight of at least this many tiles (and no K split) takes two tiles per
// workgroup (gemv_q4a_m1_pair_kernel): the output head (15520 tiles, about 15 rounds of
// the chip with one tile per workgroup) pays each workgroup's start (staging the row, the
// reduction, the stores) half as often: 248320 x 4096 at M = 1 100.5-105.7 -> 92.4-94.5
// us. Below it one tile per workgroup stays: the 9B gate_up (1536 tiles) measured the same
// or slightly slower paired (11.3-12.1 against 11.6-11.7 us), the 27B gate_up (2176
// tiles) 1 us slower alone.
constexpr int kM1PairTiles = 4096;

template <int SD, bool ACC>
static int launch_m1_pair(int tiles, int threads, size_t lds, hipStream_t st, const GemvArgs &a) {
  static LdsOptIn lds_opt;
  if (int rc = allow_large_lds(reinterpret_cast<const void *>(&gemv_q4a_m1_pair_kernel<8, SD, ACC>), lds_opt))
    return rc;
  gemv_q4a_m1_pair_kernel<8, SD, ACC><<<(tiles + 1) / 2, threads, lds, st>>>(a);
  return 0;
}

static int run_gemv(int book, const _Float16 *x, int x_stride, int M, int K, int N, const void *codes, const void *sbq,
                    int sd, const float *srow, float *y, int y_stride, int accum, int *cnt, float *part,
                    size_t part_bytes, hipStream_t st) {
  RLQ_REQUIRE(M <= kGemvMaxM, "decode kernel handles M <= %d rows (got %d)", kGemvMaxM, M);
  const int S = split_of(K, N), kw = gemv_k_per_wg(K, N);
  const int gpw = gemv_gpw(kw), waves = gemv_waves(kw);
  RLQ_REQUIRE(waves <= 16, "decode kernel: K=%d is larger than the %d it supports", K, 16 * 24 * kGroup);
  if (S > 1)
    RLQ_REQUIRE(cnt && part && part_bytes >= gemv_workspace(M, K, N),
                "decode kernel: K=%d N=%d splits K in %d and needs rlq_linear_workspace_bytes(%d, %d, %d) = %zu bytes "
                "of workspace (got %zu)", K, N, S, M, K, N, kGemvCountBytes + gemv_workspace(M, K, N),
                part_bytes + (cnt ? kGemvCountBytes : 0));
  const size_t lds = gemv_lds_bytes(M, waves, gpw);
  GemvArgs a;
  a.x = x;
  a.codes = static_cast<const u32x4 *>(codes);
  a.sb = static_cast<const u32x4 *>(sbq);
  a.srow = srow;
  a.y = y;
  a.x_stride = x_stride; a.M = M; a.K = K; a.N = N; a.y_stride = y_stride;
  a.split = S;
  a.gsplit = S == 1 ? K / kGroup : gsplit_of(K, S);
  a.part = S == 1 ? nullptr : part;
  a.cnt = S == 1 ? nullptr : cnt;
  const dim3 grid(tiles_of(N), S);
  const int threads = 64 * waves;
  int rc;
  if (M == 1 && gpw == 8 && S == 1 && book == kAffine && tiles_of(N) >= kM1PairTiles) {
    const size_t lds2 = (size_t)2 * (waves - 1) * 64 * 16 + (size_t)waves * gpw * kGroup * 2;
    rc = sd == RLQ_BF16 ? (accum ? launch_m1_pair<1, true>(tiles_of(N), threads, lds2, st, a)
                                 : launch_m1_pair<1, false>(tiles_of(N), threads, lds2, st, a))
                        : (accum ? launch_m1_pair<0, true>(tiles_of(N), threads, lds2, st, a)
                                 : launch_m1_pair<0, false>(tiles_of(N), threads, lds2, st, a));
  } else if (M == 1) rc = gpw == 8    ? launch_gemv<1, 8>(book, sd, accum, grid, threads, lds, st, a)
                   : gpw == 12 ? launch_gemv<1, 12>(book, sd, accum, grid, threads, lds, st, a)
                   : gpw == 16 ? launch_gemv<1, 16>(book, sd, accum, grid, threads, lds, st, a)
                               : launch_gemv<1, 24>(book, sd, accum, grid, threads, lds, st, a);
  else if (gpw == 8 && pair_tiles(M, K, N))   // two tiles per workgroup, activations staged in LDS
    rc = launch_gemv<kGemvMaxM, 8, true>(book, sd, accum, dim3((tiles_of(N) + 1) / 2, S), threads, lds, st, a);
  else rc = gpw == 8 ? launch_gemv<kGemvMaxM, 8>(book, sd, accum, grid, threads, lds, st, a)
            : gpw == 12 ? launch_gemv<kGemvMaxM, 12>(book, sd, accum, grid, threads, lds, st, a)
            : gpw == 16 ? launch_gemv<kGemvMaxM, 16>(book, sd, accum, grid, threads, lds, st, a)
                        : launch_gemv<kGemvMaxM, 24>(book, sd, accum, grid, threads, lds, st, a);
  if (rc) return rc;
  RLQ_HIP(hipGetLastError());
  return 0;
}

template <int SD>
static int launch_swiglu(int M, int I, int waves, const GemvArgs &a, hipStream_t st) {
  static LdsOptIn lds1, lds2;
  if (M == 1) {
    const void *fn = reinterpret_cast<const void *>(&gemv_q4a_m1_pair_kernel<8, SD, false, true>);
    if (int rc = allow_large_lds(fn, lds1)) return rc;
    const size_t lds = (size_t)2 * (waves - 1) * 64 * 16 + (size_t)waves * 8 * kGroup * 2;
    gemv_q4a_m1_pair_kernel<8, SD, false, true><<<I / 16, 64 * waves, lds, st>>>(a);
  } else {
    const void *fn = reinterpret_cast<const void *>(&gemv_q4a_pair_kernel<8, SD, false, kAffine, true>);
    if (int rc = allow_large_lds(fn, lds2)) return rc;
    gemv_q4a_pair_kernel<8, SD, false, kAffine, true><<<I / 16, 64 * waves, gemv_lds_bytes(M, waves, 8), st>>>(a);
  }
  RLQ_HIP(hipGetLastError());
  return 0;
}

int linear_swiglu_packed(const _Float16 *x, int x_stride, int M, int K, int I, const void *codes, const void *sbq,
                         int sd, _Float16 *act, int act_stride, hipStream_t st) {
  if (M < 1 || M > kGemvMaxM || I < 16 || I % 16 || gemv_gpw(K) != 8 || gemv_waves(K) > 16 || split_of(K, 2 * I) != 1)
    return 1;
  GemvArgs a = {};
  a.x = x;
  a.codes = static_cast<const u32x4 *>(codes);
  a.sb = static_cast<const u32x4 *>(sbq);
  a.x_stride = x_stride; a.M = M; a.K = K; a.N = 2 * I;
  a.split = 1;
  a.gsplit = K / kGroup;
  a.up_off = I / 16;
  a.act = act;
  a.act_stride = act_stride;
  const int waves = gemv_waves(K);
  return sd == RLQ_BF16 ? launch_swiglu<1>(M, I, waves, a, st) : launch_swiglu<0>(M, I, waves, a, st);
}

int linear_packed(int kernel, int book, const _Float16 *x, int x_stride, int M, int K, int N, const void *codes,
                  const void *sbq, int sd, const float *srow, float *y, int y_stride, int accum, void *ws,
                  size_t ws_bytes, hipStream_t st) {
  RLQ_REQUIRE(kernel >= 0 && kernel <= 2, "unknown kernel %d", kernel);
  // the workspace: split counters first, then the decode partials or the prefill kernel's data
  const bool has_ws = ws && ws_bytes >= kGemvCountBytes;
  int *cnt = has_ws ? static_cast<int *>(ws) : nullptr;
  void *rest = has_ws ? static_cast<char *>(ws) + kGemvCountBytes : nullptr;
  const size_t rest_bytes = has_ws ? ws_bytes - kGemvCountBytes : 0;
  const bool gemv = kernel == 1 || (kernel == 0 && decode_fits(M, K, N));
  if (gemv)
    return run_gemv(book, x, x_stride, M, K, N, codes, sbq, sd, srow, y, y_stride, accum, cnt,
                    static_cast<float *>(rest), rest_bytes, st);
  return run_gemm4(book, x, x_stride, M, K, N, codes, sbq, sd, srow, y, y_stride, accum, cnt, rest, rest_bytes, st);
}

// ================================================================== group sums

// gsum[m][g] and/or its transpose gsT[g][m_pad], summed sequentially in fp32 as
// group_sums does (kernels/linear.metal:34-45).
__global__ void group_sums_kernel(const _Float16 *x, int x_stride, int M, int K, float *gsum, float *gsT, int m_pad) {
  const int G = K / kGroup;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * G) return;
  const int m = idx / G, g = idx - m * G;
  const half8 *xp = reinterpret_cast<const half8 *>(x + (size_t)m * x_stride + (size_t)g * kGroup);
  float sum = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const half8 v = xp[c];
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += static_cast<float>(v[e]);
  }
  if (gsum) gsum[(size_t)m * G + g] = sum;
  if (gsT) gsT[(size_t)g * m_pad + m] = sum;
}

// asum[m] = sum over g of gsT[g][m], in order: the activation row sums the half-step
// codebook needs.
__global__ void row_sums_kernel(const float *gsT, int G, int m_pad, int M, float *asum) {
  const int m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  float s = 0.0f;
  for (int g = 0; g < G; ++g) s += gsT[(size_t)g * m_pad + m];
  asum[m] = s;
}

void launch_group_sums(const _Float16 *x, int x_stride, int M, int K, float *gsT, int m_pad, hipStream_t st) {
  const int G = K / kGroup;
  group_sums_kernel<<<(M * G + 255) / 256, 256, 0, st>>>(x, x_stride, M, K, nullptr, gsT, m_pad);
}

void launch_row_sums(const float *gsT, int G, int m_pad, int M, float *asum, hipStream_t st) {
  row_sums_kernel<<<(M + 255) / 256, 256, 0, st>>>(gsT, G, m_pad, M, asum);
}

static int check_linear_args(const char *fn, const void *x, int x_stride, int M, int K, int N, const void *packed,
                             int sd, const float *y, int y_stride) {
  RLQ_REQUIRE(M >= 1 && N >= 1 && K >= kGroup, "%s: bad sizes M=%d K=%d N=%d", fn, M, K, N);
  RLQ_REQUIRE(K % kGroup == 0, "%s: K=%d is not a multiple of the group size 64", fn, K);
  RLQ_REQUIRE(N <= 16 * kMaxTiles, "%s: N=%d exceeds the supported %d", fn, N, 16 * kMaxTiles);
  RLQ_REQUIRE(sd == RLQ_F16 || sd == RLQ_BF16, "%s: unknown scale dtype %d", fn, sd);
  RLQ_REQUIRE(x && packed && y, "%s: null pointer argument", fn);
  RLQ_REQUIRE(x_stride >= K && x_stride % 8 == 0, "%s: x_stride=%d must be >= K and a multiple of 8", fn, x_stride);
  RLQ_REQUIRE(y_stride >= N, "%s: y_stride=%d < N=%d", fn, y_stride, N);
  RLQ_REQUIRE(aligned(x, 16) && aligned(packed, 16), "%s: x and the packed weight must be 16-byte aligned", fn);
  RLQ_REQUIRE(aligned(y, 4), "%s: misaligned y", fn);
  return 0;
}

}  // namespace rlq

using namespace rlq;

extern "C" {

size_t rlq_packed_affine_bytes(int K, int N) {
  if (K <= 0 || N <= 0 || K % kGroup) return 0;
  return packed_bytes(K, N);
}

static int pack_mlx(const char *who, const uint32_t *w, const void *s, const void *b, int K, int N, int il,
                    void *packed, void *stream) {
  RLQ_REQUIRE(N >= 1 && K >= kGroup && K % kGroup == 0, "%s: bad sizes K=%d N=%d", who, K, N);
  RLQ_REQUIRE(w && s && b && packed, "%s: null pointer argument", who);
  RLQ_REQUIRE(aligned(w, 4) && aligned(packed, 16), "%s: misaligned w or packed", who);
  RLQ_REQUIRE(aligned(s, 2) && aligned(b, 2), "%s: misaligned scales or biases", who);
  const size_t pieces = (size_t)tiles_of(N) * 2 * quads_of(K) * 64;
  RLQ_REQUIRE(pieces < (1ull << 31), "%s: K=%d N=%d is too large to pack in one launch", who, K, N);
  auto codes = static_cast<u32x4 *>(packed);
  auto sb = reinterpret_cast<u32x4 *>(static_cast<char *>(packed) + packed_code_bytes(K, N));
  pack_mlx_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      w, static_cast<const uint16_t *>(s), static_cast<const uint16_t *>(b), K, N, il, codes, sb);
  RLQ_HIP(hipGetLastError());
  return 0;
}

int rlq_pack_affine(const uint32_t *w, const void *s, const void *b, int K, int N, void *packed, void *stream) {
  return pack_mlx("rlq_pack_affine", w, s, b, K, N, 0, packed, stream);
}

int rlq_pack_moe_gate_up(const uint32_t *w, const void *s, const void *b, int H, int E1, int I, void *packed,
                         void *stream) {
  RLQ_REQUIRE(E1 >= 1 && I >= 8 && I % 8 == 0, "rlq_pack_moe_gate_up: %d experts of I=%d (I must be a multiple of 8)",
              E1, I);
  RLQ_REQUIRE((long long)E1 * 2 * I <= 16LL * kMaxTiles, "rlq_pack_moe_gate_up: %d x %d rows is too many", E1, 2 * I);
  return pack_mlx("rlq_pack_moe_gate_up", w, s, b, H, E1 * 2 * I, I, packed, stream);
}

int rlq_pack_affine_blocked(const uint8_t *w_blk, const uint16_t *s_blk, const uint16_t *b_blk, int K, int n_pad,
                            int row0, int rows, void *packed, void *stream) {
  RLQ_REQUIRE(K >= kGroup && K % kGroup == 0, "rlq_pack_affine_blocked: K=%d is not a multiple of 64", K);
  RLQ_REQUIRE(n_pad % 256 == 0 && n_pad > 0, "rlq_pack_affine_blocked: n_pad=%d is not a multiple of the block 256",
              n_pad);
  RLQ_REQUIRE(row0 >= 0 && rows >= 1 && row0 + rows <= n_pad, "rlq_pack_affine_blocked: rows [%d, %d) outside [0, %d)",
              row0, row0 + rows, n_pad);
  RLQ_REQUIRE(w_blk && s_blk && b_blk && packed, "rlq_pack_affine_blocked: null pointer argument");
  RLQ_REQUIRE(aligned(packed, 16), "rlq_pack_affine_blocked: packed must be 16-byte aligned");
  const size_t pieces = (size_t)tiles_of(rows) * 2 * quads_of(K) * 64;
  auto codes = static_cast<u32x4 *>(packed);
  auto sb = reinterpret_cast<u32x4 *>(static_cast<char *>(packed) + packed_code_bytes(K, rows));
  pack_blocked_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      w_blk, s_blk, b_blk, K, row0, rows, codes, sb);
  RLQ_HIP(hipGetLastError());
  return 0;
}

size_t rlq_packed_codes_bytes(int K, int N) {
  if (K <= 0 || N <= 0 || K % kGroup) return 0;
  return packed_code_bytes(K, N);
}

int rlq_pack_codes(const uint32_t *w, int K, int N, void *packed, void *stream) {
  // N is not limited to what one linear call takes: an expert stack (rlq_moe_linear_native)
  // can hold more rows than that
  RLQ_REQUIRE(N >= 1 && K >= kGroup && K % kGroup == 0, "rlq_pack_codes: bad sizes K=%d N=%d", K, N);
  RLQ_REQUIRE(w && packed, "rlq_pack_codes: null pointer argument");
  RLQ_REQUIRE(aligned(w, 4) && aligned(packed, 16), "rlq_pack_codes: misaligned w or packed");
  const size_t pieces = (size_t)tiles_of(N) * 2 * quads_of(K) * 64;
  RLQ_REQUIRE(pieces < (1ull << 31), "rlq_pack_codes: K=%d N=%d is too large to pack in one launch", K, N);
  pack_mlx_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      w, nullptr, nullptr, K, N, 0, static_cast<u32x4 *>(packed), nullptr);
  RLQ_HIP(hipGetLastError());
  return 0;
}

int rlq_pack_native_blocked(const uint8_t *w_blk, int K, int n_pad, int row0, int rows, void *packed, void *stream) {
  RLQ_REQUIRE(K >= kGroup && K % kGroup == 0, "rlq_pack_native_blocked: K=%d is not a multiple of 64", K);
  RLQ_REQUIRE(n_pad % 256 == 0 && n_pad > 0, "rlq_pack_native_blocked: n_pad=%d is not a multiple of the block 256",
              n_pad);
  RLQ_REQUIRE(row0 >= 0 && rows >= 1 && row0 + rows <= n_pad, "rlq_pack_native_blocked: rows [%d, %d) outside [0, %d)",
              row0, row0 + rows, n_pad);
  RLQ_REQUIRE(w_blk && packed, "rlq_pack_native_blocked: null pointer argument");
  RLQ_REQUIRE(aligned(packed, 16), "rlq_pack_native_blocked: packed must be 16-byte aligned");
  const size_t pieces = (size_t)tiles_of(rows) * 2 * quads_of(K) * 64;
  pack_blocked_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      w_blk, nullptr, nullptr, K, row0, rows, static_cast<u32x4 *>(packed), nullptr);
  RLQ_HIP(hipGetLastError());
  return 0;
}

int rlq_linear_native_kernel(int kernel, const void *x, int x_stride, int M, int K, int N, const void *packed,
                             const float *s_row, int book, float *y, int y_stride, int accum, void *workspace,
                             size_t workspace_bytes, void *stream) {
  int rc = check_linear_args("rlq_linear_native", x, x_stride, M, K, N, packed, RLQ_F16, y, y_stride);
  if (rc) return rc;
  RLQ_REQUIRE(book == RLQ_BOOK_INT15 || book == RLQ_BOOK_INT16 || book == RLQ_BOOK_FP4,
              "rlq_linear_native: unknown codebook %d", book);
  RLQ_REQUIRE(s_row && aligned(s_row, 4), "rlq_linear_native: null or misaligned row scales");
  RLQ_REQUIRE(kernel >= 0 && kernel <= 2, "rlq_linear_native_kernel: unknown kernel %d", kernel);
  // native matrices have no scale/bias section: the codes stand in for it (never read)
  return linear_packed(kernel, book, static_cast<const _Float16 *>(x), x_stride, M, K, N, packed, packed, RLQ_F16,
                       s_row, y, y_stride, accum, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int rlq_linear_native_raw(const void *x, int x_stride, int M, int K, int N, const void *packed, int book, float *y,
                          int y_stride, void *workspace, size_t workspace_bytes, void *stream) {
  int rc = check_linear_args("rlq_linear_native_raw", x, x_stride, M, K, N, packed, RLQ_F16, y, y_stride);
  if (rc) return rc;
  RLQ_REQUIRE(book == RLQ_BOOK_INT15 || book == RLQ_BOOK_FP4,
              "rlq_linear_native_raw: codebook %d (int15 or fp4: the raw product has no half step)", book);
  return linear_packed(0, book, static_cast<const _Float16 *>(x), x_stride, M, K, N, packed, packed, RLQ_F16, nullptr,
                       y, y_stride, 0, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int rlq_linear_native(const void *x, int x_stride, int M, int K, int N, const void *packed, const float *s_row,
                      int book, float *y, int y_stride, int accum, void *workspace, size_t workspace_bytes,
                      void *stream) {
  return rlq_linear_native_kernel(0, x, x_stride, M, K, N, packed, s_row, book, y, y_stride, accum, workspace,
                                  workspace_bytes, stream);
}

size_t rlq_linear_workspace_bytes(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 0 || K % kGroup) return 0;
  // the split counters, then the largest of the decode partials (up to 8 rows: a workspace
  // sized for M serves every smaller M) and the books' prefill data
  return kGemvCountBytes + std::max({gemv_workspace(std::min(M, kGemvMaxM), K, N), gemm4_workspace(kAffine, M, K, N),
                                     gemm4_workspace(kInt16, M, K, N), gemm4_workspace(kInt15, M, K, N)});
}

int rlq_linear_affine_kernel(int kernel, const void *x, int x_stride, int M, int K, int N, const void *packed,
                             int scale_dtype, float *y, int y_stride, int accum, void *workspace,
                             size_t workspace_bytes, void *stream) {
  int rc = check_linear_args("rlq_linear_affine", x, x_stride, M, K, N, packed, scale_dtype, y, y_stride);
  if (rc) return rc;
  RLQ_REQUIRE(kernel >= 0 && kernel <= 2, "rlq_linear_affine_kernel: unknown kernel %d", kernel);
  const void *sbq = static_cast<const char *>(packed) + packed_code_bytes(K, N);
  return linear_packed(kernel, kAffine, static_cast<const _Float16 *>(x), x_stride, M, K, N, packed, sbq, scale_dtype,
                       nullptr, y, y_stride, accum, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int rlq_linear_affine(const void *x, int x_stride, int M, int K, int N, const void *packed, int scale_dtype, float *y,
                      int y_stride, int accum, void *workspace, size_t workspace_bytes, void *stream) {
  return rlq_linear_affine_kernel(0, x, x_stride, M, K, N, packed, scale_dtype, y, y_stride, accum, workspace,
                                  workspace_bytes, stream);
}

int rlq_group_sums(const void *x, int x_stride, int M, int K, float *gsum, void *stream) {
  RLQ_REQUIRE(M >= 1 && K >= kGroup && K % kGroup == 0, "rlq_group_sums: bad sizes M=%d K=%d", M, K);
  RLQ_REQUIRE(x && gsum, "rlq_group_sums: null pointer argument");
  RLQ_REQUIRE(x_stride >= K && x_stride % 8 == 0 && aligned(x, 16), "rlq_group_sums: x must be 16-byte aligned rows");
  const int G = K / kGroup;
  group_sums_kernel<<<(M * G + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const _Float16 *>(x), x_stride, M, K, gsum, nullptr, 0);
  RLQ_HIP(hipGetLastError());
  return 0;
}

int rlq_dequant_affine(const void *packed, int scale_dtype, int K, int N, float *out, void *stream) {
  RLQ_REQUIRE(N >= 1 && K >= kGroup && K % kGroup == 0, "rlq_dequant_affine: bad sizes K=%d N=%d", K, N);
  RLQ_REQUIRE(packed && out, "rlq_dequant_affine: null pointer argument");
  RLQ_REQUIRE(scale_dtype == RLQ_F16 || scale_dtype == RLQ_BF16, "rlq_dequant_affine: unknown scale dtype %d",
              scale_dtype);
  RLQ_REQUIRE(aligned(packed, 16), "rlq_dequant_affine: packed must be 16-byte aligned");
  const size_t pieces = (size_t)tiles_of(N) * 2 * quads_of(K) * 64;
  const unsigned blocks = (unsigned)((pieces + 255) / 256);
  auto st = static_cast<hipStream_t>(stream);
  auto codes = static_cast<const u32x4 *>(packed);
  auto sb = reinterpret_cast<const u32x4 *>(static_cast<const char *>(packed) + packed_code_bytes(K, N));
  if (scale_dtype == RLQ_F16) dequant_kernel<0><<<blocks, 256, 0, st>>>(codes, sb, K, N, out);
  else dequant_kernel<1><<<blocks, 256, 0, st>>>(codes, sb, K, N, out);
  RLQ_HIP(hipGetLastError());
  return 0;
}

int rlq_repack_blocked(const uint8_t *w_blk, const uint16_t *s_blk, const uint16_t *b_blk, int K, int n_pad, int row0,
                       int rows, uint32_t *w, uint16_t *s, uint16_t *b, void *stream) {
  RLQ_REQUIRE(K >= kGroup && K % kGroup == 0, "rlq_repack_blocked: K=%d is not a multiple of 64", K);
  RLQ_REQUIRE(n_pad % 256 == 0 && n_pad > 0, "rlq_repack_blocked: n_pad=%d is not a multiple of the block 256", n_pad);
  RLQ_REQUIRE(row0 >= 0 && rows >= 1 && row0 + rows <= n_pad, "rlq_repack_blocked: rows [%d, %d) outside [0, %d)", row0,
              row0 + rows, n_pad);
  RLQ_REQUIRE(w_blk && s_blk && b_blk && w && s && b, "rlq_repack_blocked: null pointer argument");
  auto st = static_cast<hipStream_t>(stream);
  const size_t words = (size_t)rows * (K / 8);
  repack_w_kernel<<<(unsigned)((words + 255) / 256), 256, 0, st>>>(w_blk, K, row0, rows, w);
  RLQ_HIP(hipGetLastError());
  const size_t sbn = (size_t)rows * (K / kGroup);
  repack_sb_kernel<<<(unsigned)((sbn + 255) / 256), 256, 0, st>>>(s_blk, b_blk, K / kGroup, row0, rows, s, b);
  RLQ_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
