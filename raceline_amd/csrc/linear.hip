// Affine 4-bit group-quantized linear layer on gfx950: decode GEMV, prefill GEMM,
// group sums, a dequantizing check kernel and the blocked->MLX upload repack.
//
//   y[m][n] = sum_k x[m][k] * W[n][k],   W[n][k] = s[n][g] * q[n][k] + b[n][g],  g = k / 64
//
// evaluated, like the reference kernel (kernels/linear.metal:5-9,85-101), as
//   y[m][n] = sum_g ( s[n][g] * (x_g . q_g)[m][n] + b[n][g] * gsum[m][g] )
// so the weights are never dequantized in software: the integer codes go to the
// matrix cores as exact fp16 values and the scale and bias are applied per group
// to the fp32 partial product.
//
// Matrix-core operand layout (v_mfma_f32_32x32x16_f16, wave64):
//   A (32 x 16): lane l holds row l%32, k = 8*(l/32) .. +7
//   B (16 x 32): lane l holds col l%32, k = 8*(l/32) .. +7
//   D (32 x 32): lane l, element v holds col l%32, row 8*(v/4) + 4*(l/32) + v%4
// A is the activations (rows = tokens), B the weights (cols = output features). Per
// group of 64 the lane with k-half h = l/32 feeds the four 8-element chunks
// k = 32h + 8t (t = 0..3) of one 16-byte load of its weight row, so one group is four
// MFMAs and each weight row is read as 32 contiguous bytes per group.
#include "rlq_common.h"
#include "../../include/rlq.h"

#include <algorithm>

namespace rlq {

constexpr int kGroup = 64;
constexpr int kGemvMaxGps = 128;  // groups of one split of the decode kernel (LDS bound)

// Workspace layout: a fixed area of split-K counters first (kept zero between calls, so it
// must not move with the shape of a call), then the per-call scratch (partials, group sums).
constexpr int kMaxTiles = 16384;                                   // N <= 32 * kMaxTiles
constexpr size_t kCounterBytes = (size_t)kMaxTiles * sizeof(unsigned);

// ================================================================== decode GEMV (M <= 32)
//
// Grid (ceil(N/32), ksplit); 256 threads = 4 waves. A workgroup owns 32 output
// features and `gps` consecutive groups of K; its four waves take consecutive quarters
// of those groups, and their partial sums meet in LDS in a fixed order. When K is split
// over workgroups (small N: the GPU needs >= ~1000 workgroups to fill 256 CUs), each
// writes its partial [split][M][N] to the workspace and the last one to finish a column
// tile (a counter per tile) adds them in split order and writes y. The order of every
// sum depends only on (K, N), never on M or on timing, so a token's result is the same
// whatever other tokens share the call.
struct GemvArgs {
  const _Float16 *x;
  const uint32_t *w;
  const uint16_t *s;
  const uint16_t *b;
  float *y;
  float *part;
  unsigned *counters;
  int x_stride, M, K, N, y_stride;
  int ksplit, gps;
};

template <int NV, int SD, bool ACC>
__global__ __launch_bounds__(256) void gemv_q4a_kernel(GemvArgs a) {
  constexpr int MT = 8 * NV;  // token rows covered: acc quads 0..NV-1
  __shared__ __attribute__((aligned(16))) float gs[kGemvMaxGps][MT];
  __shared__ __attribute__((aligned(16))) float red[3][64][4 * NV];
  __shared__ int last;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int n0 = blockIdx.x * 32;
  const int n = n0 + col;
  const bool nvalid = n < a.N;
  const int G = a.K / kGroup;
  const int g0 = blockIdx.y * a.gps;
  const int g1 = min(G, g0 + a.gps);
  const int ng = g1 - g0;

  // Group sums of the activations over this split's groups, summed sequentially in
  // fp32 as group_sums does (kernels/linear.metal:34-45). Rows >= M are zero.
  for (int idx = tid; idx < MT * ng; idx += 256) {
    const int m = idx / ng, gl = idx - m * ng;
    float sum = 0.0f;
    if (m < a.M) {
      const half8 *xp = reinterpret_cast<const half8 *>(a.x + (size_t)m * a.x_stride + (size_t)(g0 + gl) * kGroup);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const half8 v = xp[c];
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += static_cast<float>(v[e]);
      }
    }
    gs[gl][m] = sum;
  }
  __syncthreads();

  const int wpg = (ng + 3) >> 2;
  const int wg0 = g0 + wave * wpg;
  const int wg1 = min(g1, wg0 + wpg);

  const uint32_t *wrow = a.w + (size_t)(nvalid ? n : 0) * (a.K / 8) + 4 * h;
  const bool xvalid = col < a.M;
  const _Float16 *xrow = a.x + (size_t)(xvalid ? col : 0) * a.x_stride + 32 * h;
  const uint16_t *srow = a.s + (size_t)(nvalid ? n : 0) * G;
  const uint16_t *brow = a.b + (size_t)(nvalid ? n : 0) * G;

  f32x16 acc = {};
  const half8 hz = {};

  auto group_step = [&](int g, u32x4 wq, const half8 *xa) {
    f32x16 p = {};
#pragma unroll
    for (int t = 0; t < 4; ++t) p = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[t], nib8_to_half8(wq[t]), p, 0, 0, 0);
    const float sc = nvalid ? scale_f32<SD>(srow[g]) * kTwo24 : 0.0f;
    const float bi = nvalid ? scale_f32<SD>(brow[g]) : 0.0f;
    const float *gsg = gs[g - g0];
#pragma unroll
    for (int q = 0; q < NV; ++q) {
      const f32x4 gq = *reinterpret_cast<const f32x4 *>(gsg + 8 * q + 4 * h);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[4 * q + r] += sc * p[4 * q + r] + bi * gq[r];
    }
  };

  int g = wg0;
  for (; g + 4 <= wg1; g += 4) {
    u32x4 wq[4];
    half8 xa[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) wq[j] = nvalid ? *reinterpret_cast<const u32x4 *>(wrow + 8 * (g + j)) : u32x4{};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xa[j][t] = xvalid ? *reinterpret_cast<const half8 *>(xrow + kGroup * (g + j) + 8 * t) : hz;
#pragma unroll
    for (int j = 0; j < 4; ++j) group_step(g + j, wq[j], xa[j]);
  }
  for (; g < wg1; ++g) {
    const u32x4 wq = nvalid ? *reinterpret_cast<const u32x4 *>(wrow + 8 * g) : u32x4{};
    half8 xa[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) xa[t] = xvalid ? *reinterpret_cast<const half8 *>(xrow + kGroup * g + 8 * t) : hz;
    group_step(g, wq, xa);
  }

  // Waves 1..3 hand their partials to wave 0, which adds them in wave order.
  if (wave > 0) {
#pragma unroll
    for (int v = 0; v < 4 * NV; ++v) red[wave - 1][lane][v] = acc[v];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
      for (int v = 0; v < 4 * NV; ++v) acc[v] += red[w][lane][v];
  }

  if (a.ksplit == 1) {
    if (wave == 0 && nvalid) {
#pragma unroll
      for (int v = 0; v < 4 * NV; ++v) {
        const int m = 8 * (v >> 2) + 4 * h + (v & 3);
        if (m < a.M) {
          float *dst = a.y + (size_t)m * a.y_stride + n;
          *dst = ACC ? *dst + acc[v] : acc[v];
        }
      }
    }
    return;
  }

  // Split K: publish this split's partial, then count it. The partials are agent-scope
  // atomic stores (coherent across the XCDs' L2s) and the wave waits for them to complete
  // before the counter moves, so the last workgroup, reading them with agent-scope atomic
  // loads, sees every one. No fence: an agent-scope fence writes back and invalidates the
  // whole L2, which serialises thousands of workgroups.
  float *P = a.part + (size_t)blockIdx.y * a.M * a.N;
  if (wave == 0) {
    if (nvalid) {
#pragma unroll
      for (int v = 0; v < 4 * NV; ++v) {
        const int m = 8 * (v >> 2) + 4 * h + (v & 3);
        if (m < a.M) __hip_atomic_store(P + (size_t)m * a.N + n, acc[v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(a.counters + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      last = (prev == (unsigned)(a.ksplit - 1));
    }
  }
  __syncthreads();
  if (!last) return;
  for (int idx = tid; idx < a.M * 32; idx += 256) {
    const int m = idx >> 5, nn = n0 + (idx & 31);
    if (nn >= a.N) continue;
    float sum = 0.0f;
    const float *src = a.part + (size_t)m * a.N + nn;
    for (int sp = 0; sp < a.ksplit; ++sp)
      sum += __hip_atomic_load(src + (size_t)sp * a.M * a.N, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float *dst = a.y + (size_t)m * a.y_stride + nn;
    *dst = ACC ? *dst + sum : sum;
  }
  if (tid == 0) __hip_atomic_store(a.counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split of K over workgroups for the decode kernel. A function of (K, N) only, so the
// summation order of an output never depends on M.
struct GemvPlan {
  int ntiles, ksplit, gps;
};

static GemvPlan gemv_plan(int K, int N) {
  GemvPlan p;
  const int G = K / kGroup;
  p.ntiles = (N + 31) / 32;
  int ks = std::max(1, (1024 + p.ntiles - 1) / p.ntiles);
  ks = std::min(ks, std::max(1, G / 4));
  ks = std::max(ks, (G + kGemvMaxGps - 1) / kGemvMaxGps);
  int gps = (G + ks - 1) / ks;
  gps = (gps + 3) / 4 * 4;
  gps = std::min(gps, kGemvMaxGps);
  p.gps = gps;
  p.ksplit = (G + gps - 1) / gps;
  return p;
}

static size_t gemv_workspace(int M, int K, int N) {
  const GemvPlan p = gemv_plan(K, N);
  if (p.ksplit == 1) return 0;
  return kCounterBytes + (size_t)p.ksplit * M * N * sizeof(float);
}

template <int SD, bool ACC>
static void launch_gemv(int nv, dim3 grid, hipStream_t st, const GemvArgs &a) {
  switch (nv) {
    case 1: gemv_q4a_kernel<1, SD, ACC><<<grid, 256, 0, st>>>(a); break;
    case 2: gemv_q4a_kernel<2, SD, ACC><<<grid, 256, 0, st>>>(a); break;
    case 3: gemv_q4a_kernel<3, SD, ACC><<<grid, 256, 0, st>>>(a); break;
    default: gemv_q4a_kernel<4, SD, ACC><<<grid, 256, 0, st>>>(a); break;
  }
}

static int run_gemv(const _Float16 *x, int x_stride, int M, int K, int N, const uint32_t *w, const uint16_t *s,
                    const uint16_t *b, int sd, float *y, int y_stride, int accum, void *ws, size_t ws_bytes,
                    hipStream_t st) {
  RLQ_REQUIRE(M <= 32, "decode kernel handles M <= 32 rows (got %d)", M);
  const GemvPlan p = gemv_plan(K, N);
  const size_t need = gemv_workspace(M, K, N);
  RLQ_REQUIRE(ws_bytes >= need, "workspace of %zu bytes is smaller than the %zu this call needs", ws_bytes, need);
  RLQ_REQUIRE(need == 0 || aligned(ws, 16), "workspace must be 16-byte aligned");
  GemvArgs a;
  a.x = x; a.w = w; a.s = s; a.b = b; a.y = y;
  a.counters = static_cast<unsigned *>(ws);
  a.part = need ? reinterpret_cast<float *>(static_cast<char *>(ws) + kCounterBytes) : nullptr;
  a.x_stride = x_stride; a.M = M; a.K = K; a.N = N; a.y_stride = y_stride;
  a.ksplit = p.ksplit; a.gps = p.gps;
  const int nv = (M + 7) / 8;
  const dim3 grid(p.ntiles, p.ksplit);
  if (sd == RLQ_F16) {
    if (accum) launch_gemv<0, true>(nv, grid, st, a); else launch_gemv<0, false>(nv, grid, st, a);
  } else {
    if (accum) launch_gemv<1, true>(nv, grid, st, a); else launch_gemv<1, false>(nv, grid, st, a);
  }
  RLQ_HIP(hipGetLastError());
  return 0;
}

// ================================================================== group sums

// gsum[m][g] (row stride gs_stride) and, when gsT != null, the transpose gsT[g][m_pad].
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

// ================================================================== prefill GEMM (M > 32)
//
// Workgroup tile 128 (tokens) x 128 (features), 4 waves as 2 x 2, each 64 x 64 = 2 x 2
// MFMA tiles. Per group of 64: the activation tile goes through LDS (shared by the two
// waves of a row band); each wave loads its own 64 weight rows' 32 bytes straight into
// B operands and turns them into exact fp16 codes in registers; four MFMAs per tile
// give the group's partial product, then acc += s * part + b * gsum.
struct GemmArgs {
  const _Float16 *x;
  const uint32_t *w;
  const uint16_t *s;
  const uint16_t *b;
  const float *gsT;  // [G][m_pad]
  float *y;
  int x_stride, M, K, N, y_stride, m_pad;
};

constexpr int kBM = 128, kBN = 128, kLdsRow = 64 + 8;

template <int SD, bool ACC>
__global__ __launch_bounds__(256) void gemm_q4a_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 As[kBM * kLdsRow];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int G = a.K / kGroup;

  int nrow[2];
  bool nval[2];
  const uint32_t *wr[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    nrow[ct] = n0 + wn * 64 + ct * 32 + col;
    nval[ct] = nrow[ct] < a.N;
    wr[ct] = a.w + (size_t)(nval[ct] ? nrow[ct] : 0) * (a.K / 8) + 4 * h;
  }

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  for (int g = 0; g < G; ++g) {
    // activation tile [128][64] -> LDS: 1024 chunks of 8 halves, 4 per thread
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int chunk = tid + 256 * c;
      const int r = chunk >> 3, kc = chunk & 7;
      const int m = m0 + r;
      half8 v = {};
      if (m < a.M) v = *reinterpret_cast<const half8 *>(a.x + (size_t)m * a.x_stride + (size_t)g * kGroup + 8 * kc);
      *reinterpret_cast<half8 *>(As + r * kLdsRow + 8 * kc) = v;
    }
    u32x4 wq[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) wq[ct] = nval[ct] ? *reinterpret_cast<const u32x4 *>(wr[ct] + 8 * g) : u32x4{};
    __syncthreads();

    half8 bf[2][4];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int t = 0; t < 4; ++t) bf[ct][t] = nib8_to_half8(wq[ct][t]);

#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      half8 af[4];
      const _Float16 *arow = As + (wm * 64 + rt * 32 + col) * kLdsRow + 32 * h;
#pragma unroll
      for (int t = 0; t < 4; ++t) af[t] = *reinterpret_cast<const half8 *>(arow + 8 * t);
      const f32x4 *gsp = reinterpret_cast<const f32x4 *>(a.gsT + (size_t)g * a.m_pad + m0 + wm * 64 + rt * 32 + 4 * h);
      f32x4 gq[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) gq[q] = gsp[2 * q];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        f32x16 p = {};
#pragma unroll
        for (int t = 0; t < 4; ++t) p = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[t], bf[ct][t], p, 0, 0, 0);
        const float sc = nval[ct] ? scale_f32<SD>(a.s[(size_t)nrow[ct] * G + g]) * kTwo24 : 0.0f;
        const float bi = nval[ct] ? scale_f32<SD>(a.b[(size_t)nrow[ct] * G + g]) : 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[rt][ct][4 * q + r] += sc * p[4 * q + r] + bi * gq[q][r];
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      if (!nval[ct]) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 64 + rt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (m < a.M) {
          float *dst = a.y + (size_t)m * a.y_stride + nrow[ct];
          *dst = ACC ? *dst + acc[rt][ct][v] : acc[rt][ct][v];
        }
      }
    }
}

static size_t gemm_workspace(int M, int K) {
  const int m_pad = (M + kBM - 1) / kBM * kBM;
  return kCounterBytes + (size_t)(K / kGroup) * m_pad * sizeof(float);
}

static int run_gemm(const _Float16 *x, int x_stride, int M, int K, int N, const uint32_t *w, const uint16_t *s,
                    const uint16_t *b, int sd, float *y, int y_stride, int accum, void *ws, size_t ws_bytes,
                    hipStream_t st) {
  const size_t need = gemm_workspace(M, K);
  RLQ_REQUIRE(ws_bytes >= need, "workspace of %zu bytes is smaller than the %zu this call needs", ws_bytes, need);
  RLQ_REQUIRE(aligned(ws, 16), "workspace must be 16-byte aligned");
  const int m_pad = (M + kBM - 1) / kBM * kBM;
  float *gsT = reinterpret_cast<float *>(static_cast<char *>(ws) + kCounterBytes);
  // rows M..m_pad of gsT are never read for output rows >= M; they only need to be finite
  const int G = K / kGroup;
  group_sums_kernel<<<(M * G + 255) / 256, 256, 0, st>>>(x, x_stride, M, K, nullptr, gsT, m_pad);
  RLQ_HIP(hipGetLastError());
  GemmArgs a;
  a.x = x; a.w = w; a.s = s; a.b = b; a.gsT = gsT; a.y = y;
  a.x_stride = x_stride; a.M = M; a.K = K; a.N = N; a.y_stride = y_stride; a.m_pad = m_pad;
  const dim3 grid((N + kBN - 1) / kBN, m_pad / kBM);
  if (sd == RLQ_F16) {
    if (accum) gemm_q4a_kernel<0, true><<<grid, 256, 0, st>>>(a);
    else gemm_q4a_kernel<0, false><<<grid, 256, 0, st>>>(a);
  } else {
    if (accum) gemm_q4a_kernel<1, true><<<grid, 256, 0, st>>>(a);
    else gemm_q4a_kernel<1, false><<<grid, 256, 0, st>>>(a);
  }
  RLQ_HIP(hipGetLastError());
  return 0;
}

// ================================================================== dequant (checking)

template <int SD>
__global__ void dequant_kernel(const uint32_t *w, const uint16_t *s, const uint16_t *b, int K, int N, float *out) {
  const size_t words = (size_t)N * (K / 8);
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int n = (int)(i / (K / 8));
  const int c = (int)(i - (size_t)n * (K / 8));
  const int g = (8 * c) / kGroup;
  const float sc = scale_f32<SD>(s[(size_t)n * (K / kGroup) + g]);
  const float bi = scale_f32<SD>(b[(size_t)n * (K / kGroup) + g]);
  const uint32_t u = w[i];
  float *o = out + (size_t)n * K + 8 * c;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = __fmaf_rn(sc, (float)((u >> (4 * e)) & 15u), bi);
}

// ================================================================== blocked -> MLX repack

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

static int check_linear_args(const char *fn, const void *x, int x_stride, int M, int K, int N, const uint32_t *w,
                             const void *s, const void *b, int sd, const float *y, int y_stride) {
  RLQ_REQUIRE(M >= 1 && N >= 1 && K >= kGroup, "%s: bad sizes M=%d K=%d N=%d", fn, M, K, N);
  RLQ_REQUIRE(N <= 32 * kMaxTiles, "%s: N=%d exceeds the supported %d", fn, N, 32 * kMaxTiles);
  RLQ_REQUIRE(K % kGroup == 0, "%s: K=%d is not a multiple of the group size 64", fn, K);
  RLQ_REQUIRE(sd == RLQ_F16 || sd == RLQ_BF16, "%s: unknown scale dtype %d", fn, sd);
  RLQ_REQUIRE(x && w && s && b && y, "%s: null pointer argument", fn);
  RLQ_REQUIRE(x_stride >= K && x_stride % 8 == 0, "%s: x_stride=%d must be >= K and a multiple of 8", fn, x_stride);
  RLQ_REQUIRE(y_stride >= N, "%s: y_stride=%d < N=%d", fn, y_stride, N);
  RLQ_REQUIRE(aligned(x, 16) && aligned(w, 16), "%s: x and w must be 16-byte aligned", fn);
  RLQ_REQUIRE(aligned(s, 2) && aligned(b, 2) && aligned(y, 4), "%s: misaligned s, b or y", fn);
  return 0;
}

}  // namespace rlq

using namespace rlq;

extern "C" {

size_t rlq_linear_workspace_bytes(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 0 || K % kGroup) return 0;
  return std::max(M <= 32 ? gemv_workspace(M, K, N) : (size_t)0, gemm_workspace(M, K));
}

int rlq_linear_affine_kernel(int kernel, const void *x, int x_stride, int M, int K, int N, const uint32_t *w,
                             const void *s, const void *b, int scale_dtype, float *y, int y_stride, int accum,
                             void *workspace, size_t workspace_bytes, void *stream) {
  int rc = check_linear_args("rlq_linear_affine", x, x_stride, M, K, N, w, s, b, scale_dtype, y, y_stride);
  if (rc) return rc;
  RLQ_REQUIRE(kernel >= 0 && kernel <= 2, "rlq_linear_affine_kernel: unknown kernel %d", kernel);
  const bool gemv = kernel == 1 || (kernel == 0 && M <= 32);
  auto st = static_cast<hipStream_t>(stream);
  auto xh = static_cast<const _Float16 *>(x);
  auto sh = static_cast<const uint16_t *>(s);
  auto bh = static_cast<const uint16_t *>(b);
  if (gemv)
    return run_gemv(xh, x_stride, M, K, N, w, sh, bh, scale_dtype, y, y_stride, accum, workspace, workspace_bytes, st);
  return run_gemm(xh, x_stride, M, K, N, w, sh, bh, scale_dtype, y, y_stride, accum, workspace, workspace_bytes, st);
}

int rlq_linear_affine(const void *x, int x_stride, int M, int K, int N, const uint32_t *w, const void *s,
                      const void *b, int scale_dtype, float *y, int y_stride, int accum, void *workspace,
                      size_t workspace_bytes, void *stream) {
  return rlq_linear_affine_kernel(0, x, x_stride, M, K, N, w, s, b, scale_dtype, y, y_stride, accum, workspace,
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

int rlq_dequant_affine(const uint32_t *w, const void *s, const void *b, int scale_dtype, int K, int N, float *out,
                       void *stream) {
  RLQ_REQUIRE(N >= 1 && K >= kGroup && K % kGroup == 0, "rlq_dequant_affine: bad sizes K=%d N=%d", K, N);
  RLQ_REQUIRE(w && s && b && out, "rlq_dequant_affine: null pointer argument");
  RLQ_REQUIRE(scale_dtype == RLQ_F16 || scale_dtype == RLQ_BF16, "rlq_dequant_affine: unknown scale dtype %d",
              scale_dtype);
  const size_t words = (size_t)N * (K / 8);
  const unsigned blocks = (unsigned)((words + 255) / 256);
  auto st = static_cast<hipStream_t>(stream);
  if (scale_dtype == RLQ_F16)
    dequant_kernel<0><<<blocks, 256, 0, st>>>(w, static_cast<const uint16_t *>(s), static_cast<const uint16_t *>(b), K, N, out);
  else
    dequant_kernel<1><<<blocks, 256, 0, st>>>(w, static_cast<const uint16_t *>(s), static_cast<const uint16_t *>(b), K, N, out);
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
  const size_t sb = (size_t)rows * (K / kGroup);
  repack_sb_kernel<<<(unsigned)((sb + 255) / 256), 256, 0, st>>>(s_blk, b_blk, K / kGroup, row0, rows, s, b);
  RLQ_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
