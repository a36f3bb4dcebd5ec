// Prefill GEMM on gfx950 for the 4-bit formats (affine and native codebooks), M > 8.
//
//   affine: y[m][n] = sum_g s[n][g] * (x_g . q_g)[m][n] + b[n][g] * gsum[m][g]
//   native: y[m][n] = s[n] * (x . L(q))[m][n]  (+ 0.5 s[n] rowsum[m] for the half-step book)
//
// Workgroup tile 128 tokens x 256 features, 8 waves as 2 x 4, each 64 x 64 = 4 x 4
// v_mfma_f32_16x16x32_f16 tiles. The K loop runs over group pairs (128 inputs):
//  - the activation tile [128][128] of the next pair streams straight from memory into
//    one of two LDS buffers (buffer_load ... lds: no registers, no VALU), while the MFMAs
//    work on the other; rows are stored with their 16-byte chunks XOR-swizzled by the row
//    so the MFMA operand reads hit 16 distinct chunks;
//  - each wave's packed codes (one 16-byte load per lane per 16-row tile: the tile layout
//    of q4_tile.h) and scales of the next pair are prefetched into registers;
//  - codes become exact fp16 values in registers; a wave converts each of its 4 feature
//    tiles once per group and reuses them over its 4 token tiles.
// Affine: the activations are first rewritten by a prep pass into the operand order of
// q4_tile.h (x0, x4, x1/16, x5/16, ...), matching the cheap code conversion, and the per
// group epilogue is a single FMA per output (acc += s * part): the bias term
// sum_g b[n][g] gsum[m][g] is one more MFMA product at the end, over K' = 2G, with the
// group sums split into fp16 hi + lo (exact to 2^-22) and b as the other operand.
// Native books: activations are used as they are, codes decode in element order, and the
// products chain in the MFMA over all of K with the row scale applied at the end.
// A row's result depends only on its own activations (MFMA rows are independent).
#include "gemm.h"
#include "q4_tile.h"
#include "../../include/rlq.h"

#include <algorithm>

namespace rlq {

constexpr int kGM = 128, kGN = 256;         // workgroup tile
constexpr int kGThreads = 512;
constexpr int kARowBytes = 256;             // one pair of groups: 128 fp16
constexpr int kABufBytes = kGM * kARowBytes;

// Eight codes (oddx16 element order of q4_tile.h) -> exact normal fp16: (q0, q4),
// (16 q1, 16 q5), (q2, q6), (16 q3, 16 q7).
__device__ __forceinline__ half8 nib8_to_half8_oddx16_exact(uint32_t u) {
  const uint32_t t = u >> 8;
  u32x4 d;
  d[0] = magic_pair_to_f16(u & 0x000F000Fu);
  d[1] = magic_pair_to_f16(u & 0x00F000F0u);
  d[2] = magic_pair_to_f16(t & 0x000F000Fu);
  d[3] = magic_pair_to_f16(t & 0x00F000F0u);
  return __builtin_bit_cast(half8, d);
}

// ------------------------------------------------------------------ affine prep pass

// xp[m][k]: x in operand order (prep_x8 per 8 elements); gshl[m][2g], [2g+1]: the group
// sum (sequential fp32, as kernels/linear.metal:42-44) split into fp16 hi and lo.
__global__ void gemm_prep_kernel(const _Float16 *x, int x_stride, int M, int K, _Float16 *xp, _Float16 *gshl,
                                 int gs_stride) {
  const int G = K / kGroup;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * G) return;
  const int m = idx / G, g = idx - m * G;
  const u32x4 *src = reinterpret_cast<const u32x4 *>(x + (size_t)m * x_stride + (size_t)g * kGroup);
  u32x4 *dst = reinterpret_cast<u32x4 *>(xp + (size_t)m * K + (size_t)g * kGroup);
  float sum = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const u32x4 v = src[c];
    const half8 h = __builtin_bit_cast(half8, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += static_cast<float>(h[e]);
    dst[c] = prep_x8(v);
  }
  const _Float16 hi = static_cast<_Float16>(sum);
  const _Float16 lo = static_cast<_Float16>(sum - static_cast<float>(hi));
  gshl[(size_t)m * gs_stride + 2 * g] = hi;
  gshl[(size_t)m * gs_stride + 2 * g + 1] = lo;
  if (g == G - 1)   // the row's padding up to gs_stride is zero (no memset: this runs in graphs)
    for (int k = 2 * G; k < gs_stride; ++k) gshl[(size_t)m * gs_stride + k] = (_Float16)0.0f;
}

// ------------------------------------------------------------------ the GEMM

template <int BOOK, int SD, bool ACC>
__global__ __launch_bounds__(kGThreads) void gemm4_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, j4 = lane >> 4;
  const int wm = wave >> 2, wn = wave & 3;
  const int G = a.K / kGroup, G4 = quads_of(a.K), GP = 2 * G4;
  const int NP = (G + 1) / 2;                        // group pairs with real groups
  const int T = tiles_of(a.N);

  // Workgroups are numbered round-robin over the 8 XCDs; give each XCD a contiguous
  // range of tiles, token blocks fastest, so the workgroups of one XCD share feature
  // blocks (weights) in its L2.
  const int nwg = gridDim.x, wid = blockIdx.x;
  const int per_xcd = (nwg + 7) / 8;
  int lin = (wid % 8) * per_xcd + wid / 8;
  if (nwg % 8 != 0) lin = wid;                      // uneven grids keep the plain order
  const int mblocks = (a.M + kGM - 1) / kGM;
  const int mb = lin % mblocks, nb = lin / mblocks;
  const int m0 = mb * kGM, n0 = nb * kGN;

  // activation descriptor: the whole [M][x_stride] matrix; rows >= M read zeros
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.M * a.x_stride * 2));
  // this thread's four 16-byte chunks of each activation tile
  uint32_t a_off[4];
  bool a_row[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * (4 * wave + i) + (lane >> 4);   // row within the tile
    const int c = (lane & 15) ^ (r & 15);             // logical chunk stored at this lane's slot
    a_off[i] = (uint32_t)(((size_t)(m0 + r) * a.x_stride + 8 * c) * 2);
    a_row[i] = m0 + r < a.M;
  }
  auto issue_a = [&](int p, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * (4 * wave + i) + (lane >> 4);
      const int c = (lane & 15) ^ (r & 15);
      const bool ok = a_row[i] && 128 * p + 8 * c < a.K;   // inputs past K read zero
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rx, (__attribute__((address_space(3))) void *)(lds + (size_t)buf * kABufBytes + (size_t)(4 * wave + i) * 1024),
          16, ok ? a_off[i] + (uint32_t)(256 * p) : kFarOffset, 0, 0, 0);
    }
  };

  // weights: this wave's 4 feature tiles
  int tile[4];
#pragma unroll
  for (int ft = 0; ft < 4; ++ft) tile[ft] = (n0 >> 4) + wn * 4 + ft;
  __amdgpu_buffer_rsrc_t rw[4], rs[4];
#pragma unroll
  for (int ft = 0; ft < 4; ++ft) {
    const bool tv = tile[ft] < T;
    rw[ft] = make_rsrc(a.codes + (size_t)(tv ? tile[ft] : 0) * GP * 64, tv ? (uint32_t)GP * 1024u : 0u);
    rs[ft] = make_rsrc(a.sb + (size_t)(tv ? tile[ft] : 0) * G4 * 16, (BOOK == kAffine && tv) ? (uint32_t)G4 * 256u : 0u);
  }
  u32x4 wq[4], wq_n[4];
  uint32_t sp[4][2], sp_n[4][2];     // affine: (s|b) of groups 2p, 2p+1 per tile
  auto issue_b = [&](int p, u32x4 (&w)[4], uint32_t (&s)[4][2]) {
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) {
      w[ft] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw[ft], 16u * lane, (uint32_t)p * 1024u, 0));
      if constexpr (BOOK == kAffine) {
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                      rs[ft], 16u * c16 + 8u * (p & 1), (uint32_t)(p >> 1) * 256u, 0));
        s[ft][0] = v[0];
        s[ft][1] = v[1];
      }
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{};

  issue_a(0, 0);
  issue_b(0, wq, sp);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int p = 0; p < NP; ++p) {
    const int buf = p & 1;
    if (p + 1 < NP) {
      issue_a(p + 1, buf ^ 1);
      issue_b(p + 1, wq_n, sp_n);
    }
    const unsigned char *abuf = lds + (size_t)buf * kABufBytes;
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      half8 bf[4][2];
#pragma unroll
      for (int ft = 0; ft < 4; ++ft)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const uint32_t u = wq[ft][2 * gg + s];
          if constexpr (BOOK == kAffine) bf[ft][s] = nib8_to_half8_oddx16_exact(u);
          else bf[ft][s] = native8_to_half8<BOOK>(u);
        }
      float sc[4];
      if constexpr (BOOK == kAffine) {
#pragma unroll
        for (int ft = 0; ft < 4; ++ft) sc[ft] = scale_f32<SD>((uint16_t)(sp[ft][gg] & 0xFFFFu));
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int r = wm * 64 + mt * 16 + c16;
        half8 af[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int c = 8 * gg + 4 * s + j4;
          af[s] = *reinterpret_cast<const half8 *>(abuf + r * kARowBytes + ((c ^ c16) << 4));
        }
#pragma unroll
        for (int ft = 0; ft < 4; ++ft) {
          if constexpr (BOOK == kAffine) {
            f32x4 pp = {};
#pragma unroll
            for (int s = 0; s < 2; ++s) pp = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], bf[ft][s], pp, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[mt][ft][v] = __builtin_fmaf(sc[ft], pp[v], acc[mt][ft][v]);
          } else {
#pragma unroll
            for (int s = 0; s < 2; ++s)
              acc[mt][ft] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], bf[ft][s], acc[mt][ft], 0, 0, 0);
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);     // the next pair's activations (LDS) and weights (registers)
    __syncthreads();                   // ... are there for every wave, and this buffer is free
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) {
      wq[ft] = wq_n[ft];
      sp[ft][0] = sp_n[ft][0];
      sp[ft][1] = sp_n[ft][1];
    }
  }

  if constexpr (BOOK == kAffine) {
    // acc += sum_g b[n][g] * gsum[m][g]: an MFMA product over K' = 2G (hi, lo per group)
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(a.gshl, (uint32_t)((size_t)a.M * a.gs_stride * 2));
    const int steps = a.gs_stride / 32;
    for (int st = 0; st < steps; ++st) {
      half8 bb[4];
#pragma unroll
      for (int ft = 0; ft < 4; ++ft) {
        const int q = 4 * st + j4;                   // quad of groups 4q .. 4q+3
        const u32x4 v = q < G4 ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                               rs[ft], 16u * c16, (uint32_t)q * 256u, 0))
                               : u32x4{};
        u32x4 d;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t bbits = v[e] >> 16;
          uint32_t h;
          if constexpr (SD == 0) {
            h = bbits;
          } else {
            h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(__uint_as_float(bbits << 16)));
          }
          d[e] = h | (h << 16);                       // (b, b): times gsum hi and lo
        }
        bb[ft] = __builtin_bit_cast(half8, d);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int m = m0 + wm * 64 + mt * 16 + c16;
        const half8 ag = __builtin_bit_cast(
            half8, __builtin_amdgcn_raw_buffer_load_b128(
                       rg, m < a.M ? (uint32_t)(((size_t)m * a.gs_stride + 32 * st + 8 * j4) * 2) : kFarOffset, 0, 0));
        // the bias MFMA uses K' = 32 per step: lane (c16, j4) holds k' = 8 j4 .. +7, i.e.
        // groups 4 j4' .. +3 of this step (two k' per group)
#pragma unroll
        for (int ft = 0; ft < 4; ++ft) acc[mt][ft] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ag, bb[ft], acc[mt][ft], 0, 0, 0);
      }
    }
  }

#pragma unroll
  for (int ft = 0; ft < 4; ++ft) {
    const int n = 16 * tile[ft] + c16;
    if (n >= a.N) continue;
    const float rs_n = BOOK == kAffine ? 1.0f : a.srow[n];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm * 64 + mt * 16 + 4 * j4 + v;
        if (m < a.M) {
          float val = acc[mt][ft][v];
          if constexpr (BOOK == kInt16) val = __builtin_fmaf(0.5f, a.asum[m], val);
          if constexpr (BOOK != kAffine) val *= rs_n;
          float *dst = a.y + (size_t)m * a.y_stride + n;
          *dst = ACC ? *dst + val : val;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ host

size_t gemm4_workspace(int book, int M, int K) {
  const int G = K / kGroup;
  const size_t gs_stride = (size_t)(2 * G + 31) / 32 * 32;
  if (book == kAffine) return ((size_t)M * K * 2 + 255) / 256 * 256 + (size_t)M * gs_stride * 2;
  if (book == kInt16) return (size_t)(G + 1) * ((M + 127) / 128 * 128) * sizeof(float);
  return 0;
}

template <int BOOK, int SD>
static void launch_gemm4_inst(int accum, dim3 grid, size_t lds, hipStream_t st, const GemmArgs &a) {
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm4_kernel<BOOK, SD, true>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm4_kernel<BOOK, SD, false>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    attr_set = true;
  }
  if (accum) gemm4_kernel<BOOK, SD, true><<<grid, kGThreads, lds, st>>>(a);
  else gemm4_kernel<BOOK, SD, false><<<grid, kGThreads, lds, st>>>(a);
}

int run_gemm4(int book, const _Float16 *x, int x_stride, int M, int K, int N, const void *packed, int sd,
              const float *srow, float *y, int y_stride, int accum, void *ws, size_t ws_bytes, hipStream_t st) {
  const int G = K / kGroup;
  const size_t need = gemm4_workspace(book, M, K);
  RLQ_REQUIRE(ws_bytes >= need, "workspace of %zu bytes is smaller than the %zu this call needs", ws_bytes, need);
  RLQ_REQUIRE(need == 0 || aligned(ws, 256), "workspace must be 256-byte aligned");
  RLQ_REQUIRE((size_t)M * std::max(x_stride, K) * 2 < (1ull << 31), "prefill kernel: x spans more than 2 GiB");
  GemmArgs a = {};
  a.codes = static_cast<const u32x4 *>(packed);
  a.sb = reinterpret_cast<const u32x4 *>(static_cast<const char *>(packed) + packed_code_bytes(K, N));
  a.srow = srow;
  a.y = y;
  a.M = M; a.K = K; a.N = N; a.y_stride = y_stride;
  if (book == kAffine) {
    const int gs_stride = (2 * G + 31) / 32 * 32;
    _Float16 *xp = static_cast<_Float16 *>(ws);
    _Float16 *gshl = reinterpret_cast<_Float16 *>(static_cast<char *>(ws) + ((size_t)M * K * 2 + 255) / 256 * 256);
    gemm_prep_kernel<<<(M * G + 255) / 256, 256, 0, st>>>(x, x_stride, M, K, xp, gshl, gs_stride);
    RLQ_HIP(hipGetLastError());
    a.x = xp; a.x_stride = K; a.gshl = gshl; a.gs_stride = gs_stride;
  } else {
    a.x = x; a.x_stride = x_stride;
    if (book == kInt16) {
      const int m_pad = (M + 127) / 128 * 128;
      float *gsT = static_cast<float *>(ws);
      float *asum = gsT + (size_t)G * m_pad;
      launch_group_sums(x, x_stride, M, K, gsT, m_pad, st);
      launch_row_sums(gsT, G, m_pad, M, asum, st);
      a.asum = asum;
    }
  }
  const int mblocks = (M + kGM - 1) / kGM, nblocks = (N + kGN - 1) / kGN;
  const dim3 grid(mblocks * nblocks);
  const size_t lds = 2 * (size_t)kABufBytes;
  switch (book) {
    case kInt15: launch_gemm4_inst<kInt15, 0>(accum, grid, lds, st, a); break;
    case kInt16: launch_gemm4_inst<kInt16, 0>(accum, grid, lds, st, a); break;
    case kFp4: launch_gemm4_inst<kFp4, 0>(accum, grid, lds, st, a); break;
    default:
      if (sd == RLQ_BF16) launch_gemm4_inst<kAffine, 1>(accum, grid, lds, st, a);
      else launch_gemm4_inst<kAffine, 0>(accum, grid, lds, st, a);
  }
  RLQ_HIP(hipGetLastError());
  return 0;
}

}  // namespace rlq
