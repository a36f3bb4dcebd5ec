// Dense fp16 linear on gfx950: y = x W^T for the small matrices the reference keeps in
// half precision (kernels/linear.metal:186-225, linear_f16: the MoE router and the MTP
// head's input projection; layout tools/convert.py:218-226).
//
// Weights are repacked once at upload into MFMA operand order: for each tile t of 16 rows
// and each step s of 32 inputs, 1024 bytes in which lane l = 16j + c holds the 8 halves
// W[16t + c][32s + 8j .. +7] (the B operand of one v_mfma_f32_16x16x32_f16). A wave's
// loads are then whole consecutive kilobytes.
//
// Grid: (16-row weight tiles, 16-row token blocks). The waves of a workgroup split the K
// steps into consecutive ranges, chain their MFMAs, and add their partials in LDS in wave
// order, so a row's result depends only on K.
#include "q4_tile.h"
#include "../../include/rlq.h"

#include <algorithm>

namespace rlq {

constexpr int kStepK = 32;
constexpr int kDenseStepsPerWave = 8;    // loads in flight per wave (two per step)

inline size_t packed_f16_bytes(int K, int N) { return (size_t)tiles_of(N) * (K / kStepK) * 1024; }

// source row-major (ld = K halves per row) or blocked ([n_pad/256][K][256], rows row0..)
__global__ void pack_f16_kernel(const _Float16 *w, int K, int N, int blocked, int row0, u32x4 *out) {
  const int steps = K / kStepK;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;   // ((t * steps + s) * 64 + l)
  if (i >= (size_t)tiles_of(N) * steps * 64) return;
  const int l = (int)(i & 63);
  const size_t ts = i >> 6;
  const int t = (int)(ts / steps), s = (int)(ts - (size_t)t * steps);
  const int c = l & 15, j = l >> 4, r = 16 * t + c;
  half8 v = {};
  if (r < N) {
    const int k0 = kStepK * s + 8 * j;
    if (!blocked) {
      v = *reinterpret_cast<const half8 *>(w + (size_t)r * K + k0);
    } else {
      const int n = row0 + r, blk = n >> 8, col = n & 255;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = w[((size_t)blk * K + k0 + e) * 256 + col];
    }
  }
  out[i] = __builtin_bit_cast(u32x4, v);
}

struct DenseArgs {
  const _Float16 *x;
  const u32x4 *w;
  float *y;
  int x_stride, M, K, N, y_stride, spw;   // spw: steps per wave
};

template <bool ACC>
__global__ __launch_bounds__(1024) void dense_f16_kernel(DenseArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, j4 = lane >> 4;
  const int t = blockIdx.x, m0 = 16 * blockIdx.y;
  const int steps = a.K / kStepK;
  const int s0 = wave * a.spw, s1 = min(steps, s0 + a.spw);
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(a.w + ((size_t)t * steps + s0) * 64, (uint32_t)max(0, s1 - s0) * 1024u);
  const int rows = min(16, a.M - m0);
  const bool live = c16 < rows;
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(a.x + (size_t)m0 * a.x_stride + (size_t)s0 * kStepK,
                s1 > s0 ? (uint32_t)((rows - 1) * a.x_stride + (s1 - s0) * kStepK) * 2u : 0u);
  const uint32_t xoff = (uint32_t)c16 * a.x_stride * 2u + 16u * j4;
  f32x4 acc = {};
  for (int b0 = 0; b0 < a.spw; b0 += kDenseStepsPerWave) {
    u32x4 wb[kDenseStepsPerWave], xb[kDenseStepsPerWave];
#pragma unroll
    for (int i = 0; i < kDenseStepsPerWave; ++i) {
      const int st = b0 + i;   // relative to s0; out-of-range loads return zeros
      xb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rx, live && s0 + st < s1 ? xoff + (uint32_t)st * 64u : kFarOffset, 0, 0));
      // the whole offset in the range-checked vector operand: steps past the wave's range read zeros
      wb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, 16u * lane + (uint32_t)st * 1024u, 0,
                                                                             kNonTemporal));
    }
#pragma unroll
    for (int i = 0; i < kDenseStepsPerWave; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, xb[i]), __builtin_bit_cast(half8, wb[i]),
                                                   acc, 0, 0, 0);
  }
  acc = reduce_waves(acc, reinterpret_cast<f32x4 *>(lds), wave, waves, lane);
  const int n = 16 * t + c16;
  if (wave != 0 || n >= a.N) return;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * j4 + v;
    if (r < rows) {
      float *dst = a.y + (size_t)(m0 + r) * a.y_stride + n;
      *dst = ACC ? *dst + acc[v] : acc[v];
    }
  }
}

}  // namespace rlq

using namespace rlq;

extern "C" {

size_t rlq_packed_f16_bytes(int K, int N) {
  if (K <= 0 || N <= 0 || K % kStepK) return 0;
  return packed_f16_bytes(K, N);
}

static int pack_f16(const char *fn, const void *w, int K, int N, int blocked, int row0, void *packed, void *stream) {
  RLQ_REQUIRE(K >= kStepK && K % kStepK == 0 && N >= 1, "%s: bad sizes K=%d N=%d (K a multiple of 32)", fn, K, N);
  RLQ_REQUIRE(w && packed, "%s: null pointer argument", fn);
  RLQ_REQUIRE(aligned(w, 16) && aligned(packed, 16), "%s: w and packed must be 16-byte aligned", fn);
  const size_t pieces = (size_t)tiles_of(N) * (K / kStepK) * 64;
  pack_f16_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const _Float16 *>(w), K, N, blocked, row0, static_cast<u32x4 *>(packed));
  RLQ_HIP(hipGetLastError());
  return 0;
}

int rlq_pack_f16(const void *w, int K, int N, void *packed, void *stream) {
  return pack_f16("rlq_pack_f16", w, K, N, 0, 0, packed, stream);
}

int rlq_pack_f16_blocked(const void *w_blk, int K, int n_pad, int row0, int rows, void *packed, void *stream) {
  RLQ_REQUIRE(n_pad % 256 == 0 && n_pad > 0, "rlq_pack_f16_blocked: n_pad=%d is not a multiple of the block 256",
              n_pad);
  RLQ_REQUIRE(row0 >= 0 && rows >= 1 && row0 + rows <= n_pad, "rlq_pack_f16_blocked: rows [%d, %d) outside [0, %d)",
              row0, row0 + rows, n_pad);
  return pack_f16("rlq_pack_f16_blocked", w_blk, K, rows, 1, row0, packed, stream);
}

int rlq_linear_f16(const void *x, int x_stride, int M, int K, int N, const void *packed, float *y, int y_stride,
                   int accum, void *stream) {
  RLQ_REQUIRE(M >= 1 && N >= 1 && K >= kStepK && K % kStepK == 0, "rlq_linear_f16: bad sizes M=%d K=%d N=%d", M, K,
              N);
  RLQ_REQUIRE(x && packed && y, "rlq_linear_f16: null pointer argument");
  RLQ_REQUIRE(x_stride >= K && x_stride % 8 == 0, "rlq_linear_f16: x_stride=%d must be >= K and a multiple of 8",
              x_stride);
  RLQ_REQUIRE(y_stride >= N, "rlq_linear_f16: y_stride=%d < N=%d", y_stride, N);
  RLQ_REQUIRE(aligned(x, 16) && aligned(packed, 16) && aligned(y, 4), "rlq_linear_f16: misaligned argument");
  RLQ_REQUIRE((long long)M * x_stride * 2 < (1LL << 31), "rlq_linear_f16: x spans more than 2 GiB");
  const int steps = K / kStepK;
  const int waves = std::min(16, (steps + kDenseStepsPerWave - 1) / kDenseStepsPerWave);
  const int spw = (steps + waves - 1) / waves;
  DenseArgs a;
  a.x = static_cast<const _Float16 *>(x);
  a.w = static_cast<const u32x4 *>(packed);
  a.y = y;
  a.x_stride = x_stride; a.M = M; a.K = K; a.N = N; a.y_stride = y_stride;
  a.spw = (spw + kDenseStepsPerWave - 1) / kDenseStepsPerWave * kDenseStepsPerWave;
  const dim3 grid(tiles_of(N), (M + 15) / 16);
  const size_t lds = (size_t)(waves - 1) * 64 * 16;
  if (accum) dense_f16_kernel<true><<<grid, 64 * waves, lds, static_cast<hipStream_t>(stream)>>>(a);
  else dense_f16_kernel<false><<<grid, 64 * waves, lds, static_cast<hipStream_t>(stream)>>>(a);
  RLQ_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
