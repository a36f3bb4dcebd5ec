// Prefill GEMM on gfx950 for the 4-bit formats (affine and native codebooks), M > 8.
//
//   affine: y[m][n] = sum_g s[n][g] * (x_g . q_g)[m][n] + b[n][g] * gsum[m][g]
//   native: y[m][n] = s[n] * (x . L(q))[m][n]  (+ 0.5 s[n] rowsum[m] for the half-step book)
//
// Workgroup tile 128 tokens x 256 features, 8 waves; each wave owns 32 features over all
// 128 tokens (four v_mfma_f32_32x32x16_f16 tiles; on gfx950 this shape runs at twice the
// rate of 16x16x32), so each code is converted to fp16 once per workgroup.
//  - A 3-stage LDS ring holds, per group pair (128 inputs), the activation tile, the
//    workgroup's packed codes and its scale/bias quads, all filled by LDS-DMA
//    (buffer_load ... lds: no registers, no VALU) two pairs ahead of use. Activation rows
//    are stored with their 16-byte chunks XOR-swizzled by the row, so the MFMA operand
//    reads hit distinct banks.
//  - Codes become exact fp16 subnormals q * 2^-24 in registers (four masks and a shift per
//    eight codes: the operand trick of q4_tile.h), the scale carries the 2^24.
//  - The 32 MFMAs of a pair run in a fixed order with each A fragment read from LDS 8
//    MFMAs ahead; affine group products are scaled into the fp32 accumulators by FMAs
//    interleaved with the MFMAs of the next half-group.
// Affine: the activations are first rewritten by a prep pass (exact per-row power-of-two
// prescale, then the operand order (x0, x4, x1/16, x5/16, ...) of the five-op code
// conversion), and the outputs are scaled back at the store. The bias term
// sum_g b[n][g] gsum[m][g] is one more MFMA product at the end, over K' = 2G, with the
// group sums split into fp16 hi + lo (exact to 2^-22) and b as the other operand; the
// group sums of the tile's rows go through the LDS once per workgroup for all its waves.
// The K loop runs three group pairs per iteration, one per LDS stage, so every LDS read has
// a compile-time stage offset; workgroups are ordered in groups of 4 token blocks per XCD.
// Native books: activations are used as they are, codes decode in element order, and the
// products chain in the MFMA over all of K with the row scale applied at the end.
// A row's result depends only on its own activations (MFMA rows are independent).
#include "gemm.h"
#include "q4_tile.h"
#include "../../include/rlq.h"

#include <algorithm>
#include <type_traits>

namespace rlq {

constexpr int kGM = 128, kGN = 256;         // workgroup tile
constexpr int kGThreads = 512;
constexpr int kARowBytes = 256;             // one pair of groups: 128 fp16
constexpr int kABytes = kGM * kARowBytes;   // stage part: activation tile, 32 KB
constexpr int kBBytes = (kGN / 16) * 1024;  // stage part: the 16 tiles' code kilobytes, 16 KB
constexpr int kSBytes = (kGN / 16) * 256;   // stage part: their scale/bias quads, 4 KB
constexpr int kStageBytes = kABytes + kBBytes + kSBytes;
constexpr int kStages = 3;                  // loads run two group pairs ahead of the MFMAs
constexpr int kGroupM = 4;                  // token blocks per group of the workgroup order
constexpr int kBiasChunk = 32;              // bias product: steps of group-sum pieces staged at a time
constexpr int kMaxGemmSplit = 2;            // workgroups per output tile when K is split
constexpr int kProBiasSteps = 11;           // bias steps run in the prologue (their pieces fill 47 KB)
static_assert(kGM * (32 * kProBiasSteps + 16) <= kABytes + kBBytes, "the prologue's bias pieces fit stage 2");
// LDS by part, then stage: the three activation tiles, the three code parts, the three
// scale parts, so that with the stage known at compile time every read of a stage is a
// lane's base address plus an immediate offset
constexpr int a_part(int stage) { return stage * kABytes; }
constexpr int b_part(int stage) { return kStages * kABytes + stage * kBBytes; }
constexpr int s_part(int stage) { return kStages * (kABytes + kBBytes) + stage * kSBytes; }
// affine: the tile's 128 row scales 2^-e, after the ring (read by the stores at the end);
// 1 KB, as the one LDS-DMA that brings them writes 16 bytes for each of the 64 lanes
constexpr int kRscaleLds = kStages * kStageBytes;
constexpr int kGemmLdsBytes = kRscaleLds + 1024;
static_assert(kGemmLdsBytes <= 160 * 1024, "the row scales fit after the ring");

// ------------------------------------------------------------------ affine prep pass

// The GEMM's code conversion is the five-op form of q4_tile.h (odd codes at 16 times the
// scale), so the odd activations go in divided by 16. A division by 16 in fp16 rounds
// values below 2^-10 onto the subnormal grid, which would make the result depend on the
// activations' scale. So each row is first multiplied by a power of two, 2^e with e chosen
// from the row's largest magnitude (max |x| 2^e in [2^8, 2^9)), and the GEMM multiplies
// its outputs by 2^-e: powers of two change no bits in fp32, and after the prescale only
// elements below 2^-19 of the row's largest one reach the subnormal grid (an error below
// 2^-29 of that largest element each). 2^8 keeps each group sum of 64 scaled elements
// within fp16 range for the bias product.
constexpr int kPrepThreads = 256;

// eight consecutive activations times f (even elements) and f / 16 (odd ones) -> operand
// order (x0, x4, x1/16, x5/16, x2, x6, x3/16, x7/16), rounded to fp16 once
__device__ __forceinline__ u32x4 prep_x8_scaled(u32x4 p, float f) {
  const half8 h = __builtin_bit_cast(half8, p);
  const float fo = f * 0.0625f;
  half8 o;
  o[0] = (_Float16)((float)h[0] * f);  o[1] = (_Float16)((float)h[4] * f);
  o[2] = (_Float16)((float)h[1] * fo); o[3] = (_Float16)((float)h[5] * fo);
  o[4] = (_Float16)((float)h[2] * f);  o[5] = (_Float16)((float)h[6] * f);
  o[6] = (_Float16)((float)h[3] * fo); o[7] = (_Float16)((float)h[7] * fo);
  return __builtin_bit_cast(u32x4, o);
}

// The group sums feed the bias product sum_g b[n][g] gsum[m][g], an MFMA over K' = P G with
// each group sum split into P exact pieces of the biases' 16-bit type: fp16 biases (SD 0)
// take (hi, lo), exact to 2^-22 of the sum; bf16 biases (SD 1) take (hi, mid, lo, 0), whose
// three 8-bit pieces hold the fp32 sum exactly. The bf16 product keeps bf16 biases exact
// (converting them to fp16 would round those below 2^-14).
template <int SD> constexpr int kGsPieces = SD == 0 ? 2 : 4;
static int gs_stride_of(int G, int sd) { return ((sd == 0 ? 2 : 4) * G + 31) / 32 * 32; }

__device__ __forceinline__ uint32_t bf16_rne_bits(float v) {   // finite v
  const uint32_t u = __float_as_uint(v);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// The pieces of one group sum of the scaled row (see kGsPieces), and the zero padding of the
// row's pieces up to gs_stride after its last group.
template <int SD>
__device__ __forceinline__ void write_gs_pieces(uint16_t *gs, int gs_stride, int m, int g, int G, float sum) {
  constexpr int P = kGsPieces<SD>;
  uint16_t *dst = gs + (size_t)m * gs_stride + P * g;
  if constexpr (SD == 0) {
    const _Float16 hi = static_cast<_Float16>(sum);
    const _Float16 lo = static_cast<_Float16>(sum - static_cast<float>(hi));
    dst[0] = __builtin_bit_cast(uint16_t, hi);
    dst[1] = __builtin_bit_cast(uint16_t, lo);
  } else {
    const uint32_t hi = bf16_rne_bits(sum);
    const float r1 = sum - __uint_as_float(hi << 16);         // exact
    const uint32_t mid = bf16_rne_bits(r1);
    const uint32_t lo = bf16_rne_bits(r1 - __uint_as_float(mid << 16));   // exact: 8 bits remain
    dst[0] = (uint16_t)hi;
    dst[1] = (uint16_t)mid;
    dst[2] = (uint16_t)lo;
    dst[3] = 0;
  }
  if (g == G - 1)   // the row's padding up to gs_stride is zero (no memset: this runs in graphs)
    for (int k = P * G; k < gs_stride; ++k) gs[(size_t)m * gs_stride + k] = 0;
}

// The workgroup's max |x| of its row from each thread's partial max (THR threads).
template <int THR = kPrepThreads>
__device__ __forceinline__ float row_max(float mx, float *wmax) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, d));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < THR / 64; ++w) mx = __builtin_fmaxf(mx, wmax[w]);
  return mx;
}

// 2^e for the row's largest magnitude (max |x| 2^e in [2^8, 2^9)); 1 for a row that is all
// zeros or holds an infinity or a NaN.
__device__ __forceinline__ int row_exponent(float mx) {
  int ex = 0;
  if (mx > 0.0f && mx <= 65504.0f) {
    int k;
    (void)__builtin_frexpf(mx, &k);                     // mx = f 2^k, f in [0.5, 1)
    ex = 9 - k;                                         // mx 2^ex in [2^8, 2^9)
  }
  return ex;
}

// The prep pass with the row read once: thread i of THR holds chunks i, i + THR, ... (CPT of
// them, K <= 8 THR CPT) in registers between the max and the writes. The same arithmetic in
// the same order as gemm_prep_kernel below, so the same bits (the max does not depend on the
// order, and each group's sum is its 8 threads' fixed butterfly whatever THR is). Rows of more
// than 8192 activations take 1024 threads: with 256 threads, 16 chunks each held 154 VGPRs
// (3 waves per SIMD), and the 27B down projection's prep (K = 17408) ran at 4.1 TB/s.
template <int SD, int CPT, int THR = kPrepThreads>
__global__ __launch_bounds__(THR) void gemm_prep1_kernel(const _Float16 *x, int x_stride, int M, int K,
                                                         _Float16 *xp, uint16_t *gs, int gs_stride, float *rscale) {
  __shared__ float wmax[THR / 64];
  const int m = blockIdx.x;
  const int C = K / 8;                                  // chunks per row (a multiple of 8)
  const _Float16 *row = x + (size_t)m * x_stride;
  u32x4 v[CPT];
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = threadIdx.x + THR * j;
    v[j] = c < C ? *reinterpret_cast<const u32x4 *>(row + 8 * c) : u32x4{};
    const half8 h = __builtin_bit_cast(half8, v[j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = __builtin_fmaxf(mx, __builtin_fabsf(static_cast<float>(h[e])));
  }
  mx = row_max<THR>(mx, wmax);
  const int ex = row_exponent(mx);
  const float f = __builtin_ldexpf(1.0f, ex);
  if (threadIdx.x == 0) rscale[m] = __builtin_ldexpf(1.0f, -ex);
  const int G = C >> 3;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    if (THR * j >= C) break;                   // uniform: the butterfly needs every lane
    const int c = threadIdx.x + THR * j;
    const half8 h = __builtin_bit_cast(half8, v[j]);
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += static_cast<float>(h[e]) * f;
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    if (c >= C) continue;
    *reinterpret_cast<u32x4 *>(xp + (size_t)m * K + 8 * c) = prep_x8_scaled(v[j], f);
    if ((c & 7) == 0) write_gs_pieces<SD>(gs, gs_stride, m, c >> 3, G, sum);
  }
}

// One workgroup per token row m. Pass 1 finds max |x| of the row; pass 2 writes
// xp[m][k] (the row times 2^e, in operand order), gs[m][P g ..] (the pieces of the group
// sums of the scaled row) and rscale[m] = 2^-e. One thread per 8 activations per step
// (coalesced 16-byte loads and stores); the 8 threads of a group add their partial sums
// with a fixed butterfly. A row that is all zeros, or holds an infinity or a NaN, keeps
// e = 0.
template <int SD>
__global__ __launch_bounds__(kPrepThreads) void gemm_prep_kernel(const _Float16 *x, int x_stride, int M, int K,
                                                                 _Float16 *xp, uint16_t *gs, int gs_stride,
                                                                 float *rscale) {
  __shared__ float wmax[kPrepThreads / 64];
  const int m = blockIdx.x;
  const int C = K / 8;                                  // chunks per row (a multiple of 8)
  const _Float16 *row = x + (size_t)m * x_stride;
  float mx = 0.0f;
  for (int c = threadIdx.x; c < C; c += kPrepThreads) {
    const half8 h = __builtin_bit_cast(half8, *reinterpret_cast<const u32x4 *>(row + 8 * c));
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = __builtin_fmaxf(mx, __builtin_fabsf(static_cast<float>(h[e])));
  }
  mx = row_max(mx, wmax);
  const int ex = row_exponent(mx);
  const float f = __builtin_ldexpf(1.0f, ex);
  if (threadIdx.x == 0) rscale[m] = __builtin_ldexpf(1.0f, -ex);
  const int G = C >> 3;
  for (int c0 = 0; c0 < C; c0 += kPrepThreads) {        // uniform trip count: the butterfly needs every lane
    const int c = c0 + threadIdx.x;
    const bool in = c < C;
    u32x4 v = {};
    if (in) v = *reinterpret_cast<const u32x4 *>(row + 8 * c);
    const half8 h = __builtin_bit_cast(half8, v);
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += static_cast<float>(h[e]) * f;
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    if (!in) continue;
    *reinterpret_cast<u32x4 *>(xp + (size_t)m * K + 8 * c) = prep_x8_scaled(v, f);
    if ((c & 7) == 0) write_gs_pieces<SD>(gs, gs_stride, m, c >> 3, G, sum);
  }
}

// ------------------------------------------------------------------ the GEMM

// Where one thread's 8 LDS-DMA loads of a stage come from (see gemm4_kernel).
struct StageSrc {
  __amdgpu_buffer_rsrc_t rx, rcode, rsb;
  uint32_t a_off[4];
  bool a_row[4];
  int K, GP, G4, wave, lane;
};

__device__ __forceinline__ __attribute__((address_space(3))) void *lds_at(unsigned char *lds, int off) {
  return (__attribute__((address_space(3))) void *)(lds + off);
}

// Loads group pair p into LDS stage `stage`: 4 activation chunks (16 bytes each), 2 code
// chunks of 16 bytes (tile 2 wave + i: its pair-p kilobyte) and 2 scale words (quad p/2 of
// the same tiles). The per-lane part of each offset goes in the range-checked vector
// operand: rows past M and tiles past N read zeros. The pair's part, the same for every
// lane, goes in the scalar operand (no ALU work), which the range check does not see; so
// a pair reaching past K (an odd number of groups) takes the path with the whole offset
// checked, where inputs past K read zeros.
__device__ __forceinline__ void issue_stage(const StageSrc &s, unsigned char *lds, int p, int stage) {
  if (128 * (p + 1) <= s.K) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(s.rx, lds_at(lds, a_part(stage) + (4 * s.wave + i) * 1024), 16,
                                               s.a_off[i], 256 * p, 0, 0);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * (4 * s.wave + i) + (s.lane >> 4);
      const int c = (s.lane & 15) ^ (r & 15);
      const bool ok = s.a_row[i] && 128 * p + 8 * c < s.K;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(s.rx, lds_at(lds, a_part(stage) + (4 * s.wave + i) * 1024), 16,
                                               ok ? s.a_off[i] + (uint32_t)(256 * p) : kFarOffset, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int k = 2 * s.wave + i;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(s.rcode, lds_at(lds, b_part(stage) + k * 1024), 16,
                                             (uint32_t)k * s.GP * 1024u + 16u * s.lane, p * 1024, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int k = 2 * s.wave + i;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(s.rsb, lds_at(lds, s_part(stage) + k * 256), 4,
                                             (uint32_t)k * s.G4 * 256u + 4u * s.lane, (p >> 1) * 256, 0, 0);
  }
}


// The B reads of a pair (two 16-byte code slots) and, affine, its two scale words.
template <int BOOK, int STAGE>
__device__ __forceinline__ void read_pair_head(const unsigned char *lds, uint32_t boff, uint32_t soff, int p,
                                               u32x4 (&wq)[2], uint32_t (&sp)[2]) {
  wq[0] = *reinterpret_cast<const u32x4 *>(lds + b_part(STAGE) + boff);
  wq[1] = *reinterpret_cast<const u32x4 *>(lds + b_part(STAGE) + boff + 512);
  if constexpr (BOOK == kAffine) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = *reinterpret_cast<const u32x2 *>(lds + s_part(STAGE) + soff + 8 * (p & 1));
    sp[0] = v[0];
    sp[1] = v[1];
  }
}


// Where byte `pos` of a chunk of bias pieces lives in the LDS: from the start at the end of
// the kernel; in the prologue the first 32 KB in stage 2's activation part and the rest in
// its code part (both free until stage 2 is issued). (A lambda inside the kernel here made
// the host pass drop the kernel's launch stubs without a diagnostic.)
__device__ __forceinline__ int bias_piece_at(int pos, bool pro) {
  return !pro ? pos : pos < kABytes ? a_part(2) + pos : b_part(2) + (pos - kABytes);
}

// A fragment of step j of a pair (see gemm4_kernel): token tile 2 ((j >> 3) & 1) + (j & 1),
// 32 rows of 256 bytes apart per tile, chunk of step (j >> 1) & 3 of group j >> 4.
template <int STAGE>
__device__ __forceinline__ half8 read_frag(const unsigned char *lds, const uint32_t (&aoff)[2][4], int j) {
  const int gg = j >> 4, mt = 2 * ((j >> 3) & 1) + (j & 1), i = (j >> 1) & 3;
  return *reinterpret_cast<const half8 *>(lds + a_part(STAGE) + mt * 32 * kARowBytes + aoff[gg][i]);
}

template <int BOOK, int SD, bool ACC>
__global__ __launch_bounds__(kGThreads) void gemm4_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.K / kGroup, G4 = quads_of(a.K), GP = 2 * G4;
  const int NP = (G + 1) / 2;                        // group pairs with real groups
  const int T = tiles_of(a.N);
  // Split K (S = gridDim.y > 1, see gemm_split_of): split s takes group pairs
  // [s P, s P + P) (P = np_split, the last split the rest) and its share of the bias steps;
  // split 0 writes y (adding to it when asked), split s > 0 its partial products to
  // y_part[s - 1]; the tile's last split to arrive adds them in split order (see the end of
  // the kernel).
  const int split = blockIdx.y, S = gridDim.y;
  const int pb = split * a.np_split;
  const int NPs = min(NP, pb + a.np_split) - pb;
  const bool acc_here = ACC && split == 0;

  // Workgroups are numbered round-robin over the 8 XCDs; give each XCD a contiguous
  // range of tiles, ordered in groups of kGroupM token blocks (token blocks fastest, then
  // feature blocks), so the workgroups an XCD runs at once share both their activation
  // rows and their weights in its L2 (kGroupM 4: 4 token x 8 feature blocks per XCD).
  const int nwg = gridDim.x, wid = blockIdx.x;
  const int per_xcd = (nwg + 7) / 8;
  int lin = (wid % 8) * per_xcd + wid / 8;
  if (nwg % 8 != 0) lin = wid;                      // uneven grids keep the plain order
  const int mblocks = (a.M + kGM - 1) / kGM, nblocks = (a.N + kGN - 1) / kGN;
  const int group = lin / (kGroupM * nblocks), first_m = group * kGroupM;
  const int gm = min(mblocks - first_m, kGroupM), rem = lin - group * kGroupM * nblocks;
  const int mb = first_m + rem % gm, nb = rem / gm;
  const int m0 = mb * kGM, n0 = nb * kGN;

  // Every stage of the LDS ring holds, for one group pair: the activation tile (rows with
  // their 16-byte chunks XOR-swizzled by the row), the kilobyte of codes of each of the
  // workgroup's 16 tiles (a straight copy of the packed layout), and their scale/bias
  // quads. Every thread issues the same 8 LDS-DMA loads per stage (4 activation chunks of
  // 16 bytes, 2 code chunks of 16 bytes, 2 scale words), so waiting until 8 loads remain
  // in flight waits for exactly the older stage.
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.M * a.x_stride * 2));
  const int t0 = n0 >> 4;                                 // first 16-row tile of the workgroup
  const int tiles = max(0, min(T, t0 + 16) - t0);
  const __amdgpu_buffer_rsrc_t rcode = make_rsrc(a.codes + (size_t)min(t0, T) * GP * 64, (uint32_t)tiles * GP * 1024u);
  const __amdgpu_buffer_rsrc_t rsb =
      make_rsrc(a.sb + (size_t)min(t0, T) * G4 * 16, BOOK == kAffine ? (uint32_t)tiles * G4 * 256u : 0u);
  StageSrc src;
  src.rx = rx; src.rcode = rcode; src.rsb = rsb;
  src.K = a.K; src.GP = GP; src.G4 = G4; src.wave = wave; src.lane = lane;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * (4 * wave + i) + (lane >> 4);   // row within the tile
    const int c = (lane & 15) ^ (r & 15);             // logical chunk stored at this lane's slot
    src.a_off[i] = (uint32_t)(((size_t)(m0 + r) * a.x_stride + 8 * c) * 2);
    src.a_row[i] = m0 + r < a.M;
  }

  // Each wave owns 32 features (one 32-column MFMA tile = the workgroup's 16-row tiles
  // 2 wave and 2 wave + 1) over all 128 tokens (four 32-row MFMA tiles), so every code is
  // converted once per workgroup. The 32x32x16 MFMA only needs A and B to agree on which
  // input k sits in which lane slot: lane l (column l%32, half h = l/32) takes, for step i
  // of a group, the packed word 2i + h of its row, which the 16-row layout keeps in the
  // slot of lane 16 j + c with j = (2i + h) % 4. Two 16-byte reads per lane and pair
  // (slots h and 2 + h) bring a lane all its B operands: words h, 4 + h (first read) and
  // 2 + h, 6 + h (second) of both groups. The A operand of step i is the natural chunk of
  // inputs 16 i + 8 h .. +7, as the MFMA expects.
  const int h = lane >> 5, c32 = lane & 31;
  const int tt = c32 >> 4, cr = c32 & 15;                 // 16-row tile within the 32, row in it
  const int kt = 2 * wave + tt;                           // the lane's 16-row tile in the workgroup
  uint32_t aoff[2][4];                                    // A fragment offsets within a stage
#pragma unroll
  for (int gg = 0; gg < 2; ++gg)
#pragma unroll
    for (int i = 0; i < 4; ++i) aoff[gg][i] = (uint32_t)(c32 * kARowBytes + (((8 * gg + 2 * i + h) ^ cr) << 4));
  const uint32_t boff = (uint32_t)(kt * 1024 + 256 * h + 16 * cr);   // within a stage's code part
  const uint32_t soff = (uint32_t)(kt * 256 + 16 * cr);               // within its scale part

  // The K loop is software-pipelined over the 32 MFMAs of a group pair, in a fixed order:
  // step j = 16 gg + 8 half + 2 i + t multiplies token tile mt = 2 half + t by the codes of
  // step i of group gg. Every A fragment feeds exactly one MFMA, and is read from LDS 8
  // steps before it (a sliding window of 8 fragments in registers). Affine: each group
  // product is scaled into the accumulators by FMAs that run beside the next half's
  // MFMAs (tiles 0, 1 of a group during its steps 8..15, tiles 2, 3 during the next
  // group's steps 0..7), four FMAs per MFMA, so no instruction waits on a result issued
  // just before it. The barrier that hands stage p + 1 over sits before step 24 of pair
  // p: by then every wave has issued all its reads of stage p, and the first 8 fragments
  // of pair p + 1 are read during steps 24..31.
  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f32x16{};
  f32x16 pp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) pp[i] = f32x16{};
  float sc_prev = 0.0f;
  half8 carry[8];                                         // fragments 0..7 of the next pair
  u32x4 wq[2];
  uint32_t sp[2] = {0u, 0u};

  // Affine: acc += sum_g b[n][g] * gsum[m][g], an MFMA product over K' = P G, each group
  // sum as P pieces (gemm_prep_kernel); a split K shares its steps out evenly over the splits
  // (each split adds its share; any division covers every step once). Step st covers
  // k' = 16 st .. +15; lane half h holds k' 16 st + 8 h .. +7: for fp16 biases (P = 2) the
  // (hi, lo) of groups 8 st + 4 h .. +3, so b of those groups, each twice; for bf16 biases
  // (P = 4) the pieces of groups 4 st + 2 h and + 1, so b of those two, four times each.
  // Every wave needs the pieces of all 128 rows, so they go through the LDS: LDS-DMA'd once
  // per workgroup, cs steps at a time, rows padded by 16 bytes (an odd number of 16-byte
  // slots apart, so the fragment reads of 32 rows spread over the banks). Each wave's scale
  // quads (its own biases) come straight from memory, in flight while the pieces land.
  // The first kProBiasSteps steps run in the prologue, their loads in flight with the first
  // two stages' (one wait for both), the pieces in stage 2's activation and code parts, free
  // until stage 2 is issued: as the workgroup's last phase the bias product cost the whole
  // round trip of its loads (27B gate_up at M = 2048: 116 us of 865). Later steps (long K,
  // bf16 biases) run at the end, from the start of the LDS.
  const int bsteps = a.gs_stride / 16;
  const int st_lo = split * bsteps / S, st_hi = (split + 1) * bsteps / S;
  const int st_pro = BOOK == kAffine ? min(st_hi, st_lo + kProBiasSteps) : st_lo;
  auto bias_chunk = [&](int st0, int cs, bool pro) {
    const int tn = t0 + 2 * wave;
    const int tv = max(0, min(T, tn + 2) - tn);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.sb + (size_t)min(tn, T) * G4 * 16, (uint32_t)tv * G4 * 256u);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(a.gs, (uint32_t)((size_t)a.M * a.gs_stride * 2));
    const int rowb = 32 * cs + 16;                         // LDS bytes per row
    u32x4 v[kBiasChunk];
#pragma unroll
    for (int u = 0; u < kBiasChunk; ++u) {
      const int q = SD == 0 ? 2 * (st0 + u) + h : st0 + u;   // quad of groups 4q .. 4q+3
      const uint32_t off = u < cs && q < G4 ? (uint32_t)tt * G4 * 256u + (uint32_t)q * 256u + 16u * cr : kFarOffset;
      v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);                   // lgkmcnt(0): this wave's LDS reads are done
    asm volatile("s_barrier" ::: "memory");               // and every wave's
    // 1 KB blocks of the chunk (128 rows of rowb bytes), each lane 16 bytes; pad slots and
    // rows past M read zeros
    const int nblk = (kGM * rowb + 1023) / 1024;
    for (int blk = wave; blk < nblk; blk += kGThreads / 64) {
      const int pos = blk * 1024 + 16 * lane, row = pos / rowb, col = pos - row * rowb;
      const bool ok = row < kGM && col < 32 * cs && m0 + row < a.M;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rg, lds_at(lds, bias_piece_at(blk * 1024, pro)), 16,
          ok ? (uint32_t)(((size_t)(m0 + row) * a.gs_stride + 16 * st0) * 2 + col) : kFarOffset, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);                        // the pieces (and the scale quads) landed
    asm volatile("s_barrier" ::: "memory");
#pragma unroll
    for (int u = 0; u < kBiasChunk; ++u) {
      if (u >= cs) continue;                              // uniform
      u32x4 d;
      if constexpr (SD == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e] = (v[u][e] >> 16) * 0x10001u;       // (b, b): times hi and lo
      } else {
        const uint32_t b0 = (h ? v[u][2] : v[u][0]) >> 16, b1 = (h ? v[u][3] : v[u][1]) >> 16;
        d[0] = d[1] = b0 * 0x10001u;                                         // b of group 4q + 2h, four times
        d[2] = d[3] = b1 * 0x10001u;                                         // and of group 4q + 2h + 1
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const u32x4 ag = *reinterpret_cast<const u32x4 *>(lds + bias_piece_at((mt * 32 + c32) * rowb + 32 * u + 16 * h, pro));
        if constexpr (SD == 0)
          acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, ag),
                                                          __builtin_bit_cast(half8, d), acc[mt], 0, 0, 0);
        else
          acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ag),
                                                           __builtin_bit_cast(bf16x8, d), acc[mt], 0, 0, 0);
      }
    }
  };

  // Every stage issue loads a real pair: past the last pair the index is clamped (a
  // duplicate of the last pair into a stage nobody reads any more), so exactly two
  // stages are always in flight and one wait count fits every hand-over.
  if (BOOK == kAffine && wave == 0) {
    // the tile's row scales, first in wave 0's queue, so every wait below covers them
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.rscale + m0, (uint32_t)(min(kGM, a.M - m0) * 4));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, lds_at(lds, kRscaleLds), 16, lane < 32 ? 16u * lane : kFarOffset, 0,
                                             0, 0);
  }
  issue_stage(src, lds, pb, 0);
  issue_stage(src, lds, pb + min(1, NPs - 1), 1);
  if (st_pro > st_lo) {                                   // uniform: affine with bias steps here
    bias_chunk(st_lo, st_pro - st_lo, true);              // waits for both stages too
    __builtin_amdgcn_s_waitcnt(0xC07F);                   // lgkmcnt(0): the chunk's reads are done
  } else {
    __builtin_amdgcn_s_waitcnt(0x0F78);                   // vmcnt(8): stage 0 in place, 1 may fly
  }
  asm volatile("s_barrier" ::: "memory");
  issue_stage(src, lds, pb + min(2, NPs - 1), 2);
  read_pair_head<BOOK, 0>(lds, boff, soff, pb, wq, sp);
#pragma unroll
  for (int j = 0; j < 8; ++j) carry[j] = read_frag<0>(lds, aoff, j);

  // Pair q from stage STAGE = q % 3. The loop below runs the pairs three at a time, so the
  // stage of every LDS read is a compile-time constant.
  auto pair = [&](auto stage_c, int q) {
    constexpr int STAGE = decltype(stage_c)::value, NEXT = (STAGE + 1) % kStages;
    const bool more = q + 1 < NPs;
    half8 fr[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) fr[j] = carry[j];
    half8 bf[4];
    float sc = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int gg = j >> 4, half = (j >> 3) & 1, i = (j >> 1) & 3, t = j & 1, mt = 2 * half + t;
      if (j == 24 && more) {
        // hand over stage p + 1: this wave's reads of stage p are issued and complete,
        // and stage p + 1 has landed for every wave
        __builtin_amdgcn_s_waitcnt(0x0078);                   // lgkmcnt(0) vmcnt(8): stage p + 2 may fly
        asm volatile("s_barrier" ::: "memory");
        issue_stage(src, lds, pb + min(q + 3, NPs - 1), STAGE);   // (q + 3) % 3 == STAGE
        // the last codes of this pair were read at step 22
        read_pair_head<BOOK, NEXT>(lds, boff, soff, pb + q + 1, wq, sp);
      }
      // (past the last pair the carried reads see a stale stage, and are not used)
      if (j + 8 < 32) fr[j + 8] = read_frag<STAGE>(lds, aoff, j + 8);
      else carry[j - 24] = read_frag<NEXT>(lds, aoff, j - 24);
      if ((j & 15) == 0 && BOOK == kAffine) sc = scale_f32<SD>((uint16_t)(sp[gg] & 0xFFFFu)) * kTwo24;
      if ((j & 15) < 8 && t == 0) {
        // codes of step i, group gg: word 2i + h, i.e. read (i & 1), element 2 gg + (i >> 1)
        const uint32_t u = wq[i & 1][2 * gg + (i >> 1)];
        if constexpr (BOOK == kAffine) bf[i] = nib8_to_half8_oddx16(u);
        else bf[i] = native8_to_half8<BOOK>(u);
      }
      if constexpr (BOOK == kAffine) {
        pp[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fr[j], bf[i], i == 0 ? f32x16{} : pp[mt], 0, 0, 0);
        // four FMAs of the other half: tiles 2, 3 (previous group, scale sc_prev) during
        // steps 0..7 of a group, tiles 0, 1 (this group, scale sc) during steps 8..15
        const int k = j & 7;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int idx = 4 * k + e, ft = idx >> 4, v = idx & 15;
          if (half == 0) acc[2 + ft][v] = __builtin_fmaf(sc_prev, pp[2 + ft][v], acc[2 + ft][v]);
          else acc[ft][v] = __builtin_fmaf(sc, pp[ft][v], acc[ft][v]);
        }
        // keep the four FMAs in this step: the compiler otherwise sinks them into clumps
        // after the MFMAs, which keeps more group products alive than registers allow
        const int ft = (4 * k) >> 4;
        if (half == 0) asm volatile("" : "+v"(acc[2 + ft]));
        else asm volatile("" : "+v"(acc[ft]));
        if ((j & 15) == 15) sc_prev = sc;
      } else {
        acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fr[j], bf[i], acc[mt], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int q = 0;
  for (; q + kStages <= NPs; q += kStages) {
    pair(std::integral_constant<int, 0>{}, q);
    pair(std::integral_constant<int, 1>{}, q + 1);
    pair(std::integral_constant<int, 2>{}, q + 2);
  }
  if (q < NPs) pair(std::integral_constant<int, 0>{}, q);
  if (q + 1 < NPs) pair(std::integral_constant<int, 1>{}, q + 1);
  __builtin_amdgcn_s_waitcnt(0);                          // the clamped duplicates have landed
  if constexpr (BOOK == kAffine) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      acc[2][v] = __builtin_fmaf(sc_prev, pp[2][v], acc[2][v]);
      acc[3][v] = __builtin_fmaf(sc_prev, pp[3][v], acc[3][v]);
    }
  }

  if constexpr (BOOK == kAffine) {
    // the bias steps the prologue left (long K, bf16 biases): the LDS from its start, which
    // the ring no longer uses
    for (int st0 = st_pro; st0 < st_hi; st0 += kBiasChunk) bias_chunk(st0, min(kBiasChunk, st_hi - st0), false);
  }

  // D of a 32x32 tile: lane l holds column l%32, rows 8 (v/4) + 4 (l/32) + v%4. acc becomes
  // this split's values (split 0's with y added when asked).
  const int n = n0 + 32 * wave + c32;
  const bool col = n < a.N;
  const float rs_n = BOOK == kAffine || !a.srow || !col ? 1.0f : a.srow[n];   // no row scales: the raw product
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = m0 + mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
      if (col && m < a.M) {
        float val = acc[mt][v];
        if constexpr (BOOK == kAffine)   // undoes the prep's 2^e, exactly (the scale staged in the prologue)
          val *= reinterpret_cast<const float *>(lds + kRscaleLds)[m - m0];
        if constexpr (BOOK == kInt16) {
          if (split == 0) val = __builtin_fmaf(0.5f, a.asum[m], val);
        }
        if constexpr (BOOK != kAffine) val *= rs_n;
        if (acc_here) val = a.y[(size_t)m * a.y_stride + n] + val;
        acc[mt][v] = val;
      }
    }
  }
  if (S == 1) {
    if (!col) return;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (m < a.M) a.y[(size_t)m * a.y_stride + n] = acc[mt][v];
      }
    return;
  }

  // Split K. Every split stores its values (split 0 in y, split s in y_part[s - 1]) with
  // agent-scope atomic stores, the coherent accesses every XCD sees, waits for them, and the
  // workgroup counts its arrival on the tile's counter. The split whose arrival is the
  // S-th adds the S values in split order (its own from registers, the others by
  // agent-scope atomic loads), writes y and sets the counter back to zero. No workgroup
  // waits for another, so nothing assumes the splits run at the same time.
  float *const mine = split == 0 ? a.y : a.y_part + (size_t)(split - 1) * a.M * a.N;
  const int mstride = split == 0 ? a.y_stride : a.N;
  if (col) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (m < a.M)
          __hip_atomic_store(mine + (size_t)m * mstride + n, acc[mt][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
  }
  __builtin_amdgcn_s_waitcnt(0);                     // this wave's values are stored
  __syncthreads();                                   // and every wave's
  int *const arrival = reinterpret_cast<int *>(lds);   // the ring and the bias pieces are done with
  const int tile = mb * ((a.N + kGN - 1) / kGN) + nb;
  if (tid == 0) arrival[0] = __hip_atomic_fetch_add(a.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (arrival[0] != S - 1) return;                   // uniform: the tile's last split goes on
  if (tid == 0) __hip_atomic_store(a.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (!col) return;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    // every value of this token tile is requested before the first is added
    float p[kMaxGemmSplit][16];
#pragma unroll
    for (int s = 0; s < kMaxGemmSplit; ++s) {
      if (s >= S || s == split) continue;            // uniform
      const float *src = s == 0 ? a.y : a.y_part + (size_t)(s - 1) * a.M * a.N;
      const int sstride = s == 0 ? a.y_stride : a.N;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = min(m0 + mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3), a.M - 1);
        p[s][v] = __hip_atomic_load(src + (size_t)m * sstride + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = m0 + mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
      float sum = split == 0 ? acc[mt][v] : p[0][v];
#pragma unroll
      for (int s = 1; s < kMaxGemmSplit; ++s)
        if (s < S) sum += s == split ? acc[mt][v] : p[s][v];
      if (m < a.M) a.y[(size_t)m * a.y_stride + n] = sum;
    }
  }
}

// ------------------------------------------------------------------ host

// K is split over S = 2 workgroups per output tile where that fills the rounds of the chip
// far better and the reduction is long: the workgroup takes about the same time per group
// pair whatever the shape (one 8-wave workgroup per CU), so a launch takes ceil(tiles S /
// 256) rounds of 1/S of a tile's time, plus the partials' hand-over (each split stores its
// 128 x 256 floats, the last one loads the others: measured about 20 us per launch of the
// 27B o or down projection at M = 2048). For a 2048-token chunk (16 token blocks) the 27B
// down projection (20 feature blocks, K = 17408) has 320 tiles, 1.25 rounds unsplit, 2.5
// split (497 -> 435 us with the prep pass); the o projection (the same tiles at K = 5120)
// gains less than the hand-over costs (180 -> 183 us), and 4 splits of either were slower
// still (198 and 440 us). So S = 2 for weights of at most 32 feature blocks whose rounds at
// 16 token blocks are at least 1.25 times fuller split, and whose K holds 64 group pairs or
// more. The choice depends on the weight's shape only, never on M, so a token's result is
// the same whatever the batch.
static double round_fill(int tiles) { return tiles / (256.0 * ((tiles + 255) / 256)); }
static int gemm_split_of(int K, int N) {
  const int nblocks = (N + kGN - 1) / kGN, NP = (K / kGroup + 1) / 2;
  if (nblocks > 32 || NP < 64) return 1;
  return round_fill(32 * nblocks) >= 1.25 * round_fill(16 * nblocks) ? kMaxGemmSplit : 1;
}

static size_t books_workspace(int book, int M, int K) {
  const int G = K / kGroup;
  if (book == kAffine)   // the group-sum pieces sized for bf16 biases, the larger of the two
    return ((size_t)M * K * 2 + 255) / 256 * 256 + ((size_t)M * gs_stride_of(G, 1) * 2 + 255) / 256 * 256 +
           ((size_t)M * sizeof(float) + 255) / 256 * 256;
  if (book == kInt16) return ((size_t)(G + 1) * ((M + 127) / 128 * 128) * sizeof(float) + 255) / 256 * 256;
  return 0;
}

// Rows of one launch of a split weight: as many whole token blocks as have counters.
static int split_chunk_rows(int N) { return kGemmMaxCounters / ((N + kGN - 1) / kGN) * kGM; }

size_t gemm4_workspace(int book, int M, int K, int N) {
  const int S = gemm_split_of(K, N);
  const size_t rows = S > 1 ? (size_t)std::min(M, split_chunk_rows(N)) : 0;
  return books_workspace(book, M, K) + (size_t)(S - 1) * rows * N * sizeof(float);
}

template <int BOOK, int SD>
static int launch_gemm4_inst(int accum, dim3 grid, size_t lds, hipStream_t st, const GemmArgs &a) {
  static LdsOptIn lds_acc, lds_set;
  if (accum) {
    if (int rc = allow_large_lds(reinterpret_cast<const void *>(&gemm4_kernel<BOOK, SD, true>), lds_acc)) return rc;
    gemm4_kernel<BOOK, SD, true><<<grid, kGThreads, lds, st>>>(a);
  } else {
    if (int rc = allow_large_lds(reinterpret_cast<const void *>(&gemm4_kernel<BOOK, SD, false>), lds_set)) return rc;
    gemm4_kernel<BOOK, SD, false><<<grid, kGThreads, lds, st>>>(a);
  }
  return 0;
}

int run_gemm4(int book, const _Float16 *x, int x_stride, int M, int K, int N, const void *codes, const void *sbq,
              int sd, const float *srow, float *y, int y_stride, int accum, int *cnt, void *ws, size_t ws_bytes,
              hipStream_t st) {
  const int G = K / kGroup;
  const size_t need = gemm4_workspace(book, M, K, N);
  RLQ_REQUIRE(ws_bytes >= need, "workspace of %zu bytes is smaller than the %zu this call needs", ws_bytes, need);
  RLQ_REQUIRE(need == 0 || aligned(ws, 256), "workspace must be 256-byte aligned");
  RLQ_REQUIRE((size_t)M * std::max(x_stride, K) * 2 < (1ull << 31), "prefill kernel: x spans more than 2 GiB");
  GemmArgs a = {};
  a.codes = static_cast<const u32x4 *>(codes);
  a.sb = static_cast<const u32x4 *>(sbq);
  a.srow = srow;
  a.y = y;
  a.M = M; a.K = K; a.N = N; a.y_stride = y_stride;
  if (book == kAffine) {
    const int gs_stride = gs_stride_of(G, sd);
    _Float16 *xp = static_cast<_Float16 *>(ws);
    const size_t xp_bytes = ((size_t)M * K * 2 + 255) / 256 * 256;
    uint16_t *gs = reinterpret_cast<uint16_t *>(static_cast<char *>(ws) + xp_bytes);
    float *rscale = reinterpret_cast<float *>(static_cast<char *>(ws) + xp_bytes +
                                              ((size_t)M * gs_stride_of(G, 1) * 2 + 255) / 256 * 256);
    const int cpt = (K / 8 + kPrepThreads - 1) / kPrepThreads;   // chunks of the row per thread
#define RLQ_PREP(THR, KERNEL, ...)                                                                                     \
  (sd == RLQ_BF16 ? KERNEL<1, ##__VA_ARGS__><<<M, THR, 0, st>>>(x, x_stride, M, K, xp, gs, gs_stride, rscale)          \
                  : KERNEL<0, ##__VA_ARGS__><<<M, THR, 0, st>>>(x, x_stride, M, K, xp, gs, gs_stride, rscale))
    if (cpt <= 4) RLQ_PREP(kPrepThreads, gemm_prep1_kernel, 4);
    else if (cpt <= 16) RLQ_PREP(1024, gemm_prep1_kernel, 4, 1024);   // K <= 32768: 4 chunks per thread of 1024
    else RLQ_PREP(kPrepThreads, gemm_prep_kernel);
#undef RLQ_PREP
    RLQ_HIP(hipGetLastError());
    a.x = xp; a.x_stride = K; a.gs = gs; a.gs_stride = gs_stride; a.rscale = rscale;
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
  const int S = gemm_split_of(K, N);
  RLQ_REQUIRE(S == 1 || cnt, "prefill kernel: this weight splits K in %d, which needs the workspace's counters", S);
  a.np_split = ((G + 1) / 2 + S - 1) / S;
  a.cnt = cnt;
  if (S > 1) a.y_part = reinterpret_cast<float *>(static_cast<char *>(ws) + books_workspace(book, M, K));
  const int nblocks = (N + kGN - 1) / kGN;
  const size_t lds = (size_t)kGemmLdsBytes;
  // a split weight launches in chunks of rows whose tiles have counters; the rows are
  // independent, so chunking changes no result
  const int chunk = S > 1 ? split_chunk_rows(N) : M;
  for (int r0 = 0; r0 < M; r0 += chunk) {
    GemmArgs c = a;
    c.M = std::min(chunk, M - r0);
    c.x = a.x + (size_t)r0 * a.x_stride;
    c.y = a.y + (size_t)r0 * a.y_stride;
    if (a.gs) c.gs = a.gs + (size_t)r0 * a.gs_stride;
    if (a.rscale) c.rscale = a.rscale + r0;
    if (a.asum) c.asum = a.asum + r0;
    const dim3 grid((c.M + kGM - 1) / kGM * nblocks, S);
    int rc;
    switch (book) {
      case kInt15: rc = launch_gemm4_inst<kInt15, 0>(accum, grid, lds, st, c); break;
      case kInt16: rc = launch_gemm4_inst<kInt16, 0>(accum, grid, lds, st, c); break;
      case kFp4: rc = launch_gemm4_inst<kFp4, 0>(accum, grid, lds, st, c); break;
      default:
        rc = sd == RLQ_BF16 ? launch_gemm4_inst<kAffine, 1>(accum, grid, lds, st, c)
                            : launch_gemm4_inst<kAffine, 0>(accum, grid, lds, st, c);
    }
    if (rc) return rc;
    RLQ_HIP(hipGetLastError());
  }
  return 0;
}

}  // namespace rlq
