// The engine layer over .rlm model files: what src/engine.mm does on the quantized matmul
// path, on a HIP device.
//  - rl_open: the model file (model_file.cpp) is read; every blocked matrix is uploaded to
//    HBM and packed once into the kernels' layout (include/rlq.h); float tensors are
//    uploaded; for native files the norm weights are folded with the column scales of the
//    matrices they feed (src/engine.mm:517-530). The engine's scratch (normed rows, the
//    gate/up products, activations, MoE workspace, logits) is sized by max_chunk.
//  - rl_linear: Engine::encode_linear (engine.mm:832-906), dispatched on the tensor kind.
//  - rl_norm: Engine::encode_norm / rms_norm_rows (engine.mm:908-932, ops.metal:74-112).
//  - rl_mlp: Engine::encode_mlp and encode_moe (engine.mm:943-1059).
//  - rl_head, rl_draft_head: the output head with the draft vocabulary (engine.mm:1425-1458,
//    :1634-1638); rl_top_k and a device top-k (capi.mm:74-101).
// The attention, linear-attention, embedding and sampling parts of a forward pass are not
// part of this build: rl_forward is not provided.
#include "linear.h"
#include "model_file.h"
#include "q4_tile.h"
#include "rlq_common.h"
#include "../../include/rl_engine.h"
#include "../../include/rlq.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <numeric>
#include <string>
#include <vector>

namespace rlq {

// ------------------------------------------------------------------ device memory

// One device allocation, freed with its owner.
struct DevMem {
  void *p = nullptr;
  size_t bytes = 0;
  DevMem() = default;
  DevMem(const DevMem &) = delete;
  DevMem &operator=(const DevMem &) = delete;
  DevMem(DevMem &&o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr; o.bytes = 0; }
  DevMem &operator=(DevMem &&o) noexcept {
    if (this != &o) {
      release();
      p = o.p;
      bytes = o.bytes;
      o.p = nullptr;
      o.bytes = 0;
    }
    return *this;
  }
  ~DevMem() { release(); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  template <typename T> T *as() const { return static_cast<T *>(p); }
};

static int dev_alloc(DevMem &m, size_t bytes, const char *what) {
  m.release();
  if (bytes == 0) return 0;
  const hipError_t e = hipMalloc(&m.p, bytes);
  if (e != hipSuccess) {
    m.p = nullptr;
    return fail("rl_open: cannot allocate %zu bytes of device memory for %s (%s)", bytes, what, hipGetErrorString(e));
  }
  m.bytes = bytes;
  return 0;
}

// ------------------------------------------------------------------ kernels

constexpr int kNormThreads = 256;

constexpr int kNormMaxPer = 32;   // rows of up to 8192 take the register form

// The sum of the threads' partial sums of squares, in a fixed tree (butterfly in each wave,
// then the waves in order); every thread gets it.
__device__ __forceinline__ float norm_total(float ss, float *part) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) ss += __shfl_xor(ss, d);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int wv = 0; wv < kNormThreads / 64; ++wv) total += part[wv];
  return total;
}

// One element of a normed row, half(x * inv * w): the one expression every kernel that
// norms a row uses, so that they give the same bits.
__device__ __forceinline__ _Float16 norm_out(float x, float inv, float w) { return static_cast<_Float16>(x * inv * w); }

// out[r][i] = half(h[r][i] * inv * w[i]), inv = 1 / sqrt(sum_i h[r][i]^2 / D + eps): one
// workgroup per row. Each thread sums its elements i = tid, tid + 256, ... in order, and
// the threads' sums meet in norm_total's tree, so a row's result depends on nothing but the
// row (the property kernels/ops.metal:60-72 keeps for chunking). With PER > 0 (D <= 256 PER)
// a thread issues the loads of all its elements of h and w at once and keeps them in
// registers (buffer loads whose range check returns 0 past D; a zero adds nothing to the
// sum of squares), so the row costs one memory round trip instead of one per element; the
// arithmetic is the same. PER = 0 is the loop form for longer rows.
template <int PER>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const float *h, int h_stride, const float *w, int D,
                                                                float eps, _Float16 *out, int out_stride) {
  __shared__ float part[kNormThreads / 64];
  const float *x = h + (size_t)blockIdx.x * h_stride;
  _Float16 *o = out + (size_t)blockIdx.x * out_stride;
  float ss = 0.0f;
  if constexpr (PER > 0) {
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)D * 4u), rw = make_rsrc(w, (uint32_t)D * 4u);
    float xv[PER], wv[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j)
      xv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                            rx, 4u * (threadIdx.x + (uint32_t)j * kNormThreads), 0, 0));
#pragma unroll
    for (int j = 0; j < PER; ++j)
      wv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                            rw, 4u * (threadIdx.x + (uint32_t)j * kNormThreads), 0, 0));
#pragma unroll
    for (int j = 0; j < PER; ++j) ss = __builtin_fmaf(xv[j], xv[j], ss);
    const float inv = 1.0f / __builtin_sqrtf(norm_total(ss, part) / (float)D + eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = threadIdx.x + j * kNormThreads;
      if (i < D) o[i] = norm_out(xv[j], inv, wv[j]);
    }
  } else {
    for (int i = threadIdx.x; i < D; i += kNormThreads) ss = __builtin_fmaf(x[i], x[i], ss);
    const float inv = 1.0f / __builtin_sqrtf(norm_total(ss, part) / (float)D + eps);
    for (int i = threadIdx.x; i < D; i += kNormThreads) o[i] = norm_out(x[i], inv, w[i]);
  }
}

// One token's norm and the dense (f16b) router product in one launch, for the mixture of
// experts at decode (src/engine.mm:965-991: encode_rms, then the router linear): workgroup
// b takes router tile b, forms the normed row itself (threads 0..255 sum the squares in
// rms_norm_kernel's order, waves 0..3 meet as norm_total meets them, every element is
// norm_out's), keeps it in LDS, and multiplies it into its tile as dense_f16_kernel does
// (the waves split the K steps into ranges of spw, chain their MFMAs, add their partials in
// wave order), so logits and normed row have the bits of rl_norm followed by rl_linear.
// Workgroup 0 also writes the normed row for the expert kernels. Waves: dense_f16_kernel's
// for this K (at least 4, for the norm's 256 threads); spw <= 8 (one batch of loads).
constexpr int kDenseStep = 32;   // inputs per 1 KB block of the dense f16 layout (dense.hip)

template <int PER>
__global__ __launch_bounds__(1024) void norm_router_kernel(const float *h, const float *nw, int D, float eps,
                                                           _Float16 *xn_out, const u32x4 *w, int N, int spw,
                                                           float *y) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  float *part = reinterpret_cast<float *>(lds);                                   // [4]
  _Float16 *xs = reinterpret_cast<_Float16 *>(lds + 16);                          // [D]
  f32x4 *red = reinterpret_cast<f32x4 *>(lds + 16 + ((size_t)D * 2 + 15) / 16 * 16);   // [waves-1][64]
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, j4 = lane >> 4;
  const int t = blockIdx.x;
  const int steps = D / kDenseStep;
  const int s0 = wave * spw, s1 = min(steps, s0 + spw);
  // the norm's loads first (threads 0..255, rms_norm_kernel<PER>'s elements), then the
  // router tile's: the first wait is for the norm's only
  const bool nt = threadIdx.x < kNormThreads;
  const __amdgpu_buffer_rsrc_t rh = make_rsrc(h, nt ? (uint32_t)D * 4u : 0u), rn = make_rsrc(nw, nt ? (uint32_t)D * 4u : 0u);
  float xv[PER], wv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j)
    xv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                          rh, 4u * (threadIdx.x + (uint32_t)j * kNormThreads), 0, 0));
#pragma unroll
  for (int j = 0; j < PER; ++j)
    wv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                          rn, 4u * (threadIdx.x + (uint32_t)j * kNormThreads), 0, 0));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w + ((size_t)t * steps + s0) * 64, (uint32_t)max(0, s1 - s0) * 1024u);
  u32x4 wb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    wb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, 16u * lane + (uint32_t)i * 1024u, 0,
                                                                           kNonTemporal));
  __builtin_amdgcn_sched_barrier(0);
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) ss = __builtin_fmaf(xv[j], xv[j], ss);
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) ss += __shfl_xor(ss, d);
  if (nt && lane == 0) part[wave] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int wv4 = 0; wv4 < kNormThreads / 64; ++wv4) total += part[wv4];
  const float inv = 1.0f / __builtin_sqrtf(total / (float)D + eps);
  if (nt) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = threadIdx.x + j * kNormThreads;
      if (i < D) {
        const _Float16 v = norm_out(xv[j], inv, wv[j]);
        xs[i] = v;
        if (t == 0) xn_out[i] = v;
      }
    }
  }
  __syncthreads();
  // dense_f16_kernel's products for token row 0 (lanes c16 = 0; the other rows are zeros)
  f32x4 acc = {};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int st = s0 + i;
    const u32x4 xb = c16 == 0 && st < s1 ? *reinterpret_cast<const u32x4 *>(xs + st * kDenseStep + 8 * j4)
                                         : u32x4{0u, 0u, 0u, 0u};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, xb), __builtin_bit_cast(half8, wb[i]), acc,
                                                 0, 0, 0);
  }
  acc = reduce_waves(acc, red, wave, waves, lane);
  const int n = 16 * t + c16;
  if (wave == 0 && j4 == 0 && n < N) y[n] = acc[0];
}

// Top-k with rl_top_k's order (value descending, equal values by index ascending, NaN left
// out). Pass 1: workgroup b takes entries [b C, (b+1) C) and picks its k best by k rounds
// of a workgroup-wide best (each thread holds its entries in registers and marks the ones
// taken); merge passes then pick the k best of groups of candidates the same way until one
// workgroup is left. A round's best: the larger value, then the lower index.
constexpr int kTopkThreads = 256;
constexpr int kTopkPer = 8;                                  // entries per thread in pass 1
constexpr int kTopkChunk = kTopkThreads * kTopkPer;          // C
constexpr int kTopkMaxK = 256;
constexpr int kTopkMergeThreads = 1024;

struct Cand {
  float v;
  int i;   // -1: none
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  if (i < 0) return false;
  if (bi < 0) return true;
  return v > bv || (v == bv && i < bi);
}

// The workgroup's best (value, index) of each thread's (v, i); every thread gets it.
template <int THREADS>
__device__ __forceinline__ Cand block_best(float v, int i, Cand *scratch) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const float ov = __shfl_xor(v, d);
    const int oi = __shfl_xor(i, d);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = Cand{v, i};
  __syncthreads();
  Cand b = scratch[0];
#pragma unroll
  for (int w = 1; w < THREADS / 64; ++w)
    if (better(scratch[w].v, scratch[w].i, b.v, b.i)) b = scratch[w];
  __syncthreads();   // scratch is reused by the next round
  return b;
}

template <int PER, int THREADS>
__device__ __forceinline__ void pick_k(const float (&v)[PER], const int (&idx)[PER], int k, float *out_v, int *out_i,
                                       Cand *scratch) {
  static_assert(PER <= 64, "one bit per entry");
  uint64_t taken = 0;
  for (int r = 0; r < k; ++r) {
    // this thread's best entry not yet taken
    float bv = 0.0f;
    int bi = -1, bj = -1;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (!(taken >> j & 1ull) && better(v[j], idx[j], bv, bi)) {
        bv = v[j];
        bi = idx[j];
        bj = j;
      }
    const Cand b = block_best<THREADS>(bv, bi, scratch);
    if (b.i >= 0 && b.i == bi) taken |= 1ull << bj;   // indices are distinct: one thread owns it
    if (threadIdx.x == 0) {
      out_v[r] = b.v;
      out_i[r] = b.i;
    }
  }
}

__global__ __launch_bounds__(kTopkThreads) void topk_chunk_kernel(const float *x, int n, int k, float *cand_v,
                                                                  int *cand_i) {
  __shared__ Cand scratch[kTopkThreads / 64];
  float v[kTopkPer];
  int idx[kTopkPer];
#pragma unroll
  for (int j = 0; j < kTopkPer; ++j) {
    const int i = blockIdx.x * kTopkChunk + j * kTopkThreads + threadIdx.x;
    const float val = i < n ? x[i] : 0.0f;
    v[j] = val;
    idx[j] = i < n && !__builtin_isnan(val) ? i : -1;
  }
  pick_k<kTopkPer, kTopkThreads>(v, idx, k, cand_v + (size_t)blockIdx.x * k, cand_i + (size_t)blockIdx.x * k, scratch);
}

// Pass 2 and later: workgroup b takes candidates [b G, (b+1) G) of m, G = 1024 PER, and
// writes its k best to out + b k. The k best of a union are the k best of the groups' k
// best, so passes repeat until one workgroup is left; every candidate keeps its index
// into x, so the order (value, then index) is the same as one merge over all of them.
constexpr int kTopkMergePer = 16;
constexpr int kTopkMergeGroup = kTopkMergeThreads * kTopkMergePer;

template <int PER>
__global__ __launch_bounds__(kTopkMergeThreads) void topk_merge_kernel(const float *cand_v, const int *cand_i, int m,
                                                                       int k, float *out_v, int *out_i) {
  __shared__ Cand scratch[kTopkMergeThreads / 64];
  float v[PER];
  int idx[PER];
  const int base = blockIdx.x * kTopkMergeThreads * PER;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = base + j * kTopkMergeThreads + threadIdx.x;
    v[j] = c < m ? cand_v[c] : 0.0f;
    idx[j] = c < m ? cand_i[c] : -1;
  }
  pick_k<PER, kTopkMergeThreads>(v, idx, k, out_v + (size_t)blockIdx.x * k, out_i + (size_t)blockIdx.x * k, scratch);
}

// ------------------------------------------------------------------ the engine

// One matrix of the model in device memory.
struct EngineTensor {
  const QTensor *q = nullptr;
  DevMem packed;     // the kernels' layout of all n_pad rows (affine: codes then scale quads)
  DevMem srow;       // native: row scales [n_pad]
  DevMem col;        // native: column scales [k]
  bool moe_gate_up = false;   // an affine expert gate/up stack (rows interleaved per tile)
};

}  // namespace rlq

struct rl_engine {
  std::unique_ptr<rlq::ModelFile> model;
  int max_chunk = 0;
  std::map<std::string, rlq::EngineTensor> mats;
  std::map<std::string, rlq::DevMem> floats;     // f32 tensors as they are in the file
  std::vector<rlq::DevMem> norm_in, norm_post;   // native: folded norm weights per layer
  rlq::DevMem norm_final;
  rlq::DevMem norm_mtp_out;                      // native files with an MTP head: mtp.norm folded with lm_head's column scales
  bool has_mtp = false;
  int x_stride = 0, proj_stride = 0, act_stride = 0, router_stride = 0;
  rlq::DevMem xn, proj, act, router_logits, linear_ws, moe_ws, logits, draft_logits, slots;
  rlq::DevMem topk_v, topk_i, topk_v2, topk_i2, topk_out_v, topk_out_i;
  int head_rows_done = 0;                        // rows of the last rl_head
  hipStream_t head_stream = nullptr;             // the stream the last rl_head ran on
  int draft_vocab_rows = 0, draft_tail_first = -1;
};

namespace rlq {

static std::string lname(int layer, const char *what) { return "layers." + std::to_string(layer) + "." + what; }

static bool ends_with(const std::string &s, const char *tail) {
  const size_t n = strlen(tail);
  return s.size() >= n && s.compare(s.size() - n, n, tail) == 0;
}

static const EngineTensor *tensor_of(const rl_engine *e, const std::string &name) {
  auto it = e->mats.find(name);
  return it == e->mats.end() ? nullptr : &it->second;
}

static int copy_range(void *dst, const uint8_t *base, uint64_t off, size_t bytes) {
  RLQ_HIP(hipMemcpy(dst, base + off, bytes, hipMemcpyHostToDevice));
  return 0;
}

// Uploads and packs one blocked matrix (staging: a device buffer large enough for its file
// bytes). Expert gate/up stacks of affine files are repacked through the MLX layout so that
// each 16-row tile holds the gate and up rows of 8 features (rlq_pack_moe_gate_up).
static int upload_matrix(rl_engine *e, const std::string &name, const QTensor &q, DevMem &staging, int E1, int I) {
  const uint8_t *base = e->model->data();
  EngineTensor t;
  t.q = &q;
  const size_t K = (size_t)q.k, NP = (size_t)q.n_pad;
  if (q.kind == kKindF16b) {
    const size_t wb = NP * K * 2;
    if (int rc = copy_range(staging.p, base, q.w, wb)) return rc;
    if (int rc = dev_alloc(t.packed, rlq_packed_f16_bytes(q.k, q.n_pad), name.c_str())) return rc;
    if (int rc = rlq_pack_f16_blocked(staging.p, q.k, q.n_pad, 0, q.n_pad, t.packed.p, nullptr)) return rc;
  } else if (q.kind == kKindQ4n) {
    const size_t wb = NP * K / 2;
    if (int rc = copy_range(staging.p, base, q.w, wb)) return rc;
    if (int rc = dev_alloc(t.packed, rlq_packed_codes_bytes(q.k, q.n_pad), name.c_str())) return rc;
    if (int rc = rlq_pack_native_blocked(staging.as<uint8_t>(), q.k, q.n_pad, 0, q.n_pad, t.packed.p, nullptr)) return rc;
    if (int rc = dev_alloc(t.srow, NP * 4, name.c_str())) return rc;
    if (int rc = copy_range(t.srow.p, base, q.s, NP * 4)) return rc;
    if (int rc = dev_alloc(t.col, K * 4, name.c_str())) return rc;
    if (int rc = copy_range(t.col.p, base, q.c, K * 4)) return rc;
  } else {   // q4a
    const size_t wb = NP * K / 2, sb = NP * (K / 64) * 2;
    uint8_t *w = staging.as<uint8_t>();
    uint16_t *s = reinterpret_cast<uint16_t *>(w + wb), *b = s + sb / 2;
    if (int rc = copy_range(w, base, q.w, wb)) return rc;
    if (int rc = copy_range(s, base, q.s, sb)) return rc;
    if (int rc = copy_range(b, base, q.b, sb)) return rc;
    if (E1 > 0) {
      // an expert gate/up stack: blocked -> MLX rows (after the file bytes in staging) -> interleaved pack
      t.moe_gate_up = true;
      const int rows = E1 * 2 * I;
      RLQ_REQUIRE(q.n == rows, "%s: %d rows, the mixture of experts needs %d", name.c_str(), q.n, rows);
      uint32_t *mw = reinterpret_cast<uint32_t *>(w + wb + 2 * sb);
      uint16_t *ms = reinterpret_cast<uint16_t *>(mw + (size_t)rows * (K / 8));
      uint16_t *mb = ms + (size_t)rows * (K / 64);
      if (int rc = rlq_repack_blocked(w, s, b, q.k, q.n_pad, 0, rows, mw, ms, mb, nullptr)) return rc;
      if (int rc = dev_alloc(t.packed, rlq_packed_affine_bytes(q.k, rows), name.c_str())) return rc;
      if (int rc = rlq_pack_moe_gate_up(mw, ms, mb, q.k, E1, I, t.packed.p, nullptr)) return rc;
    } else {
      if (int rc = dev_alloc(t.packed, rlq_packed_affine_bytes(q.k, q.n_pad), name.c_str())) return rc;
      if (int rc = rlq_pack_affine_blocked(w, s, b, q.k, q.n_pad, 0, q.n_pad, t.packed.p, nullptr)) return rc;
    }
  }
  RLQ_HIP(hipDeviceSynchronize());   // staging is reused by the next matrix
  e->mats[name] = std::move(t);
  return 0;
}

// Staging bytes one matrix needs (the file bytes; for an affine expert gate/up stack also
// its MLX form).
static size_t staging_bytes(const QTensor &q, bool gate_up_stack) {
  const size_t K = (size_t)q.k, NP = (size_t)q.n_pad;
  if (q.kind == kKindF16b) return NP * K * 2;
  if (q.kind == kKindQ4n) return NP * K / 2;
  size_t b = NP * K / 2 + 2 * NP * (K / 64) * 2;
  if (gate_up_stack) b += (size_t)q.n * (K / 2 + 2 * (K / 64) * 2);
  return b + 256;
}

static int fold_norm(rl_engine *e, DevMem &dst, const FTensor &norm, const QTensor *consumer) {
  const int H = e->model->config().hidden;
  RLQ_REQUIRE((int)norm.count() >= H, "a norm weight has %zu entries, hidden size is %d", norm.count(), H);
  std::vector<float> w(H);
  memcpy(w.data(), e->model->data() + norm.offset, (size_t)H * 4);
  if (consumer && consumer->native) {
    RLQ_REQUIRE(consumer->k >= H, "a native matrix fed by a norm has k=%d < hidden %d", consumer->k, H);
    const float *cs = reinterpret_cast<const float *>(e->model->data() + consumer->c);
    for (int k = 0; k < H; ++k) w[k] *= cs[k];
  }
  if (int rc = dev_alloc(dst, (size_t)H * 4, "a norm weight")) return rc;
  RLQ_HIP(hipMemcpy(dst.p, w.data(), (size_t)H * 4, hipMemcpyHostToDevice));
  return 0;
}

static int open_engine(rl_engine *e, const char *path, int max_ctx, int max_chunk) {
  RLQ_REQUIRE(path, "rl_open: null path");
  RLQ_REQUIRE(max_chunk >= 1 && max_chunk <= (1 << 20) && max_ctx >= 0, "rl_open: max_chunk=%d max_ctx=%d", max_chunk,
              max_ctx);
  if (int rc = ModelFile::open(path, e->model)) return rc;
  const ModelConfig &c = e->model->config();
  // the geometry the reference's kernels assume (src/engine.mm:394-396)
  if (c.lin_k_dim != 128 || c.head_dim != 256 || c.rope_dims() != 64 || c.conv_taps != 4 || c.group != 64 ||
      c.block != 256 || c.lin_v_dim % 8 != 0 || c.kv_heads <= 0 || c.heads % c.kv_heads != 0)
    return fail("unsupported model geometry (kernels assume Dk=128, head_dim=256, 64 rotary dims, 4 conv taps)");
  if (c.native && c.book != "fp4" && c.book != "int15")
    return fail("codebook '%s' is not supported by this build", c.book.c_str());
  RLQ_REQUIRE(c.hidden > 0 && c.hidden % 64 == 0, "rl_open: hidden size %d is not a multiple of 64", c.hidden);
  e->max_chunk = max_chunk;
  const int E1 = c.is_moe() ? c.experts + 1 : 0;

  // every blocked matrix, packed; the largest one sizes the staging buffer
  size_t stage = 0;
  for (const auto &kv : e->model->qtensors()) {
    const QTensor &q = kv.second;
    if (!q.blocked) continue;   // token tables: not on this path
    stage = std::max(stage, staging_bytes(q, c.is_moe() && !q.native && ends_with(kv.first, ".moe.gate_up")));
  }
  DevMem staging;
  if (int rc = dev_alloc(staging, stage, "staging")) return rc;
  for (const auto &kv : e->model->qtensors()) {
    const QTensor &q = kv.second;
    if (!q.blocked) continue;
    const std::string &name = kv.first;
    const bool gu = c.is_moe() && !q.native && ends_with(name, ".moe.gate_up");
    if (int rc = upload_matrix(e, name, q, staging, gu ? E1 : 0, c.moe_inter)) return rc;
  }
  staging.release();
  for (const auto &kv : e->model->ftensors()) {
    DevMem m;
    const size_t bytes = kv.second.count() * 4;
    if (int rc = dev_alloc(m, std::max<size_t>(bytes, 4), kv.first.c_str())) return rc;
    if (bytes) RLQ_HIP(hipMemcpy(m.p, e->model->data() + kv.second.offset, bytes, hipMemcpyHostToDevice));
    e->floats[kv.first] = std::move(m);
  }
  // native files: norm weights times the column scales of the matrix each one feeds
  if (c.native) {
    e->norm_in.resize(c.layers);
    e->norm_post.resize(c.layers);
    for (int i = 0; i < c.layers; ++i) {
      const FTensor *fin = e->model->f(lname(i, "in_norm"));
      const QTensor *cin = e->model->q(lname(i, "lin.in_proj"));
      if (!cin) cin = e->model->q(lname(i, "attn.qkv"));
      if (fin)
        if (int rc = fold_norm(e, e->norm_in[i], *fin, cin)) return rc;
      const FTensor *fpost = e->model->f(lname(i, "post_norm"));
      const QTensor *cpost = e->model->q(lname(i, c.is_moe() ? "moe.gate_up" : "mlp.gate_up"));
      if (fpost)
        if (int rc = fold_norm(e, e->norm_post[i], *fpost, cpost)) return rc;
    }
    if (const FTensor *ff = e->model->f("final_norm"))
      if (int rc = fold_norm(e, e->norm_final, *ff, e->model->q("lm_head"))) return rc;
    // the MTP head's output norm, folded as src/engine.mm:534 does (has_mtp_: native files
    // with mtp.fc, :398)
    const FTensor *fm = e->model->f("mtp.norm");
    if (e->model->q("mtp.fc") && fm) {
      if (int rc = fold_norm(e, e->norm_mtp_out, *fm, e->model->q("lm_head"))) return rc;
      e->has_mtp = true;
    }
  }

  // scratch sized by max_chunk (src/engine.mm:398-449)
  const size_t R = (size_t)max_chunk;
  int xs = c.hidden;
  size_t lin_ws = 0;
  for (const auto &kv : e->mats) {
    const QTensor &q = *kv.second.q;
    xs = std::max(xs, q.k);
    // every matrix rl_linear, rl_mlp or the head runs through the linear kernels, the MoE
    // router included, at up to max_chunk rows (expert stacks run on the MoE workspace)
    const bool expert_stack = ends_with(kv.first, ".moe.gate_up") || ends_with(kv.first, ".moe.down");
    if (q.kind != kKindF16b && !expert_stack)
      lin_ws = std::max(lin_ws, rlq_linear_workspace_bytes(max_chunk, q.k, q.n_pad));
  }
  e->x_stride = (xs + 7) / 8 * 8;
  for (int i = 0; i < c.layers; ++i)
    if (const QTensor *gu = e->model->q(lname(i, "mlp.gate_up"))) e->proj_stride = std::max(e->proj_stride, gu->n_pad);
  e->act_stride = (std::max(c.intermediate, c.moe_inter) + 7) / 8 * 8;
  if (int rc = dev_alloc(e->xn, R * e->x_stride * 2 + 256, "xn")) return rc;
  if (e->proj_stride)
    if (int rc = dev_alloc(e->proj, R * e->proj_stride * 4, "proj")) return rc;
  if (int rc = dev_alloc(e->act, R * std::max(e->act_stride, 8) * 2 + 256, "act")) return rc;
  if (int rc = dev_alloc(e->linear_ws, lin_ws, "the linear workspace")) return rc;
  if (lin_ws) RLQ_HIP(hipMemset(e->linear_ws.p, 0, lin_ws));   // the decode kernel's split counters start at zero
  if (c.is_moe()) {
    const QTensor *router = e->model->q(lname(0, "moe.router"));
    RLQ_REQUIRE(router, "model has no quantized tensor '%s'", lname(0, "moe.router").c_str());
    e->router_stride = router->n_pad;
    if (int rc = dev_alloc(e->router_logits, R * e->router_stride * 4, "router logits")) return rc;
    if (int rc = dev_alloc(e->moe_ws, rlq_moe_workspace_bytes(max_chunk, c.experts, c.experts_per_tok, c.hidden,
                                                              c.moe_inter), "the MoE workspace"))
      return rc;
    std::vector<int> ident(E1);
    std::iota(ident.begin(), ident.end(), 0);
    if (int rc = dev_alloc(e->slots, (size_t)E1 * 4, "the slot table")) return rc;
    RLQ_HIP(hipMemcpy(e->slots.p, ident.data(), (size_t)E1 * 4, hipMemcpyHostToDevice));
  }
  if (const QTensor *head = e->model->q("lm_head")) {
    if (int rc = dev_alloc(e->logits, (size_t)16 * head->n_pad * 4, "logits")) return rc;
    if (int rc = dev_alloc(e->draft_logits, (size_t)head->n_pad * 4, "draft logits")) return rc;
  }
  const size_t chunks = (std::max<size_t>(e->logits.bytes / 4, 1) + kTopkChunk - 1) / kTopkChunk + 1;
  if (int rc = dev_alloc(e->topk_v, chunks * kTopkMaxK * 4, "top-k")) return rc;
  if (int rc = dev_alloc(e->topk_i, chunks * kTopkMaxK * 4, "top-k")) return rc;
  // the second merge buffer: the groups of the first merge pass, k best each (later passes
  // shrink and alternate between the two)
  const size_t groups = (chunks * kTopkMaxK + kTopkMergeGroup - 1) / kTopkMergeGroup;
  if (int rc = dev_alloc(e->topk_v2, groups * kTopkMaxK * 4, "top-k")) return rc;
  if (int rc = dev_alloc(e->topk_i2, groups * kTopkMaxK * 4, "top-k")) return rc;
  if (int rc = dev_alloc(e->topk_out_v, kTopkMaxK * 4, "top-k")) return rc;
  if (int rc = dev_alloc(e->topk_out_i, kTopkMaxK * 4, "top-k")) return rc;
  return 0;
}

// encode_linear over rows [r0, r0 + N) of a matrix (r0 a multiple of 16).
static int linear_rows(rl_engine *e, const EngineTensor &t, int r0, int N, const _Float16 *x, int x_stride, int M,
                       float *out, int out_stride, int accum, hipStream_t st) {
  const QTensor &q = *t.q;
  const ModelConfig &c = e->model->config();
  RLQ_REQUIRE(r0 % 16 == 0 && r0 >= 0 && N >= 1 && r0 + N <= q.n_pad, "rows [%d, %d) of a %d-row matrix", r0, r0 + N,
              q.n_pad);
  RLQ_REQUIRE(M >= 1 && M <= e->max_chunk && x && out, "rl_linear: %d rows (max_chunk %d) or a null buffer", M,
              e->max_chunk);
  RLQ_REQUIRE(x_stride >= q.k && x_stride % 8 == 0 && aligned(x, 16), "rl_linear: x_stride=%d for k=%d", x_stride,
              q.k);
  RLQ_REQUIRE(out_stride >= N && aligned(out, 4), "rl_linear: out_stride=%d < %d", out_stride, N);
  if (q.kind == kKindF16b) {
    RLQ_REQUIRE(r0 == 0, "a dense matrix runs whole");
    return rlq_linear_f16(x, x_stride, M, q.k, N, t.packed.p, out, out_stride, accum, st);
  }
  const int tile = r0 / 16;
  const char *codes = t.packed.as<char>() + packed_tile_code_offset(q.k, tile);
  if (q.kind == kKindQ4n) {
    const std::string &bk = q.book.empty() ? c.book : q.book;
    const int book = bk == "fp4" ? kFp4 : bk == "int16" ? kInt16 : kInt15;
    return linear_packed(0, book, x, x_stride, M, q.k, N, codes, codes, RLQ_F16, t.srow.as<float>() + r0, out,
                         out_stride, accum, e->linear_ws.p, e->linear_ws.bytes, st);
  }
  const char *sbq = t.packed.as<char>() + packed_code_bytes(q.k, q.n_pad) + packed_tile_sb_offset(q.k, tile);
  return linear_packed(0, kAffine, x, x_stride, M, q.k, N, codes, sbq, RLQ_BF16, nullptr, out, out_stride, accum,
                       e->linear_ws.p, e->linear_ws.bytes, st);
}

static int norm_with(rl_engine *e, const float *w, const float *h, int h_stride, int rows, _Float16 *xn,
                     int xn_stride, hipStream_t st) {
  const ModelConfig &c = e->model->config();
  const int per = (c.hidden + kNormThreads - 1) / kNormThreads;
  auto launch = [&](auto kernel) {
    kernel<<<rows, kNormThreads, 0, st>>>(h, h_stride, w, c.hidden, c.norm_eps, xn, xn_stride);
  };
  if (per <= 8) launch(rms_norm_kernel<8>);
  else if (per <= 16) launch(rms_norm_kernel<16>);
  else if (per <= 20) launch(rms_norm_kernel<20>);
  else if (per <= kNormMaxPer) launch(rms_norm_kernel<kNormMaxPer>);
  else launch(rms_norm_kernel<0>);
  RLQ_HIP(hipGetLastError());
  return 0;
}

// the weight of norm `which` (0 input, 1 post-attention, 2 final) of a layer: native files'
// folded copies, the file's own float tensor otherwise; nullptr when the file has none
static const float *norm_weight(rl_engine *e, int which, int layer) {
  const ModelConfig &c = e->model->config();
  if (c.native) {
    const DevMem &m = which == 2 ? e->norm_final : which == 0 ? e->norm_in[layer] : e->norm_post[layer];
    return m.as<float>();
  }
  const std::string name = which == 2 ? std::string("final_norm") : lname(layer, which == 0 ? "in_norm" : "post_norm");
  auto it = e->floats.find(name);
  return it == e->floats.end() ? nullptr : it->second.as<float>();
}

static int norm_rows(rl_engine *e, int which, int layer, const float *h, int h_stride, int rows, _Float16 *xn,
                     int xn_stride, hipStream_t st) {
  const ModelConfig &c = e->model->config();
  RLQ_REQUIRE(which >= 0 && which <= 2, "rl_norm: which=%d (0 input, 1 post-attention, 2 final)", which);
  RLQ_REQUIRE(which == 2 || (layer >= 0 && layer < c.layers), "rl_norm: layer %d of %d", layer, c.layers);
  RLQ_REQUIRE(h && xn && rows >= 1 && h_stride >= c.hidden && xn_stride >= c.hidden, "rl_norm: bad rows or strides");
  const float *w = norm_weight(e, which, layer);
  RLQ_REQUIRE(w, "model has no float tensor for norm %d of layer %d", which, layer);
  return norm_with(e, w, h, h_stride, rows, xn, xn_stride, st);
}

static int top_k_device(rl_engine *e, const float *x, int n, int k, int32_t *ids, float *vals, hipStream_t st) {
  RLQ_REQUIRE(x && ids && vals && n >= 0 && k >= 0 && k <= kTopkMaxK, "rl_top_k_device: k=%d (<= %d) n=%d", k,
              kTopkMaxK, n);
  k = std::min(k, n);
  if (k == 0) return 0;
  const int chunks = (n + kTopkChunk - 1) / kTopkChunk;
  RLQ_REQUIRE((size_t)chunks * k * 4 <= e->topk_v.bytes, "rl_top_k_device: n=%d is more than the engine's logits", n);
  topk_chunk_kernel<<<chunks, kTopkThreads, 0, st>>>(x, n, k, e->topk_v.as<float>(), e->topk_i.as<int>());
  RLQ_HIP(hipGetLastError());
  // merge passes: ping-pong between the two candidate buffers until one group is left,
  // which writes the result
  float *cv = e->topk_v.as<float>(), *tv = e->topk_v2.as<float>();
  int *ci = e->topk_i.as<int>(), *ti = e->topk_i2.as<int>();
  for (int m = chunks * k;;) {
    const int groups = (m + kTopkMergeGroup - 1) / kTopkMergeGroup;
    float *ov = groups == 1 ? e->topk_out_v.as<float>() : tv;
    int *oi = groups == 1 ? e->topk_out_i.as<int>() : ti;
    RLQ_REQUIRE((size_t)groups * k * 4 <= (groups == 1 ? e->topk_out_v.bytes : e->topk_v2.bytes),
                "rl_top_k_device: %d candidates do not fit the merge buffer", m);
    const int per = (m + kTopkMergeThreads - 1) / kTopkMergeThreads;
    if (per <= 1) topk_merge_kernel<1><<<groups, kTopkMergeThreads, 0, st>>>(cv, ci, m, k, ov, oi);
    else if (per <= 4) topk_merge_kernel<4><<<groups, kTopkMergeThreads, 0, st>>>(cv, ci, m, k, ov, oi);
    else topk_merge_kernel<kTopkMergePer><<<groups, kTopkMergeThreads, 0, st>>>(cv, ci, m, k, ov, oi);
    RLQ_HIP(hipGetLastError());
    if (groups == 1) break;
    m = groups * k;
    std::swap(cv, tv);
    std::swap(ci, ti);
  }
  std::vector<float> v(k);
  std::vector<int> i(k);
  RLQ_HIP(hipMemcpyAsync(v.data(), e->topk_out_v.p, (size_t)k * 4, hipMemcpyDeviceToHost, st));
  RLQ_HIP(hipMemcpyAsync(i.data(), e->topk_out_i.p, (size_t)k * 4, hipMemcpyDeviceToHost, st));
  RLQ_HIP(hipStreamSynchronize(st));
  int got = 0;
  for (int r = 0; r < k && i[r] >= 0; ++r, ++got) {
    ids[r] = i[r];
    vals[r] = v[r];
  }
  return got;
}

// One token of a mixture of experts: post-attention norm and router product in one launch
// (norm_router_kernel), the normed row left in e->xn and the logits in e->router_logits, as
// rl_norm and rl_linear leave them. Returns 1 (nothing launched) when the router is not a
// dense f16b matrix or its shape is outside the kernel's (fewer than 4 waves, more than 8
// K steps per wave, rows past the norm's register form).
static int norm_router_one_token(rl_engine *e, int layer, const float *h, hipStream_t st) {
  const ModelConfig &c = e->model->config();
  const EngineTensor *router = tensor_of(e, lname(layer, "moe.router"));
  const float *w = norm_weight(e, 1, layer);
  if (!router || !w || router->q->kind != kKindF16b || router->q->k != c.hidden || c.hidden % kDenseStep) return 1;
  const int H = c.hidden, steps = H / kDenseStep;
  // dense_f16_kernel's split of the K steps over the waves (rlq_linear_f16)
  const int waves = std::min(16, (steps + 7) / 8);
  const int spw = ((steps + waves - 1) / waves + 7) / 8 * 8;
  const int per = (H + kNormThreads - 1) / kNormThreads;
  if (waves < kNormThreads / 64 || spw > 8 || per > kNormMaxPer) return 1;
  RLQ_REQUIRE(router->q->n >= c.experts + 1 && router->q->n_pad == e->router_stride,
              "layer %d: router is %d x %d, needs %d x %d", layer, router->q->n, router->q->k, c.experts + 1, H);
  const size_t lds = 16 + ((size_t)H * 2 + 15) / 16 * 16 + (size_t)(waves - 1) * 64 * 16;
  auto launch = [&](auto kernel) {
    kernel<<<tiles_of(router->q->n), 64 * waves, lds, st>>>(h, w, H, c.norm_eps, e->xn.as<_Float16>(),
                                                            router->packed.as<u32x4>(), router->q->n, spw,
                                                            e->router_logits.as<float>());
  };
  if (per <= 8) launch(norm_router_kernel<8>);
  else if (per <= 16) launch(norm_router_kernel<16>);
  else if (per <= 20) launch(norm_router_kernel<20>);
  else launch(norm_router_kernel<kNormMaxPer>);
  RLQ_HIP(hipGetLastError());
  return 0;
}

// The experts of a mixture-of-experts layer once the normed rows (e->xn) and the router
// logits are in place: routing, gate/up, SwiGLU, down and the combine into h.
static int moe_experts(rl_engine *e, int layer, float *h, int h_stride, int T, hipStream_t st) {
  const ModelConfig &c = e->model->config();
  _Float16 *xn = e->xn.as<_Float16>();
  const EngineTensor *router = tensor_of(e, lname(layer, "moe.router"));
  const EngineTensor *gu = tensor_of(e, lname(layer, "moe.gate_up"));
  const EngineTensor *dn = tensor_of(e, lname(layer, "moe.down"));
  RLQ_REQUIRE(router && gu && dn, "layer %d: the mixture of experts needs moe.router, moe.gate_up and moe.down", layer);
  const int E = c.experts, E1 = E + 1, H = c.hidden, I = c.moe_inter;
  RLQ_REQUIRE(router->q->n >= E1 && router->q->k == H && router->q->n_pad == e->router_stride,
              "layer %d: router is %d x %d, needs %d x %d", layer, router->q->n, router->q->k, E1, H);
  RLQ_REQUIRE(gu->q->n == E1 * 2 * I && gu->q->k == H && dn->q->n == E1 * H && dn->q->k == I,
              "layer %d: expert stacks do not match %d experts of %d x %d", layer, E1, I, H);
  RLQ_REQUIRE(gu->q->native == dn->q->native, "layer %d: gate/up and down stacks of different formats", layer);
  const float *logits = e->router_logits.as<float>();
  if (!gu->q->native)
    return rlq_moe(xn, e->x_stride, logits, e->router_stride, T, E, c.experts_per_tok, c.norm_topk ? 1 : 0, H, I,
                   gu->packed.p, dn->packed.p, RLQ_BF16, h, h_stride, e->moe_ws.p, e->moe_ws.bytes, st);
  const std::string &bk = gu->q->book.empty() ? c.book : gu->q->book;
  return rlq_moe_native(xn, e->x_stride, logits, e->router_stride, T, E, c.experts_per_tok, c.norm_topk ? 1 : 0, H, I,
                        gu->packed.p, gu->srow.as<float>(), dn->packed.p, dn->srow.as<float>(), e->slots.as<int>(), E1,
                        bk == "fp4" ? RLQ_BOOK_FP4 : RLQ_BOOK_INT15, dn->col.as<float>(), h, h_stride, e->moe_ws.p,
                        e->moe_ws.bytes, st);
}

}  // namespace rlq

using namespace rlq;

extern "C" {

rl_engine *rl_open(const char *model_path, int max_ctx, int max_chunk) {
  std::unique_ptr<rl_engine> e(new rl_engine());
  if (open_engine(e.get(), model_path, max_ctx, max_chunk)) return nullptr;
  return e.release();
}

void rl_close(rl_engine *e) { delete e; }

int rl_vocab(const rl_engine *e) { return e ? e->model->config().vocab : 0; }
int rl_hidden_size(const rl_engine *e) { return e ? e->model->config().hidden : 0; }

int rl_linear(rl_engine *e, const char *tensor, const char *part, const void *x, int x_stride, int rows, float *out,
              int out_stride, int accum, void *stream) {
  RLQ_REQUIRE(e && tensor, "rl_linear: null engine or tensor name");
  const EngineTensor *t = tensor_of(e, tensor);
  RLQ_REQUIRE(t, "model has no quantized tensor '%s'", tensor);
  RLQ_REQUIRE(!t->moe_gate_up, "rl_linear: '%s' is an expert stack (rl_mlp runs it)", tensor);
  int r0 = 0, n = t->q->n;
  if (part) {
    const std::pair<int, int> *p = t->q->part(part);
    RLQ_REQUIRE(p, "quantized tensor has no part '%s'", part);
    r0 = p->first;
    n = p->second;
    RLQ_REQUIRE(r0 % 16 == 0, "rl_linear: part '%s' of '%s' starts at row %d, not a multiple of 16", part, tensor, r0);
  }
  return linear_rows(e, *t, r0, n, static_cast<const _Float16 *>(x), x_stride, rows, out, out_stride, accum,
                     static_cast<hipStream_t>(stream));
}

int rl_norm(rl_engine *e, int which, int layer, const float *h, int h_stride, int rows, void *xn, int xn_stride,
            void *stream) {
  RLQ_REQUIRE(e, "rl_norm: null engine");
  return norm_rows(e, which, layer, h, h_stride, rows, static_cast<_Float16 *>(xn), xn_stride,
                   static_cast<hipStream_t>(stream));
}

int rl_mlp(rl_engine *e, int layer, float *h, int h_stride, int T, void *stream) {
  RLQ_REQUIRE(e, "rl_mlp: null engine");
  const ModelConfig &c = e->model->config();
  RLQ_REQUIRE(layer >= 0 && layer < c.layers, "rl_mlp: layer %d of %d", layer, c.layers);
  RLQ_REQUIRE(h && T >= 1 && T <= e->max_chunk && h_stride >= c.hidden, "rl_mlp: T=%d (max_chunk %d) or bad h", T,
              e->max_chunk);
  auto st = static_cast<hipStream_t>(stream);
  _Float16 *xn = e->xn.as<_Float16>();
  if (c.is_moe() && T == 1) {
    // one token of a mixture of experts: the norm and the router product in one launch
    // (norm_router_kernel: the bits of the two steps)
    const int fused = norm_router_one_token(e, layer, h, st);
    if (fused < 0) return fused;
    if (fused == 0) return moe_experts(e, layer, h, h_stride, T, st);
  }
  if (int rc = norm_rows(e, 1, layer, h, h_stride, T, xn, e->x_stride, st)) return rc;
  if (!c.is_moe()) {
    // encode_mlp (src/engine.mm:943-958): gate_up, SwiGLU with down's column scale, down + h
    const EngineTensor *gu = tensor_of(e, lname(layer, "mlp.gate_up"));
    const EngineTensor *dn = tensor_of(e, lname(layer, "mlp.down"));
    RLQ_REQUIRE(gu && dn, "model has no quantized tensor '%s'", lname(layer, gu ? "mlp.down" : "mlp.gate_up").c_str());
    const int I = c.intermediate;
    const std::pair<int, int> *pg = gu->q->part("gate"), *pu = gu->q->part("up");
    RLQ_REQUIRE(pg && pu && pg->first == 0 && pg->second == I && pu->first == I && pu->second == I,
                "%s: parts gate and up must be rows [0, %d) and [%d, %d)", lname(layer, "mlp.gate_up").c_str(), I, I,
                2 * I);
    RLQ_REQUIRE(dn->q->k == I && dn->q->n == c.hidden && gu->q->k == c.hidden, "layer %d: MLP shapes do not match",
                layer);
    const float *cs = dn->q->native ? dn->col.as<float>() : nullptr;
    // decode sizes of an affine gate/up: the SwiGLU fused into the gate/up launch (the same
    // bits as the two steps below)
    int fused = 1;
    if (gu->q->kind == kKindQ4a && !cs && T <= 8) {
      const char *codes = gu->packed.as<char>();
      fused = linear_swiglu_packed(xn, e->x_stride, T, gu->q->k, I, codes,
                                   codes + packed_code_bytes(gu->q->k, gu->q->n_pad), RLQ_BF16,
                                   e->act.as<_Float16>(), e->act_stride, st);
      if (fused < 0) return fused;
    }
    if (fused) {
      float *proj = e->proj.as<float>();
      if (int rc = linear_rows(e, *gu, 0, 2 * I, xn, e->x_stride, T, proj, e->proj_stride, 0, st)) return rc;
      if (int rc = rlq_moe_swiglu(proj, e->proj_stride, T, I, cs, e->act.p, e->act_stride, st)) return rc;
    }
    return linear_rows(e, *dn, 0, c.hidden, e->act.as<_Float16>(), e->act_stride, T, h, h_stride, 1, st);
  }
  // encode_moe (src/engine.mm:965-1059)
  const EngineTensor *router = tensor_of(e, lname(layer, "moe.router"));
  RLQ_REQUIRE(router, "layer %d: the mixture of experts needs moe.router", layer);
  RLQ_REQUIRE(router->q->n >= c.experts + 1 && router->q->k == c.hidden && router->q->n_pad == e->router_stride,
              "layer %d: router is %d x %d, needs %d x %d", layer, router->q->n, router->q->k, c.experts + 1,
              c.hidden);
  float *logits = e->router_logits.as<float>();
  if (int rc = linear_rows(e, *router, 0, router->q->n, xn, e->x_stride, T, logits, e->router_stride, 0, st)) return rc;
  return moe_experts(e, layer, h, h_stride, T, st);
}

const float *rl_head(rl_engine *e, const float *h, int h_stride, int rows, void *stream) {
  if (!e) {
    fail("rl_head: null engine");
    return nullptr;
  }
  const EngineTensor *head = tensor_of(e, "lm_head");
  if (!head) {
    fail("model has no quantized tensor 'lm_head'");
    return nullptr;
  }
  if (rows < 1 || rows > 16 || rows > e->max_chunk) {
    fail("rl_head: %d rows (1..16, <= max_chunk)", rows);
    return nullptr;
  }
  auto st = static_cast<hipStream_t>(stream);
  _Float16 *xn = e->xn.as<_Float16>();
  if (norm_rows(e, 2, 0, h, h_stride, rows, xn, e->x_stride, st)) return nullptr;
  const int np = head->q->n_pad;
  if (linear_rows(e, *head, 0, np, xn, e->x_stride, rows, e->logits.as<float>(), np, 0, st)) return nullptr;
  e->head_rows_done = rows;
  e->head_stream = st;
  return e->logits.as<float>();
}

void rl_set_draft_vocab(rl_engine *e, int rows) {
  if (e) e->draft_vocab_rows = rows <= 0 ? 0 : (rows + 255) / 256 * 256;
}

void rl_set_draft_tail(rl_engine *e, int first) {
  if (e) e->draft_tail_first = first < 0 ? -1 : first / 256 * 256;
}

int rl_draft_main(const rl_engine *e) {
  const QTensor *head = e ? e->model->q("lm_head") : nullptr;
  if (!head) return 0;
  return e->draft_vocab_rows > 0 ? std::min(e->draft_vocab_rows, head->n_pad) : head->n_pad;
}

int rl_draft_tail(const rl_engine *e) {
  const QTensor *head = e ? e->model->q("lm_head") : nullptr;
  if (!head) return -1;
  const int t = e->draft_tail_first;
  // as src/engine.mm:1449-1453: only past the main rows, inside the matrix, for native heads
  if (t < 0 || t <= rl_draft_main(e) || t >= head->n_pad || !head->native) return -1;
  return t;
}

int rl_draft_vocab(const rl_engine *e) {
  const QTensor *head = e ? e->model->q("lm_head") : nullptr;
  if (!head) return 0;
  const int tail = rl_draft_tail(e);
  return rl_draft_main(e) + (tail < 0 ? 0 : head->n_pad - tail);
}

// Every expert of a mixture of experts stays resident in HBM (288 GB holds the largest
// MoE file whole), so there is no expert cache: as src/engine.mm:364-365 reports for an
// engine without one, no slots, no hits or loads, and a size of zero.
int rl_expert_cache(const rl_engine *e, unsigned long long *hits, unsigned long long *loads) {
  (void)e;
  if (hits) *hits = 0;
  if (loads) *loads = 0;
  return 0;
}

void rl_expert_cache_size(const rl_engine *e, int *experts, unsigned long long *slot_bytes) {
  (void)e;
  if (experts) *experts = 0;
  if (slot_bytes) *slot_bytes = 0;
}

size_t rl_logits_stride(const rl_engine *e) {
  const QTensor *head = e ? e->model->q("lm_head") : nullptr;
  return head ? (size_t)head->n_pad : 0;
}

const float *rl_draft_head(rl_engine *e, const float *h_row, void *stream) {
  if (!e) {
    fail("rl_draft_head: null engine");
    return nullptr;
  }
  const EngineTensor *head = tensor_of(e, "lm_head");
  if (!head) {
    fail("model has no quantized tensor 'lm_head'");
    return nullptr;
  }
  auto st = static_cast<hipStream_t>(stream);
  _Float16 *xn = e->xn.as<_Float16>();
  const ModelConfig &c = e->model->config();
  if (e->has_mtp) {
    // a file with an MTP head: the draft row is normed with mtp.norm (src/engine.mm:1419-1424);
    // a rotated file would rotate it instead, with a kernel that is not on this path
    if (c.rot_block) {
      fail("rl_draft_head: a rotated model file (rot_block %d) needs the rotation kernel, not built here", c.rot_block);
      return nullptr;
    }
    if (norm_with(e, e->norm_mtp_out.as<float>(), h_row, c.hidden, 1, xn, e->x_stride, st)) return nullptr;
  } else if (norm_rows(e, 2, 0, h_row, c.hidden, 1, xn, e->x_stride, st)) {
    return nullptr;
  }
  const int main_rows = rl_draft_main(e), tail = rl_draft_tail(e), np = head->q->n_pad;
  float *out = e->draft_logits.as<float>();
  if (linear_rows(e, *head, 0, main_rows, xn, e->x_stride, 1, out, np, 0, st)) return nullptr;
  if (tail >= 0 && linear_rows(e, *head, tail, np - tail, xn, e->x_stride, 1, out + main_rows, np, 0, st))
    return nullptr;
  return out;
}

int rl_top_k(const float *logits, int n, int k, int32_t *ids, float *vals) {
  k = std::min(k, n);
  if (k <= 0 || !logits || !ids || !vals) return 0;
  // the entries that are not NaN, in descending order of value, equal values by index
  std::vector<int32_t> idx;
  idx.reserve((size_t)n);
  for (int i = 0; i < n; ++i)
    if (!std::isnan(logits[i])) idx.push_back(i);
  const int m = std::min<int>(k, (int)idx.size());
  std::partial_sort(idx.begin(), idx.begin() + m, idx.end(), [&](int32_t a, int32_t b) {
    return logits[a] > logits[b] || (logits[a] == logits[b] && a < b);
  });
  for (int r = 0; r < m; ++r) {
    ids[r] = idx[r];
    vals[r] = logits[idx[r]];
  }
  return m;
}

int rl_top_k_device(rl_engine *e, const float *logits, int n, int k, int32_t *ids, float *vals, void *stream) {
  RLQ_REQUIRE(e, "rl_top_k_device: null engine");
  return top_k_device(e, logits, n, k, ids, vals, static_cast<hipStream_t>(stream));
}

int rl_argmax(const rl_engine *e) {
  if (!e || e->head_rows_done < 1) return 0;
  int32_t id = 0;
  float v;
  rl_engine *m = const_cast<rl_engine *>(e);   // the device top-k uses the engine's scratch
  // on the stream of the rl_head that wrote the logits, so it runs after the head's kernels
  const int got = top_k_device(m, m->logits.as<float>(), e->model->config().vocab, 1, &id, &v, e->head_stream);
  return got == 1 ? id : 0;
}

}  // extern "C"
