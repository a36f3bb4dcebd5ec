// Mixture-of-experts MLP on gfx950: routing, the grouped expert matmuls over 4-bit affine
// expert stacks, SwiGLU and the combine, following kernels/moe.metal and
// src/engine.mm:965-1059 of the reference.
//
// A token goes to `topk` of E routed experts (falling logit, equal logits: the lower
// expert first) plus the shared expert, number E; S = topk + 1 assignments per token,
// assignment a = t * S + slot. The routing sorts the assignments by expert into "rows";
// each expert's rows are consecutive, and an expert's rows are cut into work items of at
// most 16 rows (the MFMA tile height). The grouped matmuls run over the expert's matrices
// in the stacked tensors: below 8 tokens one small workgroup per (item, 16-row weight
// tile) (moe_expert_kernel), from 8 tokens one workgroup per (item, block of tiles) with
// the item's rows staged once in LDS (moe_expert_lds_kernel); both give the same bits.
// The combine adds each token's S results to its residual row in slot order. For one
// token, rlq_moe routes inside the gate/up launch; up to four tokens, it runs the down
// projection and the combine as one launch (the same bits as the separate steps).
//
// Differences from the reference, all of them MI355X choices:
//  - rows within an expert are placed in token order (the reference places them with
//    atomics in no particular order, moe.metal:133-139); nothing depends on it, but the
//    order is now reproducible run to run;
//  - the gather of the routed rows is fused into the gate/up kernel (it reads x through
//    the row -> token map), and SwiGLU into its epilogue (the gate/up stack is packed so
//    one 16-row tile holds 8 gate rows and the matching 8 up rows);
//  - there is no indirect dispatch: grids are sized for the most items a call can have,
//    and workgroups past the item count the routing wrote exit at once.
// A row's result depends only on its own token (MFMA rows are independent), so the
// layer's output for a token does not depend on the other tokens of the call.
#include "q4_tile.h"
#include "../../include/rlq.h"

#include <algorithm>
#include <mutex>
#include <cmath>

namespace rlq {

constexpr int kItemRows = 16;     // rows per work item: the MFMA tile height
constexpr int kMaxTopk = 16;
constexpr int kMaxExperts = 1023; // E; E + 1 <= 1024 (one thread per expert in the sort)
constexpr int kRouteSmallTokens = 16;   // up to this many tokens route in one launch (a wave each)
constexpr size_t kSortSmallLds = (2 * 1024 + 32) * 4;
constexpr int kDownCombineTokens = 4;   // up to this many tokens, rlq_moe runs down + combine as one launch

// Most work items a call can have: sum over experts of ceil(rows_e / 16) <= A / 16 + the
// number of experts with rows, which is at most min(E + 1, A).
static inline int moe_max_items(int T, int E, int topk) {
  const long long A = (long long)T * (topk + 1);
  return (int)(A / kItemRows + std::min<long long>(E + 1, A));
}

// ------------------------------------------------------------------ routing: top-k

// Wave-wide max and sum, every lane getting the result: rows of 16 lanes combine through
// DPP lane swizzles (quad [1,0,3,2], quad [2,3,0,1], half-row mirror, row mirror), then the
// four row results are read as scalars and combined in row order.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_lane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return fmaxf(fmaxf(row_lane(v, 0), row_lane(v, 16)), fmaxf(row_lane(v, 32), row_lane(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return (row_lane(v, 0) + row_lane(v, 16)) + (row_lane(v, 32) + row_lane(v, 48));
}

__device__ __forceinline__ int wave_min_i(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// One wave per token. Lane l holds logits l, l + 64, ...; repeated wave-wide argmax with
// ties to the lower expert (kernels/moe.metal:75-91). Weights: exp(l - max) over the
// softmax denominator of all E logits, or over the chosen ones when norm_topk
// (moe.metal:92-102); the shared slot gets sigmoid(logit[E]) (moe.metal:103-104).
// Each lane first orders its EPL logits, highest first (equal ones by expert); a round
// then takes the wave max of the lanes' first untaken logits, and the expert is the lowest
// one among the lanes holding it: the only such lane's (one ballot bit, the usual case), or
// a wave min of expert numbers. That lane drops its first entry. Entries past E and NaN
// logits are -inf; an expert < E always wins a tie with them (topk <= E). Lane r keeps
// round r's pick and logit; the exponentials are taken afterwards, one per lane, and
// summed in round order.
template <int EPL>
__device__ void topk_token(const float *row, int E, int topk, int norm_topk, int *sel_t, float *w_t, int lane) {
  const float shared_logit = row[E];
  float v[EPL];
  int ev[EPL];
  float lm = -INFINITY;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    const float l = e < E ? row[e] : -INFINITY;
    v[j] = l == l ? l : -INFINITY;            // a NaN logit ranks last
    ev[j] = e;
    lm = fmaxf(lm, v[j]);
  }
  asm volatile("" ::"s"(shared_logit));   // read beside the others, not after the rounds
  const float m = wave_max(lm);
  float z = 0.0f;
  if (!norm_topk) {
    float lz = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) lz += (lane + 64 * j < E) ? expf(v[j] - m) : 0.0f;
    z = wave_sum(lz);
  }
  // highest first; a strictly higher logit moves ahead, so equal ones stay in expert order
#pragma unroll
  for (int i = 1; i < EPL; ++i)
#pragma unroll
    for (int j = i; j > 0; --j)
      if (v[j] > v[j - 1]) {
        const float tv = v[j];
        v[j] = v[j - 1];
        v[j - 1] = tv;
        const int te = ev[j];
        ev[j] = ev[j - 1];
        ev[j - 1] = te;
      }

  int my_which = 0;
  float my_top = 0.0f;
  for (int r = 0; r < topk; ++r) {
    const float top = wave_max(v[0]);
    const uint64_t b = __ballot(v[0] == top);
    int be;
    if (__popcll(b) == 1) {
      be = __builtin_amdgcn_readlane(ev[0], (int)__builtin_ctzll(b));
    } else {
      be = wave_min_i(v[0] == top ? ev[0] : INT_MAX);
    }
    if (lane == (be & 63) && ev[0] == be) {
#pragma unroll
      for (int j = 0; j + 1 < EPL; ++j) {
        v[j] = v[j + 1];
        ev[j] = ev[j + 1];
      }
      v[EPL - 1] = -INFINITY;
      ev[EPL - 1] = INT_MAX;
    }
    if (lane == r) {
      my_which = be;
      my_top = top;
    }
  }
  const float ex = lane < topk ? expf(my_top - m) : 0.0f;
  float denom = z;
  if (norm_topk) {
    denom = 0.0f;
    for (int r = 0; r < topk; ++r) denom += row_lane(ex, r);
  }
  if (lane < topk) {
    sel_t[lane] = my_which;
    w_t[lane] = ex / denom;
  }
  if (lane == 0) {
    sel_t[topk] = E;
    w_t[topk] = 1.0f / (1.0f + expf(-shared_logit));
  }
}

template <int EPL>
__global__ __launch_bounds__(256) void moe_topk_kernel(const float *logits, int stride, int T, int E, int topk,
                                                       int norm_topk, int *sel, float *w) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const size_t a0 = (size_t)t * (topk + 1);
  topk_token<EPL>(logits + (size_t)t * stride, E, topk, norm_topk, sel + a0, w + a0, threadIdx.x & 63);
}

// ------------------------------------------------------------------ routing: sort

// Inclusive prefix sum over the wave: within rows of 16 lanes by DPP row shifts (1, 2, 4,
// 8; lanes shifted in from outside the row read 0), then each row adds the totals of the
// rows before it, read as scalars.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);   // row_shr:8
  const int t0 = __builtin_amdgcn_readlane(v, 15), t1 = __builtin_amdgcn_readlane(v, 31),
            t2 = __builtin_amdgcn_readlane(v, 47);
  const int row = (threadIdx.x & 63) >> 4;
  return v + (row >= 1 ? t0 : 0) + (row >= 2 ? t1 : 0) + (row >= 3 ? t2 : 0);
}

// Exclusive prefix sum over the workgroup (at most 16 waves) of one int per thread; *total
// gets the sum. wave_tot: 16 ints of LDS.
__device__ int block_exclusive_scan(int v, int *wave_tot, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int inc = wave_inclusive_scan(v);
  if (lane == 63) wave_tot[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    const int nw = blockDim.x >> 6;
    const int t = lane < nw ? wave_tot[lane] : 0;
    const int ti = wave_inclusive_scan(t);
    if (lane < nw) wave_tot[lane] = ti - t;
    if (lane == nw - 1) *total = ti;
  }
  __syncthreads();
  const int ex = wave_tot[wave] + inc - v;
  __syncthreads();   // wave_tot may be reused by the caller's next scan
  return ex;
}

// A workgroup barrier that orders LDS accesses only: __syncthreads also waits for every
// global store in flight (its release fence), which the sort's later phases never read back
// (the work items, rows and slots are for the next kernels); that wait took about 1 us at
// each such barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);             // lgkmcnt(0): this thread's LDS accesses are done
  asm volatile("s_barrier" ::: "memory");
}

// One workgroup of 1024 threads sorts all T*S assignments by expert (a counting sort,
// moe.metal:109-139) and writes the work list. Within an expert, rows follow token order:
// token t's row for expert e is off[e] + (tokens before t that chose e). The tokens go in
// rounds of 64 per wave (wpr waves): lane i of wave w holds token 64 w + i of the round and
// sets bit i of its wave's 64-bit mask of each expert it chose, so within the wave a token's
// rank is a popcount of the lower lanes' bits and the wave's count for the expert the
// popcount of the mask (a token chooses an expert at most once). Pass 1 adds every wave's
// counts into the experts' totals, a scan gives the row offsets and the work items; pass 2
// turns each round's per-wave counts into per-wave row bases (expert by expert, in wave
// order) and places every assignment. With one round (T <= 64 wpr) pass 2 reuses pass 1's
// masks and each lane keeps its token's experts in registers.
// LDS: off[1024], scan scratch[32], cnt[wpr][E+1] ints, then mask[wpr][E+1] 64-bit words.
__device__ void sort_assignments(const int *sel, int T, int E, int S, int wpr, int *tok, int *inv, int4 *items,
                                 int *n_items, unsigned char *lds) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E1 = E + 1;
  int *off = reinterpret_cast<int *>(lds);      // [1024]: totals, then row offsets / running bases
  int *scratch = off + 1024;                    // [32]
  int *cnt = scratch + 32;                      // [wpr][E1]
  uint64_t *mask = reinterpret_cast<uint64_t *>(lds + ((size_t)(1056 + wpr * E1) * 4 + 7) / 8 * 8);   // [wpr][E1]
  const int per_round = 64 * wpr, rounds = (T + per_round - 1) / per_round;
  const bool in_round = wave < wpr;
  uint64_t *my_mask = mask + (size_t)wave * E1;
  int *my_cnt = cnt + (size_t)wave * E1;
  int ev[kMaxTopk + 1];                         // this lane's token's experts (sel is clamped into 0..E)

  // the masks of round r for this wave: zeroed, then every chosen expert's bit of each lane
  auto build = [&](int r) {
    for (int e = lane; e < E1; e += 64) my_mask[e] = 0ull;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int t = r * per_round + 64 * wave + lane;
#pragma unroll
    for (int k = 0; k <= kMaxTopk; ++k) {
      if (k >= S) break;                        // uniform
      ev[k] = t < T ? min(max(sel[(size_t)t * S + k], 0), E) : 0;
      if (t < T) atomicOr(reinterpret_cast<unsigned long long *>(my_mask + ev[k]), 1ull << lane);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // pass 1: the experts' totals
  off[tid] = 0;
  lds_barrier();
  for (int r = 0; r < rounds; ++r) {
    if (in_round) {
      build(r);
      for (int e = lane; e < E1; e += 64) {
        const int c = __popcll(my_mask[e]);
        my_cnt[e] = c;
        if (c) atomicAdd(&off[e], c);
      }
    }
  }
  lds_barrier();
  const int c = tid < E1 ? off[tid] : 0;
  const int ni = (c + kItemRows - 1) / kItemRows;
  int o, io, n_it;
  if ((long long)T * S < (1 << 15)) {   // uniform: counts and item counts fit one scan, 16 bits each
    const int packed = block_exclusive_scan(c | (ni << 16), scratch, scratch + 16);
    o = packed & 0xFFFF;
    io = packed >> 16;
    n_it = scratch[16] >> 16;
  } else {
    o = block_exclusive_scan(c, scratch, scratch + 16);
    io = block_exclusive_scan(ni, scratch, scratch + 17);
    n_it = scratch[17];
  }
  if (tid < E1) {
    off[tid] = o;
    for (int i = 0; i < ni; ++i)
      items[io + i] = int4{tid, o + i * kItemRows, min(kItemRows, c - i * kItemRows), 0};
  }
  if (tid == 0) *n_items = n_it;
  lds_barrier();

  // pass 2: each round's per-wave row bases, then the rows
  for (int r = 0; r < rounds; ++r) {
    if (rounds > 1) {                           // uniform: one round keeps pass 1's masks and counts
      if (in_round) {
        build(r);
        for (int e = lane; e < E1; e += 64) my_cnt[e] = __popcll(my_mask[e]);
      }
      lds_barrier();
    }
    if (tid < E1) {
      // every wave's count is read before the first base is written (one LDS round trip)
      int cw[16];
#pragma unroll
      for (int w = 0; w < 16; ++w) cw[w] = w < wpr ? cnt[(size_t)w * E1 + tid] : 0;
      int run = off[tid];
#pragma unroll
      for (int w = 0; w < 16; ++w) {
        if (w < wpr) cnt[(size_t)w * E1 + tid] = run;
        run += cw[w];
      }
      off[tid] = run;                           // the next round continues the expert's rows
    }
    lds_barrier();
    const int t = r * per_round + 64 * wave + lane;
    if (in_round && t < T) {
      const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
      for (int k = 0; k <= kMaxTopk; ++k) {
        if (k >= S) break;                      // uniform
        const int e = ev[k];
        const int pos = my_cnt[e] + __popcll(my_mask[e] & below);
        inv[(size_t)t * S + k] = pos;
        tok[pos] = t;
      }
    }
    if (r + 1 < rounds) lds_barrier();        // uniform: the next round rebuilds masks and counts
  }
}

__global__ __launch_bounds__(1024) void moe_sort_kernel(const int *sel, int T, int E, int S, int wpr, int *tok,
                                                        int *inv, int4 *items, int *n_items) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  sort_assignments(sel, T, E, S, wpr, tok, inv, items, n_items, lds);
}

// The sort for a few assignments (A <= 1024, one thread each): an assignment's row within its
// expert is the number of earlier assignments to the same expert (a token picks an expert
// at most once, so this is token order, as sort_assignments places them); an expert's count
// is a loop over the assignments. One scan gives both the row offsets and the work items
// (count in the low, item count in the high 16 bits: A <= 1024 keeps both sums in range).
// LDS: sel [1024] ints, offsets [1024], scan scratch [32].
__device__ void sort_small(const int *sel, int T, int E, int S, int *tok, int *inv, int4 *items, int *n_items,
                           unsigned char *lds) {
  int *sl = reinterpret_cast<int *>(lds);       // [1024]
  int *off = sl + 1024;                         // [1024]
  int *scratch = off + 1024;                    // [32]
  const int tid = threadIdx.x;
  const int A = T * S, E1 = E + 1;
  const int ea = tid < A ? min(max(sel[tid], 0), E) : -1;
  sl[tid] = ea;
  __syncthreads();
  int c = 0;
  if (tid < E1)
    for (int b = 0; b < A; ++b) c += sl[b] == tid;
  int rank = 0;
  for (int b = 0; b < min(tid, A); ++b) rank += sl[b] == ea;
  const int ni = (c + kItemRows - 1) / kItemRows;
  const int packed = block_exclusive_scan(c | (ni << 16), scratch, scratch + 16);
  const int o = packed & 0xFFFF, io = packed >> 16;
  if (tid < E1) {
    off[tid] = o;
    for (int i = 0; i < ni; ++i) items[io + i] = int4{tid, o + i * kItemRows, min(kItemRows, c - i * kItemRows), 0};
  }
  if (tid == 0) *n_items = scratch[16] >> 16;
  __syncthreads();
  if (tid < A) {
    const int pos = off[ea] + rank;
    inv[tid] = pos;
    tok[pos] = tid / S;
  }
}

// Routing of up to 16 tokens in one launch: wave t picks token t's experts, then the whole
// workgroup sorts them (sort_small: the same rows and items as moe_sort_kernel). sel and w
// are written to memory and read back after the barrier, which makes them visible to the
// workgroup.
template <int EPL>
__global__ __launch_bounds__(1024) void moe_route_small_kernel(const float *logits, int stride, int T, int E, int topk,
                                                               int norm_topk, int *sel, float *w, int *tok, int *inv,
                                                               int4 *items, int *n_items) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int t = threadIdx.x >> 6;
  const size_t a0 = (size_t)t * (topk + 1);
  if (t < T) topk_token<EPL>(logits + (size_t)t * stride, E, topk, norm_topk, sel + a0, w + a0, threadIdx.x & 63);
  __syncthreads();
  sort_small(sel, T, E, topk + 1, tok, inv, items, n_items, lds);
}

// ------------------------------------------------------------------ grouped expert matmuls

struct MoeArgs {
  const _Float16 *x;        // gate_up: the token rows [T][x_stride]; down: act [A][x_stride]
  const int *tok;           // gate_up: row -> token (the fused gather); down: unused
  const u32x4 *codes;
  const u32x4 *sb;
  const int4 *items;
  const int *n_items;
  void *out;                // gate_up: act fp16 [A][out_stride]; down: y fp32 [A][out_stride]
  int x_rows, x_stride, K, tiles_per_expert, out_stride;
  int tiles_per_block, waves_per_tile;   // the staged kernel's workgroup shape
  const float *s_row;       // native books: row scales of the slots; slots[e]: expert e's slot
  const int *slots;
  int n_slots;
  int n_experts;            // experts a work item may name (E + 1)
  int n_rows;               // sorted rows of the call (T * S): the row -> token map and the outputs
};

// A work item as read from the list, clamped into the call's tables. The list is written
// on the device; a corrupt entry then gives bounded wrong rows instead of an access outside
// the weight stack, the row -> token map or the outputs.
__device__ __forceinline__ int4 clamp_item(int4 it, int n_experts, int n_rows) {
  it.x = min(max(it.x, 0), n_experts - 1);
  it.y = min(max(it.y, 0), n_rows - 1);
  it.z = min(max(it.z, 0), min(16, n_rows - it.y));
  return it;
}

// The token of sorted row r, clamped to the call's tokens (see clamp_item).
__device__ __forceinline__ int token_of(const int *tok, int r, int T) { return min(max(tok[r], 0), T - 1); }


// One item's products for one 16-row weight tile (tile = blockIdx.x) by all the workgroup's
// waves, each a range of GPW groups of K; the waves meet in LDS in wave order and wave 0
// writes. KIND 0: gate/up with the gather and SwiGLU fused (interleaved stack); the rows'
// tokens come from the row -> token map, or (ONE_TOKEN) are all token 0. KIND 1: down.
// ONE_TOKEN forms accumulator row 0 only; with PRE it takes the token's group sums from gs
// (all groups of K, formed by row0_group_sums).
template <int GPW, int SD, int KIND, bool ONE_TOKEN, bool PRE = false>
__device__ __forceinline__ void expert_tile(const MoeArgs &a, int e, int r0, int rows, unsigned char *lds,
                                            const float *gs = nullptr) {
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, j4 = lane >> 4;
  const int G = a.K / kGroup, G4 = quads_of(a.K);
  const int tile = blockIdx.x;
  const int t = e * a.tiles_per_expert + tile;
  const int wg0 = wave * GPW;
  const int wn = max(0, min(G, wg0 + GPW) - wg0);
  const WaveTile wt = wave_tile(a.codes, a.sb, t, G4, wg0, GPW);

  const bool live = c16 < rows;
  int xrow = r0 + (live ? c16 : 0);
  if constexpr (KIND == 0) xrow = ONE_TOKEN ? 0 : token_of(a.tok, xrow, a.x_rows);
  const uint32_t xrange = wn > 0 ? (uint32_t)((a.x_rows - 1) * a.x_stride + wn * kGroup) * 2u : 0u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (size_t)min(wg0, G) * kGroup, xrange);
  f32x4 acc = tile_dot_rows<GPW, SD, kAffine, ONE_TOKEN ? 1 : 4, PRE>(
      wt, rx, (uint32_t)xrow * a.x_stride * 2u + 16u * j4, live, wn, lane, PRE ? gs + min(wg0, G) : nullptr);
  acc = reduce_waves(acc, reinterpret_cast<f32x4 *>(lds), wave, waves, lane);
  if (wave != 0) return;
  if constexpr (KIND == 0) {
    // lanes c16 < 8 hold gate features 8 tile + c16, lanes c16 + 8 the matching up ones
    _Float16 *act = static_cast<_Float16 *>(a.out);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float u = __shfl_xor(acc[v], 8);
      const int r = 4 * j4 + v;
      if (c16 < 8 && r < rows)
        act[(size_t)(r0 + r) * a.out_stride + 8 * tile + c16] = static_cast<_Float16>(silu(acc[v]) * u);
    }
  } else {
    float *y = static_cast<float *>(a.out);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * j4 + v;
      if (r < rows) y[(size_t)(r0 + r) * a.out_stride + 16 * tile + c16] = acc[v];
    }
  }
}

// grid (tiles_per_expert, max_items); block 64 * ceil(4 G4 / GPW).
template <int GPW, int SD, int KIND>
__global__ __launch_bounds__(1024) void moe_expert_kernel(MoeArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int item = blockIdx.y;
  // the item entry is read together with the count (the list holds the most items a call
  // can have, so the read is in bounds; entries past the count are not used)
  const int4 it = a.items[item];
  const int n_items = *a.n_items;
  asm volatile("" ::"s"(it.x), "s"(it.y), "s"(it.z), "s"(n_items));   // both loads before the branch
  if (item >= n_items) return;                  // uniform: the whole workgroup leaves
  const int4 ic = clamp_item(it, a.n_experts, a.n_rows);
  expert_tile<GPW, SD, KIND, false>(a, ic.x, ic.y, ic.z, lds);
}

// One token: its routing and the gate/up products in one launch. Every workgroup picks the
// token's experts itself (wave 0, topk_token, as moe_topk_kernel does) and takes its item
// from them: with one token each chosen expert has one row, and the sort orders experts by
// number, so item i (= blockIdx.y, S of them) is the i-th smallest chosen expert, at row i;
// the shared expert, number E, is always the last, so its workgroups skip the routing.
// Workgroup (0, 0) also writes the routing tables (sel, w, tok, inv, items, n_items) as the
// sort writes them for one token, for the down and combine launch. While wave 0 routes, the
// other waves form the token's group sums for every wave's range (the products then need
// only the code MFMAs). LDS: the reduction, then sel [S], w [S], the chosen experts in
// ascending order [S] and the group sums [K / 64].
template <int GPW, int SD, int EPL>
__global__ __launch_bounds__(1024) void moe_gate_up_one_token_kernel(MoeArgs a, const float *logits, int E, int topk,
                                                                     int norm_topk, int *sel, float *w, int *tok,
                                                                     int *inv, int4 *items, int *n_items) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int S = topk + 1;
  if (blockIdx.y == S - 1 && blockIdx.y != 0) {
    // the shared expert (number E) is the largest chosen one, so always the last item:
    // its workgroups need no routing and stream their weights at once
    expert_tile<GPW, SD, 0, true>(a, E, S - 1, 1, lds);
    return;
  }
  const int waves = blockDim.x >> 6;
  int *sel_l = reinterpret_cast<int *>(lds + (size_t)(waves - 1) * 64 * 16);
  float *w_l = reinterpret_cast<float *>(sel_l + S);
  int *order = reinterpret_cast<int *>(w_l + S);   // the chosen experts in ascending order
  float *gs_l = reinterpret_cast<float *>(order + S);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // the sums of range r (groups [r GPW, r GPW + GPW) of K) of the token row, as expert_tile reads it
  auto range_sums = [&](int r) {
    const int G = a.K / kGroup, wg0 = min(r * GPW, G), wn = max(0, min(G, wg0 + GPW) - wg0);
    const uint32_t xrange = wn > 0 ? (uint32_t)((a.x_rows - 1) * a.x_stride + wn * kGroup) * 2u : 0u;
    row0_group_sums<GPW>(make_rsrc(a.x + (size_t)wg0 * kGroup, xrange), 16u * (uint32_t)(lane >> 4), wn, lane,
                         gs_l + wg0);
  };
  if (wave == 0) topk_token<EPL>(logits, E, topk, norm_topk, sel_l, w_l, lane);
  // ranges: wave v >= 1 takes range v - 1, the last wave also the last range; a lone wave
  // takes its own range after routing
  const int r_lo = wave == 0 ? (waves == 1 ? 0 : waves) : wave - 1;
  const int r_hi = wave == 0 ? (waves == 1 ? 1 : waves) : (wave == waves - 1 ? waves : wave);
  for (int r = r_lo; r < r_hi; ++r) range_sums(r);
  __syncthreads();
  // thread s ranks slot s's expert among the S distinct chosen experts
  const int s = threadIdx.x;
  if (s < S) {
    const int es = sel_l[s];
    int rank = 0;
    for (int q = 0; q < S; ++q) rank += sel_l[q] < es;
    order[rank] = es;
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      sel[s] = es;
      w[s] = w_l[s];
      inv[s] = rank;
      tok[rank] = 0;
      items[rank] = int4{es, rank, 1, 0};
      if (s == 0) *n_items = S;
    }
  }
  __syncthreads();
  const int i = blockIdx.y;
  expert_tile<GPW, SD, 0, true, true>(a, order[i], i, 1, lds, gs_l);
}

// tile_dot_lds for two blocks of 16 staged rows at once (xs: row 0 of the first block, the
// second 16 rows further; gs: the first block's sums of group wg0, 16 NB = 32 floats per
// group, the second block's 16 after them). The codes of each group are converted once and
// multiplied into both blocks; each block's products, sums and order are tile_dot_lds's, so
// each gets the bits it gets alone. two = false: the second block is empty and skipped.
template <int GPW, int SD, int SUB, int BOOK = kAffine, bool FULL = false>
__device__ __forceinline__ void tile_dot_lds2(const u32x4 (&wq)[GPW / 2], const u32x4 (&sq)[GPW / 4],
                                              const _Float16 *xs, const float *gs, int rstride, int wn, int lane,
                                              bool two, f32x4 (&acc0)[SUB], f32x4 (&acc1)[SUB]) {
  const _Float16 *xa0 = xs + (lane & 15) * rstride + 8 * (lane >> 4);
  const _Float16 *xa1 = xa0 + 16 * rstride;
  const float *ga0 = gs + 4 * (lane >> 4);
  const float *ga1 = ga0 + 16;
#pragma unroll
  for (int s = 0; s < SUB; ++s) {
    acc0[s] = f32x4{};
    acc1[s] = f32x4{};
  }
#pragma unroll
  for (int jg = 0; jg < GPW; ++jg) {
    if (FULL || jg < wn) {   // uniform: the groups past the wave's range add nothing (FULL: wn == GPW)
      constexpr int per = GPW / SUB;
      half8 bq[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t u = wq[jg >> 1][2 * (jg & 1) + s];
        if constexpr (BOOK == kAffine) bq[s] = nib8_to_half8_sub(u);
        else bq[s] = native8_operand<BOOK>(u);
      }
      auto block = [&](const _Float16 *xa, const float *ga, f32x4 &acc) {
        half8 af[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) af[s] = *reinterpret_cast<const half8 *>(xa + jg * kGroup + 32 * s);
        if constexpr (BOOK == kAffine) {
          const f32x4 gsv = *reinterpret_cast<const f32x4 *>(ga + 32 * jg);
          group_step_gs_b<GPW, SD, 4>(acc, af, gsv, bq, sq, jg);
        } else {
#pragma unroll
          for (int s = 0; s < 2; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], bq[s], acc, 0, 0, 0);
        }
        asm volatile("" : "+v"(acc));
      };
      block(xa0, ga0, acc0[jg / per]);
      if (two) block(xa1, ga1, acc1[jg / per]);   // uniform
    }
  }
}

// The same products with the item's token rows staged once per workgroup: a workgroup
// takes one work item and `tiles_per_block` consecutive 16-row weight tiles of its expert,
// each split over K between `waves_per_tile` waves (wave = tile * waves_per_tile + part).
// Wave w stages rows w, w + waves, ... of the item (one token index per row, a uniform
// load through the row -> token map for gate/up): its first row's loads are issued, then
// every weight load of the wave, and the row goes to LDS in operand order while the
// weights are in flight. The group sums of the 16 rows are then formed once for all the
// workgroup's tiles (group_sums), and every tile reads rows and sums from LDS. (The
// per-tile kernel above reads each row once per tile and wave from L2 and forms the sums
// per tile: the same products, so the two kernels give the same bits.) LDS: 16 rows of
// K + 8 halves (the pad keeps the 16 rows of an operand read in distinct banks), the
// group sums [G][16] floats, then the partials of parts 1.. of every tile. CPL: chunks of
// 8 halves per lane and row (K / 512, rounded up). SUB: a part is summed as SUB sub-parts of
// GPW / SUB groups (the per-tile kernel's groups per wave), added in sub-part order, so the
// sums are the per-tile kernel's. Up to K = 2048 (CPL <= 4) the kernel is held to 80 VGPRs (six
// waves per SIMD), which lets two 12-wave workgroups share a CU; at K = 4096 LDS allows one
// workgroup per CU and the registers are left free.
// BOOK: kAffine, or (KIND 1 only) a native book: expert e's matrix sits at slot
// a.slots[e] with row scales a.s_row, the products chain as moe_native_kernel's do and the
// row scale is applied at the store (a slot outside the table gives zero rows).
// NB = 2: an expert's first two work items run in one workgroup as two blocks of 16 rows
// (item i leads when the item before it belongs to another expert, and takes item i + 1 when
// that one is its expert's too; the second item's own workgroup leaves at once). Both blocks
// use the codes as converted once, and each block's products, sums and order are those of
// the item alone, so the bits do not change; what it saves is the second reading and
// conversion of the expert's weights, which otherwise a few rows pay in full (at T = 512,
// 120 of the 256 routed experts have a second item, of 3.3 rows on average). An expert's
// third and later items (only the shared expert has them at these sizes) run alone.
// LDS with NB blocks: 16 NB rows, the group sums [G][16 NB], the partials of NB blocks.
template <int GPW, int SD, int KIND, int CPL, int SUB, int BOOK = kAffine, int NB = 1, bool FULL = false>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(CPL < 8 && NB == 1 ? 6 : 1))) void
moe_expert_lds_kernel(MoeArgs a) {
  static_assert(BOOK == kAffine || KIND == 1, "native books: the down kind only");
  static_assert(NB == 1 || NB == 2, "one or two row blocks");
  constexpr int NR = 16 * NB;                     // staged rows
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int item = blockIdx.y;
  // the item entry is read together with the count (the list holds the most items a call
  // can have, so the read is in bounds; entries past the count are not used)
  const int4 it = a.items[item];
  const int n_items = *a.n_items;
  asm volatile("" ::"s"(it.x), "s"(it.y), "s"(it.z), "s"(n_items));   // both loads before the branch
  if (item >= n_items) return;                  // uniform: the whole workgroup leaves
  const int4 ic = clamp_item(it, a.n_experts, a.n_rows);
  int e = ic.x;
  const int r0 = ic.y, rows = ic.z;
  int r1 = 0, rows1 = 0;                        // the second block (NB = 2): its first row and count
  if constexpr (NB == 2) {
    const int ep = item > 0 ? a.items[item - 1].x : -1;
    const int ep2 = item > 1 ? a.items[item - 2].x : -1;
    if (ep == it.x && ep2 != it.x) return;      // uniform: the second item of its expert, taken by the first
    if (ep != it.x && item + 1 < n_items) {
      const int4 nx = a.items[item + 1];
      if (nx.x == it.x) {
        const int4 nc = clamp_item(nx, a.n_experts, a.n_rows);
        r1 = nc.y;
        rows1 = nc.z;
      }
    }
  }
  bool slot_ok = true;
  if constexpr (BOOK != kAffine) {
    const int slot = __builtin_amdgcn_readfirstlane(a.slots[e]);
    slot_ok = slot >= 0 && slot < a.n_slots;    // uniform; a bad slot reads slot 0, writes zeros
    e = slot_ok ? slot : 0;
  }
  const int tid = threadIdx.x, nthreads = blockDim.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, j4 = lane >> 4;
  const int G = a.K / kGroup, G4 = quads_of(a.K);
  const int W = a.waves_per_tile;
  const int tt = wave / W, part = wave - tt * W;
  const int tile = blockIdx.x * a.tiles_per_block + tt;
  const bool tile_ok = tile < a.tiles_per_expert;
  const int t = e * a.tiles_per_expert + min(tile, a.tiles_per_expert - 1);
  const int wg0 = part * GPW;
  const int wn = tile_ok ? max(0, min(G, wg0 + GPW) - wg0) : 0;
  const int rstride = a.K + 8;
  _Float16 *xs = reinterpret_cast<_Float16 *>(lds);
  float *gsl = reinterpret_cast<float *>(lds + (size_t)NR * rstride * 2);
  f32x4 *red = reinterpret_cast<f32x4 *>(gsl + (size_t)G * NR);
  const int nw = nthreads >> 6, cpr = a.K / 8;

  // 1. the wave's first row (lane l: chunks l, l + 64, ... of 8 halves); rows past the
  // item's read zeros. Staged row r < 16 is row r of the first block, r >= 16 row r - 16 of
  // the second.
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.x_rows * a.x_stride * 2));
  auto load_row = [&](int row, u32x4 (&xr)[CPL]) {
    int blk_r0 = r0, blk_rows = rows, br = row;
    if constexpr (NB == 2) {
      blk_r0 = row < 16 ? r0 : r1;
      blk_rows = row < 16 ? rows : rows1;
      br = row & 15;
    }
    const bool ok = br < blk_rows;
    const int src = KIND == 0 ? token_of(a.tok, blk_r0 + (ok ? br : 0), a.x_rows) : blk_r0 + br;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      const uint32_t off = ok && c < cpr ? (uint32_t)(((size_t)src * a.x_stride + 8 * c) * 2) : kFarOffset;
      xr[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
    }
  };
  auto store_row = [&](int row, const u32x4 (&xr)[CPL]) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c < cpr) *reinterpret_cast<u32x4 *>(xs + (size_t)row * rstride + 8 * c) = prep_act<BOOK>(xr[j]);
    }
  };
  u32x4 xr[CPL];
  load_row(wave, xr);
  // 2. every weight load of this wave's part of its tile
  u32x4 wq[GPW / 2], sq[GPW / 4];
  const WaveTile wt = wave_tile(a.codes, BOOK == kAffine ? a.sb : a.codes, t, G4, wg0, wn > 0 ? GPW : 0);
  issue_tile_loads<GPW, BOOK>(wt, lane, wq, sq);
  __builtin_amdgcn_sched_barrier(0);
  // 3. rows -> LDS in operand order (loads complete in issue order: the first row waits
  // for its own loads only); a workgroup of fewer than NR waves stages the rest in turn
  store_row(wave, xr);
  for (int row = wave + nw; row < NR; row += nw) {
    load_row(row, xr);
    store_row(row, xr);
  }
  __syncthreads();
  // 4. the group sums of the staged rows, once for every tile: wave w forms groups w, w + nw,
  // ... of each block
  for (int gb = wave; BOOK == kAffine && gb < G * NB; gb += nw) {
    const int b = NB == 1 ? 0 : gb >= G, g = gb - b * G;
    const _Float16 *xa = xs + (size_t)(16 * b + c16) * rstride + 8 * j4 + (size_t)g * kGroup;
    half8 af[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) af[s] = *reinterpret_cast<const half8 *>(xa + 32 * s);
    const f32x4 gsv = group_sums(af);
    if (c16 == 0) *reinterpret_cast<f32x4 *>(gsl + (size_t)g * NR + 16 * b + 4 * j4) = gsv;
  }
  __syncthreads();
  // 5. products, then the sub-parts of each tile meet in order (only those with groups)
  f32x4 accs[NB][SUB];
  if constexpr (NB == 1) {
    if constexpr (FULL) {
      // every part of K holds GPW groups: the only wave without groups is one past the
      // expert's last tile
      if (wn > 0) {   // uniform
        tile_dot_lds<GPW, SD, SUB, BOOK, true>(wq, sq, xs + (size_t)wg0 * kGroup, gsl + (size_t)wg0 * 16, rstride, wn,
                                               lane, accs[0]);
      } else {
#pragma unroll
        for (int s = 0; s < SUB; ++s) accs[0][s] = f32x4{};
      }
    } else {
      tile_dot_lds<GPW, SD, SUB, BOOK>(wq, sq, xs + (size_t)wg0 * kGroup, gsl + (size_t)wg0 * 16, rstride, wn, lane,
                                       accs[0]);
    }
  } else if constexpr (FULL) {
    if (wn > 0) {   // uniform
      tile_dot_lds2<GPW, SD, SUB, BOOK, true>(wq, sq, xs + (size_t)wg0 * kGroup, gsl + (size_t)wg0 * NR, rstride, wn,
                                              lane, rows1 > 0, accs[0], accs[1]);
    } else {
#pragma unroll
      for (int s = 0; s < SUB; ++s) accs[0][s] = accs[1][s] = f32x4{};
    }
  } else {
    tile_dot_lds2<GPW, SD, SUB, BOOK>(wq, sq, xs + (size_t)wg0 * kGroup, gsl + (size_t)wg0 * NR, rstride, wn, lane,
                                      rows1 > 0, accs[0], accs[1]);
  }
  constexpr int per = GPW / SUB;
  if (part > 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int s = 0; s < SUB; ++s) red[((((size_t)tt * (W - 1) + part - 1) * NB + b) * SUB + s) * 64 + lane] = accs[b][s];
  }
  __syncthreads();
  if (part != 0 || !tile_ok) return;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int br0 = b ? r1 : r0, brows = b ? rows1 : rows;
    if (b > 0 && brows == 0) continue;            // uniform: no second block
    f32x4 acc = accs[b][0];
#pragma unroll
    for (int s = 1; s < SUB; ++s) {
      if (s * per < G) {
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] += accs[b][s][v];
      }
    }
    for (int p = 1; p < W; ++p) {
#pragma unroll
      for (int s = 0; s < SUB; ++s) {
        if ((p * SUB + s) * per >= G) break;
        const f32x4 o = red[((((size_t)tt * (W - 1) + p - 1) * NB + b) * SUB + s) * 64 + lane];
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] += o[v];
      }
    }
    if constexpr (KIND == 0) {
      _Float16 *act = static_cast<_Float16 *>(a.out);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float u = __shfl_xor(acc[v], 8);
        const int r = 4 * j4 + v;
        if (c16 < 8 && r < brows)
          act[(size_t)(br0 + r) * a.out_stride + 8 * tile + c16] = static_cast<_Float16>(silu(acc[v]) * u);
      }
    } else {
      float *y = static_cast<float *>(a.out);
      float sn = 1.0f;
      if constexpr (BOOK != kAffine) sn = a.s_row[(size_t)e * a.tiles_per_expert * 16 + 16 * tile + c16];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = 4 * j4 + v;
        if (r < brows)
          y[(size_t)(br0 + r) * a.out_stride + 16 * tile + c16] =
              BOOK == kAffine ? acc[v] : slot_ok ? sn * acc[v] : 0.0f;
      }
    }
  }
}

// Down projection and combine in one launch, for a few tokens whose items fit one wave's
// groups (K = I <= 64 * GPW): one workgroup per 16-feature tile of H; wave w takes items
// w, w + waves, ... and forms the tile's outputs for each item's rows exactly as
// moe_expert_kernel does (one wave per tile there too); the outputs meet in LDS by row, and
// the workgroup then adds each token's S slots into its residual row in slot order, with
// moe_combine_kernel's fused multiply-adds. Same bits as the two launches, without the
// second one and without writing y. LDS: [A rows][16] floats, then inv [A] and w [A].
// BOOK: kAffine, or a native book (int15, fp4) whose expert e sits at slot slots[e] with row
// scales s_row (the products are then moe_native_kernel's, scaled at the row as there; a
// slot outside [0, n_slots) contributes zero rows).
template <int GPW, int SD, int BOOK = kAffine>
__global__ __launch_bounds__(1024) void moe_down_combine_kernel(MoeArgs a, const int *inv, const float *w, int T,
                                                                int S, float *h, int h_stride, const float *s_row,
                                                                const int *slots, int n_slots) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  float *ys = reinterpret_cast<float *>(lds);
  const int A = T * S;
  const int t = threadIdx.x >> 4, c = threadIdx.x & 15;
  // Every global read that does not depend on the routing result is issued first, so that
  // its latency overlaps the weight stream: the wave's first item with the count (the list
  // holds at least as many entries as there are waves), this thread's routing-table entry
  // and, for the combining threads, the residual value the sum is added to.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool table = (int)threadIdx.x < A;
  const int inv_r = table ? min(max(inv[threadIdx.x], 0), A - 1) : 0;
  const float w_r = table ? w[threadIdx.x] : 0.0f;
  float *hp = h + (size_t)t * h_stride + 16 * blockIdx.x + c;
  const float h_r = t < T ? *hp : 0.0f;
  const int4 it0 = a.items[wave];
  const int n_items = *a.n_items;
  asm volatile("" ::"s"(it0.x), "s"(it0.y), "s"(it0.z), "s"(n_items));   // both loads before the branch
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int c16 = lane & 15, j4 = lane >> 4;
  const int G = a.K / kGroup, G4 = quads_of(a.K);
  const int tile = blockIdx.x;
  const int wn = min(G, GPW);
  const uint32_t xrange = (uint32_t)((a.x_rows - 1) * a.x_stride + wn * kGroup) * 2u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, xrange);
  for (int item = wave; item < n_items; item += waves) {
    const int4 it = clamp_item(item == wave ? it0 : a.items[item], a.n_experts, A);
    int e = it.x;
    const int r0 = it.y, rows = it.z;
    bool ok = true;
    float sn = 1.0f;
    if constexpr (BOOK != kAffine) {
      const int slot = __builtin_amdgcn_readfirstlane(slots[e]);
      ok = slot >= 0 && slot < n_slots;
      e = ok ? slot : 0;
      sn = ok ? s_row[(size_t)e * a.tiles_per_expert * 16 + 16 * tile + c16] : 0.0f;
    }
    const WaveTile wt = wave_tile(a.codes, BOOK == kAffine ? a.sb : a.codes, e * a.tiles_per_expert + tile, G4, 0,
                                  ok ? GPW : 0);
    const bool live = c16 < rows;
    const int xrow = r0 + (live ? c16 : 0);
    const f32x4 acc = tile_dot_rows<GPW, SD, BOOK>(wt, rx, (uint32_t)xrow * a.x_stride * 2u + 16u * j4, live, wn, lane);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * j4 + v;
      if (r < rows) ys[(size_t)(r0 + r) * 16 + c16] = BOOK == kAffine ? acc[v] : ok ? sn * acc[v] : 0.0f;
    }
  }
  int *inv_l = reinterpret_cast<int *>(ys + (size_t)A * 16);
  float *w_l = reinterpret_cast<float *>(inv_l + A);
  if (table) {
    inv_l[threadIdx.x] = inv_r;
    w_l[threadIdx.x] = w_r;
  }
  __syncthreads();
  if (t < T) {
    float acc = 0.0f;
    for (int s = 0; s < S; ++s) {
      const int as = t * S + s;
      acc = __builtin_fmaf(w_l[as], ys[(size_t)inv_l[as] * 16 + c], acc);
    }
    *hp = h_r + acc;
  }
}

// ------------------------------------------------------------------ combine

// h[t][d] += sum over slots s of w[t*S + s] * y[inv[t*S + s]][d], the slots in order
// (moe.metal:157-174). A thread takes V consecutive d (V = 4 when rows and pointers allow
// 16-byte accesses); every component follows the same order of fused multiply-adds.
template <int V>
__global__ void moe_combine_kernel(const float *y, int y_stride, const int *inv, const float *w, int T, int S, int H,
                                   float *h, int h_stride) {
  typedef float fvec __attribute__((ext_vector_type(V)));
  const int d = (blockIdx.x * blockDim.x + threadIdx.x) * V, t = blockIdx.y;
  if (d >= H || t >= T) return;
  fvec acc = {};
  for (int s = 0; s < S; ++s) {
    const int a = t * S + s;
    const float ws = w[a];
    const fvec yv = *reinterpret_cast<const fvec *>(y + (size_t)inv[a] * y_stride + d);
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = __builtin_fmaf(ws, yv[v], acc[v]);
  }
  fvec *hp = reinterpret_cast<fvec *>(h + (size_t)t * h_stride + d);
  fvec hv = *hp;
#pragma unroll
  for (int v = 0; v < V; ++v) hv[v] += acc[v];
  *hp = hv;
}

// ------------------------------------------------------------------ host side

// Groups per wave of the per-tile kernel: 8 up to K = 2048 (more waves per tile: measured
// 26.2 -> 23.8 us per MoE layer at T = 1 with H = 2048), then 16, then 24. The staged kernel
// sums in sub-parts of this many groups, so both give the same bits.
static int expert_gpw(int K) { return K <= 2048 ? 8 : 4 * quads_of(K) <= 16 * 16 ? 16 : 24; }
static int expert_waves(int K) { const int g = expert_gpw(K); return (4 * quads_of(K) + g - 1) / g; }

template <int GPW, int SD, int KIND>
static int launch_expert_inst(dim3 grid, int threads, hipStream_t st, const MoeArgs &a) {
  const size_t lds = (size_t)(threads / 64 - 1) * 64 * 16;
  moe_expert_kernel<GPW, SD, KIND><<<grid, threads, lds, st>>>(a);
  RLQ_HIP(hipGetLastError());
  return 0;
}

// The staged kernel takes K <= kStagedMaxK (its 16 rows of K halves fit LDS: two workgroups
// per CU up to K = 2048, one at 4096) and calls of at least kStagedMinTokens tokens: with
// fewer, items hold a row or two, there is nothing to reuse, and the per-tile kernel's many
// small workgroups spread the weight stream over more CUs (measured at T = 1: 31.4 against
// 33.0 us per layer). Groups per wave: 8 up to K = 1024, then 16.
constexpr int kStagedMaxK = 4096;
constexpr int kStagedMinTokens = 8;
static int staged_gpw(int K) { return K <= 1024 ? 8 : 16; }

// Waves per workgroup. Two workgroups per CU let one stream weights while the other stages
// rows or multiplies. With 16 groups per wave the kernel holds 80 VGPRs (6 waves per SIMD,
// 24 per CU), so where LDS leaves room for two workgroups they take 12 waves each; with 8
// groups per wave (about 52 VGPRs) two workgroups of 16 waves fit. Measured on the MoE
// layer at T = 512 (H = 2048, I = 512): gate/up 206 -> 184 us per layer going from 16 to
// 12 waves; 8 and 16 waves for down within 2 us.
static int staged_waves(int gpw, int W, int sub, int nb, size_t lds_rows) {
  const size_t lds12 = lds_rows + (size_t)(12 / W) * (W - 1) * nb * sub * 64 * 16;   // a 12-wave workgroup
  return gpw == 16 && 2 * lds12 <= kMaxLdsBytes ? 12 : 16;
}

// LDS of the staged kernel: NB blocks of 16 rows of K + 8 halves, their group sums, and the
// partials of parts 1.. of tpb tiles
static size_t staged_lds_bytes(int K, int GPW, int SUB, int NB, int tpb) {
  const int G = K / kGroup, W = (G + GPW - 1) / GPW;
  return (size_t)16 * NB * (K + 8) * 2 + (size_t)G * 16 * NB * 4 + (size_t)tpb * (W - 1) * NB * SUB * 64 * 16;
}

// tiles per workgroup: as many as staged_waves allows, fewer where the LDS would not hold them
static int staged_tpb(int K, int GPW, int SUB, int NB, int tpe) {
  const int G = K / kGroup, W = (G + GPW - 1) / GPW;
  int tpb = std::max(1, std::min(tpe, staged_waves(GPW, W, SUB, NB, staged_lds_bytes(K, GPW, SUB, NB, 0)) / W));
  while (tpb > 1 && staged_lds_bytes(K, GPW, SUB, NB, tpb) > kMaxLdsBytes) --tpb;
  return tpb;
}

template <int GPW, int SD, int KIND, int SUB, int BOOK, int NB, bool FULL = false>
static int launch_staged_nb(int tpe, hipStream_t st, MoeArgs a, int items) {
  const int G = a.K / kGroup, W = (G + GPW - 1) / GPW;
  const int tpb = staged_tpb(a.K, GPW, SUB, NB, tpe);
  a.tiles_per_block = tpb;
  a.waves_per_tile = W;
  const int threads = 64 * W * tpb;
  const int xpt = (a.K / 8 + 63) / 64;   // chunks of 8 halves per lane and row
  const size_t lds = staged_lds_bytes(a.K, GPW, SUB, NB, tpb);
  RLQ_REQUIRE(lds <= kMaxLdsBytes, "moe: the staged kernel needs %zu bytes of LDS (K=%d)", lds, a.K);
  const dim3 grid((tpe + tpb - 1) / tpb, items);
  static LdsOptIn lds_opt[4];
  const void *fns[4] = {reinterpret_cast<const void *>(&moe_expert_lds_kernel<GPW, SD, KIND, 1, SUB, BOOK, NB, FULL>),
                        reinterpret_cast<const void *>(&moe_expert_lds_kernel<GPW, SD, KIND, 2, SUB, BOOK, NB, FULL>),
                        reinterpret_cast<const void *>(&moe_expert_lds_kernel<GPW, SD, KIND, 4, SUB, BOOK, NB, FULL>),
                        reinterpret_cast<const void *>(&moe_expert_lds_kernel<GPW, SD, KIND, 8, SUB, BOOK, NB, FULL>)};
  const int which = xpt <= 1 ? 0 : xpt <= 2 ? 1 : xpt <= 4 ? 2 : 3;
  if (xpt <= 8)
    if (int rc = allow_large_lds(fns[which], lds_opt[which])) return rc;
  if (xpt <= 1) moe_expert_lds_kernel<GPW, SD, KIND, 1, SUB, BOOK, NB, FULL><<<grid, threads, lds, st>>>(a);
  else if (xpt <= 2) moe_expert_lds_kernel<GPW, SD, KIND, 2, SUB, BOOK, NB, FULL><<<grid, threads, lds, st>>>(a);
  else if (xpt <= 4) moe_expert_lds_kernel<GPW, SD, KIND, 4, SUB, BOOK, NB, FULL><<<grid, threads, lds, st>>>(a);
  else if (xpt <= 8) moe_expert_lds_kernel<GPW, SD, KIND, 8, SUB, BOOK, NB, FULL><<<grid, threads, lds, st>>>(a);
  else return fail("moe: %d activation chunks per thread (K=%d) is more than the staged kernel takes", xpt, a.K);
  RLQ_HIP(hipGetLastError());
  return 0;
}

template <int GPW, int SD, int KIND, int SUB, int BOOK = kAffine>
static int launch_staged_inst(int tpe, hipStream_t st, MoeArgs a, int items) {
  // Two row blocks per workgroup for the down projection, where the LDS holds them (measured
  // at T = 512: 180.1 and 181.2 -> 179.8 and 178.0 us per layer, alternating on one box). Not
  // for gate/up: 32 rows of K = 2048 leave room for one workgroup per CU (224 us per layer).
  const bool pair = KIND == 1 && staged_lds_bytes(a.K, GPW, SUB, 2, staged_tpb(a.K, GPW, SUB, 2, tpe)) <= kMaxLdsBytes;
  // every part of K whole (G a multiple of GPW, as at every BASELINE shape): the kernel
  // without per-group branches (the same bits; the gate/up kernel's VALU instructions 848 ->
  // 661, the register moves of the branches' merge points 211 -> 29)
  const bool full = (a.K / kGroup) % GPW == 0;
  if (pair) return full ? launch_staged_nb<GPW, SD, KIND, SUB, BOOK, 2, true>(tpe, st, a, items)
                        : launch_staged_nb<GPW, SD, KIND, SUB, BOOK, 2>(tpe, st, a, items);
  return full ? launch_staged_nb<GPW, SD, KIND, SUB, BOOK, 1, true>(tpe, st, a, items)
              : launch_staged_nb<GPW, SD, KIND, SUB, BOOK, 1>(tpe, st, a, items);
}

template <int KIND>
static int launch_expert(int K, int sd, int tpe, int items, int tokens, hipStream_t st, const MoeArgs &a) {
  if (K <= kStagedMaxK && tokens >= kStagedMinTokens) {
    // sub-parts of the per-tile kernel's groups per wave (staged_gpw is a multiple of it)
    const int sub = staged_gpw(K) / expert_gpw(K);
    if (staged_gpw(K) == 8) return sd == RLQ_F16 ? launch_staged_inst<8, 0, KIND, 1>(tpe, st, a, items)
                                                 : launch_staged_inst<8, 1, KIND, 1>(tpe, st, a, items);
    if (sub == 2) return sd == RLQ_F16 ? launch_staged_inst<16, 0, KIND, 2>(tpe, st, a, items)
                                       : launch_staged_inst<16, 1, KIND, 2>(tpe, st, a, items);
    return sd == RLQ_F16 ? launch_staged_inst<16, 0, KIND, 1>(tpe, st, a, items)
                         : launch_staged_inst<16, 1, KIND, 1>(tpe, st, a, items);
  }
  const dim3 grid(tpe, items);
  const int gpw = expert_gpw(K), threads = 64 * expert_waves(K);
  if (gpw == 8) return sd == RLQ_F16 ? launch_expert_inst<8, 0, KIND>(grid, threads, st, a)
                                     : launch_expert_inst<8, 1, KIND>(grid, threads, st, a);
  if (gpw == 16) return sd == RLQ_F16 ? launch_expert_inst<16, 0, KIND>(grid, threads, st, a)
                                      : launch_expert_inst<16, 1, KIND>(grid, threads, st, a);
  return sd == RLQ_F16 ? launch_expert_inst<24, 0, KIND>(grid, threads, st, a)
                       : launch_expert_inst<24, 1, KIND>(grid, threads, st, a);
}

// the sort's waves per round of tokens: 16, or as many as the LDS holds (12 bytes per wave
// and expert)
static size_t sort_lds_bytes(int E, int wpr) { return ((size_t)(1056 + wpr * (E + 1)) * 4 + 7) / 8 * 8 + (size_t)wpr * (E + 1) * 8; }
static int sort_wpr(int E) {
  int w = 16;                                   // at most 16 (the sort's per-expert pass holds 16 counts)
  while (w > 1 && sort_lds_bytes(E, w) > 160 * 1024) --w;
  return w;
}

static int check_moe_shape(const char *fn, int T, int E, int topk, int H, int I) {
  RLQ_REQUIRE(T >= 1 && E >= 1 && E <= kMaxExperts, "%s: T=%d E=%d (1 <= E <= %d)", fn, T, E, kMaxExperts);
  RLQ_REQUIRE(topk >= 1 && topk <= kMaxTopk && topk <= E, "%s: topk=%d (1..%d, <= E)", fn, topk, kMaxTopk);
  RLQ_REQUIRE((long long)T * (topk + 1) < (1LL << 30), "%s: T=%d is too large", fn, T);
  if (H > 0) RLQ_REQUIRE(H % 64 == 0 && H <= 16 * 24 * kGroup, "%s: H=%d must be a multiple of 64 and <= %d", fn, H,
                         16 * 24 * kGroup);
  if (I > 0) RLQ_REQUIRE(I % 64 == 0 && I <= 16 * 24 * kGroup, "%s: I=%d must be a multiple of 64 and <= %d", fn, I,
                         16 * 24 * kGroup);
  return 0;
}

// The argument checks and kernel arguments of rlq_moe_gate_up.
static int gate_up_args(const void *x, int x_stride, int T, int H, int I, int E, int topk, const void *packed_gu,
                        int scale_dtype, const int *tok, const int *items, const int *n_items, void *act,
                        int act_stride, MoeArgs &a) {
  if (int rc = check_moe_shape("rlq_moe_gate_up", T, E, topk, H, I)) return rc;
  RLQ_REQUIRE(scale_dtype == RLQ_F16 || scale_dtype == RLQ_BF16, "rlq_moe_gate_up: unknown scale dtype %d", scale_dtype);
  RLQ_REQUIRE(x && packed_gu && tok && items && n_items && act, "rlq_moe_gate_up: null pointer argument");
  RLQ_REQUIRE(x_stride >= H && x_stride % 8 == 0 && aligned(x, 16), "rlq_moe_gate_up: x must be 16-byte aligned "
              "with x_stride >= H and a multiple of 8 (got %d)", x_stride);
  RLQ_REQUIRE(act_stride >= I && aligned(act, 2), "rlq_moe_gate_up: act_stride=%d < I=%d", act_stride, I);
  RLQ_REQUIRE((long long)T * x_stride * 2 < (1LL << 31), "rlq_moe_gate_up: x spans more than 2 GiB");
  RLQ_REQUIRE(aligned(packed_gu, 16) && aligned(items, 16), "rlq_moe_gate_up: packed and items must be 16-byte aligned");
  const int N = (E + 1) * 2 * I;
  a = MoeArgs{};
  a.x = static_cast<const _Float16 *>(x);
  a.tok = tok;
  a.codes = static_cast<const u32x4 *>(packed_gu);
  a.sb = reinterpret_cast<const u32x4 *>(static_cast<const char *>(packed_gu) + packed_code_bytes(H, N));
  a.items = reinterpret_cast<const int4 *>(items);
  a.n_items = n_items;
  a.out = act;
  a.x_rows = T;
  a.x_stride = x_stride;
  a.K = H;
  a.tiles_per_expert = 2 * I / 16;
  a.out_stride = act_stride;
  a.n_experts = E + 1;
  a.n_rows = T * (topk + 1);
  return 0;
}

// One token, routing and gate/up in one launch (moe_gate_up_one_token_kernel); returns 1
// when the shape has no such kernel (E > 256 or K past 16 groups per wave), and the caller
// routes and multiplies in two launches.
template <int GPW, int SD, int EPL>
static void launch_one_token_inst(const MoeArgs &a, const float *logits, int E, int topk, int norm_topk, int *sel,
                                  float *w, int *tok, int *inv, int *items, int *n_items, hipStream_t st) {
  const int waves = expert_waves(a.K), S = topk + 1;
  const size_t lds = (size_t)(waves - 1) * 64 * 16 + (size_t)S * 12 + (size_t)(a.K / kGroup) * 4;
  moe_gate_up_one_token_kernel<GPW, SD, EPL><<<dim3(a.tiles_per_expert, S), 64 * waves, lds, st>>>(
      a, logits, E, topk, norm_topk, sel, w, tok, inv, reinterpret_cast<int4 *>(items), n_items);
}

template <int GPW, int SD>
static int launch_one_token_epl(int epl, const MoeArgs &a, const float *logits, int E, int topk, int norm_topk,
                                int *sel, float *w, int *tok, int *inv, int *items, int *n_items, hipStream_t st) {
  if (epl <= 1) launch_one_token_inst<GPW, SD, 1>(a, logits, E, topk, norm_topk, sel, w, tok, inv, items, n_items, st);
  else if (epl <= 2) launch_one_token_inst<GPW, SD, 2>(a, logits, E, topk, norm_topk, sel, w, tok, inv, items, n_items, st);
  else launch_one_token_inst<GPW, SD, 4>(a, logits, E, topk, norm_topk, sel, w, tok, inv, items, n_items, st);
  RLQ_HIP(hipGetLastError());
  return 0;
}

static int route_gate_up_one_token(const MoeArgs &a, int sd, const float *logits, int E, int topk, int norm_topk,
                                   int *sel, float *w, int *tok, int *inv, int *items, int *n_items, hipStream_t st) {
  const int epl = (E + 63) / 64, gpw = expert_gpw(a.K);
  if (epl > 4 || (gpw != 8 && gpw != 16)) return 1;
  if (gpw == 8)
    return sd == RLQ_F16 ? launch_one_token_epl<8, 0>(epl, a, logits, E, topk, norm_topk, sel, w, tok, inv, items, n_items, st)
                         : launch_one_token_epl<8, 1>(epl, a, logits, E, topk, norm_topk, sel, w, tok, inv, items, n_items, st);
  return sd == RLQ_F16 ? launch_one_token_epl<16, 0>(epl, a, logits, E, topk, norm_topk, sel, w, tok, inv, items, n_items, st)
                       : launch_one_token_epl<16, 1>(epl, a, logits, E, topk, norm_topk, sel, w, tok, inv, items, n_items, st);
}


// ------------------------------------------------------------------ native experts

// The experts of one kind in the native format, all in one launch (linear_q4n_moe,
// kernels/linear.metal:254-308): grid (Ne / 16 tiles, max_items); item i < *n_items, for
// expert e = items[i].x, reads slot = slots[e] (where the expert's matrix sits: the stacked
// tensor, slot = expert, or an expert cache) and computes its 16-row tile blockIdx.x:
//   c[r][n] = s[slot * Ne + n] * (a[src(r)] . L(q_slot[n])^T)   for the item's rows r
// with src(r) = tok[r] (GATHER: the gather of moe.metal:143-155 fused, a holds the tokens)
// or r (a holds sorted rows). Waves split K as in the affine expert kernel (expert_gpw)
// and meet in LDS in wave order; no per-group scale, so each wave's products chain in
// the MFMA (native_step) and the row scale is applied at the store, as the reference
// applies it to its matmul result. A slot outside [0, n_slots) reads nothing and gives
// zero rows.
template <int GPW, int BOOK, bool GATHER>
__global__ __launch_bounds__(1024) void moe_native_kernel(const _Float16 *a, int a_stride, int a_rows, const int *tok,
                                                          int K, int Ne, const u32x4 *codes, const float *s,
                                                          const int *slots, int n_slots, const int4 *items,
                                                          const int *n_items_p, float *c, int c_stride) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int item = blockIdx.y;
  // the list holds max_items entries (the grid's height), so the read is in bounds
  const int4 it = items[item];
  const int n_items = *n_items_p;
  asm volatile("" ::"s"(it.x), "s"(it.y), "s"(it.z), "s"(n_items));   // both loads before the branch
  if (item >= n_items) return;                  // uniform: the whole workgroup leaves
  const int r0 = it.y, rows = it.z;
  const int slot = __builtin_amdgcn_readfirstlane(slots[it.x]);
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, j4 = lane >> 4;
  const int n = 16 * blockIdx.x + c16;
  if (slot < 0 || slot >= n_slots) {            // uniform
    if (wave == 0)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (4 * j4 + v < rows) c[(size_t)(r0 + 4 * j4 + v) * c_stride + n] = 0.0f;
    return;
  }
  const int G = K / kGroup, G4 = quads_of(K);
  const int wg0 = wave * GPW;
  const int wn = max(0, min(G, wg0 + GPW) - wg0);
  const WaveTile wt = wave_tile(codes, codes, slot * (Ne / 16) + (int)blockIdx.x, G4, wg0, GPW);
  const bool live = c16 < rows;
  int xrow = r0 + (live ? c16 : 0);
  if constexpr (GATHER) xrow = min(max(tok[xrow], 0), a_rows - 1);
  const uint32_t xrange = wn > 0 ? (uint32_t)((a_rows - 1) * a_stride + wn * kGroup) * 2u : 0u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a + (size_t)min(wg0, G) * kGroup, xrange);
  f32x4 acc = tile_dot_rows<GPW, 0, BOOK>(wt, rx, (uint32_t)xrow * a_stride * 2u + 16u * j4, live, wn, lane);
  acc = reduce_waves(acc, reinterpret_cast<f32x4 *>(lds), wave, waves, lane);
  if (wave != 0) return;
  const float sn = s[(size_t)slot * Ne + n];
#pragma unroll
  for (int v = 0; v < 4; ++v)
    if (4 * j4 + v < rows) c[(size_t)(r0 + 4 * j4 + v) * c_stride + n] = sn * acc[v];
}

// act[r][i] = half(silu(gu[r][i]) * gu[r][I + i] * cs[i]) (kernels/ops.metal:446-455); cs is
// the down projection's column scale (ones for affine matrices: cs == nullptr).
__global__ void moe_swiglu_kernel(const float *gu, int gu_stride, int A, int I, const float *cs, _Float16 *act,
                                  int act_stride) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
  if (i >= I || r >= A) return;
  const float *row = gu + (size_t)r * gu_stride;
  const float v = silu(row[i]) * row[I + i];
  act[(size_t)r * act_stride + i] = static_cast<_Float16>(cs ? v * cs[i] : v);
}

template <int GPW, int BOOK>
static void launch_native_inst(dim3 grid, int threads, bool gather, hipStream_t st, const _Float16 *a, int a_stride,
                               int a_rows, const int *tok, int K, int Ne, const u32x4 *codes, const float *s,
                               const int *slots, int n_slots, const int4 *items, const int *n_items, float *c,
                               int c_stride) {
  const size_t lds = (size_t)(threads / 64 - 1) * 64 * 16;
  if (gather)
    moe_native_kernel<GPW, BOOK, true><<<grid, threads, lds, st>>>(a, a_stride, a_rows, tok, K, Ne, codes, s, slots,
                                                                   n_slots, items, n_items, c, c_stride);
  else
    moe_native_kernel<GPW, BOOK, false><<<grid, threads, lds, st>>>(a, a_stride, a_rows, tok, K, Ne, codes, s, slots,
                                                                    n_slots, items, n_items, c, c_stride);
}


// The native gate/up product with the SwiGLU in its epilogue: workgroup (i, item) takes
// the gate tile i and the up tile i + I/16 of the item's expert slot (the reference's
// gate rows [0, I) then up rows [I, 2I) of each expert), reads each activation operand
// once for both (tile_dot_rows2: each tile's sums are tile_dot_rows's) and writes
//   act[r][n] = half(silu(sg[n] * g) * (su[n] * u) * cs[n])
// with the products and the order of moe_native_kernel followed by moe_swiglu_kernel, so
// the bits are the two launches' without the fp32 gate/up rows in between. The gather is
// fused (rows are read through tok).
// One workgroup's part: slot `slot`, rows r0 .. r0 + rows - 1 (token tok[r], or token 0
// when ONE_TOKEN), gate tile blockIdx.x. LDS: the two tiles' reductions, 2 (waves-1) KB.
template <int GPW, int BOOK, bool ONE_TOKEN>
__device__ __forceinline__ void native_gate_up_tile(const _Float16 *x, int x_stride, int T, const int *tok, int H,
                                                    int I, const u32x4 *codes, const float *s, int slot, int n_slots,
                                                    int r0, int rows, const float *cs, _Float16 *act, int act_stride,
                                                    unsigned char *lds) {
  const int waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, j4 = lane >> 4;
  const int n = 16 * blockIdx.x + c16;          // feature of the gate and up halves
  if (slot < 0 || slot >= n_slots) {            // uniform: zero rows, as the two launches give
    if (wave == 0)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (4 * j4 + v < rows) {
          const float z = silu(0.0f) * 0.0f;
          act[(size_t)(r0 + 4 * j4 + v) * act_stride + n] = static_cast<_Float16>(cs ? z * cs[n] : z);
        }
    return;
  }
  const int G = H / kGroup, G4 = quads_of(H);
  const int wg0 = wave * GPW;
  const int wn = max(0, min(G, wg0 + GPW) - wg0);
  const int tg = slot * (2 * I / 16) + (int)blockIdx.x;
  const WaveTile wgt = wave_tile(codes, codes, tg, G4, wg0, GPW);
  const WaveTile wut = wave_tile(codes, codes, tg + I / 16, G4, wg0, GPW);
  const bool live = c16 < rows;
  const int xrow = ONE_TOKEN ? 0 : min(max(tok[r0 + (live ? c16 : 0)], 0), T - 1);
  const uint32_t xrange = wn > 0 ? (uint32_t)((T - 1) * x_stride + wn * kGroup) * 2u : 0u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (size_t)min(wg0, G) * kGroup, xrange);
  f32x4 ag, au;
  tile_dot_rows2<GPW, 0, BOOK>(wgt, wut, rx, (uint32_t)xrow * x_stride * 2u + 16u * j4, live, wn, lane, ag, au);
  f32x4 *red = reinterpret_cast<f32x4 *>(lds);  // [2][waves-1][64]
  if (wave > 0) {
    red[(wave - 1) * 64 + lane] = ag;
    red[(waves - 1 + wave - 1) * 64 + lane] = au;
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < waves; ++w) {
    const f32x4 og = red[(w - 1) * 64 + lane], ou = red[(waves - 1 + w - 1) * 64 + lane];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      ag[v] += og[v];
      au[v] += ou[v];
    }
  }
  const size_t srow = (size_t)slot * 2 * I + n;
  const float sg = s[srow], su = s[srow + I];
#pragma unroll
  for (int v = 0; v < 4; ++v)
    if (4 * j4 + v < rows) {
      const float z = silu(sg * ag[v]) * (su * au[v]);
      act[(size_t)(r0 + 4 * j4 + v) * act_stride + n] = static_cast<_Float16>(cs ? z * cs[n] : z);
    }
}

template <int GPW, int BOOK>
__global__ __launch_bounds__(1024) void moe_native_gate_up_kernel(const _Float16 *x, int x_stride, int T,
                                                                  const int *tok, int H, int I, const u32x4 *codes,
                                                                  const float *s, const int *slots, int n_slots,
                                                                  const int4 *items, const int *n_items_p,
                                                                  const float *cs, _Float16 *act, int act_stride) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int item = blockIdx.y;
  const int4 it = items[item];
  const int n_items = *n_items_p;
  asm volatile("" ::"s"(it.x), "s"(it.y), "s"(it.z), "s"(n_items));   // both loads before the branch
  if (item >= n_items) return;                  // uniform: the whole workgroup leaves
  const int slot = __builtin_amdgcn_readfirstlane(slots[it.x]);
  native_gate_up_tile<GPW, BOOK, false>(x, x_stride, T, tok, H, I, codes, s, slot, n_slots, it.y, it.z, cs, act,
                                        act_stride, lds);
}

// One token: the routing inside the native gate/up launch, as moe_gate_up_one_token_kernel
// does for affine experts (wave 0 picks the token's experts; item i is the i-th smallest
// chosen expert, at row i; workgroup (0, 0) writes the routing tables). LDS: the
// reductions, then sel [S], w [S] and the chosen experts in ascending order [S].
template <int GPW, int BOOK, int EPL>
__global__ __launch_bounds__(1024) void moe_native_gate_up_one_token_kernel(
    const _Float16 *x, int x_stride, int H, int I, const u32x4 *codes, const float *s, const int *slots, int n_slots,
    const float *cs, _Float16 *act, int act_stride, const float *logits, int E, int topk, int norm_topk, int *sel,
    float *w, int *tok, int *inv, int4 *items, int *n_items) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int S = topk + 1;
  if (blockIdx.y == S - 1 && blockIdx.y != 0) {
    // the shared expert (number E) is always the last item: no routing to wait for
    const int slot = __builtin_amdgcn_readfirstlane(slots[E]);
    native_gate_up_tile<GPW, BOOK, true>(x, x_stride, 1, nullptr, H, I, codes, s, slot, n_slots, S - 1, 1, cs, act,
                                         act_stride, lds);
    return;
  }
  const int waves = blockDim.x >> 6;
  int *sel_l = reinterpret_cast<int *>(lds + (size_t)2 * (waves - 1) * 64 * 16);
  float *w_l = reinterpret_cast<float *>(sel_l + S);
  int *order = reinterpret_cast<int *>(w_l + S);
  if (threadIdx.x < 64) topk_token<EPL>(logits, E, topk, norm_topk, sel_l, w_l, threadIdx.x);
  __syncthreads();
  const int t = threadIdx.x;
  if (t < S) {
    const int es = sel_l[t];
    int rank = 0;
    for (int q = 0; q < S; ++q) rank += sel_l[q] < es;
    order[rank] = es;
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      sel[t] = es;
      w[t] = w_l[t];
      inv[t] = rank;
      tok[rank] = 0;
      items[rank] = int4{es, rank, 1, 0};
      if (t == 0) *n_items = S;
    }
  }
  __syncthreads();
  const int i = blockIdx.y;
  const int slot = __builtin_amdgcn_readfirstlane(slots[order[i]]);
  native_gate_up_tile<GPW, BOOK, true>(x, x_stride, 1, nullptr, H, I, codes, s, slot, n_slots, i, 1, cs, act,
                                       act_stride, lds);
}

template <int GPW, int BOOK, int EPL>
static void launch_native_one_token_inst(int S, hipStream_t st, const _Float16 *x, int x_stride, int H, int I,
                                         const u32x4 *codes, const float *s, const int *slots, int n_slots,
                                         const float *cs, _Float16 *act, int act_stride, const float *logits, int E,
                                         int topk, int norm_topk, int *sel, float *w, int *tok, int *inv, int4 *items,
                                         int *n_items) {
  const int waves = expert_waves(H);
  const size_t lds = (size_t)2 * (waves - 1) * 64 * 16 + (size_t)S * 12;
  moe_native_gate_up_one_token_kernel<GPW, BOOK, EPL><<<dim3(I / 16, S), 64 * waves, lds, st>>>(
      x, x_stride, H, I, codes, s, slots, n_slots, cs, act, act_stride, logits, E, topk, norm_topk, sel, w, tok, inv,
      items, n_items);
}

// Routing and the native gate/up + SwiGLU of one token in one launch; returns 1 when the
// shape has no such kernel (E > 256 or more than 16 groups per wave).
static int native_one_token(int book, const _Float16 *x, int x_stride, int H, int I, const u32x4 *codes,
                            const float *s, const int *slots, int n_slots, const float *cs, _Float16 *act,
                            const float *logits, int E, int topk, int norm_topk, int *sel, float *w, int *tok,
                            int *inv, int4 *items, int *n_items, hipStream_t st) {
  const int epl = (E + 63) / 64, gpw = expert_gpw(H), S = topk + 1;
  if (epl > 4 || (gpw != 8 && gpw != 16)) return 1;
#define RLQ_NOT(G, B, P)                                                                                           \
  launch_native_one_token_inst<G, B, P>(S, st, x, x_stride, H, I, codes, s, slots, n_slots, cs, act, I, logits, E, \
                                        topk, norm_topk, sel, w, tok, inv, items, n_items)
#define RLQ_NOT_EPL(G, B) (epl <= 1 ? RLQ_NOT(G, B, 1) : epl <= 2 ? RLQ_NOT(G, B, 2) : RLQ_NOT(G, B, 4))
  if (book == RLQ_BOOK_INT15) {
    if (gpw == 8) RLQ_NOT_EPL(8, kInt15);
    else RLQ_NOT_EPL(16, kInt15);
  } else {
    if (gpw == 8) RLQ_NOT_EPL(8, kFp4);
    else RLQ_NOT_EPL(16, kFp4);
  }
#undef RLQ_NOT_EPL
#undef RLQ_NOT
  RLQ_HIP(hipGetLastError());
  return 0;
}

template <int GPW, int BOOK>
static void launch_native_gate_up_inst(dim3 grid, int threads, hipStream_t st, const _Float16 *x, int x_stride, int T,
                                       const int *tok, int H, int I, const u32x4 *codes, const float *s,
                                       const int *slots, int n_slots, const int4 *items, const int *n_items,
                                       const float *cs, _Float16 *act, int act_stride) {
  const size_t lds = (size_t)2 * (threads / 64 - 1) * 64 * 16;
  moe_native_gate_up_kernel<GPW, BOOK><<<grid, threads, lds, st>>>(x, x_stride, T, tok, H, I, codes, s, slots, n_slots,
                                                                   items, n_items, cs, act, act_stride);
}

}  // namespace rlq

using namespace rlq;

extern "C" {

size_t rlq_moe_max_items(int T, int E, int topk) {
  if (T < 1 || E < 1 || topk < 1) return 0;
  return (size_t)moe_max_items(T, E, topk);
}

int rlq_moe_route(const float *logits, int logit_stride, int T, int E, int topk, int norm_topk, int *sel, float *w,
                  int *tok, int *inv, int *items, int *n_items, void *stream) {
  if (int rc = check_moe_shape("rlq_moe_route", T, E, topk, 0, 0)) return rc;
  RLQ_REQUIRE(logit_stride >= E + 1, "rlq_moe_route: logit_stride=%d < E + 1 = %d", logit_stride, E + 1);
  RLQ_REQUIRE(logits && sel && w && tok && inv && items && n_items, "rlq_moe_route: null pointer argument");
  RLQ_REQUIRE(aligned(items, 16), "rlq_moe_route: items must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int epl = (E + 63) / 64;
  const int wpr = sort_wpr(E);
  const size_t lds = sort_lds_bytes(E, wpr);
  if (T <= kRouteSmallTokens) {
    // one launch: the top-k of each token by its own wave, then the sort (8 KB of LDS)
    int4 *it4 = reinterpret_cast<int4 *>(items);
#define RLQ_ROUTE_SMALL(N)                                                                                             \
  moe_route_small_kernel<N><<<1, 1024, kSortSmallLds, st>>>(logits, logit_stride, T, E, topk, norm_topk, sel, w, tok,  \
                                                            inv, it4, n_items)
    if (epl <= 1) RLQ_ROUTE_SMALL(1);
    else if (epl <= 2) RLQ_ROUTE_SMALL(2);
    else if (epl <= 4) RLQ_ROUTE_SMALL(4);
    else if (epl <= 8) RLQ_ROUTE_SMALL(8);
    else RLQ_ROUTE_SMALL(16);
#undef RLQ_ROUTE_SMALL
    RLQ_HIP(hipGetLastError());
    return 0;
  }
  const dim3 g1((T + 3) / 4);
  if (epl <= 1) moe_topk_kernel<1><<<g1, 256, 0, st>>>(logits, logit_stride, T, E, topk, norm_topk, sel, w);
  else if (epl <= 2) moe_topk_kernel<2><<<g1, 256, 0, st>>>(logits, logit_stride, T, E, topk, norm_topk, sel, w);
  else if (epl <= 4) moe_topk_kernel<4><<<g1, 256, 0, st>>>(logits, logit_stride, T, E, topk, norm_topk, sel, w);
  else if (epl <= 8) moe_topk_kernel<8><<<g1, 256, 0, st>>>(logits, logit_stride, T, E, topk, norm_topk, sel, w);
  else moe_topk_kernel<16><<<g1, 256, 0, st>>>(logits, logit_stride, T, E, topk, norm_topk, sel, w);
  RLQ_HIP(hipGetLastError());
  static LdsOptIn lds_opt;
  if (int rc = allow_large_lds(reinterpret_cast<const void *>(&moe_sort_kernel), lds_opt)) return rc;
  moe_sort_kernel<<<1, 1024, lds, st>>>(sel, T, E, topk + 1, wpr, tok, inv, reinterpret_cast<int4 *>(items), n_items);
  RLQ_HIP(hipGetLastError());
  return 0;
}

int rlq_moe_gate_up(const void *x, int x_stride, int T, int H, int I, int E, int topk, const void *packed_gu,
                    int scale_dtype, const int *tok, const int *items, const int *n_items, void *act, int act_stride,
                    void *stream) {
  MoeArgs a;
  if (int rc = gate_up_args(x, x_stride, T, H, I, E, topk, packed_gu, scale_dtype, tok, items, n_items, act, act_stride,
                            a))
    return rc;
  return launch_expert<0>(H, scale_dtype, a.tiles_per_expert, moe_max_items(T, E, topk), T,
                          static_cast<hipStream_t>(stream), a);
}

int rlq_moe_down(const void *act, int act_stride, int T, int H, int I, int E, int topk, const void *packed_dn,
                 int scale_dtype, const int *items, const int *n_items, float *y, int y_stride, void *stream) {
  if (int rc = check_moe_shape("rlq_moe_down", T, E, topk, H, I)) return rc;
  RLQ_REQUIRE(scale_dtype == RLQ_F16 || scale_dtype == RLQ_BF16, "rlq_moe_down: unknown scale dtype %d", scale_dtype);
  RLQ_REQUIRE(act && packed_dn && items && n_items && y, "rlq_moe_down: null pointer argument");
  RLQ_REQUIRE(act_stride >= I && act_stride % 8 == 0 && aligned(act, 16), "rlq_moe_down: act must be 16-byte aligned "
              "with act_stride >= I and a multiple of 8 (got %d)", act_stride);
  RLQ_REQUIRE(y_stride >= H, "rlq_moe_down: y_stride=%d < H=%d", y_stride, H);
  const long long A = (long long)T * (topk + 1);
  RLQ_REQUIRE(A * act_stride * 2 < (1LL << 31), "rlq_moe_down: act spans more than 2 GiB");
  RLQ_REQUIRE(aligned(packed_dn, 16) && aligned(items, 16), "rlq_moe_down: packed and items must be 16-byte aligned");
  const int N = (E + 1) * H;
  MoeArgs a = {};
  a.x = static_cast<const _Float16 *>(act);
  a.tok = nullptr;
  a.codes = static_cast<const u32x4 *>(packed_dn);
  a.sb = reinterpret_cast<const u32x4 *>(static_cast<const char *>(packed_dn) + packed_code_bytes(I, N));
  a.items = reinterpret_cast<const int4 *>(items);
  a.n_items = n_items;
  a.out = y;
  a.x_rows = (int)A;
  a.x_stride = act_stride;
  a.K = I;
  a.tiles_per_expert = H / 16;
  a.out_stride = y_stride;
  a.n_experts = E + 1;
  a.n_rows = (int)A;
  return launch_expert<1>(I, scale_dtype, a.tiles_per_expert, moe_max_items(T, E, topk), T,
                          static_cast<hipStream_t>(stream), a);
}

int rlq_moe_combine(const float *y, int y_stride, const int *inv, const float *w, int T, int topk, int H, float *h,
                    int h_stride, void *stream) {
  RLQ_REQUIRE(T >= 1 && H >= 1 && topk >= 1 && topk <= kMaxTopk, "rlq_moe_combine: T=%d H=%d topk=%d", T, H, topk);
  RLQ_REQUIRE(y && inv && w && h, "rlq_moe_combine: null pointer argument");
  RLQ_REQUIRE(y_stride >= H && h_stride >= H, "rlq_moe_combine: strides must be >= H");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (H % 4 == 0 && y_stride % 4 == 0 && h_stride % 4 == 0 && aligned(y, 16) && aligned(h, 16))
    moe_combine_kernel<4><<<dim3((H + 1023) / 1024, T), 256, 0, st>>>(y, y_stride, inv, w, T, topk + 1, H, h, h_stride);
  else
    moe_combine_kernel<1><<<dim3((H + 255) / 256, T), 256, 0, st>>>(y, y_stride, inv, w, T, topk + 1, H, h, h_stride);
  RLQ_HIP(hipGetLastError());
  return 0;
}

// Workspace of rlq_moe, in order: sel, w, tok, inv [A] (4 bytes each), items [max_items][4]
// ints, n_items (padded to 16 bytes), act fp16 [A][I], y fp32 [A][H]; each part 256-byte aligned.
static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t rlq_moe_workspace_bytes(int T, int E, int topk, int H, int I) {
  if (T < 1 || E < 1 || topk < 1 || H < 1 || I < 1) return 0;
  const size_t A = (size_t)T * (topk + 1);
  return 4 * align256(A * 4) + align256((size_t)moe_max_items(T, E, topk) * 16) + 256 + align256(A * I * 2) +
         align256(A * H * 4);
}

int rlq_moe(const void *x, int x_stride, const float *logits, int logit_stride, int T, int E, int topk, int norm_topk,
            int H, int I, const void *packed_gu, const void *packed_dn, int scale_dtype, float *h, int h_stride,
            void *workspace, size_t workspace_bytes, void *stream) {
  if (int rc = check_moe_shape("rlq_moe", T, E, topk, H, I)) return rc;
  const size_t need = rlq_moe_workspace_bytes(T, E, topk, H, I);
  RLQ_REQUIRE(workspace && workspace_bytes >= need, "rlq_moe: workspace of %zu bytes is smaller than the %zu this call "
              "needs", workspace_bytes, need);
  RLQ_REQUIRE(aligned(workspace, 256), "rlq_moe: workspace must be 256-byte aligned");
  const size_t A = (size_t)T * (topk + 1);
  char *p = static_cast<char *>(workspace);
  int *sel = reinterpret_cast<int *>(p);            p += align256(A * 4);
  float *w = reinterpret_cast<float *>(p);          p += align256(A * 4);
  int *tok = reinterpret_cast<int *>(p);            p += align256(A * 4);
  int *inv = reinterpret_cast<int *>(p);            p += align256(A * 4);
  int *items = reinterpret_cast<int *>(p);          p += align256((size_t)moe_max_items(T, E, topk) * 16);
  int *n_items = reinterpret_cast<int *>(p);        p += 256;
  _Float16 *act = reinterpret_cast<_Float16 *>(p);  p += align256(A * I * 2);
  float *y = reinterpret_cast<float *>(p);
  int fused = 1;
  if (T == 1) {
    // one token: routing and gate/up in one launch where a kernel covers the shape
    RLQ_REQUIRE(logits && logit_stride >= E + 1, "rlq_moe: logits null or logit_stride=%d < E + 1 = %d", logit_stride,
                E + 1);
    MoeArgs a;
    if (int rc = gate_up_args(x, x_stride, T, H, I, E, topk, packed_gu, scale_dtype, tok, items, n_items, act, I, a))
      return rc;
    fused = route_gate_up_one_token(a, scale_dtype, logits, E, topk, norm_topk, sel, w, tok, inv, items, n_items,
                                    static_cast<hipStream_t>(stream));
    if (fused < 0) return fused;
  }
  if (fused) {
    if (int rc = rlq_moe_route(logits, logit_stride, T, E, topk, norm_topk, sel, w, tok, inv, items, n_items, stream))
      return rc;
    if (int rc = rlq_moe_gate_up(x, x_stride, T, H, I, E, topk, packed_gu, scale_dtype, tok, items, n_items, act, I,
                                 stream))
      return rc;
  }
  if (T <= kDownCombineTokens && expert_gpw(I) == 8 && I / kGroup <= 8) {
    // a few tokens: down and combine in one launch (the same bits as the two below)
    RLQ_REQUIRE(h && h_stride >= H, "rlq_moe: h is null or h_stride=%d < H=%d", h_stride, H);
    RLQ_REQUIRE(packed_dn && aligned(packed_dn, 16), "rlq_moe: the down stack is null or not 16-byte aligned");
    RLQ_REQUIRE(scale_dtype == RLQ_F16 || scale_dtype == RLQ_BF16, "rlq_moe: unknown scale dtype %d", scale_dtype);
    MoeArgs a = {};
    a.x = act;
    a.codes = static_cast<const u32x4 *>(packed_dn);
    a.sb = reinterpret_cast<const u32x4 *>(static_cast<const char *>(packed_dn) + packed_code_bytes(I, (E + 1) * H));
    a.items = reinterpret_cast<const int4 *>(items);
    a.n_items = n_items;
    a.x_rows = (int)A;
    a.x_stride = I;
    a.K = I;
    a.tiles_per_expert = H / 16;
    a.n_experts = E + 1;
    a.n_rows = (int)A;
    const int waves = (int)std::min<size_t>(std::min<size_t>(16, A), moe_max_items(T, E, topk));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (scale_dtype == RLQ_F16)
      moe_down_combine_kernel<8, 0><<<H / 16, 64 * waves, A * 72, st>>>(a, inv, w, T, topk + 1, h, h_stride,
                                                                           nullptr, nullptr, 0);
    else
      moe_down_combine_kernel<8, 1><<<H / 16, 64 * waves, A * 72, st>>>(a, inv, w, T, topk + 1, h, h_stride,
                                                                           nullptr, nullptr, 0);
    RLQ_HIP(hipGetLastError());
    return 0;
  }
  if (int rc = rlq_moe_down(act, I, T, H, I, E, topk, packed_dn, scale_dtype, items, n_items, y, H, stream)) return rc;
  return rlq_moe_combine(y, H, inv, w, T, topk, H, h, h_stride, stream);
}


}  // extern "C"

namespace rlq {

// The scratch of rlq_moe_no_alloc: the workspace of one MoE layer call (routing tables,
// SwiGLU activations, expert outputs) in a file-scope device array. Each GPU the library
// runs on holds its own copy from the first use there until the process ends. 48 MiB
// holds the BASELINE MoE layer up to 512 tokens (rlq_moe_workspace_bytes(512, 256, 8,
// 2048, 512) is 42.5 MB) and any decode batch.
constexpr size_t kMoeScratchBytes = (size_t)48 << 20;
__device__ __align__(256) unsigned char scratch[kMoeScratchBytes];

// The array's device address on the current device, looked up once per device. In host
// code `scratch` names a host-side stand-in, not device memory: only this address may be
// handed to kernels.
constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxScratchDevices];

static int scratch_address(void **out) {
  int dev = -1;
  RLQ_HIP(hipGetDevice(&dev));
  RLQ_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "rlq_moe_no_alloc: device %d is past the %d it supports", dev,
              kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    RLQ_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    RLQ_REQUIRE(p != nullptr && aligned(p, 256), "rlq_moe_no_alloc: no usable scratch address on device %d", dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace rlq

extern "C" {

size_t rlq_moe_no_alloc_max_bytes(void) { return rlq::kMoeScratchBytes; }

int rlq_moe_no_alloc(const void *x, int x_stride, const float *logits, int logit_stride, int T, int E, int topk,
                     int norm_topk, int H, int I, const void *packed_gu, const void *packed_dn, int scale_dtype,
                     float *h, int h_stride, void *stream) {
  using namespace rlq;
  if (int rc = check_moe_shape("rlq_moe_no_alloc", T, E, topk, H, I)) return rc;
  const size_t need = rlq_moe_workspace_bytes(T, E, topk, H, I);
  RLQ_REQUIRE(need <= kMoeScratchBytes,
              "rlq_moe_no_alloc: T=%d E=%d topk=%d H=%d I=%d needs %zu bytes of scratch, more than the %zu it holds "
              "(use rlq_moe with a workspace)", T, E, topk, H, I, need, kMoeScratchBytes);
  void *ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  // rlq_moe needs no initialised workspace: every table and intermediate it reads is
  // written earlier in the same call
  return rlq_moe(x, x_stride, logits, logit_stride, T, E, topk, norm_topk, H, I, packed_gu, packed_dn, scale_dtype, h,
                 h_stride, ws, kMoeScratchBytes, stream);
}

int rlq_moe_linear_native(const void *a, int a_stride, int a_rows, const int *tok, int K, int Ne, const void *packed,
                          const float *s, const int *slots, int n_slots, int book, const int *items, const int *n_items,
                          int max_items, float *c, int c_stride, void *stream) {
  using namespace rlq;
  RLQ_REQUIRE(a && packed && s && slots && items && n_items && c, "rlq_moe_linear_native: null pointer argument");
  RLQ_REQUIRE(book == RLQ_BOOK_INT15 || book == RLQ_BOOK_FP4,
              "rlq_moe_linear_native: book %d (int15 or fp4; the reference's expert kernel has no int16 half step)",
              book);
  RLQ_REQUIRE(K >= kGroup && K % kGroup == 0 && K <= 16 * 24 * kGroup,
              "rlq_moe_linear_native: K=%d must be a multiple of 64 and <= %d", K, 16 * 24 * kGroup);
  RLQ_REQUIRE(Ne >= 16 && Ne % 16 == 0, "rlq_moe_linear_native: Ne=%d must be a multiple of 16", Ne);
  RLQ_REQUIRE(n_slots >= 1 && (long long)n_slots * Ne <= (1LL << 30), "rlq_moe_linear_native: %d slots of %d rows",
              n_slots, Ne);
  RLQ_REQUIRE(a_rows >= 1 && a_stride >= K && a_stride % 8 == 0 && aligned(a, 16) && aligned(packed, 16),
              "rlq_moe_linear_native: a must be 16-byte aligned rows of >= K halves (a_rows=%d a_stride=%d)", a_rows,
              a_stride);
  RLQ_REQUIRE((long long)a_rows * a_stride * 2 < (1LL << 31), "rlq_moe_linear_native: a is too large");
  RLQ_REQUIRE(c_stride >= Ne && max_items >= 0, "rlq_moe_linear_native: c_stride=%d < Ne=%d or max_items=%d",
              c_stride, Ne, max_items);
  RLQ_REQUIRE(aligned(items, 16), "rlq_moe_linear_native: items must be 16-byte aligned");
  if (max_items == 0) return 0;
  const dim3 grid(Ne / 16, max_items);
  const int gpw = expert_gpw(K), threads = 64 * expert_waves(K);
  auto st = static_cast<hipStream_t>(stream);
  auto ah = static_cast<const _Float16 *>(a);
  auto codes = static_cast<const u32x4 *>(packed);
  auto it = reinterpret_cast<const int4 *>(items);
  const bool gather = tok != nullptr;
  if (!gather && K <= kStagedMaxK && a_rows >= 64) {
    // sorted rows in bulk (the down kind of a batch): the staged kernel, whose sub-parts
    // give the per-tile kernel's sums, so the choice does not change a row's bits
    MoeArgs m = {};
    m.x = ah;
    m.codes = codes;
    m.sb = codes;
    m.items = it;
    m.n_items = n_items;
    m.out = c;
    m.x_rows = a_rows;
    m.x_stride = a_stride;
    m.K = K;
    m.tiles_per_expert = Ne / 16;
    m.out_stride = c_stride;
    m.s_row = s;
    m.slots = slots;
    m.n_slots = n_slots;
    m.n_experts = 1 << 30;                     // the slot table's size is the caller's; slots are checked
    m.n_rows = a_rows;
    const int sub = staged_gpw(K) / expert_gpw(K);
    int rc;
    if (staged_gpw(K) == 8)
      rc = book == RLQ_BOOK_INT15 ? launch_staged_inst<8, 0, 1, 1, kInt15>(Ne / 16, st, m, max_items)
                                  : launch_staged_inst<8, 0, 1, 1, kFp4>(Ne / 16, st, m, max_items);
    else if (sub == 2)
      rc = book == RLQ_BOOK_INT15 ? launch_staged_inst<16, 0, 1, 2, kInt15>(Ne / 16, st, m, max_items)
                                  : launch_staged_inst<16, 0, 1, 2, kFp4>(Ne / 16, st, m, max_items);
    else
      rc = book == RLQ_BOOK_INT15 ? launch_staged_inst<16, 0, 1, 1, kInt15>(Ne / 16, st, m, max_items)
                                  : launch_staged_inst<16, 0, 1, 1, kFp4>(Ne / 16, st, m, max_items);
    return rc;
  }
#define RLQ_NATIVE(G, B) \
  launch_native_inst<G, B>(grid, threads, gather, st, ah, a_stride, a_rows, tok, K, Ne, codes, s, slots, n_slots, it, \
                           n_items, c, c_stride)
  if (book == RLQ_BOOK_INT15) {
    if (gpw == 8) RLQ_NATIVE(8, kInt15);
    else if (gpw == 16) RLQ_NATIVE(16, kInt15);
    else RLQ_NATIVE(24, kInt15);
  } else {
    if (gpw == 8) RLQ_NATIVE(8, kFp4);
    else if (gpw == 16) RLQ_NATIVE(16, kFp4);
    else RLQ_NATIVE(24, kFp4);
  }
#undef RLQ_NATIVE
  RLQ_HIP(hipGetLastError());
  return 0;
}

int rlq_moe_swiglu(const float *gu, int gu_stride, int A, int I, const float *cs, void *act, int act_stride,
                   void *stream) {
  using namespace rlq;
  RLQ_REQUIRE(gu && act, "rlq_moe_swiglu: null pointer argument");
  RLQ_REQUIRE(A >= 0 && I >= 1 && gu_stride >= 2 * I && act_stride >= I,
              "rlq_moe_swiglu: A=%d I=%d gu_stride=%d act_stride=%d", A, I, gu_stride, act_stride);
  if (A == 0) return 0;
  moe_swiglu_kernel<<<dim3((I + 255) / 256, A), 256, 0, static_cast<hipStream_t>(stream)>>>(
      gu, gu_stride, A, I, cs, static_cast<_Float16 *>(act), act_stride);
  RLQ_HIP(hipGetLastError());
  return 0;
}


int rlq_moe_gate_up_native(const void *x, int x_stride, int T, const int *tok, int H, int I, const void *packed_gu,
                           const float *s_gu, const int *slots, int n_slots, int book, const int *items,
                           const int *n_items, int max_items, const float *cs, void *act, int act_stride,
                           void *stream) {
  using namespace rlq;
  RLQ_REQUIRE(x && tok && packed_gu && s_gu && slots && items && n_items && act,
              "rlq_moe_gate_up_native: null pointer argument");
  RLQ_REQUIRE(book == RLQ_BOOK_INT15 || book == RLQ_BOOK_FP4,
              "rlq_moe_gate_up_native: book %d (int15 or fp4; the reference's expert kernel has no int16 half step)",
              book);
  RLQ_REQUIRE(H >= kGroup && H % kGroup == 0 && H <= 16 * 24 * kGroup,
              "rlq_moe_gate_up_native: H=%d must be a multiple of 64 and <= %d", H, 16 * 24 * kGroup);
  RLQ_REQUIRE(I >= 16 && I % 16 == 0 && act_stride >= I, "rlq_moe_gate_up_native: I=%d (a multiple of 16), act_stride=%d",
              I, act_stride);
  RLQ_REQUIRE(n_slots >= 1 && (long long)n_slots * 2 * I <= (1LL << 30), "rlq_moe_gate_up_native: %d slots", n_slots);
  RLQ_REQUIRE(T >= 1 && x_stride >= H && x_stride % 8 == 0 && aligned(x, 16) && aligned(packed_gu, 16) &&
                  aligned(items, 16),
              "rlq_moe_gate_up_native: x must be 16-byte aligned rows of >= H halves (T=%d x_stride=%d)", T, x_stride);
  RLQ_REQUIRE((long long)T * x_stride * 2 < (1LL << 31) && max_items >= 0, "rlq_moe_gate_up_native: x is too large");
  if (max_items == 0) return 0;
  const dim3 grid(I / 16, max_items);
  const int gpw = expert_gpw(H), threads = 64 * expert_waves(H);
  auto st = static_cast<hipStream_t>(stream);
  auto xh = static_cast<const _Float16 *>(x);
  auto codes = static_cast<const u32x4 *>(packed_gu);
  auto it = reinterpret_cast<const int4 *>(items);
  auto ah = static_cast<_Float16 *>(act);
#define RLQ_NATIVE_GU(G, B) \
  launch_native_gate_up_inst<G, B>(grid, threads, st, xh, x_stride, T, tok, H, I, codes, s_gu, slots, n_slots, it, \
                                   n_items, cs, ah, act_stride)
  if (book == RLQ_BOOK_INT15) {
    if (gpw == 8) RLQ_NATIVE_GU(8, kInt15);
    else if (gpw == 16) RLQ_NATIVE_GU(16, kInt15);
    else RLQ_NATIVE_GU(24, kInt15);
  } else {
    if (gpw == 8) RLQ_NATIVE_GU(8, kFp4);
    else if (gpw == 16) RLQ_NATIVE_GU(16, kFp4);
    else RLQ_NATIVE_GU(24, kFp4);
  }
#undef RLQ_NATIVE_GU
  RLQ_HIP(hipGetLastError());
  return 0;
}


int rlq_moe_native(const void *x, int x_stride, const float *logits, int logit_stride, int T, int E, int topk,
                   int norm_topk, int H, int I, const void *packed_gu, const float *s_gu, const void *packed_dn,
                   const float *s_dn, const int *slots, int n_slots, int book, const float *cs, float *h,
                   int h_stride, void *workspace, size_t workspace_bytes, void *stream) {
  using namespace rlq;
  if (int rc = check_moe_shape("rlq_moe_native", T, E, topk, H, I)) return rc;
  const size_t need = rlq_moe_workspace_bytes(T, E, topk, H, I);
  RLQ_REQUIRE(workspace && workspace_bytes >= need,
              "rlq_moe_native: workspace of %zu bytes is smaller than the %zu this call needs", workspace_bytes, need);
  RLQ_REQUIRE(aligned(workspace, 256), "rlq_moe_native: workspace must be 256-byte aligned");
  RLQ_REQUIRE(h && h_stride >= H, "rlq_moe_native: h is null or h_stride=%d < H=%d", h_stride, H);
  // the slot-stack bounds of the step-by-step entry points, ahead of the fused paths
  RLQ_REQUIRE(n_slots >= 1 && (long long)n_slots * 2 * I <= (1LL << 30) && (long long)n_slots * H <= (1LL << 30),
              "rlq_moe_native: %d slots of %d gate/up and %d down rows", n_slots, 2 * I, H);
  const size_t A = (size_t)T * (topk + 1);
  char *p = static_cast<char *>(workspace);
  int *sel = reinterpret_cast<int *>(p);            p += align256(A * 4);
  float *w = reinterpret_cast<float *>(p);          p += align256(A * 4);
  int *tok = reinterpret_cast<int *>(p);            p += align256(A * 4);
  int *inv = reinterpret_cast<int *>(p);            p += align256(A * 4);
  int *items = reinterpret_cast<int *>(p);          p += align256((size_t)moe_max_items(T, E, topk) * 16);
  int *n_items = reinterpret_cast<int *>(p);        p += 256;
  _Float16 *act = reinterpret_cast<_Float16 *>(p);  p += align256(A * I * 2);
  float *y = reinterpret_cast<float *>(p);
  const int max_items = moe_max_items(T, E, topk);
  int separate = 1;
  if (T == 1) {
    // one token: routing inside the gate/up launch where a kernel covers the shape
    RLQ_REQUIRE(book == RLQ_BOOK_INT15 || book == RLQ_BOOK_FP4, "rlq_moe_native: book %d (int15 or fp4)", book);
    RLQ_REQUIRE(x && logits && logit_stride >= E + 1 && packed_gu && s_gu && slots && x_stride >= H &&
                    x_stride % 8 == 0 && aligned(x, 16) && aligned(packed_gu, 16) && n_slots >= 1 && I % 16 == 0,
                "rlq_moe_native: bad one-token arguments");
    separate = native_one_token(book, static_cast<const _Float16 *>(x), x_stride, H, I,
                                static_cast<const u32x4 *>(packed_gu), s_gu, slots, n_slots, cs, act, logits, E,
                                topk, norm_topk, sel, w, tok, inv, reinterpret_cast<int4 *>(items), n_items,
                                static_cast<hipStream_t>(stream));
    if (separate < 0) return separate;
  }
  if (separate) {
    if (int rc = rlq_moe_route(logits, logit_stride, T, E, topk, norm_topk, sel, w, tok, inv, items, n_items, stream))
      return rc;
    if (int rc = rlq_moe_gate_up_native(x, x_stride, T, tok, H, I, packed_gu, s_gu, slots, n_slots, book, items,
                                        n_items, max_items, cs, act, I, stream))
      return rc;
  }
  if (T <= kDownCombineTokens && expert_gpw(I) == 8 && I / kGroup <= 8) {
    // a few tokens: down and combine in one launch (the same bits as the two below)
    RLQ_REQUIRE(book == RLQ_BOOK_INT15 || book == RLQ_BOOK_FP4, "rlq_moe_native: book %d", book);
    RLQ_REQUIRE(packed_dn && s_dn && aligned(packed_dn, 16), "rlq_moe_native: down stack null or misaligned");
    MoeArgs a = {};
    a.x = act;
    a.codes = static_cast<const u32x4 *>(packed_dn);
    a.sb = a.codes;
    a.items = reinterpret_cast<const int4 *>(items);
    a.n_items = n_items;
    a.x_rows = (int)A;
    a.x_stride = I;
    a.K = I;
    a.tiles_per_expert = H / 16;
    a.n_experts = E + 1;
    a.n_rows = (int)A;
    const int waves = (int)std::min<size_t>(std::min<size_t>(16, A), moe_max_items(T, E, topk));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (book == RLQ_BOOK_INT15)
      moe_down_combine_kernel<8, 0, kInt15><<<H / 16, 64 * waves, A * 72, st>>>(a, inv, w, T, topk + 1, h, h_stride,
                                                                                s_dn, slots, n_slots);
    else
      moe_down_combine_kernel<8, 0, kFp4><<<H / 16, 64 * waves, A * 72, st>>>(a, inv, w, T, topk + 1, h, h_stride,
                                                                              s_dn, slots, n_slots);
    RLQ_HIP(hipGetLastError());
    return 0;
  }
  if (int rc = rlq_moe_linear_native(act, I, (int)A, nullptr, I, H, packed_dn, s_dn, slots, n_slots, book, items,
                                     n_items, max_items, y, H, stream))
    return rc;
  return rlq_moe_combine(y, H, inv, w, T, topk, H, h, h_stride, stream);
}

}  // extern "C"
