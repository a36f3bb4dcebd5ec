// The prefill GEMM of the 4-bit formats (gemm.hip), called by the entry points of
// linear.hip, and the small activation-sum kernels it shares with them.
#pragma once

#include "rlq_common.h"

namespace rlq {

struct GemmArgs {
  const _Float16 *x;    // affine: the prepped activations [M][K]; native: x [M][x_stride]
  const u32x4 *codes;
  const u32x4 *sb;      // affine: scale/bias quads
  const uint16_t *gs;   // affine: the group sums' pieces, fp16 or bf16 bits [M][gs_stride]
  const float *srow;    // native books: row scales [N]
  const float *asum;    // kInt16: activation row sums [M]
  const float *rscale;  // affine: 2^-e per row, undoing the prep pass's prescale [M]
  float *y;
  float *y_part;        // split K: splits 1 .. S-1's partial products [S-1][M][N]
  int *cnt;             // split K: arrivals per output tile (zero between calls)
  int x_stride, M, K, N, y_stride, gs_stride;
  int np_split;         // group pairs per split (all of them when not split)
};

// Output tiles of one prefill launch whose K is split can count their arrivals in the
// workspace's counter bytes (see rlq_linear_workspace_bytes); larger calls launch in row
// chunks.
constexpr int kGemmMaxCounters = 1024;

// Bytes of workspace run_gemm4 needs (affine: the prepped activations and the split group
// sums; kInt16: group and row sums; a shape whose K is split: the partial products).
size_t gemm4_workspace(int book, int M, int K, int N);

// codes, sbq: the two sections of a packed matrix (q4_tile.h), or of rows [r0, r0 + N) of a
// larger one (r0 a multiple of 16: see packed_tile_offsets in linear.h). cnt: the
// kGemmMaxCounters arrival counters at the start of the linear workspace (zero).
int run_gemm4(int book, const _Float16 *x, int x_stride, int M, int K, int N, const void *codes, const void *sbq, int sd,
              const float *srow, float *y, int y_stride, int accum, int *cnt, void *ws, size_t ws_bytes,
              hipStream_t st);

// defined in linear.hip
void launch_group_sums(const _Float16 *x, int x_stride, int M, int K, float *gsT, int m_pad, hipStream_t st);
void launch_row_sums(const float *gsT, int G, int m_pad, int M, float *asum, hipStream_t st);

}  // namespace rlq
