// The quantized linear over packed weights, for callers inside the library (the engine
// layer): the entry points of include/rlq.h take a whole packed matrix; these take its two
// sections separately, so that a row range of a matrix (the output head's draft rows) runs
// without a copy.
#pragma once

#include "q4_tile.h"

namespace rlq {

// Byte offsets of 16-row tile t in the code and scale/bias sections of a packed matrix of
// K inputs (include/rlq.h): rows [16 t, ...) of the matrix start there in each section.
inline size_t packed_tile_code_offset(int K, int t) { return (size_t)t * quads_of(K) * 2048; }
inline size_t packed_tile_sb_offset(int K, int t) { return (size_t)t * quads_of(K) * 256; }

// y (+)= x W^T for the packed matrix (or row range) whose sections start at codes and sbq
// (sbq unused for native books, whose row scales are srow). kernel: 0 automatic, 1 decode,
// 2 prefill; book: kAffine or a native codebook; sd: RLQ_F16 / RLQ_BF16. Arguments are
// the caller's to check (the entry points of linear.hip do).
int linear_packed(int kernel, int book, const _Float16 *x, int x_stride, int M, int K, int N, const void *codes,
                  const void *sbq, int sd, const float *srow, float *y, int y_stride, int accum, void *ws,
                  size_t ws_bytes, hipStream_t st);

// A dense MLP's gate/up product with the SwiGLU fused, for an affine packed matrix of 2I
// rows (gate rows [0, I), up rows [I, 2I)): act[m][i] = half(silu(g[m][i]) * u[m][i]) with
// g, u the rows of x W^T, the same bits as linear_packed followed by the SwiGLU kernel.
// For the decode sizes (M <= 8) whose K the decode kernel covers with 8 groups per wave
// and no K split; returns 1 (nothing launched) for other shapes, 0 when launched.
int linear_swiglu_packed(const _Float16 *x, int x_stride, int M, int K, int I, const void *codes, const void *sbq,
                         int sd, _Float16 *act, int act_stride, hipStream_t st);

}  // namespace rlq
