/* Kernel-level C ABI of the MI355X (gfx950) 4-bit group-quantized matmul path.
 *
 * This is the drop-in boundary for raceline's quantized linear and mixture-of-experts
 * matmuls. In the reference these are reached through Engine::encode_linear and
 * Engine::encode_moe (src/engine.mm:832-906, :965-1071), which bind Metal buffers and
 * dispatch kernels/linear.metal and kernels/moe.metal with the POD parameter blocks of
 * kernels/params.h:6-32. Here the same operations are plain C functions over device
 * pointers, so an engine, ctypes (raceline/engine.py:67-125 style) or a test can call them.
 *
 * Conventions
 *  - Every pointer argument is device memory (hipMalloc'd or a torch CUDA tensor), except
 *    where a comment says host. The library allocates nothing: scratch space is passed in
 *    as `workspace`, sized by the matching *_workspace_bytes() query.
 *  - `stream` is a hipStream_t (NULL: the default stream). Calls are asynchronous.
 *  - Weight layout "MLX affine" (tools/convert.py:82-89, the BASELINE configs): codes
 *    uint32 [N][K/8], element k of row n at bits 4*(k%8).. of word k/8; scales and biases
 *    [N][K/64] 16-bit floats (RLQ_F16 or RLQ_BF16). Dequantized weight:
 *      W[n][k] = float(s[n][k/64]) * q[n][k] + float(b[n][k/64])     (kernels/linear.metal:3-4)
 *  - Errors: by default an error prints "raceline: fatal: <message>" and exits with status 1,
 *    as every error of the reference does (src/metal_rt.mm:16-24, src/capi.h:12-15).
 *    rlq_set_fatal(0) switches this thread to returning a nonzero status instead, with the
 *    message in rlq_last_error(); the Python layer does that and raises.
 */
#ifndef RLQ_H
#define RLQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { RLQ_F16 = 0, RLQ_BF16 = 1 };  /* 16-bit float type of scales and biases */

/* ---------------------------------------------------------------- library */

/* ABI version of this header (bumped on any signature change). */
int rlq_abi_version(void);
/* 1: errors are fatal (default, as in the reference); 0: return a status. Returns the old value. */
int rlq_set_fatal(int on);
/* Message of the last failed call on this thread ("" if none). */
const char *rlq_last_error(void);
/* Selects the GPU for this thread's later calls (hipSetDevice). */
int rlq_set_device(int device);

/* ---------------------------------------------------------------- packed weights */

/* The kernels read weights in a packed device layout made once at upload (the reference maps
 * its file without a copy, src/model_file.mm:89-100; MI355X has to upload it, and does so into
 * the layout its kernels stream best). For T = ceil(N/16) tiles of 16 rows, G = K/64 groups
 * padded to G4 = ceil(G/4) quads, and group pairs p (groups 2p, 2p+1):
 *   codes:       T*2*G4 kilobytes; the kilobyte of (tile t, pair p) holds, for lane l = 16j + c
 *                (j = 0..3, c = 0..15), four uint32 words of row 16t + c: word 8g + 4s + j for
 *                (g, s) = (2p,0), (2p,1), (2p+1,0), (2p+1,1), in MLX nibble order (element k at
 *                bits 4*(k%8) of word k/8);
 *   scale/bias:  after the codes, T*G4*16 entries of 16 bytes, ((t*G4 + q)*16 + c): for groups
 *                4q .. 4q+3, s bits | b bits << 16;
 * rows beyond N and groups beyond G are zero. Total rlq_packed_affine_bytes(K, N) =
 * T*G4*2304 bytes: exactly K*N/2 + 4*N*K/64 when N % 16 == 0 and K % 256 == 0. */
size_t rlq_packed_affine_bytes(int K, int N);

/* MLX layout -> packed. Replaces the affine part of tools/convert.py's pack_blocked
 * (:92-117) as the producer of the kernels' layout. */
int rlq_pack_affine(const uint32_t *w, const void *s, const void *b, int K, int N, void *packed, void *stream);

/* Blocked q4a file layout (tools/convert.py:92-117: bytes [n_pad/256][K][128], 16-bit s and b
 * [n_pad/256][K/64][256]) rows [row0, row0+rows) -> packed matrix of N = rows, e.g. one part of
 * a stacked tensor (src/model_file.h:52, QTensor::parts). */
int rlq_pack_affine_blocked(const uint8_t *w_blk, const uint16_t *s_blk, const uint16_t *b_blk,
                            int K, int n_pad, int row0, int rows, void *packed, void *stream);

/* Blocked q4a file layout -> MLX layout (the interchange format), rows [row0, row0+rows). */
int rlq_repack_blocked(const uint8_t *w_blk, const uint16_t *s_blk, const uint16_t *b_blk,
                       int K, int n_pad, int row0, int rows,
                       uint32_t *w, uint16_t *s, uint16_t *b, void *stream);

/* ---------------------------------------------------------------- dense affine linear */

/* Bytes of scratch rlq_linear_affine needs for these sizes (0 for the decode kernel; the
 * prefill kernel stages the activations' group sums there). Contents need no initialisation
 * and are not kept between calls; calls that share one workspace must not overlap. */
size_t rlq_linear_workspace_bytes(int M, int K, int N);

/* y[m][n] = sum_k x[m][k] * W[n][k]   (accum = 0)
 * y[m][n] += that                      (accum = 1: the residual add, ACCUM in the reference)
 * x: fp16 [M][x_stride]; W packed as above; y: fp32 [M][y_stride]. K % 64 == 0, M, N >= 1.
 * Replaces group_sums + linear_q4a (kernels/linear.metal:34-116, dispatched by
 * src/engine.mm:875-905). M <= 8 runs the decode kernel (MFMA GEMV), larger M the prefill
 * kernel (LDS-staged MFMA GEMM). */
int rlq_linear_affine(const void *x, int x_stride, int M, int K, int N,
                      const void *packed, int scale_dtype,
                      float *y, int y_stride, int accum,
                      void *workspace, size_t workspace_bytes, void *stream);

/* Forces one kernel family for tests and measurement: 0 = automatic, 1 = decode GEMV
 * (M <= 8), 2 = prefill GEMM. Same contract as rlq_linear_affine. */
int rlq_linear_affine_kernel(int kernel, const void *x, int x_stride, int M, int K, int N,
                             const void *packed, int scale_dtype,
                             float *y, int y_stride, int accum,
                             void *workspace, size_t workspace_bytes, void *stream);

/* gsum[m][g] = sum_{k<64} x[m][64g+k], summed in order in fp32 (kernels/linear.metal:34-45). */
int rlq_group_sums(const void *x, int x_stride, int M, int K, float *gsum, void *stream);

/* W[n][k] as fp32 [N][K] from a packed matrix, bit-exact to float(s)*q + float(b). A checking
 * entry point: the matmuls never materialise W. */
int rlq_dequant_affine(const void *packed, int scale_dtype, int K, int N, float *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RLQ_H */
