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
/* Codebooks of the native 4-bit format (tools/quantlib.py:23-28): two's complement -8..7,
 * the same plus 0.5, and fp4 e2m1. */
enum { RLQ_BOOK_INT15 = 1, RLQ_BOOK_INT16 = 2, RLQ_BOOK_FP4 = 3 };

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

/* Bytes of scratch rlq_linear_affine and rlq_linear_native need for these sizes (and for
 * any smaller M). The first 4096 bytes hold the decode kernel's counters for weights whose
 * K it splits across workgroups (few tiles, long K: the down projections); they must be
 * zero before the workspace's first use, and every call leaves them zero; the prefill
 * kernel counts in the same bytes for weights whose K it splits in two (at most 32 blocks of
 * 256 outputs and 64 pairs of groups or more, such as the 27B down projection). The rest
 * holds the decode kernel's partial sums for such weights, or the prefill kernel's prepared
 * activations and group sums (and, for a weight whose K it splits, the second half's
 * partial products), and is not kept between calls. Calls that share one
 * workspace must not overlap. Pass NULL and 0 only where this query returns 0. */
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

/* ---------------------------------------------------------------- native 4-bit linear */

/* The native ("q4n") format: a 4-bit codebook value per weight, one fp32 scale per output
 * row and one per input column, W[n][k] = L[q[n][k]] * s[n] * c[k] (tools/quantlib.py:62-64,
 * tools/convert.py:197-216). The column scale is folded into the activations by whichever
 * kernel produces them (src/engine.mm:515-530), as in the reference; the kernels apply s.
 * Codes are packed into the same tile layout as the affine codes, without the scale/bias
 * section: rlq_packed_codes_bytes(K, N) = T*G4*2048 bytes. */
size_t rlq_packed_codes_bytes(int K, int N);

/* Row-major codes, uint32 [N][K/8] with element k at bits 4*(k%8) -> packed codes. */
int rlq_pack_codes(const uint32_t *w, int K, int N, void *packed, void *stream);

/* Blocked q4n file layout (bytes [n_pad/256][K][128], tools/convert.py:197-216) rows
 * [row0, row0+rows) -> packed codes. */
int rlq_pack_native_blocked(const uint8_t *w_blk, int K, int n_pad, int row0, int rows, void *packed, void *stream);

/* y[m][n] (+)= s_row[n] * sum_k x[m][k] * L[q[n][k]]  (+ 0.5 * sum_k x[m][k] inside the row
 * scale for RLQ_BOOK_INT16). Replaces linear_q4n (kernels/linear.metal:118-184). x fp16
 * [M][x_stride] (column scale already applied); s_row fp32 [N]; y fp32 [M][y_stride]. The
 * workspace (rlq_linear_workspace_bytes) is used for M > 8 by RLQ_BOOK_INT16 and by weights
 * whose K the prefill kernel splits. */
int rlq_linear_native(const void *x, int x_stride, int M, int K, int N, const void *packed, const float *s_row,
                      int book, float *y, int y_stride, int accum, void *workspace, size_t workspace_bytes,
                      void *stream);
int rlq_linear_native_kernel(int kernel, const void *x, int x_stride, int M, int K, int N, const void *packed,
                             const float *s_row, int book, float *y, int y_stride, int accum, void *workspace,
                             size_t workspace_bytes, void *stream);

/* y[m][n] = sum_k x[m][k] * L[q[n][k]]: the native product without the row scale (or any
 * other epilogue), as linear_q4n_raw computes it to measure what linear_q4n's epilogue costs
 * (kernels/linear.metal:226-252). book RLQ_BOOK_INT15 or RLQ_BOOK_FP4 (that kernel's W_T has
 * no half step); other arguments as rlq_linear_native. */
int rlq_linear_native_raw(const void *x, int x_stride, int M, int K, int N, const void *packed, int book, float *y,
                          int y_stride, void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------- dense fp16 linear */

/* Half-precision matrices (the MoE router, the MTP head's input projection) in MFMA
 * operand order: rlq_packed_f16_bytes(K, N) = ceil(N/16) * (K/32) * 1024 bytes, K % 32 == 0. */
size_t rlq_packed_f16_bytes(int K, int N);
/* Row-major fp16 [N][K] -> packed. */
int rlq_pack_f16(const void *w, int K, int N, void *packed, void *stream);
/* Blocked f16b file layout ([n_pad/256][K][256] halves, tools/convert.py:218-226) rows
 * [row0, row0+rows) -> packed. */
int rlq_pack_f16_blocked(const void *w_blk, int K, int n_pad, int row0, int rows, void *packed, void *stream);
/* y[m][n] (+)= sum_k x[m][k] * W[n][k], fp32 accumulation. Replaces linear_f16
 * (kernels/linear.metal:186-225). x fp16 [M][x_stride]; y fp32 [M][y_stride]. */
int rlq_linear_f16(const void *x, int x_stride, int M, int K, int N, const void *packed, float *y, int y_stride,
                   int accum, void *stream);

/* gsum[m][g] = sum_{k<64} x[m][64g+k], summed in order in fp32 (kernels/linear.metal:34-45). */
int rlq_group_sums(const void *x, int x_stride, int M, int K, float *gsum, void *stream);

/* W[n][k] as fp32 [N][K] from a packed matrix, bit-exact to float(s)*q + float(b). A checking
 * entry point: the matmuls never materialise W. */
int rlq_dequant_affine(const void *packed, int scale_dtype, int K, int N, float *out, void *stream);

/* Reads `bytes` bytes of device memory at p as a plain stream (16-byte non-temporal loads from
 * every CU, nothing else), the read rate this device gives a kernel that only streams: the
 * context for the decode kernels' fraction of the 8 TB/s peak. out (one float) is written only
 * for data no real buffer holds. p 16-byte aligned, bytes a multiple of 16. A measurement
 * helper with no counterpart in the reference (its bench/hw/gpu_probe.py:33-103 plays this
 * part on Apple GPUs). */
int rlq_stream_read(const void *p, size_t bytes, float *out, void *stream);

/* ---------------------------------------------------------------- mixture of experts */

/* A MoE MLP of E routed experts plus one shared expert (number E), each a gate/up matrix
 * [2I][H] (I gate rows, then I up rows) and a down matrix [H][I], stacked over the E + 1
 * experts as the reference stacks them (tools/quantize.py:168-228, shared expert last):
 * gate_up [(E+1)*2I][H], down [(E+1)*H][I], 4-bit affine with groups of 64. A token goes
 * to its topk best experts and the shared one: S = topk + 1 assignments, a = t*S + slot.
 * Replaces Engine::encode_moe (src/engine.mm:965-1059) with kernels/moe.metal and
 * linear_q4n_moe (kernels/linear.metal:254-308) for the affine format. Sizes: E <= 1023,
 * topk <= 16, H and I multiples of 64 up to 24576. */

/* The gate/up stack (MLX layout, codes [(E+1)*2I][H/8], s and b [(E+1)*2I][H/64]) ->
 * packed, with each expert's gate and up rows interleaved 8 and 8 per 16-row tile (so one
 * tile yields both halves of SwiGLU). Bytes: rlq_packed_affine_bytes(H, (E+1)*2I). The
 * down stack is packed with rlq_pack_affine(w, s, b, I, (E+1)*H, ...). */
int rlq_pack_moe_gate_up(const uint32_t *w, const void *s, const void *b, int H, int E1, int I, void *packed,
                         void *stream);

/* Upper bound on the work items of a call (size of `items`, in units of 4 ints). */
size_t rlq_moe_max_items(int T, int E, int topk);

/* Routing (kernels/moe.metal:40-140). logits fp32 [T][logit_stride], columns 0..E-1 the
 * router's, column E the shared expert's gate. Writes, for a = t*S + slot:
 *   sel[a], w[a]  the expert and weight of each assignment: slots 0..topk-1 the chosen
 *                 experts in falling order of logit (equal logits: lower expert first),
 *                 weights softmax over all E logits, renormalised over the chosen ones
 *                 when norm_topk; slot topk the shared expert, weight sigmoid(logit[E]);
 *   tok[r], inv[a] the counting sort by expert: sorted row r holds token tok[r], and
 *                 assignment a is sorted row inv[a]; within an expert, rows in token order;
 *   items         (expert, first row, rows <= 16, 0) per work item, experts ascending;
 *   *n_items      their number (device memory).
 * sel, w, tok, inv: T*S entries; items: rlq_moe_max_items(T, E, topk) * 4 ints, 16-byte aligned. */
int rlq_moe_route(const float *logits, int logit_stride, int T, int E, int topk, int norm_topk, int *sel, float *w,
                  int *tok, int *inv, int *items, int *n_items, void *stream);

/* act[r][i] = half(silu(g) * u) for every sorted row r, where (g, u) = x[tok[r]] times the
 * gate and up rows i of the row's expert (kernels/ops.metal:446-455 with unit column
 * scales, as for affine matrices, src/engine.mm:937-940). x fp16 [T][x_stride]; act fp16
 * [T*S][act_stride]. The gather of kernels/moe.metal:143-155 is fused (rows are read
 * through tok). */
int rlq_moe_gate_up(const void *x, int x_stride, int T, int H, int I, int E, int topk, const void *packed_gu,
                    int scale_dtype, const int *tok, const int *items, const int *n_items, void *act, int act_stride,
                    void *stream);

/* y[r][d] = act[r] times down row d of the row's expert, fp32 [T*S][y_stride]. */
int rlq_moe_down(const void *act, int act_stride, int T, int H, int I, int E, int topk, const void *packed_dn,
                 int scale_dtype, const int *items, const int *n_items, float *y, int y_stride, void *stream);

/* h[t][d] += sum over slots s (in order) of w[t*S+s] * y[inv[t*S+s]][d]
 * (kernels/moe.metal:157-174). */
int rlq_moe_combine(const float *y, int y_stride, const int *inv, const float *w, int T, int topk, int H, float *h,
                    int h_stride, void *stream);

/* The whole MoE MLP: route, gate/up + SwiGLU, down, combine into h (fp32 [T][h_stride],
 * accumulated like the reference's residual stream). The workspace holds the routing,
 * act and y; rlq_moe_workspace_bytes sizes it (256-byte aligned, no initialisation). */
size_t rlq_moe_workspace_bytes(int T, int E, int topk, int H, int I);
int rlq_moe(const void *x, int x_stride, const float *logits, int logit_stride, int T, int E, int topk, int norm_topk,
            int H, int I, const void *packed_gu, const void *packed_dn, int scale_dtype, float *h, int h_stride,
            void *workspace, size_t workspace_bytes, void *stream);

/* rlq_moe without a workspace argument. It has no counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops
 * and harnesses that forbid hipMalloc). Its scratch is a static device array of
 * rlq_moe_no_alloc_max_bytes() bytes (48 MiB: the BASELINE MoE layer up to 512 tokens) that
 * each GPU holds from the library's first use there until the process ends; a call whose
 * rlq_moe_workspace_bytes exceeds it fails with an error. The call allocates nothing. Every
 * call on one GPU shares that array, so calls that overlap on one GPU (two streams or two
 * threads) race; calls in order on one stream do not. Same results as rlq_moe. */
size_t rlq_moe_no_alloc_max_bytes(void);
int rlq_moe_no_alloc(const void *x, int x_stride, const float *logits, int logit_stride, int T, int E, int topk,
                     int norm_topk, int H, int I, const void *packed_gu, const void *packed_dn, int scale_dtype,
                     float *h, int h_stride, void *stream);

/* ---------------------------------------------------------------- native experts */

/* The experts of one kind (gate_up or down) in the native format, one launch: replaces
 * linear_q4n_moe (kernels/linear.metal:254-308; MoeLinearParams, kernels/params.h:28-31),
 * which src/engine.mm:1019-1048 dispatches twice per MoE layer. The matrices sit in
 * n_slots slots of Ne rows each (the stacked tensor, slot = expert, or an expert cache),
 * packed together with rlq_pack_codes(w, K, n_slots*Ne, ...) or rlq_pack_native_blocked,
 * with one fp32 scale per row s[n_slots*Ne]. For work item i < *n_items of
 * items[max_items][4] = (e, r0, rows, 0) (rlq_moe_route writes them):
 *   c[r0+j][n] = s[slot*Ne + n] * (a[src(r0+j)] . L(q[slot*Ne + n])^T),  slot = slots[e],
 * for j < rows and n < Ne, with src(r) = tok[r] (a holds the T tokens: the gather of
 * kernels/moe.metal:143-155 fused) or, tok == NULL, src(r) = r (a holds sorted rows, as
 * act does). a fp16 [a_rows][a_stride], already multiplied by the matrix's column scale
 * (the reference folds it upstream); c fp32 [.][c_stride]. book: RLQ_BOOK_INT15 or
 * RLQ_BOOK_FP4 (the reference's W_T for experts; its expert kernel has no int16 half
 * step, so RLQ_BOOK_INT16 is refused). A slot outside [0, n_slots) gives zero rows.
 * K a multiple of 64 up to 24576, Ne a multiple of 16. */
int rlq_moe_linear_native(const void *a, int a_stride, int a_rows, const int *tok, int K, int Ne, const void *packed,
                          const float *s, const int *slots, int n_slots, int book, const int *items, const int *n_items,
                          int max_items, float *c, int c_stride, void *stream);

/* The native gate/up product with the SwiGLU folded in: for the items as above and the
 * stacked gate_up tensor of n_slots slots of 2I rows (gate rows [0, I), up rows [I, 2I)),
 *   act[r][i] = half(silu(g) * u * cs[i]),  g = gu-product row i, u = row I + i,
 * the same bits as rlq_moe_linear_native (tok given) followed by rlq_moe_swiglu, in one
 * launch and without the fp32 gate/up rows. x fp16 [T][x_stride] (the tokens, read
 * through tok); act fp16 [T*S][act_stride]; cs as for rlq_moe_swiglu. I a multiple of 16. */
int rlq_moe_gate_up_native(const void *x, int x_stride, int T, const int *tok, int H, int I, const void *packed_gu,
                           const float *s_gu, const int *slots, int n_slots, int book, const int *items,
                           const int *n_items, int max_items, const float *cs, void *act, int act_stride,
                           void *stream);

/* The whole native MoE MLP in one call (Engine::encode_moe, src/engine.mm:965-1059, for
 * native files): route, gate/up with the gather and the SwiGLU, down, combine into h (fp32
 * [T][h_stride], accumulated). Stacks as for rlq_moe_gate_up_native (gate_up: n_slots
 * slots of 2I rows, K = H) and rlq_moe_linear_native (down: n_slots slots of H rows,
 * K = I); slots [E+1]; cs the down matrix's column scale or NULL. The workspace is the
 * one rlq_moe_workspace_bytes(T, E, topk, H, I) sizes (256-byte aligned, no
 * initialisation). Up to four tokens the down product and the combine run as one launch,
 * with the same bits as the step-by-step entry points. */
int rlq_moe_native(const void *x, int x_stride, const float *logits, int logit_stride, int T, int E, int topk,
                   int norm_topk, int H, int I, const void *packed_gu, const float *s_gu, const void *packed_dn,
                   const float *s_dn, const int *slots, int n_slots, int book, const float *cs, float *h,
                   int h_stride, void *workspace, size_t workspace_bytes, void *stream);

/* act[r][i] = half(silu(gu[r][i]) * gu[r][I + i] * cs[i]) for r < A, i < I: the SwiGLU of
 * kernels/ops.metal:446-455 between the native gate_up and down products. cs is the down
 * matrix's column scale (fp32 [I]; NULL means ones, as for affine matrices). gu fp32
 * [A][gu_stride >= 2I]; act fp16 [A][act_stride]. */
int rlq_moe_swiglu(const float *gu, int gu_stride, int A, int I, const float *cs, void *act, int act_stride,
                   void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RLQ_H */
