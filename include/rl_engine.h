/* Engine layer of the MI355X (gfx950) build over .rlm model files: the model file reader,
 * the upload of a model's matrices to HBM in the kernels' packed layouts, and the engine
 * steps on the quantized matmul path (Engine::encode_linear / encode_mlp / encode_moe and
 * the output head, src/engine.mm:824-1071,1425-1458,1634-1638), behind the reference's
 * rl_* C API where it has a counterpart (src/capi.h).
 *
 * Conventions are those of include/rlq.h: device pointers unless a comment says host, a
 * hipStream_t argument (NULL: the default stream), errors fatal by default ("raceline:
 * fatal: ..." and exit status 1, src/capi.h:12-15) or returned with rlq_set_fatal(0).
 * The engine allocates its device memory at rl_open (the weights, its scratch) and frees
 * it at rl_close; the engine steps take the caller's residual stream h.
 */
#ifndef RL_ENGINE_H
#define RL_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- model file (host only) */

/* The .rlm reader alone (src/model_file.mm:28-137; no GPU work): maps the file and parses
 * its header. Fails (fatal by default; NULL otherwise) on the reference's cases: a file
 * that is not "RLM1", a header that is not valid JSON, a missing config or quant field, an
 * unsupported mixture of experts or rotation, a section past the end of the file; and on a
 * header or tensor that reaches past the end of the file. */
typedef struct rlm_file rlm_file;
rlm_file *rlm_open(const char *path);
void rlm_close(rlm_file *f);

/* A config value by its header name ("hidden_size", "num_hidden_layers", "vocab_size",
 * "num_experts", "num_experts_per_tok", "moe_intermediate_size", "norm_topk_prob",
 * "intermediate_size", "head_dim", "eos_token_id"; "block", "group", "native" from the quant
 * object; "version"; "sections": their count). -1 for a name it does not know. */
int rlm_config_int(const rlm_file *f, const char *key);

/* Tensor kinds (tools/convert.py:165-250): q4a, q4n, q4a_rows, q4n_rows, f16b, f32. */
enum { RLM_Q4A = 1, RLM_Q4N = 2, RLM_Q4A_ROWS = 3, RLM_Q4N_ROWS = 4, RLM_F16B = 5, RLM_F32 = 6 };

/* One entry of the tensor table (src/model_file.h:40-62): absolute file offsets of the
 * codes (or halves, or floats) w, scales s, biases b and column scales c; for f32 tensors
 * w is the data's offset and n its element count. */
typedef struct {
  int kind, section, k, n, n_pad, n_parts;
  uint64_t w, s, b, c;
} rlm_tensor_info;
int rlm_tensor(const rlm_file *f, const char *name, rlm_tensor_info *out);
/* Rows of one part of a stacked tensor (QTensor::part_offset, src/model_file.mm:11-15). */
int rlm_tensor_part(const rlm_file *f, const char *name, const char *part, int *offset, int *rows);
int rlm_section(const rlm_file *f, int index, uint64_t *offset, uint64_t *nbytes);

/* ---------------------------------------------------------------- engine (src/capi.h) */

typedef struct rl_engine rl_engine;

/* Opens a .rlm model (src/capi.h:16-19): reads it, checks the geometry the engine supports
 * (src/engine.mm:394-396) and the codebook of native files (:516), and uploads every blocked
 * matrix (q4a, q4n, f16b) and float tensor to the current GPU, packed for the kernels
 * (affine matrices through rlq_pack_affine_blocked, expert stacks with their gate/up rows
 * interleaved, native codes through rlq_pack_native_blocked); for native files the norm
 * weights are folded with the column scales of the matrices they feed (engine.mm:517-530).
 * max_chunk bounds the rows of one engine step; max_ctx is kept for the reference's
 * signature (the attention cache is not part of this build). */
rl_engine *rl_open(const char *model_path, int max_ctx, int max_chunk);
void rl_close(rl_engine *e);
int rl_vocab(const rl_engine *e);                 /* src/capi.h:21 */
int rl_hidden_size(const rl_engine *e);           /* src/capi.h:98 */

/* Engine::encode_linear (src/engine.mm:832-906) on a named tensor of the model: out[r][n]
 * (+= with accum) sum_k x[r][k] W[n][k] for rows r < rows, dispatched on the tensor's kind:
 * q4a (affine, rlq_linear_affine's kernels), q4n (native codebook: x already carries the
 * matrix's column scale, as the engine's normed rows do), f16b (half). part: NULL for the
 * whole stacked tensor, or the name of one part (its first row must be a multiple of 16).
 * x fp16 [rows][x_stride]; out fp32 [rows][out_stride]. */
int rl_linear(rl_engine *e, const char *tensor, const char *part, const void *x, int x_stride, int rows, float *out,
              int out_stride, int accum, void *stream);

/* Engine::encode_norm (src/engine.mm:908-917, kernels/ops.metal:74-112): xn[r][i] =
 * half(h[r][i] * rsqrt(mean_i h[r]^2 + eps) * w[i]) for the layer's input norm (which 0),
 * its post-attention norm (1) or the final norm (2, layer ignored); for native files w is
 * the norm weight times the column scales of the matrix the norm feeds. h fp32
 * [rows][h_stride]; xn fp16 [rows][xn_stride]. A row's result does not depend on rows. */
int rl_norm(rl_engine *e, int which, int layer, const float *h, int h_stride, int rows, void *xn, int xn_stride,
            void *stream);

/* Engine::encode_mlp / encode_moe (src/engine.mm:943-1059): h[t] += MLP(norm_post(h[t])) for
 * t < T <= max_chunk, the layer's dense SwiGLU MLP (gate_up, SwiGLU with the down matrix's
 * column scale, down with ACCUM) or its mixture of experts (router, routing, experts, combine;
 * affine experts through rlq_moe, native ones through rlq_moe_native). h fp32 [T][h_stride]. */
int rl_mlp(rl_engine *e, int layer, float *h, int h_stride, int T, void *stream);

/* The output head (src/engine.mm:1634-1638): the final norm of rows [0, rows) of h
 * (rows <= 16) and lm_head over them, into the engine's logits (device memory, row r at
 * r * rl_logits_stride() floats; the first rl_vocab() of a row are the vocabulary's).
 * Returns that device pointer, or NULL on error in non-fatal mode. */
const float *rl_head(rl_engine *e, const float *h, int h_stride, int rows, void *stream);

/* The draft head's vocabulary (src/capi.h:75-84, src/engine.mm:1425-1458): the drafts see
 * token ids below rl_draft_main() (rl_set_draft_vocab: a multiple of 256 rows, 0 = all),
 * followed by the ids from rl_draft_tail() on (rl_set_draft_tail: the block holding that
 * id; -1 = none). */
void rl_set_draft_vocab(rl_engine *e, int rows);
void rl_set_draft_tail(rl_engine *e, int first);
int rl_draft_main(const rl_engine *e);
int rl_draft_tail(const rl_engine *e);
int rl_draft_vocab(const rl_engine *e);
size_t rl_logits_stride(const rl_engine *e);

/* src/capi.h:79-83: the expert cache of a mixture of experts kept on disk. This engine
 * keeps every expert resident in device memory, so it has none: rl_expert_cache returns 0
 * slots with *hits = *loads = 0, and rl_expert_cache_size gives 0 experts of 0 bytes, as
 * the reference reports for an engine without a cache (src/engine.mm:364-365). Null
 * pointers are allowed. */
int rl_expert_cache(const rl_engine *e, unsigned long long *hits, unsigned long long *loads);
void rl_expert_cache_size(const rl_engine *e, int *experts, unsigned long long *slot_bytes);

/* The head over the draft vocabulary for one row of h (the logits part of
 * Engine::encode_mtp_layer, src/engine.mm:1419-1436): the RMS norm, lm_head rows
 * [0, rl_draft_main()) and, when a tail is set, rows [rl_draft_tail(), n_pad) right after
 * them: rl_draft_vocab() logits in the engine's draft logits (device memory). The norm is
 * the reference's for the row: mtp.norm folded with lm_head's column scales in a native
 * file with an MTP head (src/engine.mm:534); in a file without one, final_norm (this
 * engine's extension: the reference has no draft head there). A rotated file with an MTP
 * head is refused (its rotation kernel is not on this path). */
const float *rl_draft_head(rl_engine *e, const float *h_row, void *stream);

/* The k largest of n logits in descending order, ties to the lowest index, NaN skipped
 * (src/capi.h:88-93; src/capi.mm:74-101): host memory, returns how many it wrote. */
int rl_top_k(const float *logits, int n, int k, int32_t *ids, float *vals);

/* rl_top_k over n device logits, on the GPU: ids and vals (host) receive the result; the
 * call waits for the stream. k <= 256, n <= 16 * rl_logits_stride() (the engine's logits
 * buffer). Same order and ties as rl_top_k. */
int rl_top_k_device(rl_engine *e, const float *logits, int n, int k, int32_t *ids, float *vals, void *stream);

/* src/capi.h:39: the index of the largest of the first rl_vocab() logits of row 0 of the last
 * rl_head call (the lowest index among equal ones). Runs on the stream that rl_head call ran
 * on (which must still exist), and waits for it. */
int rl_argmax(const rl_engine *e);

#ifdef __cplusplus
}
#endif

#endif /* RL_ENGINE_H */
