/*
 * vtq_runtime.h -- C ABI of libvtq_runtime, the end-to-end decode driver
 * that calls libvtq for every linear layer.
 *
 * It replaces the reference's quantized inference entry points:
 *   inference::run_quantized            src/model/inference.rs:274-345
 *   forward_quantized::step             src/model/forward_quantized.rs:288-655
 *   GgufFile::parse / Config::from_gguf src/model/gguf.rs:305-421,
 *                                       src/model/config.rs:156-213
 *   QuantizedWeights::from_gguf         src/model/quant_weights.rs:121-181
 *   blake3::hash of the GGUF blob       src/bin/vitni-receipt.rs:31
 * with the same results bit for bit: logits of every decode step, the
 * generated tokens and the `vitnify-receipt v2` model digest
 * (src/cert/builder.rs:458-471).
 *
 * The GGUF blob is parsed on the host once (every length, count and offset
 * checked as the reference checks them; a malformed file never reaches the
 * device) and each tensor the step reads is uploaded to device memory once.
 * The whole decode step runs on the GPU: the embedding row, RMSNorm, the
 * linears (the libvtq kernels, with the k-quant GEMVs of a layer fused: q|k|v
 * in one launch, the residual adds into Wo and W2, SwiGLU into W1|W3), RoPE,
 * attention over the KV cache and the argmax, in the reference's operation
 * order.  Activations, the KV cache, the token sequence and the step
 * position stay in device memory; one step is captured once in a HIP graph
 * and replayed per position, and the host reads the tokens (and the logits
 * history, when asked for) once at the end.
 *
 * Status codes are those of include/vtq.h; vtqrt_last_error() gives text.
 */
#ifndef VTQ_RUNTIME_H
#define VTQ_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct vtqrt_model vtqrt_model;

/* GgufFile::parse (level 0: src/model/gguf.rs:305-421), or the parse plus
 * Config::from_gguf and QuantizedWeights::from_gguf (level 1:
 * src/model/config.rs:156-213, src/model/quant_weights.rs:121-181), on the
 * host only: no device is touched, so it runs without a GPU.  Returns VTQ_OK
 * or the status of the first check that fails (VTQ_E_MALFORMED /
 * VTQ_E_TRUNCATED / VTQ_E_OVERFLOW for the file, VTQ_E_INTERNAL for the
 * model tables, as the reference's Error variants) with the reference's
 * text in err (optional, NUL-terminated, at most err_cap bytes).  dims
 * (optional, level 1) receives dim, hidden, layers, heads, kv_heads, vocab,
 * seq_len.  vtqrt_load runs the same checks first. */
int vtqrt_parse(const uint8_t *gguf, size_t len, int level, int dims[7], char *err, size_t err_cap);

/* Parse a GGUF v2/v3 blob (vtqrt_parse level 1) and upload the tensors the
 * decode step reads to HIP device `device`.  The blob is copied; the caller
 * may free it afterwards.  On failure *out still holds a model whose
 * vtqrt_last_error() explains it; free it with vtqrt_free. */
int vtqrt_load(int device, const uint8_t *gguf, size_t len, vtqrt_model **out);
void vtqrt_free(vtqrt_model *m);
const char *vtqrt_last_error(const vtqrt_model *m);
/* dim, hidden, layers, heads, kv_heads, vocab, seq_len */
int vtqrt_dims(const vtqrt_model *m, int dims[7]);

/* rms_norm_slice (src/ops/rms_norm.rs:60-110) on device memory: d_y[i] =
 * d_x[i] * scale * d_w[i], scale = 1 / sqrt(sum(x*x) / n + eps) with the
 * sum of squares in the reference's serial order, enqueued on `stream` (a
 * hipStream_t on the current device, NULL for the null stream).  The decode
 * step uses the same sum (fused into the GEMV that consumes the norm).
 * 1 <= n <= 32768; d_x, d_w, d_y 4-byte aligned. */
int vtqrt_rms_norm_device(const float *d_x, const float *d_w, size_t n, float eps, float *d_y, void *stream);

/* The single-precision libm functions the decode step evaluates on the
 * device (the `libm = "0.2"` crate's expf, sqrtf, cosf, sinf, powf; RoPE,
 * softmax, SwiGLU and RMSNorm call them, src/model/forward_quantized.rs:
 * 423-559, src/ops/rms_norm.rs:102), over d_x[0..n): d_y[7i + k] = f_k(d_x[i])
 * for the seven evaluations of the reference's transcendental sweep in its
 * order (tests/transcendental_determinism.rs:34-42): expf(x), sqrtf(|x|),
 * cosf(x), sinf(x), powf(1e4, x/64), powf(1e6, x/64), 1/(1+expf(-x)).
 * Enqueued on `stream`; it exists so the device code can be pinned by the
 * reference's PINNED_TRANSCENDENTAL hash.  n < 2^31 / 7. */
int vtqrt_transcendentals_device(const float *d_x, size_t n, float *d_y, void *stream);

/* inference::run_quantized.  regime: VTQ_REGIME_INTEGER (std-parallel
 * build) or VTQ_REGIME_FLOAT_FUSED (default build) for the Q4_K arm.
 * logits (optional) receives (prompt_len + n_new) * vocab floats, one row per
 * decode step; tokens receives the n_new generated ids; digest the
 * `vitnify-receipt v2` model digest (compute_digest, src/cert/builder.rs:
 * 458-471); digest_v1 (optional) the frozen `vitnify-receipt v1` digest of
 * the same cert (compute_digest_v1, :476-487), which vitni-receipt prints
 * as model_digest_v1 (src/bin/vitni-receipt.rs:40-55).  weights_hash is
 * BLAKE3 of the whole GGUF blob (vtqrt_blake3).  Errors, in the reference's
 * order: VTQ_E_INVALID_SHAPE for an empty prompt or prompt_len + n_new past
 * seq_len; then what step 0 would report (embedding_row's texts, a norm
 * weight of the wrong length as VTQ_E_SHAPE_MISMATCH, each linear's
 * linear_dispatch error); then a prompt or generated token past the
 * embedding table.  Nothing is launched until these checks pass.
 * digest_v1 arrived in ABI 0.2.0 (vtq_version); NULL skips it. */
int vtqrt_run(vtqrt_model *m, int regime, const char *model_id, const uint8_t weights_hash[32],
              const uint32_t *prompt, int prompt_len, int n_new, float *logits, uint32_t *tokens,
              uint8_t digest[32], uint8_t digest_v1[32]);

/* How vtqrt_run processes the prompt.  VTQRT_PROMPT_BATCHED (the default):
 * positions 0 .. prompt_len-1 in one pass, every linear over all prompt
 * rows at once (the prefill GEMM for Q4_K), then the decode steps from
 * position prompt_len; where the pass's attention does not fit in LDS (a
 * position's scores and one tile of cached rows: prompts beyond about 39,800
 * positions at head_dim 64), or with a one-token prompt, it steps as below.  VTQRT_PROMPT_STEPWISE: one
 * forward_quantized::step per position, as run_quantized's loop
 * (src/model/inference.rs:313-329).  Both give the same tokens, digests and
 * logits bit for bit: the reference's batch rows are independent, and each
 * position's norm, cache write and attention are its own step's.
 * vtqrt_run_recorded always steps.  No counterpart in the reference (its
 * loop only steps); added in ABI 0.3.0. */
#define VTQRT_PROMPT_BATCHED 0
#define VTQRT_PROMPT_STEPWISE 1
int vtqrt_set_prompt_mode(vtqrt_model *m, int mode);

/* run_quantized with a PerOpRecorder and/or a PerActivationRecorder attached
 * to every step (src/model/forward_quantized.rs:64-132, :260-284,
 * step_with_recorders :329-655): per op, BLAKE3 of its f32 input and output
 * and of its weights (hash_f32_slice for norms); per checkpoint (post_embed,
 * post_attn, post_ffn, pre_lm_head, post_lm_head) BLAKE3 of the residual
 * stream.  The records enter the v2 digest in declaration order
 * (src/cert/builder.rs:251-305, :489-560).  op_name is "rms_norm" or
 * "linear_q4_0" (the reference's name for every linear); layer is
 * 0xFFFFFFFF for the model-level ops.  ops / acts (optional) receive up to
 * *_cap records, *n_ops / *n_acts the counts (9*layers + 2 and
 * 2*layers + 3 per step). */
#define VTQRT_RECORD_OPS 1
#define VTQRT_RECORD_ACTIVATIONS 2
typedef struct {
    uint32_t op_index, layer;
    char op_name[16];
    uint8_t input_hash[32], params_hash[32], output_hash[32];
} vtqrt_op_record;
typedef struct {
    uint32_t act_index, token_index, layer;
    char checkpoint[16];
    uint8_t tensor_hash[32];
} vtqrt_act_record;
int vtqrt_run_recorded(vtqrt_model *m, int regime, const char *model_id, const uint8_t weights_hash[32],
                       const uint32_t *prompt, int prompt_len, int n_new, int flags, uint32_t *tokens,
                       vtqrt_op_record *ops, size_t ops_cap, vtqrt_act_record *acts, size_t acts_cap,
                       size_t *n_ops, size_t *n_acts, uint8_t digest[32]);

/* BLAKE3-256 (crate blake3 = "1" as the reference uses it). */
void vtqrt_blake3(const void *data, size_t len, uint8_t out[32]);

#ifdef __cplusplus
}
#endif
#endif
