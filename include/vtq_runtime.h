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
 * The GGUF blob is parsed once and uploaded to device memory once; every
 * linear runs on the GPU through vtq_linear_device (include/vtq.h) on
 * device-resident weights.  The rest of the step (embedding row, RMSNorm,
 * RoPE, attention over the KV cache, SwiGLU, argmax) runs on the host in
 * the reference's operation order.
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

/* Parse a GGUF v2/v3 blob and upload it to HIP device `device`.  The blob is
 * copied; the caller may free it afterwards. */
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

/* inference::run_quantized.  regime: VTQ_REGIME_INTEGER (std-parallel
 * build) or VTQ_REGIME_FLOAT_FUSED (default build) for the Q4_K arm.
 * logits (optional) receives (prompt_len + n_new) * vocab floats, one row per
 * decode step; tokens receives the n_new generated ids; digest the v2 model
 * digest.  weights_hash is BLAKE3 of the whole GGUF blob (vtqrt_blake3). */
int vtqrt_run(vtqrt_model *m, int regime, const char *model_id, const uint8_t weights_hash[32],
              const uint32_t *prompt, int prompt_len, int n_new, float *logits, uint32_t *tokens,
              uint8_t digest[32]);

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
