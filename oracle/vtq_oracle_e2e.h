/*
 * vtq_oracle_e2e.h -- CPU restatement of the reference's end-to-end decode
 * path around the quantized linears (config 5).  TEST INFRASTRUCTURE ONLY:
 * the checker for the GPU runtime, never linked into the product.
 *
 *  - Rust `libm = "0.2"` single-precision functions used by the forward
 *    step (expf, powf, sinf, cosf; sqrtf is IEEE), restated from the
 *    FreeBSD msun algorithms the crate ports.  Pinned by the reference's
 *    PINNED_TRANSCENDENTAL hash (tests/transcendental_determinism.rs:62-63).
 *  - BLAKE3 (crate `blake3 = "1"`), restated from the published
 *    specification.  Pinned by the empty-input test vector and the
 *    reference's v2 digest pin (src/cert/builder.rs:719-741).
 *  - `vitnify-receipt v2` digest (src/cert/builder.rs:440-597).
 *  - GGUF v2/v3 parsing (src/model/gguf.rs:305-421), Config::from_gguf
 *    (src/model/config.rs:156-213), QuantizedWeights::from_gguf
 *    (src/model/quant_weights.rs:121-181).
 *  - forward_quantized::step (src/model/forward_quantized.rs:288-655) and
 *    inference::run_quantized (src/model/inference.rs:274-345).
 */
#ifndef VTQ_ORACLE_E2E_H
#define VTQ_ORACLE_E2E_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- libm (Rust libm 0.2, FreeBSD msun algorithms) ---- */
float vtqo_expf(float x);
float vtqo_powf(float x, float y);
float vtqo_sinf(float x);
float vtqo_cosf(float x);
float vtqo_sqrtf(float x);

/* ---- BLAKE3 ---- */
typedef struct {
    uint32_t cv[8];
    uint64_t chunk_counter;
    uint8_t block[64];
    uint8_t block_len;
    uint8_t blocks_compressed;
    uint32_t cv_stack[54][8];
    uint8_t cv_stack_len;
} vtqo_blake3;
void vtqo_blake3_init(vtqo_blake3 *h);
void vtqo_blake3_update(vtqo_blake3 *h, const void *data, size_t len);
void vtqo_blake3_final(const vtqo_blake3 *h, uint8_t out[32]);
void vtqo_blake3_hash(const void *data, size_t len, uint8_t out[32]);

/* BLAKE3 over every f32 result of the reference's transcendental sweep
 * (tests/transcendental_determinism.rs:14-63). Returns the input count. */
size_t vtqo_transcendental_hash(uint8_t out[32]);

/* `vitnify-receipt v2` digest of inputs/outputs (no op/activation records):
 * names[i] NUL-terminated, data[i]/lens[i] the field bytes. */
void vtqo_digest_v2(int n_in, const char *const *in_names, const uint8_t *const *in_data, const size_t *in_lens,
                    int n_out, const char *const *out_names, const uint8_t *const *out_data,
                    const size_t *out_lens, uint8_t out[32]);

/* ---- model + decode ---- */
typedef struct vtqo_model vtqo_model;
/* Status codes of the model functions, as the reference's Error variants
 * (the numbering of include/vtq.h): 1 Internal, 3 NotImplemented,
 * 5 Malformed, 6 Truncated, 7 Overflow, 8 ShapeMismatch, 9 InvalidShape. */

/* GgufFile::parse (level 0, src/model/gguf.rs:305-421), plus
 * Config::from_gguf and QuantizedWeights::from_gguf (level 1).  0 or the
 * status of the first failing check, with the reference's text in msg. */
int vtqo_gguf_parse(const uint8_t *blob, size_t len, int level, const char **msg);
/* Parse a GGUF blob (borrowed; must outlive the model): vtqo_gguf_parse
 * level 1.  0 on success, a status with msg set otherwise. */
int vtqo_model_load(const uint8_t *blob, size_t len, vtqo_model **out, const char **msg);
void vtqo_model_free(vtqo_model *m);
/* dim, hidden, layers, heads, kv_heads, vocab, seq_len */
void vtqo_model_dims(const vtqo_model *m, int dims[7]);

/* inference::run_quantized: regime 0 = std-parallel integer Q4_K,
 * 1 = float-fused Q4_K.  logits (may be NULL) receives
 * (prompt_len + n_new) * vocab floats, one row per decode step.
 * tokens receives n_new ids; digest the v2 model digest, digest_v1 (may be
 * NULL) the v1 digest of the same cert.  weights_hash is BLAKE3 of the whole
 * GGUF blob.  0 on success, a status with msg set otherwise. */
int vtqo_run_quantized(const vtqo_model *m, int regime, const char *model_id, const uint8_t weights_hash[32],
                       const uint32_t *prompt, int prompt_len, int n_new, int threads, float *logits,
                       uint32_t *tokens, uint8_t digest[32], uint8_t digest_v1[32], const char **msg);

/* PerOp / activation receipts (src/model/forward_quantized.rs:64-132,
 * :260-284; src/cert/builder.rs:251-305, :489-560).  op_name is
 * "rms_norm" or "linear_q4_0" (the reference's name for every linear);
 * layer is 0xFFFFFFFF for the model-level ops and checkpoints. */
#define VTQO_RECORD_OPS 1
#define VTQO_RECORD_ACTIVATIONS 2
typedef struct {
    uint32_t op_index, layer;
    char op_name[16];
    uint8_t input_hash[32], params_hash[32], output_hash[32];
} vtqo_op_record;
typedef struct {
    uint32_t act_index, token_index, layer;
    char checkpoint[16];
    uint8_t tensor_hash[32];
} vtqo_act_record;

/* compute_digest_v2 with op and activation sections (no interventions) */
void vtqo_digest_v2_full(int n_in, const char *const *in_names, const uint8_t *const *in_data, const size_t *in_lens,
                         int n_out, const char *const *out_names, const uint8_t *const *out_data,
                         const size_t *out_lens, size_t n_ops, const vtqo_op_record *ops, size_t n_acts,
                         const vtqo_act_record *acts, uint8_t out[32]);

/* compute_digest_v1 (src/cert/builder.rs:476-487): the frozen v1 domain, no
 * regime, the same sections */
void vtqo_digest_v1_full(int n_in, const char *const *in_names, const uint8_t *const *in_data, const size_t *in_lens,
                         int n_out, const char *const *out_names, const uint8_t *const *out_data,
                         const size_t *out_lens, size_t n_ops, const vtqo_op_record *ops, size_t n_acts,
                         const vtqo_act_record *acts, uint8_t out[32]);

/* run_quantized's cert with a PerOpRecorder and/or a PerActivationRecorder
 * attached to every step (flags: VTQO_RECORD_*).  ops / acts (optional)
 * receive up to *_cap records; *n_ops / *n_acts the counts. */
int vtqo_run_quantized_recorded(const vtqo_model *m, int regime, const char *model_id,
                                const uint8_t weights_hash[32], const uint32_t *prompt, int prompt_len, int n_new,
                                int threads, int flags, uint32_t *tokens, vtqo_op_record *ops, size_t ops_cap,
                                vtqo_act_record *acts, size_t acts_cap, size_t *n_ops, size_t *n_acts,
                                uint8_t digest[32], const char **msg);

/* forward-step helpers, exported for their known-answer tests */
void vtqo_rms_norm(const float* x, const float* w, int n, float eps, float* out);
void vtqo_softmax(float* x, int n);
uint32_t vtqo_argmax(const float* v, int n);

#ifdef __cplusplus
}
#endif
#endif
