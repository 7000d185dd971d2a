/*
 * vtq_oracle.h -- CPU restatement of vitni-tensor's quantized linear path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT.  This library is the checker that the HIP
 * backend (libvtq) is compared against.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it.  libvtq never links it and has
 * no CPU fallback.
 *
 * Every function restates one Rust function of the reference crate
 * vitni-tensor 0.2.1 (the citation is on each declaration, path:line relative
 * to the reference root).  The reference is Rust and no Rust toolchain exists
 * in this image, so the reference itself cannot be built; this restatement is
 * pinned instead by the reference's own published constants and known-answer
 * tests (see tests/test_oracle_pins.py).
 *
 * Numerics: every float operation is one separately rounded IEEE binary32
 * operation, evaluated in source order, as in the Rust reference (Rust never
 * contracts a*b+c into an FMA).  The Makefile builds with -ffp-contract=off
 * -fno-fast-math; x86-64 SSE evaluates float in float (FLT_EVAL_METHOD 0).
 *
 * Status codes mirror the reference's Result: 0 = Ok, 1 = Error::Internal,
 * 3 = Error::NotImplemented.  On error *msg (when non-null) receives the
 * reference's &'static str verbatim.
 */
#ifndef VTQ_ORACLE_H
#define VTQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VTQO_OK 0
#define VTQO_E_INTERNAL 1
#define VTQO_E_NOT_IMPLEMENTED 3

/* src/ops/quant.rs:452, :457 */
#define VTQO_CANON_LANES 8
#define VTQO_CANON_CHUNK 8192

/* src/ops/quant.rs:738-743 */
typedef struct vtqo_q8block {
    float d;
    int8_t qs[256];
    int32_t bsums[8];
} vtqo_q8block;

/* src/ops/quant.rs:40-66 */
float vtqo_f16_to_f32(uint16_t half);
/* Same, returned as raw bits (a float return value would be quieted by callers' conversions). */
uint32_t vtqo_f16_to_f32_bits(uint16_t half);
/* src/ops/quant.rs:68-83 (the reference's truncating encoder, used by its tests) */
uint16_t vtqo_f32_to_f16(float f);

/* src/ops/quant.rs:461-476 */
float vtqo_fixed_tree(float *part, size_t n);
/* src/ops/quant.rs:482-505 */
float vtqo_canonical_chunk(const float *x, const float *w, size_t n);
/* src/ops/quant.rs:547-566 */
float vtqo_canonical_dot(const float *x, const float *w, size_t n);
/* src/ops/quant.rs:572-574 */
float vtqo_canonical_combine(float *chunk_sums, size_t n);
/* src/ops/quant.rs:579-608 (test-only regime-2 order) */
float vtqo_canonical_dot_regime2(const float *x, const float *w, size_t n);

/* src/ops/quant.rs:91-111, :160-186, :193-210, :280-319, :337-386.
 * out must hold (len/block_bytes)*block_numel floats. */
int vtqo_dequantize_q4_0(const uint8_t *w, size_t len, float *out, const char **msg);
int vtqo_dequantize_q5_0(const uint8_t *w, size_t len, float *out, const char **msg);
int vtqo_dequantize_q8_0(const uint8_t *w, size_t len, float *out, const char **msg);
int vtqo_dequantize_q4_k(const uint8_t *w, size_t len, float *out, const char **msg);
int vtqo_dequantize_q6_k(const uint8_t *w, size_t len, float *out, const char **msg);
/* src/ops/quant.rs:115-150, :213-241 (encoders used by the reference's tests) */
int vtqo_quantize_q4_0(const float *x, size_t n, uint8_t *out, const char **msg);
int vtqo_quantize_q8_0(const float *x, size_t n, uint8_t *out, const char **msg);

/* src/ops/quant.rs:750-771 (n <= 256) */
void vtqo_quantize_block_q8(const float *x, size_t n, vtqo_q8block *out);
/* src/ops/quant.rs:849-898 */
float vtqo_dot_q4k_q8_block(const uint8_t *w, const vtqo_q8block *xq, size_t n);
/* src/ops/quant.rs:995-1057 */
float vtqo_dot_q6k_q8_block(const uint8_t *w, const vtqo_q8block *xq, size_t n);
/* src/ops/quant.rs:904-928 */
int vtqo_integer_dot_q4k(const float *x, const uint8_t *w, size_t w_len, size_t n,
                         float *out, const char **msg);
/* src/ops/quant.rs:616-702 */
int vtqo_canonical_dot_q4k_fused(const float *x, const uint8_t *w, size_t w_len, size_t n,
                                 float *out, const char **msg);
/* src/ops/quant.rs:1212-1300 */
int vtqo_canonical_dot_q6k_fused(const float *x, const uint8_t *w, size_t w_len, size_t n,
                                 float *out, const char **msg);

/* Linear layers: y[batch][out_feat] = x[batch][in_feat] . W[out_feat][in_feat]^T.
 * threads <= 1 selects the serial function; otherwise the row-parallel twin
 * with the reference's grain max(1, ceil(out_feat / (4*threads))).
 * src/ops/quant.rs:936-980 / :1149-1196 */
int vtqo_linear_q4_k_integer(const float *x, const uint8_t *w, size_t w_len, float *y,
                             size_t batch, size_t in_feat, size_t out_feat, int threads,
                             const char **msg);
/* src/ops/quant.rs:1060-1096 / :1099-1146 */
int vtqo_linear_q6_k_integer(const float *x, const uint8_t *w, size_t w_len, float *y,
                             size_t batch, size_t in_feat, size_t out_feat, int threads,
                             const char **msg);
/* src/ops/quant.rs:1433-1453 / :1386-1430 */
int vtqo_linear_q4_k_fused(const float *x, const uint8_t *w, size_t w_len, float *y,
                           size_t batch, size_t in_feat, size_t out_feat, int threads,
                           const char **msg);
/* src/ops/quant.rs:1304-1327 / :1331-1369 */
int vtqo_linear_q6_k_fused(const float *x, const uint8_t *w, size_t w_len, float *y,
                           size_t batch, size_t in_feat, size_t out_feat, int threads,
                           const char **msg);
/* src/ops/quant.rs:1456-1482, :1485-1511 (dequantize whole matrix, then canonical dot) */
int vtqo_linear_q4_k_cpu(const float *x, size_t x_len, const uint8_t *w, size_t w_len,
                         float *y, size_t y_len, size_t batch, size_t in_feat,
                         size_t out_feat, const char **msg);
int vtqo_linear_q6_k_cpu(const float *x, size_t x_len, const uint8_t *w, size_t w_len,
                         float *y, size_t y_len, size_t batch, size_t in_feat,
                         size_t out_feat, const char **msg);
/* src/ops/quant.rs:1529-1565 */
int vtqo_linear_q4_0_cpu(const float *x, size_t x_len, const uint8_t *w, size_t w_len,
                         float *y, size_t y_len, size_t batch, size_t in_feat,
                         size_t out_feat, const char **msg);

/* src/model/forward_quantized.rs:663-785 (linear_dispatch), generalised from
 * the reference's batch = 1 to any batch by treating rows independently as
 * the per-dtype kernels already do (src/ops/quant.rs:952-978).
 * ggml_type: 0 F32, 1 F16, 2 Q4_0, 6 Q5_0, 8 Q8_0, 12 Q4_K, 14 Q6_K (src/model/gguf.rs:127-139).
 * regime 0 = std-parallel build (integer Q4_K), regime 1 = default build
 * (float-fused Q4_K).  threads as above; the reference uses the parallel
 * twins only for out_feat >= 512 (forward_quantized.rs:710, :734). */
int vtqo_linear_dispatch(int ggml_type, int regime, const float *x, size_t x_len,
                         const uint8_t *w, size_t w_len, float *y, size_t y_len,
                         size_t batch, size_t in_feat, size_t out_feat, int threads,
                         const char **msg);

/* src/ops/matmul.rs:30-129: rank-2 f32 matmul through canonical_dot with the
 * rhs column gathered.  a[m][k], b[k][n], out[m][n]. */
void vtqo_matmul_f32(const float *a, const float *b, float *out, size_t m, size_t k, size_t n);

#ifdef __cplusplus
}
#endif
#endif
