/*
 * vtq.h -- C ABI of libvtq, the MI355X (gfx950) backend for vitni-tensor's
 * quantized linear layer.
 *
 * The reference seam is the uniform Rust signature every dtype arm of
 * `linear_dispatch` calls (src/model/forward_quantized.rs:663-785), e.g.
 *
 *   pub fn linear_q4_k_integer(x: &[f32], w_q4k: &[u8], y_out: &mut [f32],
 *                              batch: usize, in_feat: usize, out_feat: usize)
 *       -> Result<()>                                  (src/ops/quant.rs:936-943)
 *
 * Each entry point below replaces one such function (citation on each) with
 * the same argument meaning: x[batch][in_feat] f32 row-major, w the GGUF
 * blocks of W[out_feat][in_feat] row-major, y[batch][out_feat] f32, all
 * outputs written.  Results are bit-identical to the reference CPU path.
 * Slices become (pointer, length) pairs; lengths are checked here where the
 * reference would panic on a short slice.
 *
 * Status codes mirror vitni_tensor::error::Error (src/error.rs:7-63):
 *   VTQ_OK                 Ok(())
 *   VTQ_E_INTERNAL         Error::Internal(&'static str)  (shape/length;
 *                          vtq_last_error() returns the reference's text)
 *   VTQ_E_GPU              Error::GpuError                (HIP failure)
 *   VTQ_E_NOT_IMPLEMENTED  Error::NotImplemented          (F16/other dtypes; a
 *                          request beyond the no-alloc entry point's scratch)
 *   VTQ_E_INVALID_ARGUMENT null pointer or context; Rust's types rule these out
 *   VTQ_E_MALFORMED        Error::Malformed               (GGUF parse, libvtq_runtime)
 *   VTQ_E_TRUNCATED        Error::Truncated               (GGUF parse, libvtq_runtime)
 *   VTQ_E_OVERFLOW         Error::Overflow                (GGUF parse, libvtq_runtime)
 *   VTQ_E_SHAPE_MISMATCH   Error::ShapeMismatch           (a norm weight whose length
 *                          is not the model dimension, rms_norm.rs:80-85)
 *   VTQ_E_INVALID_SHAPE    Error::InvalidShape            (empty prompt, prompt + new
 *                          tokens past seq_len, inference.rs:301-311)
 * No entry point aborts or panics.
 *
 * Threading: a context is used by one host thread at a time (the reference's
 * Accelerator takes &mut self, src/accel/mod.rs:82).  Contexts on different
 * threads are independent.
 */
#ifndef VTQ_H
#define VTQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VTQ_OK 0
#define VTQ_E_INTERNAL 1
#define VTQ_E_GPU 2
#define VTQ_E_NOT_IMPLEMENTED 3
#define VTQ_E_INVALID_ARGUMENT 4
#define VTQ_E_MALFORMED 5
#define VTQ_E_TRUNCATED 6
#define VTQ_E_OVERFLOW 7
#define VTQ_E_SHAPE_MISMATCH 8
#define VTQ_E_INVALID_SHAPE 9

/* GGUF tensor type tags (src/model/gguf.rs:127-139). */
#define VTQ_TYPE_F32 0
#define VTQ_TYPE_F16 1
#define VTQ_TYPE_Q4_0 2
#define VTQ_TYPE_Q5_0 6
#define VTQ_TYPE_Q8_0 8
#define VTQ_TYPE_Q4_K 12
#define VTQ_TYPE_Q6_K 14

/* Numerical regime of the Q4_K arm, chosen by a Cargo feature in the
 * reference (src/model/forward_quantized.rs:704-725):
 *   VTQ_REGIME_INTEGER      `std-parallel` build: linear_q4_k_integer[_parallel]
 *   VTQ_REGIME_FLOAT_FUSED  default build:        linear_q4_k_fused
 * All other dtypes compute the same bits in both regimes. */
#define VTQ_REGIME_INTEGER 0
#define VTQ_REGIME_FLOAT_FUSED 1

typedef struct vtq_ctx vtq_ctx;

/* Create a context bound to HIP device `device`.  Replaces constructing the
 * reference's accelerator value (CpuAccelerator, src/accel/mod.rs:102-120). */
int vtq_create(int device, vtq_ctx **out);
void vtq_destroy(vtq_ctx *ctx);
/* Text of the last error on this context ("" after success); for
 * VTQ_E_INTERNAL it is the reference's Error::Internal message. */
const char *vtq_last_error(const vtq_ctx *ctx);
/* Library version string, "vtq <major>.<minor>.<patch> (gfx950)".  It names
 * the ABI of this header and of vtq_runtime.h together; 0.2.0 added the
 * trailing digest_v1 argument of vtqrt_run (a caller built against 0.1.0
 * headers must not load this library); 0.3.0 added vtqrt_set_prompt_mode
 * (no existing signature changed). */
const char *vtq_version(void);

/* ---- host-pointer entry points (synchronous; y is complete on return) ----
 * x, w, y are host memory owned by the caller.  w is uploaded once and cached
 * on the device keyed by (pointer, length): the reference's weights are
 * zero-copy views into a GGUF blob that lives for the model's lifetime
 * (src/model/quant_weights.rs:47-52), so the bytes behind a cached key must
 * not change until vtq_release_weights() drops it. */

/* src/model/forward_quantized.rs:663-785 linear_dispatch, for any batch. */
int vtq_linear(vtq_ctx *ctx, int ggml_type, int regime, const float *x, size_t x_len,
               const uint8_t *w, size_t w_len, float *y, size_t y_len, size_t batch,
               size_t in_feat, size_t out_feat);

/* src/ops/quant.rs:936-980 linear_q4_k_integer (and its row-parallel twin
 * :1149-1196, which computes the same bits). */
int vtq_linear_q4_k_integer(vtq_ctx *ctx, const float *x, size_t x_len, const uint8_t *w,
                            size_t w_len, float *y, size_t y_len, size_t batch, size_t in_feat,
                            size_t out_feat);
/* src/ops/quant.rs:1060-1096 linear_q6_k_integer (twin :1099-1146). */
int vtq_linear_q6_k_integer(vtq_ctx *ctx, const float *x, size_t x_len, const uint8_t *w,
                            size_t w_len, float *y, size_t y_len, size_t batch, size_t in_feat,
                            size_t out_feat);
/* src/ops/quant.rs:1433-1453 linear_q4_k_fused (twin :1386-1430). */
int vtq_linear_q4_k_fused(vtq_ctx *ctx, const float *x, size_t x_len, const uint8_t *w,
                          size_t w_len, float *y, size_t y_len, size_t batch, size_t in_feat,
                          size_t out_feat);
/* src/ops/quant.rs:1529-1565 linear_q4_0_cpu (exact-length checks kept). */
int vtq_linear_q4_0(vtq_ctx *ctx, const float *x, size_t x_len, const uint8_t *w, size_t w_len,
                    float *y, size_t y_len, size_t batch, size_t in_feat, size_t out_feat);

/* Drop the device copy cached for host weight pointer w (any length), or
 * every cached weight when w is NULL. */
int vtq_release_weights(vtq_ctx *ctx, const uint8_t *w);

/* ---- device-pointer entry point (asynchronous) ----
 * Same computation as vtq_linear, but d_x, d_w, d_y are device memory on the
 * context's device and the work is enqueued on `stream` (a hipStream_t, NULL
 * for the null stream) without synchronising.  d_x and d_w must be 16-byte
 * aligned, and d_w readable up to the next multiple of 16 bytes past w_len
 * (every hipMalloc or torch device allocation is: the kernels fetch whole
 * 16-byte chunks and ignore the bytes past the blob).  This is what a device-resident forward step calls; it replaces
 * the same linear_dispatch arm as vtq_linear.  Calls that overlap in time on
 * one context race on the context's workspace. */
int vtq_linear_device(vtq_ctx *ctx, int ggml_type, int regime, const float *d_x,
                      const uint8_t *d_w, size_t w_len, float *d_y, size_t batch, size_t in_feat,
                      size_t out_feat, void *stream);

/* ---- allocation-free device entry point ----
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same computation, arguments and
 * errors as vtq_linear_device, but it calls no hipMalloc / hipFree: the
 * prefill GEMM's workspace (the quantized activations, batch >= 32 on Q4_K
 * in the integer regime) lives in a fixed 32 MiB array on each GPU,
 * allocated when the library loads.  Requests whose workspace would exceed
 * it (vtq::q4k_gemm_workspace_bytes: about batch x in_feat x 1.14 bytes,
 * batch capped at 8192 per chunk) return VTQ_E_NOT_IMPLEMENTED with a
 * message and launch nothing.  Rows longer than the kernels hold (k-quant
 * beyond 32768 inputs, the canonical dot beyond 65536) keep their
 * segments' sums there too (segments x batch x out_feat x 4 bytes, plus one
 * gathered segment of x per batch row for the canonical dot), with the
 * batch split into passes that fit; a single batch row that does not fit
 * is refused the same way.  All calls on one GPU share that array:
 * calls that overlap in time on one device (any context, any stream) race
 * on it and must be serialised by the caller.  Every byte a call reads from
 * the array is written earlier in the same call, so nothing needs clearing
 * between calls. */
int vtq_linear_device_noalloc(vtq_ctx *ctx, int ggml_type, int regime, const float *d_x,
                              const uint8_t *d_w, size_t w_len, float *d_y, size_t batch,
                              size_t in_feat, size_t out_feat, void *stream);

#ifdef __cplusplus
}
#endif
#endif
