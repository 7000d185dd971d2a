// vtq_kernels.h -- internal launcher interface between the C ABI layer and
// the HIP kernels.  Pointers are device pointers; launches are asynchronous
// on `stream`.  Shapes have been validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vtq {

// Canonical-dot weight formats (8-lane pinned fp32 dot, src/ops/quant.rs:482-566).
enum CanonFormat { kCanonQ8_0 = 0, kCanonQ5_0 = 1, kCanonQ4_0 = 2, kCanonF32 = 3, kCanonQ4KFloat = 4 };

size_t act_lds_bytes(int R);
int kquant_max_in_feat();
int canon_max_in_feat();

hipError_t launch_q4k_gemv(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           int num_cus, hipStream_t stream);
hipError_t launch_q6k_gemv(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           int num_cus, hipStream_t stream);
hipError_t launch_canon_gemv(CanonFormat fmt, const float* x, const uint8_t* w, size_t row_bytes, float* y,
                             int batch, int in_feat, int out_feat, int num_cus, hipStream_t stream);
// Decode-step GEMV (integer regime, Q4_K = 12 / Q6_K = 14, batch 1): the
// output rows are the concatenation of up to three matrices that share x
// (unused slots have rows 0).  Epilogues: store, accumulate into y (the
// residual add), or SwiGLU of two equal-row matrices (y[i] = silu(g_i)*u_i).
// With norm_w set (store and SwiGLU only), x is first replaced by
// rms_norm(x, norm_w, eps) (src/ops/rms_norm.rs:60-110), computed by every
// workgroup from the raw x.
enum RowsEpilogue { kEpiStore = 0, kEpiAccumulate = 1, kEpiSwiGLU = 2 };
struct RowsArgs {
    const uint8_t* w[3];
    int rows[3];
    const float* norm_w = nullptr;
    float eps = 0.0f;
};
bool kquant_fused_supported(int ggml_type, int in_feat, int epi, const RowsArgs& a);
hipError_t launch_kquant_fused(int ggml_type, int epi, const float* x, const RowsArgs& a, float* y, int in_feat,
                               int num_cus, hipStream_t stream);

hipError_t launch_fill(float* y, size_t n, float v, hipStream_t stream);

// Raise `kernel`'s dynamic-LDS limit to at least `bytes` on the current
// device (gfx950 has 160 KiB per CU; the default limit is 64 KiB).  The
// attribute is set once per (device, kernel) and size, not per launch.
hipError_t allow_dynamic_lds(const void* kernel, size_t bytes);

// Prefill GEMM (batch >= kGemmMinBatch): activation pre-pass into `workspace`
// (q4k_gemm_workspace_bytes) followed by the i8-MFMA kernel.
constexpr int kGemmMinBatch = 32;
size_t q4k_gemm_workspace_bytes(int batch, int in_feat);
int q4k_gemm_max_in_feat();
hipError_t launch_q4k_gemm(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           void* workspace, hipStream_t stream);

}  // namespace vtq
