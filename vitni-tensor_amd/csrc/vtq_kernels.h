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
hipError_t launch_fill(float* y, size_t n, float v, hipStream_t stream);

// Prefill GEMM (batch >= kGemmMinBatch): activation pre-pass into `workspace`
// (q4k_gemm_workspace_bytes) followed by the i8-MFMA kernel.
constexpr int kGemmMinBatch = 32;
size_t q4k_gemm_workspace_bytes(int batch, int in_feat);
int q4k_gemm_max_in_feat();
hipError_t launch_q4k_gemm(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           void* workspace, hipStream_t stream);

}  // namespace vtq
