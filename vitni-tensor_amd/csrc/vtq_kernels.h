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
    // A row segment of a longer matrix: bytes between consecutive weight
    // rows and floats between consecutive batch rows of x (0: the dense
    // R * block bytes and R * 256 of an unsegmented launch).
    uint32_t row_stride = 0;
    int x_stride = 0;
};
bool kquant_fused_supported(int ggml_type, int in_feat, int epi, const RowsArgs& a);
hipError_t launch_kquant_fused(int ggml_type, int epi, const float* x, const RowsArgs& a, float* y, int in_feat,
                               int num_cus, hipStream_t stream);

hipError_t launch_fill(float* y, size_t n, float v, hipStream_t stream);

// Rows longer than the kernels hold (k-quant: kquant_max_in_feat(); the
// canonical dot: canon_max_in_feat()) run as aligned segments of that many
// inputs, each writing its own y slice; fixed_tree over the segments'
// sums then gives the row's value, because the reference's pairwise tree
// only pairs blocks (chunks) inside an aligned power-of-two group before it
// pairs the groups' sums.
// One k-quant segment (Q4_K = 12 / Q6_K = 14): seg_in inputs starting at x
// and w, x rows x_stride floats apart, weight rows row_stride bytes apart.
hipError_t launch_kquant_segment(int ggml_type, const float* x, int x_stride, const uint8_t* w, size_t row_stride,
                                 float* y, int batch, int seg_in, int out_feat, int num_cus, hipStream_t stream);
// One canonical-dot segment: seg_in inputs of contiguous x rows (seg_in
// floats apart), weight rows row_bytes apart, w_avail bytes readable from w.
hipError_t launch_canon_segment(CanonFormat fmt, const float* x, const uint8_t* w, size_t row_bytes, size_t w_avail,
                                float* y, int batch, int seg_in, int out_feat, hipStream_t stream);
// out[b][0..ncol) = x[b][col0 .. col0 + ncol) for b < batch (rows ld floats apart).
hipError_t launch_gather_cols(const float* x, size_t ld, size_t col0, int ncol, int batch, float* out,
                              hipStream_t stream);
// y[i] = fixed_tree(part[0][i], part[1][i], ..., part[nseg-1][i]) for i < n
// (part[s] is n floats, the slices one after another).
hipError_t launch_segment_tree(const float* part, size_t n, int nseg, float* y, hipStream_t stream);

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
