// canon_gemv.hip -- exact-decode weights + the pinned 8-lane fp32 dot.
//
// Replaces the per-row `dequantize_*` + `canonical_dot_pub` arms of
// linear_dispatch (src/model/forward_quantized.rs:671-697, :751-776) and the
// float-fused Q4_K regime (canonical_dot_q4k_fused, src/ops/quant.rs:616-702).
//
// The contract (src/ops/quant.rs:429-448, :482-566): a row of n elements is
// cut into chunks of 8192; inside a chunk, lane j accumulates from +0.0, in
// increasing i, every product x_i * w_i with i % 8 == j (the product rounded
// before the add, never fused); the 8 lanes and then the chunk sums are
// combined with fixed_tree.  Each chain is mapped to one GPU lane, so the
// 8 lanes of a row's chunk are 8 adjacent lanes of a wave and the two trees
// are shuffles between them.  Every decoded weight is exact in binary32
// (f16 scale times a small integer), so decoding order is free.
#include "vtq_device.h"
#include "vtq_kernels.h"

namespace vtq {

constexpr int kChunk = 8192;
constexpr int kMaxChunkSlots = 8;  // in_feat <= 65536

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// Each decoder yields the weights of lane j's elements of one block:
// elements kBlock*bi + j + 8m, m = 0 .. kBlock/8 - 1.
struct DecQ8_0 {  // src/ops/quant.rs:193-210
    static constexpr int kBlock = 32;
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        const uint8_t* blk = row + 34 * bi;
        const float d = f16_to_f32(ld_u16(blk));
#pragma unroll
        for (int m = 0; m < 4; m++) w[m] = d * (float)(int8_t)blk[2 + j + 8 * m];
    }
};

struct DecQ5_0 {  // src/ops/quant.rs:160-186
    static constexpr int kBlock = 32;
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        const uint8_t* blk = row + 22 * bi;
        const float d = f16_to_f32(ld_u16(blk));
        const uint32_t qh = ld_u16(blk + 2) | (ld_u16(blk + 4) << 16);
        const uint8_t* qs = blk + 6;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int e = j + 8 * m;
            const uint32_t nib = (e < 16) ? (qs[e] & 0x0Fu) : (uint32_t)(qs[e - 16] >> 4);
            const int q = (int)(nib | (((qh >> e) & 1u) << 4)) - 16;
            w[m] = d * (float)q;
        }
    }
};

struct DecQ4_0 {  // src/ops/quant.rs:91-111 (element 2k low nibble, 2k+1 high)
    static constexpr int kBlock = 32;
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        const uint8_t* blk = row + 18 * bi;
        const float d = f16_to_f32(ld_u16(blk));
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int e = j + 8 * m;
            const uint32_t byte = blk[2 + (e >> 1)];
            const int q = (int)((e & 1) ? (byte >> 4) : (byte & 0x0Fu)) - 8;
            w[m] = d * (float)q;
        }
    }
};

struct DecQ4KFloat {  // src/ops/quant.rs:649-667: w = d1*q - m1f per sub-block
    static constexpr int kBlock = 32;
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        const int sb = bi >> 3, sj = bi & 7;
        const uint8_t* blk = row + 144 * sb;
        const float d = f16_to_f32(ld_u16(blk));
        const float dmin = f16_to_f32(ld_u16(blk + 2));
        const uint8_t* s = blk + 4;
        uint32_t sc, mn;
        if (sj < 4) {
            sc = s[sj] & 0x3Fu;
            mn = s[sj + 4] & 0x3Fu;
        } else {
            sc = (s[sj + 4] & 0x0Fu) | ((uint32_t)(s[sj - 4] >> 6) << 4);
            mn = (uint32_t)(s[sj + 4] >> 4) | ((uint32_t)(s[sj] >> 6) << 4);
        }
        const float d1 = d * (float)sc;
        const float m1f = dmin * (float)mn;
        const uint8_t* qs = blk + 16 + 32 * (sj >> 1);
        const bool hi = (sj & 1) != 0;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t b = qs[j + 8 * m];
            const uint32_t q = hi ? (b >> 4) : (b & 0x0Fu);
            w[m] = d1 * (float)q - m1f;
        }
    }
};

struct DecF32 {  // src/model/forward_quantized.rs:674-697
    static constexpr int kBlock = 8;
    __device__ static void decode(const uint8_t* row, int bi, int j, float* w) {
        w[0] = reinterpret_cast<const float*>(row)[8 * bi + j];
    }
};

// Wave layout: 8 lane groups of 8 lanes; group u = (row slot u / CPW,
// chunk slot u % CPW); lane j of a group is chain j.
template <class Dec, int CPW>
__global__ __launch_bounds__(256) void canon_gemv_kernel(const float* __restrict__ x,
                                                          const uint8_t* __restrict__ W, size_t row_bytes,
                                                          float* __restrict__ y, int n, int out_feat,
                                                          int nchunks) {
    constexpr int kRowsPerWave = 8 / CPW;
    constexpr int P = Dec::kBlock / 8;
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int j = lane & 7, u = lane >> 3;
    const int c = u % CPW;
    const int o = (blockIdx.x * 4 + wave) * kRowsPerWave + u / CPW;
    const float* xb = x + (size_t)blockIdx.y * n;
    float acc = -0.0f;  // padding value for chunk slots past the row's end
    if (o < out_feat && c < nchunks) {
        acc = 0.0f;
        const uint8_t* wrow = W + (size_t)o * row_bytes;
        const int cs = c * kChunk;
        const int ce = min(cs + kChunk, n);
        for (int bi = cs / Dec::kBlock; bi * Dec::kBlock < ce; ++bi) {
            float wv[P];
            if (Dec::kBlock == 8 && bi * 8 + j >= ce) break;  // f32 tail: lane j has no element
            Dec::decode(wrow, bi, j, wv);
#pragma unroll
            for (int m = 0; m < P; m++) {
                const float p = xb[bi * Dec::kBlock + j + 8 * m] * wv[m];
                acc = acc + p;
            }
        }
    }
    // fixed_tree over the 8 lanes (chunk sum), then over the chunk slots.
    float v = group_tree<1, 8>(acc);
    v = group_tree<8, CPW>(v);
    if (c == 0 && j == 0 && o < out_feat) y[(size_t)blockIdx.y * out_feat + o] = v;
}

template <class Dec>
static hipError_t launch_dec(const float* x, const uint8_t* w, size_t row_bytes, float* y, int batch, int n,
                             int out_feat, hipStream_t stream) {
    const int nchunks = (n + kChunk - 1) / kChunk;
    int cpw = 1;
    while (cpw < nchunks) cpw <<= 1;
    const int rows_per_wg = 4 * (8 / cpw);
    dim3 grid((unsigned)((out_feat + rows_per_wg - 1) / rows_per_wg), (unsigned)batch, 1);
    switch (cpw) {
    case 1: hipLaunchKernelGGL((canon_gemv_kernel<Dec, 1>), grid, dim3(256), 0, stream, x, w, row_bytes, y, n, out_feat, nchunks); break;
    case 2: hipLaunchKernelGGL((canon_gemv_kernel<Dec, 2>), grid, dim3(256), 0, stream, x, w, row_bytes, y, n, out_feat, nchunks); break;
    case 4: hipLaunchKernelGGL((canon_gemv_kernel<Dec, 4>), grid, dim3(256), 0, stream, x, w, row_bytes, y, n, out_feat, nchunks); break;
    case 8: hipLaunchKernelGGL((canon_gemv_kernel<Dec, 8>), grid, dim3(256), 0, stream, x, w, row_bytes, y, n, out_feat, nchunks); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_canon_gemv(CanonFormat fmt, const float* x, const uint8_t* w, size_t row_bytes, float* y,
                             int batch, int in_feat, int out_feat, int num_cus, hipStream_t stream) {
    (void)num_cus;
    switch (fmt) {
    case kCanonQ8_0: return launch_dec<DecQ8_0>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    case kCanonQ5_0: return launch_dec<DecQ5_0>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    case kCanonQ4_0: return launch_dec<DecQ4_0>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    case kCanonF32: return launch_dec<DecF32>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    case kCanonQ4KFloat: return launch_dec<DecQ4KFloat>(x, w, row_bytes, y, batch, in_feat, out_feat, stream);
    }
    return hipErrorInvalidValue;
}

int canon_max_in_feat() { return kMaxChunkSlots * kChunk; }

__global__ void fill_kernel(float* __restrict__ y, size_t n, float v) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = v;
}

hipError_t launch_fill(float* y, size_t n, float v, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, y, n, v);
    return hipGetLastError();
}

}  // namespace vtq
