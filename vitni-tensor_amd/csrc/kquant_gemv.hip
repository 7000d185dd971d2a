// kquant_gemv.hip -- exact-integer Q4_K / Q6_K decode GEMV for gfx950.
//
// Replaces linear_q4_k_integer[_parallel] (src/ops/quant.rs:936-980,
// :1149-1196) and linear_q6_k_integer[_parallel] (:1060-1146) for any batch;
// each batch row is one grid.y slice.
//
// One workgroup = NW waves.  It first quantizes its batch row of x into LDS
// (quantize_block_q8, src/ops/quant.rs:750-771: one wave per 256-element
// block), then streams a contiguous range of weight rows.  A wave owns one
// output row at a time and walks it in windows of 16 super-blocks: lane
// 4g+h handles quarter h of super-block 16w+g, so the 64 lanes cover 2304
// contiguous bytes of Q4_K (3360 of Q6_K) per window.  Integer partial sums
// are combined across the 4 lanes of a block with DPP (exact in any order),
// the per-block float epilogue is evaluated exactly as the reference writes
// it, and the block parts are combined with the pinned fixed_tree:
//   fixed_tree(p[0..R)) == fixed_tree over windows of fixed_tree(window),
// because the first four tree levels only ever pair blocks inside an aligned
// 16-block window (padded slots hold -0.0, the exact identity of +).
#include "vtq_device.h"
#include "vtq_kernels.h"

namespace vtq {

constexpr int kMaxWindows = 16;  // R <= 256 super-blocks: in_feat <= 65536

struct ActLds {
    uint32_t* qs;  // [R*64] packed int8 codes, word = 4 elements
    float* d;      // [R]
    int* s16;      // [R*16] sums of 16-element runs
    int* s32;      // [R*8]  sums of 32-element sub-blocks (bsums)
};

__device__ __forceinline__ ActLds act_lds_layout(unsigned char* base, int R) {
    ActLds a;
    a.qs = reinterpret_cast<uint32_t*>(base);
    a.d = reinterpret_cast<float*>(base + (size_t)R * 256);
    a.s16 = reinterpret_cast<int*>(base + (size_t)R * 260);
    a.s32 = reinterpret_cast<int*>(base + (size_t)R * 324);
    return a;
}

size_t act_lds_bytes(int R) { return (size_t)R * 356; }

template <int NW>
__device__ __forceinline__ void quantize_row_to_lds(const float* __restrict__ xb, int R, ActLds a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int b = wave; b < R; b += NW) {
        const float4 v = reinterpret_cast<const float4*>(xb + (size_t)b * 256)[lane];
        uint32_t packed;
        int s16, s32;
        const float d = quant_block_wave(v, &packed, &s16, &s32);
        a.qs[b * 64 + lane] = packed;
        if ((lane & 3) == 0) a.s16[b * 16 + (lane >> 2)] = s16;
        if ((lane & 7) == 0) a.s32[b * 8 + (lane >> 3)] = s32;
        if (lane == 0) a.d[b] = d;
    }
}

// fixed_tree over the per-window sums ws[0..nwin) (stride form, static indices).
__device__ __forceinline__ float window_tree(float (&ws)[kMaxWindows], int nwin) {
    if (nwin == 0) return 0.0f;
#pragma unroll
    for (int s = 1; s < kMaxWindows; s <<= 1) {
#pragma unroll
        for (int i = 0; i + s < kMaxWindows; i += 2 * s) {
            if (i + s < nwin) ws[i] = ws[i] + ws[i + s];
        }
    }
    return ws[0];
}

// ------------------------------------------------------------------ Q4_K

// Integer part of one Q4_K super-block for quarter h (sub-blocks 2h, 2h+1)
// (src/ops/quant.rs:849-898).  Returns acc and acc_m contributions.
__device__ __forceinline__ void q4k_quarter(const uint8_t* __restrict__ blk, int h, const uint32_t* xw,
                                            const int* s32, uint4& hdr, int& acc, int& accm) {
    hdr = *reinterpret_cast<const uint4*>(blk);
    const uint4 qa = *reinterpret_cast<const uint4*>(blk + 16 + 32 * h);
    const uint4 qb = *reinterpret_cast<const uint4*>(blk + 32 + 32 * h);
    const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    int s_lo = 0, s_hi = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        s_lo = __builtin_amdgcn_sdot4((int)(qw[i] & 0x0F0F0F0Fu), (int)xw[16 * h + i], s_lo, false);
        s_hi = __builtin_amdgcn_sdot4((int)((qw[i] >> 4) & 0x0F0F0F0Fu), (int)xw[16 * h + 8 + i], s_hi, false);
    }
    // get_scale_min_k4 (src/ops/quant.rs:267-276) for j = 2h, 2h+1, two bytes at a time.
    const int sh = 16 * (h & 1);
    const uint32_t A = hdr.w >> sh, B = hdr.y >> sh, C = hdr.z >> sh;
    uint32_t scp, mp;
    if (h < 2) {
        scp = B & 0x3F3Fu;
        mp = C & 0x3F3Fu;
    } else {
        scp = (A & 0x0F0Fu) | ((B & 0xC0C0u) >> 2);
        mp = ((A >> 4) & 0x0F0Fu) | ((C & 0xC0C0u) >> 2);
    }
    const int sc_lo = (int)(scp & 0xFFu), sc_hi = (int)((scp >> 8) & 0xFFu);
    const int m_lo = (int)(mp & 0xFFu), m_hi = (int)((mp >> 8) & 0xFFu);
    acc = sc_lo * s_lo + sc_hi * s_hi;
    accm = m_lo * s32[2 * h] + m_hi * s32[2 * h + 1];
}

template <int NW>
__global__ __launch_bounds__(NW * 64) void q4k_gemv_kernel(const float* __restrict__ x,
                                                           const uint8_t* __restrict__ W,
                                                           float* __restrict__ y, int R, int out_feat,
                                                           int rows_per_wg) {
    extern __shared__ __align__(16) unsigned char lds[];
    const ActLds act = act_lds_layout(lds, R);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* xb = x + (size_t)blockIdx.y * R * 256;
    float* yb = y + (size_t)blockIdx.y * out_feat;
    quantize_row_to_lds<NW>(xb, R, act);
    __syncthreads();

    const int g = lane >> 2, h = lane & 3;
    const int nwin = (R + 15) >> 4;
    const size_t row_bytes = (size_t)R * 144;
    const int row0 = blockIdx.x * rows_per_wg;
    const int row1 = min(row0 + rows_per_wg, out_feat);
    for (int o = row0 + wave; o < row1; o += NW) {
        const uint8_t* wrow = W + (size_t)o * row_bytes;
        float ws[kMaxWindows];
#pragma unroll
        for (int w = 0; w < kMaxWindows; w++) {
            ws[w] = -0.0f;
            if (w < nwin) {
                const int b = 16 * w + g;
                const bool valid = b < R;
                int acc = 0, accm = 0;
                uint4 hdr = make_uint4(0, 0, 0, 0);
                if (valid) q4k_quarter(wrow + (size_t)b * 144, h, act.qs + b * 64, act.s32 + b * 8, hdr, acc, accm);
                acc = quad_sum_i(acc);
                accm = quad_sum_i(accm);
                float part = -0.0f;
                if (valid) {
                    const float dx = act.d[b];
                    const float d = f16_to_f32(hdr.x & 0xFFFFu);
                    const float dmin = f16_to_f32(hdr.x >> 16);
                    const float t1 = (d * dx) * (float)acc;
                    const float t2 = (dmin * dx) * (float)accm;
                    part = t1 - t2;
                }
                ws[w] = group_tree<4, 16>(part);
            }
        }
        const float r = window_tree(ws, nwin);
        if (lane == 0) yb[o] = r;
    }
}

// ------------------------------------------------------------------ Q6_K

// 16 bytes starting at a 2-byte-aligned address.  Reads stay inside
// [p - 2, p + 18) and only extend past [p, p + 16) when p is not 4-aligned.
__device__ __forceinline__ uint4 load16_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t off = (uint32_t)(a & 3u);
    const uint32_t* p4 = reinterpret_cast<const uint32_t*>(a - off);
    const u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p4);
    if (off == 0) return make_uint4(v.x, v.y, v.z, v.w);
    const uint32_t e = p4[4];
    return make_uint4(__builtin_amdgcn_alignbyte(v.y, v.x, off), __builtin_amdgcn_alignbyte(v.z, v.y, off),
                      __builtin_amdgcn_alignbyte(v.w, v.z, off), __builtin_amdgcn_alignbyte(e, v.w, off));
}

// Bytes [p, p+8) from a 2-byte-aligned address, reads inside [p-2, p+10).
__device__ __forceinline__ uint2 load8_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t off = (uint32_t)(a & 3u);
    const uint32_t* p4 = reinterpret_cast<const uint32_t*>(a - off);
    const uint32_t w0 = p4[0], w1 = p4[1];
    if (off == 0) return make_uint2(w0, w1);
    const uint32_t w2 = p4[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, off), __builtin_amdgcn_alignbyte(w2, w1, off));
}

__device__ __forceinline__ int sext8(uint32_t v, int byte) { return (int)(int8_t)((v >> (8 * byte)) & 0xFFu); }

// Lane k of a Q6_K block: hf = k>>1 (128-element half), t = k&1 (l in
// [16t, 16t+16)).  Returns its share of acc = sum_j sc_j * sums_j
// (src/ops/quant.rs:995-1057): buckets 8hf+t+2q for q = 0..3, each exactly
// one 16-element run, with (code - 32) folded as sum(code*x) - 32*sum(x).
__device__ __forceinline__ int q6k_lane(const uint8_t* __restrict__ blk, int k, const uint32_t* xw,
                                        const int* s16) {
    const int hf = k >> 1, t = k & 1;
    const uint4 b0 = load16_a2(blk + 64 * hf + 16 * t);
    const uint4 b1 = load16_a2(blk + 64 * hf + 32 + 16 * t);
    const uint4 hh = load16_a2(blk + 128 + 32 * hf + 16 * t);
    const uint2 scw = load8_a2(blk + 192 + 8 * hf);
    const uint32_t B0[4] = {b0.x, b0.y, b0.z, b0.w};
    const uint32_t B1[4] = {b1.x, b1.y, b1.z, b1.w};
    const uint32_t H[4] = {hh.x, hh.y, hh.z, hh.w};
    // activation words: element 128hf + 16t + 32q + 4i -> word 32hf + 4t + 8q + i
    const int xw0 = 32 * hf + 4 * t;
    int S1 = 0, S2 = 0, S3 = 0, S4 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t q1 = (B0[i] & 0x0F0F0F0Fu) | ((H[i] & 0x03030303u) << 4);
        const uint32_t q2 = (B1[i] & 0x0F0F0F0Fu) | ((H[i] & 0x0C0C0C0Cu) << 2);
        const uint32_t q3 = ((B0[i] >> 4) & 0x0F0F0F0Fu) | (H[i] & 0x30303030u);
        const uint32_t q4 = ((B1[i] >> 4) & 0x0F0F0F0Fu) | ((H[i] >> 2) & 0x30303030u);
        S1 = __builtin_amdgcn_sdot4((int)q1, (int)xw[xw0 + i], S1, false);
        S2 = __builtin_amdgcn_sdot4((int)q2, (int)xw[xw0 + 8 + i], S2, false);
        S3 = __builtin_amdgcn_sdot4((int)q3, (int)xw[xw0 + 16 + i], S3, false);
        S4 = __builtin_amdgcn_sdot4((int)q4, (int)xw[xw0 + 24 + i], S4, false);
    }
    const int j0 = 8 * hf + t;  // bucket of q1; q2..q4 at +2, +4, +6
    const int sum1 = S1 - 32 * s16[j0 + 0];
    const int sum2 = S2 - 32 * s16[j0 + 2];
    const int sum3 = S3 - 32 * s16[j0 + 4];
    const int sum4 = S4 - 32 * s16[j0 + 6];
    // scales: i8 at 192 + 8hf + t + 2q  ->  bytes t, t+2 of scw.x and of scw.y
    const int c1 = sext8(scw.x, t), c2 = sext8(scw.x, t + 2);
    const int c3 = sext8(scw.y, t), c4 = sext8(scw.y, t + 2);
    return c1 * sum1 + c2 * sum2 + c3 * sum3 + c4 * sum4;
}

template <int NW>
__global__ __launch_bounds__(NW * 64) void q6k_gemv_kernel(const float* __restrict__ x,
                                                           const uint8_t* __restrict__ W,
                                                           float* __restrict__ y, int R, int out_feat,
                                                           int rows_per_wg) {
    extern __shared__ __align__(16) unsigned char lds[];
    const ActLds act = act_lds_layout(lds, R);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* xb = x + (size_t)blockIdx.y * R * 256;
    float* yb = y + (size_t)blockIdx.y * out_feat;
    quantize_row_to_lds<NW>(xb, R, act);
    __syncthreads();

    const int g = lane >> 2, k = lane & 3;
    const int nwin = (R + 15) >> 4;
    const size_t row_bytes = (size_t)R * 210;
    const int row0 = blockIdx.x * rows_per_wg;
    const int row1 = min(row0 + rows_per_wg, out_feat);
    for (int o = row0 + wave; o < row1; o += NW) {
        const uint8_t* wrow = W + (size_t)o * row_bytes;
        float ws[kMaxWindows];
#pragma unroll
        for (int w = 0; w < kMaxWindows; w++) {
            ws[w] = -0.0f;
            if (w < nwin) {
                const int b = 16 * w + g;
                const bool valid = b < R;
                int acc = 0;
                uint32_t dbits = 0;
                if (valid) {
                    const uint8_t* blk = wrow + (size_t)b * 210;
                    acc = q6k_lane(blk, k, act.qs + b * 64, act.s16 + b * 16);
                    dbits = *reinterpret_cast<const uint16_t*>(blk + 208);
                }
                acc = quad_sum_i(acc);
                float part = -0.0f;
                if (valid) {
                    const float d = f16_to_f32(dbits);
                    part = (d * act.d[b]) * (float)acc;
                }
                ws[w] = group_tree<4, 16>(part);
            }
        }
        const float r = window_tree(ws, nwin);
        if (lane == 0) yb[o] = r;
    }
}

// ------------------------------------------------------------- launchers

static constexpr int kNW = 4;

static void grid_for(int out_feat, int num_cus, int batch, dim3& grid, int& rows_per_wg) {
    // Two workgroups per CU in one wave of dispatch, contiguous row ranges.
    int target = 2 * num_cus;
    int rpw = (out_feat + target - 1) / target;
    if (rpw < kNW) rpw = kNW;
    rows_per_wg = rpw;
    grid = dim3((unsigned)((out_feat + rpw - 1) / rpw), (unsigned)batch, 1);
}

hipError_t launch_q4k_gemv(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           int num_cus, hipStream_t stream) {
    const int R = in_feat / 256;
    dim3 grid;
    int rpw;
    grid_for(out_feat, num_cus, batch, grid, rpw);
    hipLaunchKernelGGL(q4k_gemv_kernel<kNW>, grid, dim3(kNW * 64), act_lds_bytes(R), stream, x, w, y, R,
                       out_feat, rpw);
    return hipGetLastError();
}

hipError_t launch_q6k_gemv(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           int num_cus, hipStream_t stream) {
    const int R = in_feat / 256;
    dim3 grid;
    int rpw;
    grid_for(out_feat, num_cus, batch, grid, rpw);
    hipLaunchKernelGGL(q6k_gemv_kernel<kNW>, grid, dim3(kNW * 64), act_lds_bytes(R), stream, x, w, y, R,
                       out_feat, rpw);
    return hipGetLastError();
}

int kquant_max_in_feat() { return kMaxWindows * 16 * 256; }

}  // namespace vtq
