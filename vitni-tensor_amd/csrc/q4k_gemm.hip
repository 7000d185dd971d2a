// q4k_gemm.hip -- exact-integer Q4_K prefill GEMM on i8 MFMA (gfx950).
//
// Replaces linear_q4_k_integer (src/ops/quant.rs:936-980) for large batch:
// y[b][o] = fixed_tree_s part(b, o, s) with, per super-block s,
//   acc  = sum_j sc_j * sum_{k in j} q_k * xq_k          (j = 8 sub-blocks of 32)
//   accm = sum_j m_j  * bsum_j
//   part = (d*dx) * f32(acc) - (dmin*dx) * f32(accm)
//
// Integer work on v_mfma_i32_32x32x32_i8:
//  * the 6-bit sub-block scale is folded into the weight operand by a 3+3 bit
//    split, sc = 8*sh + sl: A1 = q*sh and A0 = q*sl are both <= 105 (i8), and
//    acc = 8*C1 + C0 exactly (|C1| <= 256*105*127), so one super-block is 16
//    MFMAs whose accumulators run over all 256 elements;
//  * the min term is one more pair of MFMAs over the 8 sub-blocks with
//    bsum = 64*bh + bl split into two i8 operands (bl in [0,63], bh in [-64,63]);
//    accm = 64*Ch + Cl exactly.
// Integer sums are exact in any order, so the MFMA reduction order is free.
// The float epilogue is the reference's, per (b, o, s), in VALU, and the
// fixed_tree over super-blocks is kept in registers as a binary counter:
// fixed_tree(p[0..R)) == fold-right over the balanced trees of the binary
// digits of R, each built left to right as parts arrive.
//
// Tile: a workgroup of 4 waves owns 32 weight rows x 128 tokens; wave w owns
// tokens 32w..32w+31 of the tile.  Per super-block the workgroup stages the
// 32 rows' 144-byte blocks in LDS and builds the MFMA weight operands there
// once; each wave reads its token operands (the pre-quantized activation)
// straight from global memory.
#include "vtq_device.h"
#include "vtq_kernels.h"

namespace vtq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ------------------------------------------------ activation pre-pass

// quantize_block_q8 (src/ops/quant.rs:750-771) of every 256-block of every
// batch row: one wave per (row, block).  Writes the codes row-major
// [M][K], d [M][R], and the split sub-block sums [M][R][16] = bl[8], bh[8].
__global__ __launch_bounds__(256) void act_quant_rows_kernel(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                              float* __restrict__ xd, int8_t* __restrict__ xb,
                                                              int R, int M) {
    const int lane = threadIdx.x & 63;
    const long blk = (long)blockIdx.x * 4 + wave_id();
    if (blk >= (long)R * M) return;
    const long b = blk / R, s = blk % R;
    const long K = (long)R * 256;
    const float4 v = reinterpret_cast<const float4*>(x + b * K + s * 256)[lane];
    uint32_t packed;
    int s16, s32;
    const float d = quant_block_wave(v, &packed, &s16, &s32);
    reinterpret_cast<uint32_t*>(xq + b * K + s * 256)[lane] = packed;
    if (lane == 0) xd[b * R + s] = d;
    if ((lane & 7) == 0) {
        const int j = lane >> 3;
        int8_t* o = xb + (b * R + s) * 16;
        o[j] = (int8_t)(s32 & 63);       // bl
        o[8 + j] = (int8_t)(s32 >> 6);   // bh (arithmetic shift: s32 = 64*bh + bl)
    }
}

// ---------------------------------------------------------------- GEMM

constexpr int kTO = 32;   // weight rows per workgroup
constexpr int kTB = 128;  // tokens per workgroup (4 waves x 32)

template <int LV>
__global__ __launch_bounds__(256, 2) void q4k_gemm_kernel(const uint8_t* __restrict__ W,
                                                          const int8_t* __restrict__ xq,
                                                          const float* __restrict__ xd,
                                                          const int8_t* __restrict__ xb, float* __restrict__ y,
                                                          int R, int N, int M) {
    __shared__ __align__(16) uint8_t raw[kTO * 144];  // 32 rows' blocks of super-block s
    __shared__ v4i opA1[8][64];                         // weight operands per k-step (sub-block) and lane
    __shared__ v4i opA0[8][64];
    __shared__ v4i opAm[64];                            // min-term operand
    __shared__ float dsh[kTO], dminsh[kTO];

    const int t = threadIdx.x, lane = t & 63, wave = wave_id();
    const int o0 = blockIdx.x * kTO;
    const int g = lane >> 5, n = lane & 31;
    const int tok = min(blockIdx.y * kTB + wave * 32 + n, M - 1);  // clamped: tail tokens are discarded
    const long K = (long)R * 256;
    const size_t row_bytes = (size_t)R * 144;

    float stk[LV][16];
#pragma unroll
    for (int l = 0; l < LV; l++)
#pragma unroll
        for (int i = 0; i < 16; i++) stk[l][i] = 0.0f;

    for (int s = 0; s < R; s++) {
        // token operands of this super-block (global, issued before the LDS phase)
        const v4i* xrow = reinterpret_cast<const v4i*>(xq + (long)tok * K + (long)s * 256);
        v4i bop[8];
#pragma unroll
        for (int j = 0; j < 8; j++) bop[j] = xrow[2 * j + g];  // elements 32j + 16g .. +16
        const int8_t* bs = xb + ((long)tok * R + s) * 16;
        const int2 bsl = *reinterpret_cast<const int2*>(bs);      // bl[0..8)
        const int2 bsh = *reinterpret_cast<const int2*>(bs + 8);  // bh[0..8)
        const float dx = xd[(long)tok * R + s];

        __syncthreads();  // previous super-block's operands are consumed
        // stage 32 rows x 144 B (288 chunks of 16 B)
        for (int c = t; c < kTO * 9; c += 256) {
            const int r = c / 9, q = c % 9;
            const int orow = min(o0 + r, N - 1);
            *reinterpret_cast<uint4*>(raw + r * 144 + q * 16) =
                *reinterpret_cast<const uint4*>(W + (size_t)orow * row_bytes + (size_t)s * 144 + q * 16);
        }
        __syncthreads();
        // build operands: thread (row r = t%32, sub-block j = t/32) writes the two lanes (r, g=0/1)
        {
            const int r = t & 31, j = t >> 5;
            const uint8_t* blk = raw + r * 144;
            const uint8_t* sb = blk + 4;
            uint32_t sc, mn;
            if (j < 4) {
                sc = sb[j] & 63u;
                mn = sb[j + 4] & 63u;
            } else {
                sc = (sb[j + 4] & 15u) | ((uint32_t)(sb[j - 4] >> 6) << 4);
                mn = (uint32_t)(sb[j + 4] >> 4) | ((uint32_t)(sb[j] >> 6) << 4);
            }
            const uint32_t sh = sc >> 3, sl = sc & 7u;
            const uint4* q4 = reinterpret_cast<const uint4*>(blk + 16 + 32 * (j >> 1));
            const bool hi = (j & 1) != 0;
#pragma unroll
            for (int gg = 0; gg < 2; gg++) {
                const uint4 qv = q4[gg];
                const uint32_t w0 = (hi ? qv.x >> 4 : qv.x) & 0x0F0F0F0Fu, w1 = (hi ? qv.y >> 4 : qv.y) & 0x0F0F0F0Fu;
                const uint32_t w2 = (hi ? qv.z >> 4 : qv.z) & 0x0F0F0F0Fu, w3 = (hi ? qv.w >> 4 : qv.w) & 0x0F0F0F0Fu;
                // byte-wise products stay below 256: no carry between bytes
                opA1[j][r + 32 * gg] = v4i{(int)(w0 * sh), (int)(w1 * sh), (int)(w2 * sh), (int)(w3 * sh)};
                opA0[j][r + 32 * gg] = v4i{(int)(w0 * sl), (int)(w1 * sl), (int)(w2 * sl), (int)(w3 * sl)};
            }
            // min-term operand: lane (r, g=0) bytes 0..7 = m_0..m_7 (one byte per thread j)
            reinterpret_cast<uint8_t*>(&opAm[r])[j] = (uint8_t)mn;
            reinterpret_cast<uint8_t*>(&opAm[r])[8 + j] = 0;
            reinterpret_cast<uint8_t*>(&opAm[r + 32])[j] = 0;
            reinterpret_cast<uint8_t*>(&opAm[r + 32])[8 + j] = 0;
            if (j == 0) {
                dsh[r] = f16_to_f32(blk[0] | (blk[1] << 8));
                dminsh[r] = f16_to_f32(blk[2] | (blk[3] << 8));
            }
        }
        __syncthreads();

        v16i c1 = {}, c0 = {}, cl = {}, ch = {};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(opA1[j][lane], bop[j], c1, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(opA0[j][lane], bop[j], c0, 0, 0, 0);
        }
        const v4i am = opAm[lane];
        const v4i bl = g == 0 ? v4i{bsl.x, bsl.y, 0, 0} : v4i{0, 0, 0, 0};
        const v4i bh = g == 0 ? v4i{bsh.x, bsh.y, 0, 0} : v4i{0, 0, 0, 0};
        cl = __builtin_amdgcn_mfma_i32_32x32x32_i8(am, bl, cl, 0, 0, 0);
        ch = __builtin_amdgcn_mfma_i32_32x32x32_i8(am, bh, ch, 0, 0, 0);

        // epilogue: element i of this lane is row 8*(i/4) + 4*g + i%4, token n
        float p[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = 8 * (i >> 2) + 4 * g + (i & 3);
            const int acc = 8 * c1[i] + c0[i];
            const int accm = 64 * ch[i] + cl[i];
            const float t1 = (dsh[r] * dx) * (float)acc;
            const float t2 = (dminsh[r] * dx) * (float)accm;
            p[i] = t1 - t2;
        }
        // fixed_tree, streamed: combine with the stored block of each level while bit l of s is set
        bool carry = true;
#pragma unroll
        for (int l = 0; l < LV; l++) {
            if (carry) {
                if ((s >> l) & 1) {
#pragma unroll
                    for (int i = 0; i < 16; i++) p[i] = stk[l][i] + p[i];
                } else {
#pragma unroll
                    for (int i = 0; i < 16; i++) stk[l][i] = p[i];
                    carry = false;
                }
            }
        }
    }
    // fold the remaining blocks right to left (smaller, later blocks first)
    float r16[16];
    bool have = false;
#pragma unroll
    for (int l = 0; l < LV; l++) {
        if ((R >> l) & 1) {
#pragma unroll
            for (int i = 0; i < 16; i++) r16[i] = have ? stk[l][i] + r16[i] : stk[l][i];
            have = true;
        }
    }
    const int tok_real = blockIdx.y * kTB + wave * 32 + n;
    if (tok_real < M) {
        float* yrow = y + (long)tok_real * N;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int r = 8 * q + 4 * g;
            const int o = o0 + r;
            if (o + 3 < N) {
                *reinterpret_cast<float4*>(yrow + o) = make_float4(r16[4 * q], r16[4 * q + 1], r16[4 * q + 2], r16[4 * q + 3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (o + e < N) yrow[o + e] = r16[4 * q + e];
            }
        }
    }
}

size_t q4k_gemm_workspace_bytes(int batch, int in_feat) {
    const size_t R = in_feat / 256;
    return ((size_t)batch * in_feat + 255) / 256 * 256 + ((size_t)batch * R * 4 + 255) / 256 * 256 +
           (size_t)batch * R * 16 + 256;
}

int q4k_gemm_max_in_feat() { return 127 * 256; }

hipError_t launch_q4k_gemm(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           void* workspace, hipStream_t stream) {
    const int R = in_feat / 256;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    int8_t* xq = reinterpret_cast<int8_t*>(ws);
    float* xd = reinterpret_cast<float*>(ws + ((size_t)batch * in_feat + 255) / 256 * 256);
    int8_t* xb = reinterpret_cast<int8_t*>(reinterpret_cast<uint8_t*>(xd) + ((size_t)batch * R * 4 + 255) / 256 * 256);
    const long blocks = (long)batch * R;
    hipLaunchKernelGGL(act_quant_rows_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, stream, x, xq, xd,
                       xb, R, batch);
    if (hipError_t e = hipGetLastError()) return e;
    dim3 grid((unsigned)((out_feat + kTO - 1) / kTO), (unsigned)((batch + kTB - 1) / kTB), 1);
    int lv = 0;
    while ((1 << lv) <= R) lv++;  // bit length of R: R < 2^lv
    switch (lv) {
    case 1: hipLaunchKernelGGL(q4k_gemm_kernel<1>, grid, dim3(256), 0, stream, w, xq, xd, xb, y, R, out_feat, batch); break;
    case 2: hipLaunchKernelGGL(q4k_gemm_kernel<2>, grid, dim3(256), 0, stream, w, xq, xd, xb, y, R, out_feat, batch); break;
    case 3: hipLaunchKernelGGL(q4k_gemm_kernel<3>, grid, dim3(256), 0, stream, w, xq, xd, xb, y, R, out_feat, batch); break;
    case 4: hipLaunchKernelGGL(q4k_gemm_kernel<4>, grid, dim3(256), 0, stream, w, xq, xd, xb, y, R, out_feat, batch); break;
    case 5: hipLaunchKernelGGL(q4k_gemm_kernel<5>, grid, dim3(256), 0, stream, w, xq, xd, xb, y, R, out_feat, batch); break;
    case 6: hipLaunchKernelGGL(q4k_gemm_kernel<6>, grid, dim3(256), 0, stream, w, xq, xd, xb, y, R, out_feat, batch); break;
    case 7: hipLaunchKernelGGL(q4k_gemm_kernel<7>, grid, dim3(256), 0, stream, w, xq, xd, xb, y, R, out_feat, batch); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace vtq
