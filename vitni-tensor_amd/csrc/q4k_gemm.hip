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
// tokens 32w..32w+31 of the tile.  The activation pre-pass writes the token
// codes in the MFMA operand order, so each wave's operand loads are contiguous.
#include "vtq_device.h"
#include "vtq_kernels.h"

namespace vtq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ------------------------------------------------ activation pre-pass

// Workspace layout, in tiles of 32 tokens (Mp = batch rounded up to 32; the
// padding tokens hold zeros):
//   xqt [Mp/32][R][8][64] x 16 B   k-step j, lane 32g+n: codes 32j+16g .. +15
//                                   of token 32T+n (the MFMA B operand, so one
//                                   wave reads 1 KB contiguous per k-step)
//   xdt [Mp/32][R][32] f32          d of each (token, super-block)
//   xbt [Mp/32][R][32] x 16 B       bl[8] = bsum & 63, bh[8] = bsum >> 6
struct GemmWs {
    v4i* xqt;
    float* xdt;
    v4i* xbt;
};

inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }

inline GemmWs gemm_ws(void* base, int Mp, int R) {
    uint8_t* p = static_cast<uint8_t*>(base);
    GemmWs w;
    w.xqt = reinterpret_cast<v4i*>(p);
    p += align256((size_t)Mp * R * 256);
    w.xdt = reinterpret_cast<float*>(p);
    p += align256((size_t)Mp * R * 4);
    w.xbt = reinterpret_cast<v4i*>(p);
    return w;
}

// quantize_block_q8 (src/ops/quant.rs:750-771) of every 256-block of every
// batch row: one wave per (token, super-block), written in the tiled layout.
// Workgroup (s, q) holds the 16 consecutive tokens 16q..16q+15 of
// super-block s, so each 256-byte run of the token operands (and the 16
// d / bsum entries beside it) is written by one workgroup at once.
constexpr int kQuantWaves = 16;
__global__ __launch_bounds__(kQuantWaves * 64) void act_quant_tiles_kernel(const float* __restrict__ x, GemmWs ws,
                                                                           int R, int M) {
    const int lane = threadIdx.x & 63;
    const int s = (int)blockIdx.x;
    const int b = (int)blockIdx.y * kQuantWaves + wave_id();  // < Mp: the grid covers Mp / 16 groups
    const int tile = (b >> 5) * R + s;
    const int n = b & 31;
    uint32_t packed = 0;
    int s16 = 0, s32 = 0;
    float d = 0.0f;
    if (b < M) {  // uniform per wave
        const float4 v = reinterpret_cast<const float4*>(x + (size_t)b * R * 256 + (size_t)s * 256)[lane];
        d = quant_block_wave(v, &packed, &s16, &s32);
    }
    // lane holds elements 4*lane .. +3: k-step j = lane/8, half g = (lane/4)&1
    const int j = lane >> 3, g = (lane >> 2) & 1;
    uint8_t* dst = reinterpret_cast<uint8_t*>(ws.xqt + ((size_t)tile * 8 + j) * 64 + 32 * g + n) + 4 * (lane & 3);
    *reinterpret_cast<uint32_t*>(dst) = packed;
    if (lane == 0) ws.xdt[(size_t)tile * 32 + n] = d;
    if ((lane & 7) == 0) {
        int8_t* o = reinterpret_cast<int8_t*>(ws.xbt + (size_t)tile * 32 + n);
        o[j] = (int8_t)(s32 & 63);      // bl
        o[8 + j] = (int8_t)(s32 >> 6);  // bh (arithmetic shift: s32 = 64*bh + bl)
    }
}

// ---------------------------------------------------------------- GEMM

constexpr int kTO = 32;        // weight rows per workgroup
constexpr int kTB = 128;       // tokens per workgroup (4 waves x 32)
constexpr int kChunkM = 8192;  // tokens per launch pair (bounds the workspace)

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

// Byte-wise product of four nibbles (each <= 15) with m <= 7: every byte
// stays below 256, so one packed 16-bit multiply carries nothing across bytes.
__device__ __forceinline__ int nib_mul(uint32_t w, us2 m) {
    return (int)__builtin_bit_cast(uint32_t, __builtin_bit_cast(us2, w) * m);
}

// One workgroup: 32 weight rows x 128 tokens; wave w owns tokens 32w..32w+31.
// Per super-block the workgroup builds the weight operands once in LDS
// (double-buffered: one barrier per super-block), while each wave's token
// operands and the next super-block's weight bytes are prefetched into
// registers during the current super-block's MFMAs and epilogue.
template <int LV>
__global__ __launch_bounds__(256, 2) void q4k_gemm_kernel(const uint8_t* __restrict__ W, GemmWs ws,
                                                          float* __restrict__ y, int R, int N, int M, int NR,
                                                          int TT) {
    __shared__ v4i opA1[2][8][64];  // weight operands per buffer, k-step (sub-block) and lane
    __shared__ v4i opA0[2][8][64];
    __shared__ uint2 opAm[2][64];   // min-term operand: bytes m_0..m_7 of each row; lanes 32..63 zero
    __shared__ float dd[2][2][32];  // d, dmin of each row

    const int t = threadIdx.x, lane = t & 63, wave = wave_id();
    // Tile order: workgroup i runs on XCD i % 8, so the TT token tiles of one
    // row tile are given consecutive slots of one XCD and share its L2.
    const int id = blockIdx.x, full = (NR / 8) * 8 * TT;
    int rt, tt;
    if (id < full) {
        const int k = id >> 3;
        rt = (k / TT) * 8 + (id & 7);
        tt = k % TT;
    } else {
        rt = (NR / 8) * 8 + (id - full) / TT;
        tt = (id - full) % TT;
    }
    const int o0 = rt * kTO;
    const int g = lane >> 5, n = lane & 31;
    const int Tw = tt * 4 + wave;                  // this wave's 32-token tile
    const int T = min(Tw, (M + 31) / 32 - 1);      // past-the-end waves recompute the last tile
    const v4i* xq_w = ws.xqt + (size_t)T * R * 512 + lane;
    const v4i* xb_w = ws.xbt + (size_t)T * R * 32 + n;
    const float* xd_w = ws.xdt + (size_t)T * R * 32 + n;

    // operand builder: thread (row br, sub-block bj)
    const int br = lane & 31, bj = t >> 5;
    const uint8_t* wrow = W + (size_t)min(o0 + br, N - 1) * ((size_t)R * 144);
    const uint32_t nsh = 4 * (bj & 1), ssh = 8 * (bj & 3);

    uint4 h, q0, q1;
    auto wload = [&](int s) {
        const uint8_t* blk = wrow + (size_t)s * 144;
        h = *reinterpret_cast<const uint4*>(blk);
        const uint4* qp = reinterpret_cast<const uint4*>(blk + 16 + 32 * (bj >> 1));
        q0 = qp[0];
        q1 = qp[1];
    };
    auto build = [&](int buf) {
        // get_scale_min_k4 (src/ops/quant.rs:267-276) for sub-block bj: scale bytes 0..11 = h.y, h.z, h.w
        const uint32_t by = (h.y >> ssh) & 255u, bz = (h.z >> ssh) & 255u, bw = (h.w >> ssh) & 255u;
        const uint32_t up = bj >= 4 ? ~0u : 0u;  // sub-blocks 4..7 take the split encoding
        const uint32_t sc = ((by & 63u) & ~up) | (((bw & 15u) | ((by >> 6) << 4)) & up);
        const uint32_t mn = ((bz & 63u) & ~up) | (((bw >> 4) | ((bz >> 6) << 4)) & up);
        const us2 mh = {(unsigned short)(sc >> 3), (unsigned short)(sc >> 3)};
        const us2 ml = {(unsigned short)(sc & 7u), (unsigned short)(sc & 7u)};
        const uint32_t w[8] = {(q0.x >> nsh) & 0x0F0F0F0Fu, (q0.y >> nsh) & 0x0F0F0F0Fu, (q0.z >> nsh) & 0x0F0F0F0Fu,
                               (q0.w >> nsh) & 0x0F0F0F0Fu, (q1.x >> nsh) & 0x0F0F0F0Fu, (q1.y >> nsh) & 0x0F0F0F0Fu,
                               (q1.z >> nsh) & 0x0F0F0F0Fu, (q1.w >> nsh) & 0x0F0F0F0Fu};
        opA1[buf][bj][br] = v4i{nib_mul(w[0], mh), nib_mul(w[1], mh), nib_mul(w[2], mh), nib_mul(w[3], mh)};
        opA1[buf][bj][br + 32] = v4i{nib_mul(w[4], mh), nib_mul(w[5], mh), nib_mul(w[6], mh), nib_mul(w[7], mh)};
        opA0[buf][bj][br] = v4i{nib_mul(w[0], ml), nib_mul(w[1], ml), nib_mul(w[2], ml), nib_mul(w[3], ml)};
        opA0[buf][bj][br + 32] = v4i{nib_mul(w[4], ml), nib_mul(w[5], ml), nib_mul(w[6], ml), nib_mul(w[7], ml)};
        reinterpret_cast<uint8_t*>(&opAm[buf][br])[bj] = (uint8_t)mn;
        if (bj < 2) dd[buf][bj][br] = f16_to_f32_sel((h.x >> (16 * bj)) & 0xFFFFu);  // wave 0 only
    };

    // Token operands of the current super-block (reloaded for the next one
    // as soon as the current MFMAs are issued).
    v4i bop[8], bsv;
    float dx;
    auto tload = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 8; j++) bop[j] = xq_w[(s * 8 + j) * 64];
        bsv = xb_w[s * 32];
        dx = xd_w[s * 32];
    };

    // One super-block s from LDS buffer `buf`; prefetches the tokens of s+1
    // and the weights of s+2, and builds the weight operands of s+1 into the
    // other buffer.  Writes the per-(row, token) parts of s to p.  (Past the
    // end the loads repeat the last super-block: every load is
    // unconditional, so the wait counts stay exact across the back edge.)
    auto sblock = [&](int s, int buf, float (&p)[16]) __attribute__((always_inline)) {
        // acc = 8*C1 + C0 from two interleaved accumulator chains; token
        // register j is reloaded for super-block s+1 as soon as its two
        // MFMAs have been issued.  accm = 64*Ch + Cl is chained through one
        // accumulator (Ch scaled in place becomes the C input of Cl).
        const int sn = min(s + 1, R - 1);
        v16i c1 = {}, c0 = {}, cm = {};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(opA1[buf][j][lane], bop[j], c1, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(opA0[buf][j][lane], bop[j], c0, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            bop[j] = xq_w[(sn * 8 + j) * 64];
        }
        const uint2 amv = opAm[buf][lane];  // zero for lanes 32..63
        const v4i am = v4i{(int)amv.x, (int)amv.y, 0, 0};
        const v4i bh = g == 0 ? v4i{bsv.z, bsv.w, 0, 0} : v4i{0, 0, 0, 0};
        const v4i bl = g == 0 ? v4i{bsv.x, bsv.y, 0, 0} : v4i{0, 0, 0, 0};
        cm = __builtin_amdgcn_mfma_i32_32x32x32_i8(am, bh, cm, 0, 0, 0);
        const float dxs = dx;
        __builtin_amdgcn_sched_barrier(0);
        bsv = xb_w[sn * 32];
        dx = xd_w[sn * 32];
        int acc[16];
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] = 8 * c1[i] + c0[i];
#pragma unroll
        for (int i = 0; i < 16; i++) cm[i] *= 64;
        cm = __builtin_amdgcn_mfma_i32_32x32x32_i8(am, bl, cm, 0, 0, 0);
        // epilogue (src/ops/quant.rs:849-898): element i of this lane is row 8*(i/4) + 4*g + i%4, token n
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 dv = *reinterpret_cast<const float4*>(&dd[buf][0][8 * q + 4 * g]);
            const float4 mv = *reinterpret_cast<const float4*>(&dd[buf][1][8 * q + 4 * g]);
            const float dr[4] = {dv.x, dv.y, dv.z, dv.w}, mr[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int i = 4 * q + e;
                const float t1 = (dr[e] * dxs) * (float)acc[i];
                const float t2 = (mr[e] * dxs) * (float)cm[i];
                p[i] = t1 - t2;
            }
        }
        build(buf ^ 1);
        wload(min(s + 2, R - 1));
        __syncthreads();
    };

    // fixed_tree (src/ops/quant.rs:461-476) streamed as a binary counter:
    // level l holds the completed 2^l-block, combined as the left operand
    // with the block that completes it.  After leaf s, the levels below
    // L = (trailing ones of s) merge into level L; L is uniform, and each
    // case writes its chain straight into its level (no register shuffles).
    float stk[LV][16];
#pragma unroll
    for (int l = 0; l < LV; l++)
#pragma unroll
        for (int i = 0; i < 16; i++) stk[l][i] = 0.0f;

    if (t < 64) opAm[t >> 5][32 + (t & 31)] = make_uint2(0u, 0u);
    tload(0);
    wload(0);
    build(0);
    wload(min(1, R - 1));
    __syncthreads();

    for (int s = 0; s < R; s++) {
        float p[16];
        sblock(s, s & 1, p);
        const int L = __builtin_ctz(~s);
#pragma unroll
        for (int LL = 0; LL < LV; LL++) {
            if (L == LL) {
#pragma unroll
                for (int l = 0; l < LL; l++)
#pragma unroll
                    for (int i = 0; i < 16; i++) p[i] = stk[l][i] + p[i];
#pragma unroll
                for (int i = 0; i < 16; i++) stk[LL][i] = p[i];
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
    const int tok = Tw * 32 + n;
    if (tok < M) {
        float* yrow = y + (size_t)tok * N;
        const bool vec = (N & 3) == 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int o = o0 + 8 * q + 4 * g;
            if (vec && o + 3 < N) {
                *reinterpret_cast<float4*>(yrow + o) =
                    make_float4(r16[4 * q], r16[4 * q + 1], r16[4 * q + 2], r16[4 * q + 3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (o + e < N) yrow[o + e] = r16[4 * q + e];
            }
        }
    }
}

size_t q4k_gemm_workspace_bytes(int batch, int in_feat) {
    const int Mp = (min(batch, kChunkM) + 31) / 32 * 32;
    const size_t R = in_feat / 256;
    return align256((size_t)Mp * R * 256) + align256((size_t)Mp * R * 4) + (size_t)Mp * R * 16;
}

int q4k_gemm_max_in_feat() { return 127 * 256; }

template <int LV>
static void launch_gemm_lv(dim3 grid, hipStream_t stream, const uint8_t* w, GemmWs ws, float* y, int R, int N, int M,
                           int NR, int TT) {
    hipLaunchKernelGGL(q4k_gemm_kernel<LV>, grid, dim3(256), 0, stream, w, ws, y, R, N, M, NR, TT);
}

hipError_t launch_q4k_gemm(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           void* workspace, hipStream_t stream) {
    const int R = in_feat / 256;
    int lv = 0;
    while ((1 << lv) <= R) lv++;  // bit length of R: R < 2^lv
    if (lv < 1 || lv > 7) return hipErrorInvalidValue;
    const int NR = (out_feat + kTO - 1) / kTO;
    for (int b0 = 0; b0 < batch; b0 += kChunkM) {
        const int M = min(batch - b0, kChunkM), Mp = (M + 31) / 32 * 32;
        const GemmWs ws = gemm_ws(workspace, Mp, R);
        // Mp is a multiple of 32, so Mp / 16 groups cover every token slot
        hipLaunchKernelGGL(act_quant_tiles_kernel, dim3((unsigned)R, (unsigned)(Mp / kQuantWaves)),
                           dim3(kQuantWaves * 64), 0, stream, x + (size_t)b0 * in_feat, ws, R, M);
        if (hipError_t e = hipGetLastError()) return e;
        const int TT = (M + kTB - 1) / kTB;
        const dim3 grid((unsigned)NR * (unsigned)TT);
        float* yb = y + (size_t)b0 * out_feat;
        switch (lv) {
        case 1: launch_gemm_lv<1>(grid, stream, w, ws, yb, R, out_feat, M, NR, TT); break;
        case 2: launch_gemm_lv<2>(grid, stream, w, ws, yb, R, out_feat, M, NR, TT); break;
        case 3: launch_gemm_lv<3>(grid, stream, w, ws, yb, R, out_feat, M, NR, TT); break;
        case 4: launch_gemm_lv<4>(grid, stream, w, ws, yb, R, out_feat, M, NR, TT); break;
        case 5: launch_gemm_lv<5>(grid, stream, w, ws, yb, R, out_feat, M, NR, TT); break;
        case 6: launch_gemm_lv<6>(grid, stream, w, ws, yb, R, out_feat, M, NR, TT); break;
        default: launch_gemm_lv<7>(grid, stream, w, ws, yb, R, out_feat, M, NR, TT); break;
        }
        if (hipError_t e = hipGetLastError()) return e;
    }
    return hipSuccess;
}

}  // namespace vtq
