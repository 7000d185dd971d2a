// q4k_gemm.hip -- exact-integer Q4_K prefill GEMM on i8 MFMA (gfx950).
//
// Replaces linear_q4_k_integer (src/ops/quant.rs:936-980) for large batch:
// y[b][o] = fixed_tree_s part(b, o, s) with, per super-block s,
//   acc  = sum_j sc_j * sum_{k in j} q_k * xq_k          (j = 8 sub-blocks of 32)
//   accm = sum_j m_j  * bsum_j
//   part = (d*dx) * f32(acc) - (dmin*dx) * f32(accm)
//
// Integer work on the matrix cores:
//  * the 6-bit sub-block scale is folded into the weight operand by a 3+3 bit
//    split, sc = 8*sh + sl: A1 = q*sh and A0 = q*sl are both <= 105 (i8), and
//    acc = 8*C1 + C0 exactly (|C1| <= 256*105*127), so one super-block is 16
//    v_mfma_i32_32x32x32_i8 whose accumulators run over all 256 elements;
//  * the min term pairs m_j with bsum_j = 64*bh_j + bl_j: two i8 MFMAs and
//    accm = 64*Ch + Cl in the LDS-operand kernel, one f16 MFMA in the
//    per-wave and split-K kernels (see the per-wave kernel for why that is
//    exact).
// Integer sums are exact in any order, so the MFMA reduction order is free.
// The float epilogue is the reference's, per (b, o, s), in VALU, and the
// fixed_tree over super-blocks is a streamed binary counter:
// fixed_tree(p[0..R)) == fold-right over the balanced trees of the binary
// digits of R, each built left to right as parts arrive.
//
// Three kernels share the activation pre-pass, which writes the token codes
// in the MFMA operand order (gemm_form picks one per launch):
//  * q4k_gemm_pw_kernel (rows of at most 16 super-blocks): each wave forms
//    its own weight operands in registers, no barriers;
//  * q4k_gemm_sk_kernel (grids too small to fill the chip): the same
//    per-wave fold over whole fixed_tree subtrees of a row, one per wave of
//    a workgroup, combined in the tree's order;
//  * q4k_gemm_kernel (longer rows): a workgroup of 4 waves owns 32 weight
//    rows x 128 tokens and builds the weight operands once per super-block
//    in LDS.
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
// and one min-term operand, whichever the launch's GEMM kernel reads (the two
// share their space):
//   xbt [Mp/32][R][32] x 16 B       bl[8] = bsum & 63, bh[8] = bsum >> 6 (i8)
//   xmt [Mp/32][R][64] x 16 B       lane n: f16(64*bh_0..7) of token 32T+n,
//                                   lane 32+n: f16(bl_0..7)
struct GemmWs {
    v4i* xqt;
    float* xdt;
    v4i* xbt;
    v4i* xmt;
};

// Descriptor word 3 of a raw (untyped, stride 0) buffer on gfx9-family parts.
constexpr int kGemmWord3 = 0x00020000;

inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }

inline GemmWs gemm_ws(void* base, int Mp, int R) {
    uint8_t* p = static_cast<uint8_t*>(base);
    GemmWs w;
    w.xqt = reinterpret_cast<v4i*>(p);
    p += align256((size_t)Mp * R * 256);
    w.xdt = reinterpret_cast<float*>(p);
    p += align256((size_t)Mp * R * 4);
    w.xbt = reinterpret_cast<v4i*>(p);
    w.xmt = reinterpret_cast<v4i*>(p);
    return w;
}

// quantize_block_q8 (src/ops/quant.rs:750-771) of every 256-block of every
// batch row: one wave per (token, super-block), written in the tiled layout.
// Workgroup (s, q) holds the 16 consecutive tokens 16q..16q+15 of
// super-block s, so each 256-byte run of the token operands (and the 16
// d / bsum entries beside it) is written by one workgroup at once.
constexpr int kQuantWaves = 16;
__global__ __launch_bounds__(kQuantWaves * 64) void act_quant_tiles_kernel(const float* __restrict__ x, GemmWs ws,
                                                                           int R, int M, int f16_min) {
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
        if (f16_min) {
            // exact in f16: |64*bh| <= 4096 is a multiple of 64, 0 <= bl <= 63
            _Float16* o = reinterpret_cast<_Float16*>(ws.xmt + (size_t)tile * 64 + n);
            o[j] = (_Float16)(float)(s32 - (s32 & 63));  // 64*bh
            o[32 * 8 + j] = (_Float16)(float)(s32 & 63);  // bl, lane 32 + n
        } else {
            int8_t* o = reinterpret_cast<int8_t*>(ws.xbt + (size_t)tile * 32 + n);
            o[j] = (int8_t)(s32 & 63);      // bl
            o[8 + j] = (int8_t)(s32 >> 6);  // bh (arithmetic shift: s32 = 64*bh + bl)
        }
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

// ------------------------------------------- per-wave operand formation

// Rows of at most 16 super-blocks (in_feat <= 4096).  Each wave owns 32
// weight rows x 64 tokens (two 32-token tiles; one tile where two would
// leave the CUs idle) and forms the split weight
// operands of its rows in registers, straight from the 144-byte blocks: no
// LDS operand buffers and no workgroup barrier, so the two waves sharing a
// SIMD drift out of phase and one's MFMAs run beside the other's epilogue.
// One formed operand feeds the MFMAs of both tiles.
//
// A workgroup is four waves on four consecutive 32-row tiles and the same 64
// tokens, so the token operands of a super-block are fetched from L2 once per
// workgroup and the other three waves can hit L1.  Every operand load is a
// raw buffer load whose per-lane part is a fixed register and whose per-step
// part is a scalar offset, so the loop spends no vector instructions on
// addresses.  The token operands run in a ring of four k-steps.
//
// The min term runs on one v_mfma_f32_32x32x16_f16: k 0..7 pair m_j with
// 64*bh_j, k 8..15 pair m_j with bl_j (bsum_j = 64*bh_j + bl_j).  Every
// operand is an integer that f16 holds exactly (m <= 63, |64*bh| <= 4096,
// bl <= 63), every product is exact in f32, and every partial sum is an
// integer below 2^22 in magnitude, so the f32 result is accm exactly, the
// value f32(accm) of the reference (|accm| < 2^24).  The accumulator input
// is +0.0, so a sum with no nonzero term is +0.0, as f32(0) is.
//
// fixed_tree as a binary counter: levels 0 and 1 in registers, levels 2 and
// 3 in the wave's own LDS (each written and read a few times per row); at
// the last super-block the counter folds straight into the result, so level
// 4 (R = 16) is never stored.
//
// Template parameter NT: token tiles per wave (2 in q4k_gemm_pw_kernel; the
// split-K kernel folds one tile per wave with pw_tree<1>).
constexpr int kPwWaves = 4;
constexpr int kPwMaxR = 16;
__host__ __device__ constexpr int pw_level_bytes(int NT) { return NT * 4 * 64 * 16; }  // one tree level of NT tiles
__host__ __device__ constexpr int pw_lds_per_wave(int NT) {
    return 2 * pw_level_bytes(NT) + 2 * 32 * 4;  // levels 2 and 3, then d and dmin of the rows
}

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t rep_byte16(uint32_t v, int j) {
    // byte j of v into both 16-bit halves: {b_j, 0, b_j, 0}
    return __builtin_amdgcn_perm(0u, v, (uint32_t)j | 0x0C000C00u | ((uint32_t)j << 16));
}
__device__ __forceinline__ v4i bload16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0));
}
__device__ __forceinline__ uint32_t pk_f16(uint32_t a, uint32_t b) {  // two small integers as packed f16 (exact)
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz((float)a, (float)b));
}

// The per-wave work: rows o0 .. o0+31 and token tiles NT*tp .. NT*tp+NT-1,
// the parts of super-blocks s0 .. s0+Rl-1 folded by fixed_tree over those Rl
// leaves into res (the row's result when s0 = 0 and Rl = R; the value of one
// subtree when Rl is a power of two and s0 a multiple of it).  Rl <= 16.
// lv: this wave's LDS tree levels 2 and 3; dd: its d / dmin slots.
template <int NT>
__device__ __forceinline__ void pw_tree(const uint8_t* __restrict__ W, const GemmWs& ws, int R, int N, int M, int o0,
                                        int tp, int s0, int Rl, float4* lv, float* dd, float (&res)[NT][16]) {
    constexpr int D = 4;  // k-steps of token operands in flight
    const int lane = threadIdx.x & 63;
    const int r = lane & 31, g = lane >> 5;
    const int Mt = (M + 31) / 32;

    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(ws.xqt, (short)0, Mt * R * 8192, kGemmWord3);
    const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(ws.xmt, (short)0, Mt * R * 1024, kGemmWord3);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(ws.xdt, (short)0, Mt * R * 128, kGemmWord3);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), (short)0, N * R * 144, kGemmWord3);
    uint32_t q0[NT], m0[NT], d0[NT];  // tile bases (scalar); past the end a tile recomputes the last one
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const uint32_t T = (uint32_t)min(NT * tp + t, Mt - 1);
        q0[t] = (T * R + s0) * 8192;
        m0[t] = (T * R + s0) * 1024;
        d0[t] = (T * R + s0) * 128;
    }
    const uint32_t vq = 16u * lane, vd = 4u * r;
    // lane (r, g): header of row r, and code bytes 32h + 16g .. +15 of each
    // quarter h: low nibbles are k-step 2h, high nibbles k-step 2h + 1, both
    // at k = 16g .. 16g + 15 of the step (the B operand's order)
    const uint32_t vh = (uint32_t)min(o0 + r, N - 1) * ((uint32_t)R * 144) + (uint32_t)s0 * 144, vc = vh + 16 + 16 * g;

    uint4 hdr = __builtin_bit_cast(uint4, bload16(rw, vh, 0));
    uint4 qw[4];
#pragma unroll
    for (int h = 0; h < 4; h++) qw[h] = __builtin_bit_cast(uint4, bload16(rw, vc + 32 * h, 0));
    v4i bq[NT][D];  // token operands: ring of D k-steps
#pragma unroll
    for (int j = 0; j < D; j++)
#pragma unroll
        for (int t = 0; t < NT; t++) bq[t][j] = bload16(rq, vq, q0[t] + j * 1024);
    v4i bm[NT];
    float dx[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        bm[t] = bload16(rm, vq, m0[t]);
        dx[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, vd, d0[t], 0));
    }

    float L0[NT][16], L1[NT][16];

    // one super-block: the parts of every tile into p
    auto sblock = [&](int s, float (&p)[NT][16]) __attribute__((always_inline)) {
        const int sn = min(s + 1, Rl - 1);
        // get_scale_min_k4 (src/ops/quant.rs:267-276) of all eight sub-blocks, a byte each
        const uint32_t Y = hdr.y, Z = hdr.z, Wd = hdr.w;
        const uint32_t SCl = Y & 0x3F3F3F3Fu, Ml = Z & 0x3F3F3F3Fu;
        const uint32_t SCh = (Wd & 0x0F0F0F0Fu) | ((Y >> 2) & 0x30303030u);
        const uint32_t Mh = ((Wd >> 4) & 0x0F0F0F0Fu) | ((Z >> 2) & 0x30303030u);
        const uint32_t SHl = (SCl >> 3) & 0x07070707u, SLl = SCl & 0x07070707u;
        const uint32_t SHh = (SCh >> 3) & 0x07070707u, SLh = SCh & 0x07070707u;
        if (g == 0) {
            dd[r] = f16_to_f32_sel(hdr.x & 0xFFFFu);
            dd[32 + r] = f16_to_f32_sel(hdr.x >> 16);
        }
        const uint32_t am0 = pk_f16(Ml & 255u, (Ml >> 8) & 255u), am1 = pk_f16((Ml >> 16) & 255u, Ml >> 24);
        const uint32_t am2 = pk_f16(Mh & 255u, (Mh >> 8) & 255u), am3 = pk_f16((Mh >> 16) & 255u, Mh >> 24);
        const v8h am = __builtin_bit_cast(v8h, v4i{(int)am0, (int)am1, (int)am2, (int)am3});
        hdr = __builtin_bit_cast(uint4, bload16(rw, vh, (uint32_t)sn * 144));
        v16i c1[NT], c0[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) c1[t] = c0[t] = v16i{};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int h = j >> 1, sh = 4 * (j & 1);
            const uint32_t SH = j < 4 ? SHl : SHh, SL = j < 4 ? SLl : SLh;
            const us2 mh = __builtin_bit_cast(us2, rep_byte16(SH, j & 3));
            const us2 ml = __builtin_bit_cast(us2, rep_byte16(SL, j & 3));
            const uint32_t w0 = (qw[h].x >> sh) & 0x0F0F0F0Fu, w1 = (qw[h].y >> sh) & 0x0F0F0F0Fu;
            const uint32_t w2 = (qw[h].z >> sh) & 0x0F0F0F0Fu, w3 = (qw[h].w >> sh) & 0x0F0F0F0Fu;
            const v4i a1 = v4i{nib_mul(w0, mh), nib_mul(w1, mh), nib_mul(w2, mh), nib_mul(w3, mh)};
            const v4i a0 = v4i{nib_mul(w0, ml), nib_mul(w1, ml), nib_mul(w2, ml), nib_mul(w3, ml)};
            if (j & 1) qw[h] = __builtin_bit_cast(uint4, bload16(rw, vc + 32 * h, (uint32_t)sn * 144));
#pragma unroll
            for (int t = 0; t < NT; t++) c1[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bq[t][j % D], c1[t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < NT; t++) c0[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bq[t][j % D], c0[t], 0, 0, 0);
            // refill the ring slot: k-step j + D of this super-block, or of the next
            const uint32_t kk = (uint32_t)(j + D < 8 ? s * 8 + j + D : sn * 8 + j + D - 8) * 1024;
#pragma unroll
            for (int t = 0; t < NT; t++) bq[t][j % D] = bload16(rq, vq, q0[t] + kk);
        }
        // min term (src/ops/quant.rs:876-883): accm = sum_j m_j * bsum_j
        v16f cm[NT];
        float ds[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            cm[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, __builtin_bit_cast(v8h, bm[t]), v16f{}, 0, 0, 0);
            ds[t] = dx[t];
            bm[t] = bload16(rm, vq, m0[t] + (uint32_t)sn * 1024);
            dx[t] = __builtin_bit_cast(float,
                                       __builtin_amdgcn_raw_buffer_load_b32(rd, vd, d0[t] + (uint32_t)sn * 128, 0));
        }
        // epilogue (src/ops/quant.rs:849-898): element i of a lane is row 8*(i/4) + 4*g + i%4, token r
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 dv = *reinterpret_cast<const float4*>(dd + 8 * q + 4 * g);
            const float4 mv = *reinterpret_cast<const float4*>(dd + 32 + 8 * q + 4 * g);
            const float dr[4] = {dv.x, dv.y, dv.z, dv.w}, mr[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int i = 4 * q + e;
#pragma unroll
                for (int t = 0; t < NT; t++)
                    p[t][i] = ((dr[e] * ds[t]) * (float)(8 * c1[t][i] + c0[t][i])) - ((mr[e] * ds[t]) * cm[t][i]);
            }
        }
    };
    auto lds_store = [&](int l, const float (&v)[NT][16]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                lv[((l - 2) * NT + t) * 256 + q * 64 + lane] =
                    make_float4(v[t][4 * q], v[t][4 * q + 1], v[t][4 * q + 2], v[t][4 * q + 3]);
    };
    // v = (level l) + v: the stored block is the left operand
    auto lds_merge = [&](int l, float (&v)[NT][16]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 u = lv[((l - 2) * NT + t) * 256 + q * 64 + lane];
                v[t][4 * q] = u.x + v[t][4 * q];
                v[t][4 * q + 1] = u.y + v[t][4 * q + 1];
                v[t][4 * q + 2] = u.z + v[t][4 * q + 2];
                v[t][4 * q + 3] = u.w + v[t][4 * q + 3];
            }
    };
    auto reg_merge = [&](const float (&l)[NT][16], float (&v)[NT][16]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) v[t][i] = l[t][i] + v[t][i];
    };
    auto reg_copy = [&](float (&l)[NT][16], const float (&v)[NT][16]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 16; i++) l[t][i] = v[t][i];
    };

    // fixed_tree (src/ops/quant.rs:461-476) as a binary counter over s: after
    // leaf s the levels below L = (trailing ones of s) merge into level L.
    int s = 0;
    for (; s + 1 < Rl; s++) {
        float p[NT][16];
        sblock(s, p);
        const int L = __builtin_ctz(~s);
        if (L == 0) {
            reg_copy(L0, p);
        } else {
            reg_merge(L0, p);
            if (L == 1) {
                reg_copy(L1, p);
            } else {
                reg_merge(L1, p);
                if (L == 2) {
                    lds_store(2, p);
                } else {  // L == 3 (s = 7: R <= 16 leaves no higher level open before the last leaf)
                    lds_merge(2, p);
                    lds_store(3, p);
                }
            }
        }
    }
    {
        // last leaf: merge the levels below L, then fold the blocks still open
        // (the set bits of R above L) right to left
        sblock(s, res);
        const int L = __builtin_ctz(~s);
        if (L >= 1) reg_merge(L0, res);
        if (L >= 2) reg_merge(L1, res);
        if (L >= 3) lds_merge(2, res);
        if (L >= 4) lds_merge(3, res);
        if (L < 1 && ((Rl >> 1) & 1)) reg_merge(L1, res);
        if (L < 2 && ((Rl >> 2) & 1)) lds_merge(2, res);
        if (L < 3 && ((Rl >> 3) & 1)) lds_merge(3, res);
    }
}

template <int NT>
__global__ __launch_bounds__(kPwWaves * 64, 2) void q4k_gemm_pw_kernel(const uint8_t* __restrict__ W, GemmWs ws,
                                                                       float* __restrict__ y, int R, int N, int M,
                                                                       int NG, int TP) {
    constexpr int NW = kPwWaves;
    constexpr int kLds = pw_lds_per_wave(NT);
    extern __shared__ __align__(16) unsigned char lds[];
    const int lane = threadIdx.x & 63, wave = wave_id();
    float4* lv = reinterpret_cast<float4*>(lds + (size_t)wave * kLds);  // [level 2..][tile][q][lane]
    float* dd = reinterpret_cast<float*>(lds + (size_t)wave * kLds + 2 * pw_level_bytes(NT));  // d[32], dmin[32]

    // Workgroup i runs on XCD i % 8: consecutive slots of one XCD take its
    // 128-row groups in turn with the same token group, so the workgroups
    // running there at once share their token operands in that XCD's L2 (a
    // row group's weights come back for the next token group from the
    // memory-side cache).  With 14336 x 4096 at 512 tokens: 100.3 against
    // 102.0 us per call for row groups as the inner index (four rounds).
    const int id = blockIdx.x, full = (NG / 8) * 8 * TP;
    int rg, tp;
    if (id < full) {
        const int k = id >> 3, NGx = NG / 8;
        rg = (k % NGx) * 8 + (id & 7);
        tp = k / NGx;
    } else {
        rg = (NG / 8) * 8 + (id - full) / TP;
        tp = (id - full) % TP;
    }
    const int o0 = (rg * NW + wave) * 32;
    const int r = lane & 31, g = lane >> 5;
    const int Mt = (M + 31) / 32;
    float res[NT][16];
    pw_tree<NT>(W, ws, R, N, M, o0, tp, 0, R, lv, dd, res);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int T = NT * tp + t, tok = T * 32 + r;
        if (T < Mt && tok < M) {
            float* yrow = y + (size_t)tok * N;
            const bool vec = (N & 3) == 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int o = o0 + 8 * q + 4 * g;
                if (vec && o + 3 < N) {
                    *reinterpret_cast<float4*>(yrow + o) =
                        make_float4(res[t][4 * q], res[t][4 * q + 1], res[t][4 * q + 2], res[t][4 * q + 3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (o + e < N) yrow[o + e] = res[t][4 * q + e];
                }
            }
        }
    }
}

// Split-K for grids too small to fill the chip (prompt-sized batches): a
// workgroup owns one 32-row tile and one 32-token tile, and wave w folds
// chunk w of the row's super-blocks with pw_tree.  The chunks are whole
// subtrees of fixed_tree: the balanced trees of R's binary digits (from the
// highest), each cut into pieces of C leaves (a tree smaller than C is one
// piece).  Wave 0 then combines the chunk values as fixed_tree does: within
// each tree pairwise, level by level, and the trees folded right to left
// (fixed_tree(p[0..R)) == T_high + (... + T_low)).  Any row length to 127
// super-blocks: C <= 16 keeps pw_tree's counter within its four levels.
constexpr int kSkMaxWaves = 12;

__host__ __device__ inline int sk_chunks(int R, int C) {
    int n = 0;
    for (int k = 6; k >= 0; k--)
        if ((R >> k) & 1) n += (1 << k) >= C ? (1 << k) / C : 1;
    return n;
}

// The piece size for a grid of T tiles: the smallest that keeps the launch
// within 2048 waves (8 per CU), else the smallest that needs at most
// kSkMaxWaves chunks (every row length below 128 super-blocks has one).
static int sk_piece(int R, int T) {
    int first = 0;
    for (int C = 1; C <= 16; C <<= 1) {
        const int n = sk_chunks(R, C);
        if (n > kSkMaxWaves) continue;
        if (!first) first = C;
        if ((long)T * n <= 2048) return C;
    }
    return first;
}

__global__ __launch_bounds__(kSkMaxWaves * 64, 1) void q4k_gemm_sk_kernel(const uint8_t* __restrict__ W, GemmWs ws,
                                                                           float* __restrict__ y, int R, int N, int M,
                                                                           int C) {
    constexpr int kW = pw_lds_per_wave(1);
    extern __shared__ __align__(16) unsigned char lds[];
    const int lane = threadIdx.x & 63, wave = wave_id(), nw = (int)(blockDim.x >> 6);
    float4* lv = reinterpret_cast<float4*>(lds + (size_t)wave * kW);
    float* dd = reinterpret_cast<float*>(lds + (size_t)wave * kW + 2 * pw_level_bytes(1));
    float4* cv = reinterpret_cast<float4*>(lds + (size_t)nw * kW);  // [chunk][q][lane]
    const int Mt = (M + 31) / 32, rt = (int)blockIdx.x / Mt, tt = (int)blockIdx.x % Mt;
    const int r = lane & 31, g = lane >> 5;
    // this wave's chunk
    int s0 = 0, len = 0;
    {
        int i = wave, base = 0;
        for (int k = 6; k >= 0; k--) {
            if (!((R >> k) & 1)) continue;
            const int size = 1 << k, n = size >= C ? size / C : 1, sz = size >= C ? C : size;
            if (i < n) {
                s0 = base + i * sz;
                len = sz;
                break;
            }
            i -= n;
            base += size;
        }
    }
    float res[1][16];
    pw_tree<1>(W, ws, R, N, M, rt * 32, tt, s0, len, lv, dd, res);
#pragma unroll
    for (int q = 0; q < 4; q++)
        cv[(wave * 4 + q) * 64 + lane] = make_float4(res[0][4 * q], res[0][4 * q + 1], res[0][4 * q + 2], res[0][4 * q + 3]);
    __syncthreads();
    if (wave != 0) return;
    // the trees from the lowest binary digit up (the fold runs right to
    // left); a tree's first chunk follows the chunks of the digits above it
    auto pieces = [&](int k) { return (1 << k) >= C ? (1 << k) / C : 1; };
    float acc[16];
    bool first = true;
    for (int k = 0; k < 7; k++) {
        if (!((R >> k) & 1)) continue;
        int c0 = 0;
        for (int k2 = k + 1; k2 < 7; k2++)
            if ((R >> k2) & 1) c0 += pieces(k2);
        const int n = pieces(k);
        for (int st = 1; st < n; st <<= 1)
            for (int i = 0; i + st < n; i += 2 * st)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    float4& a = cv[((c0 + i) * 4 + q) * 64 + lane];
                    const float4 b = cv[((c0 + i + st) * 4 + q) * 64 + lane];
                    a = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
                }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 tv = cv[(c0 * 4 + q) * 64 + lane];
            const float t4[4] = {tv.x, tv.y, tv.z, tv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) acc[4 * q + e] = first ? t4[e] : t4[e] + acc[4 * q + e];
        }
        first = false;
    }
    const int tok = tt * 32 + r;
    if (tok < M) {
        float* yrow = y + (size_t)tok * N;
        const bool vec = (N & 3) == 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int o = rt * 32 + 8 * q + 4 * g;
            if (vec && o + 3 < N) {
                *reinterpret_cast<float4*>(yrow + o) = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (o + e < N) yrow[o + e] = acc[4 * q + e];
            }
        }
    }
}

size_t q4k_gemm_workspace_bytes(int batch, int in_feat) {
    const int Mp = (min(batch, kChunkM) + 31) / 32 * 32;
    const size_t R = in_feat / 256;
    return align256((size_t)Mp * R * 256) + align256((size_t)Mp * R * 4) + (size_t)Mp * R * 32;
}

int q4k_gemm_max_in_feat() { return 127 * 256; }

template <int LV>
static void launch_gemm_lv(dim3 grid, hipStream_t stream, const uint8_t* w, GemmWs ws, float* y, int R, int N, int M,
                           int NR, int TT) {
    hipLaunchKernelGGL(q4k_gemm_kernel<LV>, grid, dim3(256), 0, stream, w, ws, y, R, N, M, NR, TT);
}

template <int NT>
static hipError_t launch_pw_t(hipStream_t stream, const uint8_t* w, GemmWs ws, float* y, int R, int N, int M, int NG,
                              int TP) {
    const size_t lds = (size_t)kPwWaves * pw_lds_per_wave(NT);
    if (hipError_t e = allow_dynamic_lds(reinterpret_cast<const void*>(&q4k_gemm_pw_kernel<NT>), lds)) return e;
    hipLaunchKernelGGL((q4k_gemm_pw_kernel<NT>), dim3((unsigned)NG * (unsigned)TP), dim3(kPwWaves * 64), lds,
                       stream, w, ws, y, R, N, M, NG, TP);
    return hipGetLastError();
}

// Which kernel takes a launch (M tokens in Mt 32-token tiles): 3 the
// split-K kernel, for grids too small to fill the chip; else 2 the per-wave
// kernel with two token tiles per wave for rows of at most 16 super-blocks,
// 0 the LDS-operand kernel for longer rows.  Split-K takes rows of at most 16
// super-blocks up to 1024 tiles of 32 x 32, and longer rows where the
// LDS-operand kernel would launch fewer than 256 workgroups (measured
// crossovers, pre-pass included: 4096 x 4096 at 256 tokens 25.5 against
// 26.3 us for the LDS-operand kernel, 11264 x 2048 at 96 tokens 19.5 against
// 18.8 us for the per-wave kernel; 4096 x 11008 at 128 tokens 43.4 against
// 56.5 us, at 256 tokens 76.6 against 59.3 us).  The split-K and per-wave
// forms address the weights with 32-bit buffer offsets.
static int gemm_form(int R, int N, int M, int Mt) {
    if ((size_t)N * R * 144 >= ((size_t)1 << 31)) return 0;
    if (R <= kPwMaxR) return (long)((N + 31) / 32) * Mt <= 1024 ? 3 : 2;
    return (long)((N + kTO - 1) / kTO) * ((M + kTB - 1) / kTB) < 256 ? 3 : 0;
}

static hipError_t launch_sk(hipStream_t stream, const uint8_t* w, GemmWs ws, float* y, int R, int N, int M, int Mt) {
    const unsigned NR = (unsigned)((N + 31) / 32);
    const int C = sk_piece(R, (int)NR * Mt), nw = sk_chunks(R, C);
    if (C == 0 || nw > kSkMaxWaves) return hipErrorInvalidValue;
    const size_t lds = (size_t)nw * pw_lds_per_wave(1) + (size_t)nw * 4 * 64 * 16;
    if (hipError_t e = allow_dynamic_lds(reinterpret_cast<const void*>(&q4k_gemm_sk_kernel), lds)) return e;
    hipLaunchKernelGGL(q4k_gemm_sk_kernel, dim3(NR * (unsigned)Mt), dim3((unsigned)nw * 64), lds, stream, w, ws, y, R,
                       N, M, C);
    return hipGetLastError();
}

static hipError_t launch_pw(hipStream_t stream, const uint8_t* w, GemmWs ws, float* y, int R, int N, int M, int Mt) {
    const int NG = (N + 32 * kPwWaves - 1) / (32 * kPwWaves);
    return launch_pw_t<2>(stream, w, ws, y, R, N, M, NG, (Mt + 1) / 2);
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
        // the per-wave forms where gemm_form allows them (both read the
        // f16 min-term operand); Mp is a multiple of 32, so Mp / 16 pre-pass
        // groups cover every token slot
        const int form = gemm_form(R, out_feat, M, Mp / 32);
        const bool pw = form != 0;
        hipLaunchKernelGGL(act_quant_tiles_kernel, dim3((unsigned)R, (unsigned)(Mp / kQuantWaves)),
                           dim3(kQuantWaves * 64), 0, stream, x + (size_t)b0 * in_feat, ws, R, M, pw ? 1 : 0);
        if (hipError_t e = hipGetLastError()) return e;
        float* yb = y + (size_t)b0 * out_feat;
        if (pw) {
            const hipError_t e = form == 3 ? launch_sk(stream, w, ws, yb, R, out_feat, M, Mp / 32)
                                           : launch_pw(stream, w, ws, yb, R, out_feat, M, Mp / 32);
            if (e) return e;
            continue;
        }
        const int TT = (M + kTB - 1) / kTB;
        const dim3 grid((unsigned)NR * (unsigned)TT);
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
