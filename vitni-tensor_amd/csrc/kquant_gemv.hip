// kquant_gemv.hip -- exact-integer Q4_K / Q6_K decode GEMV for gfx950.
//
// Replaces linear_q4_k_integer[_parallel] (src/ops/quant.rs:936-980,
// :1149-1196) and linear_q6_k_integer[_parallel] (:1060-1146) for any batch;
// each batch row is one grid.y slice.
//
// Lane mapping (both kernels): a window is 16 consecutive super-blocks of one
// weight row; lane 4g+k of a wave handles quarter k of the window's block g,
// so the 64 lanes together read the window's 2304 (Q4_K) or 3360 (Q6_K)
// contiguous bytes.  Per window: integer sums with v_dot4_i32_i8, reduced over
// the 4 lanes of a block with DPP (exact in any order); the per-block float
// epilogue evaluated exactly as the reference writes it; then the pinned
// fixed_tree over the window's 16 blocks and over the row's windows.
// fixed_tree(p[0..R)) equals fixed_tree over 16-aligned windows of
// fixed_tree(window), because the first four levels of the reference's tree
// only pair blocks inside an aligned window; padded slots hold -0.0, the
// exact identity of +.
//
// Every workgroup quantizes the whole activation row into LDS
// (quantize_block_q8, src/ops/quant.rs:750-771) before it can use a weight.
//
// kquant_rows_kernel (rows of at most 3 windows for Q4_K, in_feat <= 12288,
// and 2 for Q6_K, in_feat <= 8192; matrices under 2 GiB): each
// lane copies its activation quarter of every window from LDS into registers
// once, then streams whole rows (all windows of a row per step, static window
// indices) through a ring of D register buffers.  Rows are dealt to waves
// round-robin, so at any moment the chip reads one contiguous band of the
// matrix.  Weight loads are raw buffer loads: a slot past the wave's last row
// gets an offset beyond the buffer's size, which the hardware answers with
// zeros and no memory traffic, so every load stays unconditional (vmcnt
// waits stay exact) without re-reading any row.
//
// kquant_windows_kernel (any in_feat up to 32768): the unit is one window;
// the activation quarter is re-read from LDS per unit.
#include "vtq_device.h"
#include "vtq_kernels.h"
#include "vtq_libm.h"
#include "vtq_sumsq.h"

#include <type_traits>

namespace vtq {

constexpr int kMaxWindows = 8;  // R <= 128 super-blocks: in_feat <= 32768 (LDS: 1 KiB per block)

// ------------------------------------------------ activation in LDS

// Every lane of the quantizing wave stores its copy of d and of its run
// sums (unconditional stores, no exec-mask branches); readers pick lane 4r
// for the sum of 16-element run r and lane 8j for sub-block j.
struct ActLds {
    uint32_t* qs;  // [R*64] packed int8 codes, word = 4 elements
    float* d;      // [R*64] d of block b at [64b + any lane]
    int* s16;      // [R*64] sum of run r at [64b + 4r]
    int* s32;      // [R*64] bsum of sub-block j at [64b + 8j]
    float* ws;     // [NW*8] per-wave window sums (windows kernel)
};

// Byte offsets of the activation arrays; every array starts 16-byte aligned.
__host__ __device__ constexpr size_t act_off_d(int R) { return (size_t)R * 256; }
__host__ __device__ constexpr size_t act_off_s16(int R) { return (size_t)R * 512; }
__host__ __device__ constexpr size_t act_off_s32(int R) { return (size_t)R * 768; }
__host__ __device__ constexpr size_t act_off_ws(int R) { return (size_t)R * 1024; }

__device__ __forceinline__ ActLds act_lds_layout(unsigned char* base, int R) {
    ActLds a;
    a.qs = reinterpret_cast<uint32_t*>(base);
    a.d = reinterpret_cast<float*>(base + act_off_d(R));
    a.s16 = reinterpret_cast<int*>(base + act_off_s16(R));
    a.s32 = reinterpret_cast<int*>(base + act_off_s32(R));
    a.ws = reinterpret_cast<float*>(base + act_off_ws(R));
    return a;
}

constexpr int kNW = 16;        // waves per workgroup; one workgroup per CU
constexpr int kXPerWave = 4;   // activation blocks each wave loads up front (R <= 64 fully overlapped)
__host__ __device__ constexpr size_t act_lds_end(int R) { return act_off_ws(R) + kNW * kMaxWindows * 4; }
size_t act_lds_bytes(int R) { return act_lds_end(R); }
// the sum-of-squares walk's tables: past the products (npass x 16 KiB) and the scale
__host__ __device__ constexpr size_t norm_walk_off(int R) { return act_lds_end(R) + (size_t)(R + 15) / 16 * 16384 + 16; }

// quantize_block_q8 (src/ops/quant.rs:750-771) of 256-block b, held as one
// float4 per lane (elements 4L..4L+3), into the LDS activation arrays.
__device__ __forceinline__ void quantize_block_to_lds(float4 v, int b, const ActLds& a) {
    const int lane = threadIdx.x & 63;
    uint32_t packed;
    int s16, s32;
    const float d = quant_block_wave(v, &packed, &s16, &s32);
    a.qs[b * 64 + lane] = packed;
    a.s16[b * 64 + lane] = s16;
    a.s32[b * 64 + lane] = s32;
    a.d[b * 64 + lane] = d;
}

// The activation blocks of wave `wave`: b = wave + kNW*j.  The first
// kXPerWave are loaded by load_act (issued before any weight load), the rest
// are loaded where they are quantized.
template <int XPW>
__device__ __forceinline__ void load_act(float4 (&xv)[XPW], const float* __restrict__ xb, int R, int wave) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < XPW; j++) {
        const int b = wave + kNW * j;
        if (b < R) xv[j] = reinterpret_cast<const float4*>(xb + (size_t)b * 256)[lane];
    }
}
template <int XPW>
__device__ __forceinline__ void quantize_act(const float4 (&xv)[XPW], const float* __restrict__ xb, int R, int wave,
                                             const ActLds& act) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < XPW; j++) {
        const int b = wave + kNW * j;
        if (b < R) quantize_block_to_lds(xv[j], b, act);
    }
    for (int b = wave + kNW * XPW; b < R; b += kNW)
        quantize_block_to_lds(reinterpret_cast<const float4*>(xb + (size_t)b * 256)[lane], b, act);
}

// fixed_tree over the per-window sums wv[0..nwin) (stride form, static indices).
__device__ __forceinline__ float window_tree(float (&wv)[kMaxWindows], int nwin) {
#pragma unroll
    for (int s = 1; s < kMaxWindows; s <<= 1) {
#pragma unroll
        for (int i = 0; i + s < kMaxWindows; i += 2 * s) {
            if (i + s < nwin) wv[i] = wv[i] + wv[i + s];
        }
    }
    return wv[0];
}
template <int N>
__device__ __forceinline__ float windows_tree(float (&wv)[N]) {
#pragma unroll
    for (int s = 1; s < N; s <<= 1)
#pragma unroll
        for (int i = 0; i + s < N; i += 2 * s) wv[i] = wv[i] + wv[i + s];
    return wv[0];
}

// fixed_tree over the 16 block slots of a window; slot g lives in lanes
// 4g..4g+3 and slots past the row's end hold -0.0.  The stride form pairs
// slot i with i+s for i a multiple of 2s; the sum is formed in the higher
// slot instead (IEEE addition is commutative, so a+b and b+a are the same
// bits and only the association has to match the reference):
//   stride 1, 2: row_shr:4, row_shr:8 inside each 16-lane row -> row sums at lane 15
//   stride 4:    row_bcast:15 adds row 0 into row 1 and row 2 into row 3
//   stride 8:    row_bcast:31 adds (row0+row1) into row 3
// The window sum ends in lane 63 and is read out once.
//
// Each step is one v_add_f32_dpp with the destination equal to the unshifted
// operand and bound_ctrl off: a lane whose source lane is outside its row, or
// whose row is masked off, is not written and keeps v, which is v + (-0.0)
// bit for bit (f32 denormals are not flushed).  The s_nop 1 ahead of each
// step covers the two wait states between a VALU write of a VGPR and a DPP
// read of it; the one at the end covers the readlane that follows.
#define VTQ_DPP_ADD(ctrl) "s_nop 1\n\tv_add_f32_dpp %0, %0, %0 " ctrl " bank_mask:0xf\n\t"
__device__ __forceinline__ float window16_tree(float v) {
    asm(VTQ_DPP_ADD("row_shr:4 row_mask:0xf")      // lanes 0..3 of a row keep v
        VTQ_DPP_ADD("row_shr:8 row_mask:0xf")      //
        VTQ_DPP_ADD("row_bcast:15 row_mask:0xa")   // row 0 into row 1, row 2 into row 3
        VTQ_DPP_ADD("row_bcast:31 row_mask:0x8")   // (row0+row1) into row 3
        "s_nop 1"
        : "+v"(v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// The same for two rows of at most 8 block slots each, row h in lanes
// 32h..32h+31: strides 1, 2 and 4 of window16_tree; the sums end in lanes 31
// (row 0) and 63 (row 1).
__device__ __forceinline__ float2 window8x2_tree(float v) {
    asm(VTQ_DPP_ADD("row_shr:4 row_mask:0xf")
        VTQ_DPP_ADD("row_shr:8 row_mask:0xf")
        VTQ_DPP_ADD("row_bcast:15 row_mask:0xa")
        "s_nop 1"
        : "+v"(v));
    return make_float2(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63)));
}
#undef VTQ_DPP_ADD

// ------------------------------------------------------- raw buffer loads

// Descriptor word 3 for raw (untyped, stride 0) buffers on gfx9-family parts.
constexpr int kBufferWord3 = 0x00020000;
// A load at this offset or beyond is out of range for every buffer the rows
// kernel accepts (size < 2 GiB): it returns zeros without touching memory.
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load2(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
}

// ------------------------------------------------------------------ Q4_K

struct Q4K {
    static constexpr int kBytes = 144;
    static constexpr int kRowsMaxWindows = 3;  // rows kernel without register spills
    struct Regs {
        uint4 hdr, qa, qb;
    };
    // the lane's activation quarter: sub-blocks 2k (xl) and 2k+1 (xh) of block g
    struct X {
        uint32_t xl[8], xh[8];
        int bs_lo, bs_hi;
        float dx;
    };
    // get_scale_min_k4 (src/ops/quant.rs:267-276) for j = 2k, 2k+1, two
    // bytes at a time, without branching on the lane's k:
    //   j < 4:  sc = s[j] & 63,                       m = s[j+4] & 63
    //   j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4, m = (s[j+4] >> 4) | (s[j] >> 6) << 4
    struct Lane {
        int sh;
        bool hi;
        uint32_t lowmask, topmask;
    };
    __device__ static Lane lane_consts(int k) {
        Lane c;
        c.sh = 16 * (k & 1);
        c.hi = k >= 2;
        c.lowmask = c.hi ? 0x0F0Fu : 0x3F3Fu;
        c.topmask = c.hi ? 0x3030u : 0u;
        return c;
    }
    __device__ static void load(Regs& r, const uint8_t* __restrict__ blk, int k) {
        r.hdr = *reinterpret_cast<const uint4*>(blk);
        r.qa = *reinterpret_cast<const uint4*>(blk + 16 + 32 * k);
        r.qb = *reinterpret_cast<const uint4*>(blk + 32 + 32 * k);
    }
    __device__ static void bload(Regs& r, __amdgpu_buffer_rsrc_t rs, uint32_t off, int k) {
        r.hdr = buf_load16(rs, off);
        r.qa = buf_load16(rs, off + 16 + 32 * k);
        r.qb = buf_load16(rs, off + 32 + 32 * k);
    }
    __device__ static void load_x(X& x, const ActLds& act, int b, int k) {
        const uint4* xw4 = reinterpret_cast<const uint4*>(act.qs + b * 64 + 16 * k);
        const uint4 l0 = xw4[0], l1 = xw4[1], h0 = xw4[2], h1 = xw4[3];
        x.xl[0] = l0.x; x.xl[1] = l0.y; x.xl[2] = l0.z; x.xl[3] = l0.w;
        x.xl[4] = l1.x; x.xl[5] = l1.y; x.xl[6] = l1.z; x.xl[7] = l1.w;
        x.xh[0] = h0.x; x.xh[1] = h0.y; x.xh[2] = h0.z; x.xh[3] = h0.w;
        x.xh[4] = h1.x; x.xh[5] = h1.y; x.xh[6] = h1.z; x.xh[7] = h1.w;
        x.bs_lo = act.s32[b * 64 + 16 * k];
        x.bs_hi = act.s32[b * 64 + 16 * k + 8];
        x.dx = act.d[b * 64];
    }
    // dot_q4k_q8_block (src/ops/quant.rs:849-898) for quarter k = sub-blocks
    // 2k, 2k+1; returns this block's part (identical in the 4 lanes).
    __device__ static float part(const Regs& r, const X& x, const Lane& c, bool valid) {
        const uint32_t qw[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        int s_lo = 0, s_hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s_lo = __builtin_amdgcn_sdot4((int)(qw[i] & 0x0F0F0F0Fu), (int)x.xl[i], s_lo, false);
            s_hi = __builtin_amdgcn_sdot4((int)((qw[i] >> 4) & 0x0F0F0F0Fu), (int)x.xh[i], s_hi, false);
        }
        const uint32_t A = r.hdr.w >> c.sh, B = r.hdr.y >> c.sh, C = r.hdr.z >> c.sh;
        const uint32_t scp = ((c.hi ? A : B) & c.lowmask) | ((B >> 2) & c.topmask);
        const uint32_t mp = ((c.hi ? (A >> 4) : C) & c.lowmask) | ((C >> 2) & c.topmask);
        // every factor fits 24 bits (sc, m <= 63; |s| <= 60960; |bsum| <= 4064): full-rate v_mad_i32_i24
        int acc = __mul24((int)(scp & 0xFFu), s_lo) + __mul24((int)(scp >> 8), s_hi);
        int accm = __mul24((int)(mp & 0xFFu), x.bs_lo) + __mul24((int)(mp >> 8), x.bs_hi);
        acc = quad_sum_i(acc);
        accm = quad_sum_i(accm);
        const float d = f16_hw(r.hdr.x & 0xFFFFu);
        const float dmin = f16_hw(r.hdr.x >> 16);
        const float t1 = (d * x.dx) * (float)acc;
        const float t2 = (dmin * x.dx) * (float)accm;
        return valid ? t1 - t2 : -0.0f;
    }
};

// ------------------------------------------------------------------ Q6_K

// 16 bytes from a 2-byte-aligned address, as one global_load_dwordx4 (the
// vector memory path runs in unaligned mode on this target).
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
__device__ __forceinline__ uint4 load16_u(const uint8_t* p) {
    const u32x4_a2 v = *reinterpret_cast<const u32x4_a2*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ int sext8(uint32_t v, int byte) { return (int)(int8_t)((v >> (8 * byte)) & 0xFFu); }

struct Q6K {
    static constexpr int kBytes = 210;
    static constexpr int kRowsMaxWindows = 2;
    struct Regs {
        uint4 b0, b1, hh;
        uint4 sc;      // scale bytes 192..207 (funnel-shifted)
        uint32_t d;    // f16 bits of d
    };
    // the lane's activation: runs 8hf+t+2q (q = 0..3) of block g, with
    // m_q = -32 * (sum of run q) to fold the code offset -32 in exactly
    struct X {
        uint4 x1, x2, x3, x4;
        int m1, m2, m3, m4;
        float dx;
    };
    // Lane k: hf = k>>1 (128-element half), t = k&1 (positions l in [16t, 16t+16)).
    struct Lane {
        int hf, t;
    };
    __device__ static Lane lane_consts(int k) { return Lane{k >> 1, k & 1}; }
    // One unaligned 16-byte load per run (see bload); every read stays
    // inside the 210-byte block.
    __device__ static void load(Regs& r, const uint8_t* __restrict__ blk, int k) {
        const int hf = k >> 1, t = k & 1;
        r.b0 = load16_u(blk + 64 * hf + 16 * t);
        r.b1 = load16_u(blk + 64 * hf + 32 + 16 * t);
        r.hh = load16_u(blk + 128 + 32 * hf + 16 * t);
        r.sc = load16_u(blk + 192);
        r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
    }
    // Buffer loads at 2-byte-aligned offsets: the HSA runtime runs the shader
    // memory path in unaligned mode (the compiler itself emits dwordx4 loads
    // for byte-aligned memcpy on this target), so each 16-byte run is one
    // load with no funnel shift.
    __device__ static void bload(Regs& r, __amdgpu_buffer_rsrc_t rs, uint32_t blk, int k) {
        const int hf = k >> 1, t = k & 1;
        r.b0 = buf_load16(rs, blk + 64 * hf + 16 * t);
        r.b1 = buf_load16(rs, blk + 64 * hf + 32 + 16 * t);
        r.hh = buf_load16(rs, blk + 128 + 32 * hf + 16 * t);
        r.sc = buf_load16(rs, blk + 192);
        r.d = buf_load2(rs, blk + 208);
    }
    // activation words: element 128hf + 16t + 32q + 4i -> word 32hf + 4t + 8q + i;
    // run (bucket) of q is 8hf + t + 2q, its sum sits at lane 4 * run
    __device__ static void load_x(X& x, const ActLds& act, int b, int k) {
        const int hf = k >> 1, t = k & 1;
        const uint32_t* xw = act.qs + b * 64 + 32 * hf + 4 * t;
        x.x1 = *reinterpret_cast<const uint4*>(xw);
        x.x2 = *reinterpret_cast<const uint4*>(xw + 8);
        x.x3 = *reinterpret_cast<const uint4*>(xw + 16);
        x.x4 = *reinterpret_cast<const uint4*>(xw + 24);
        const int* s16 = act.s16 + b * 64 + 4 * (8 * hf + t);
        x.m1 = -32 * s16[0];
        x.m2 = -32 * s16[8];
        x.m3 = -32 * s16[16];
        x.m4 = -32 * s16[24];
        x.dx = act.d[b * 64];
    }
    // dot_q6k_q8_block (src/ops/quant.rs:995-1057): buckets 8hf+t+2q (q = 0..3)
    // are exactly one 16-element run each; (code - 32) is folded in as
    // sum(code*x) - 32*sum(x) with the run sums from the activation pass,
    // the second term as the starting value of the dot accumulator.
    __device__ static float part(const Regs& r, const X& x, const Lane& c, bool valid) {
        const uint32_t B0[4] = {r.b0.x, r.b0.y, r.b0.z, r.b0.w};
        const uint32_t B1[4] = {r.b1.x, r.b1.y, r.b1.z, r.b1.w};
        const uint32_t H[4] = {r.hh.x, r.hh.y, r.hh.z, r.hh.w};
        const uint32_t X1[4] = {x.x1.x, x.x1.y, x.x1.z, x.x1.w}, X2[4] = {x.x2.x, x.x2.y, x.x2.z, x.x2.w};
        const uint32_t X3[4] = {x.x3.x, x.x3.y, x.x3.z, x.x3.w}, X4[4] = {x.x4.x, x.x4.y, x.x4.z, x.x4.w};
        int S1 = x.m1, S2 = x.m2, S3 = x.m3, S4 = x.m4;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q1 = (B0[i] & 0x0F0F0F0Fu) | ((H[i] & 0x03030303u) << 4);
            const uint32_t q2 = (B1[i] & 0x0F0F0F0Fu) | ((H[i] & 0x0C0C0C0Cu) << 2);
            const uint32_t q3 = ((B0[i] >> 4) & 0x0F0F0F0Fu) | (H[i] & 0x30303030u);
            const uint32_t q4 = ((B1[i] >> 4) & 0x0F0F0F0Fu) | ((H[i] >> 2) & 0x30303030u);
            S1 = __builtin_amdgcn_sdot4((int)q1, (int)X1[i], S1, false);
            S2 = __builtin_amdgcn_sdot4((int)q2, (int)X2[i], S2, false);
            S3 = __builtin_amdgcn_sdot4((int)q3, (int)X3[i], S3, false);
            S4 = __builtin_amdgcn_sdot4((int)q4, (int)X4[i], S4, false);
        }
        // scales: i8 at 192 + 8hf + t + 2q -> bytes t, t+2 of dwords 2hf and 2hf+1
        const uint32_t sa = c.hf ? r.sc.z : r.sc.x, sb = c.hf ? r.sc.w : r.sc.y;
        // |sc| <= 64 and |sum| <= 16*31*127: every product fits v_mad_i32_i24
        int acc = __mul24(sext8(sa, c.t), S1) + __mul24(sext8(sa, c.t + 2), S2) +
                  __mul24(sext8(sb, c.t), S3) + __mul24(sext8(sb, c.t + 2), S4);
        acc = quad_sum_i(acc);
        const float d = f16_hw(r.d);
        return valid ? (d * x.dx) * (float)acc : -0.0f;
    }
};

// ------------------------------------------------------------ rows kernel

// Row j of wave gw is gw + j*tw (tw = waves in the grid); lane j keeps that
// row's result and the wave stores its rows once at the end.  Waves are
// numbered in groups of four: wave w of workgroup b is
// gw = 4*(b + G*(w/4)) + w%4 (G workgroups), so each workgroup reads four
// bands of four consecutive rows, and consecutive 4-row bands fall on
// consecutive workgroups (hence on different XCDs).  Measured faster than
// 16 consecutive rows per workgroup.
//
// Weight loads issued before the activation is quantized share the memory
// system with the activation reads and delay them (the activation is needed
// by every workgroup before any weight can be used), so how much is issued
// early is tuned per shape:
//   PRE   ring slots (whole rows) loaded before the activation reads return;
//   PREW  (PRE = 0 only) windows of row 0 loaded before the activation reads
//         return, the rest of the row after the workgroup's quantization;
//   POSTX the remaining D - PRE slots are issued as soon as this wave's own
//         activation reads have returned (before quantizing), instead of
//         after the workgroup barrier.
// With PREW, a workgroup barrier right after the activation loads are issued
// makes every wave's activation requests precede every weight request of the
// workgroup in the CU's memory pipeline.
//
// The output rows are the concatenation of up to three weight matrices that
// share the activation (RowsArgs); EPI selects what is stored:
//   kEpiStore       y[r] = row r . x
//   kEpiAccumulate  y[r] = y[r] + row r . x   (the reference's residual add)
//   kEpiSwiGLU      two matrices of equal rows; y[i] = silu(g) * u with
//                   g = W0 row i . x, u = W1 row i . x and silu(g) =
//                   g / (1 + expf(-g))  (forward_quantized.rs SwiGLU)
//
// HALF (rows of at most 8 super-blocks): a wave step takes a pair of rows,
// lanes 32h + 4g + k on row 2p + h, so no lane holds a padding slot; the
// unit dealt to waves is the pair, and lane j stores pair j's two results.
template <class Fmt, int NWIN, int D, int PRE, int PREW, bool POSTX, int EPI, bool MULTI, bool NORM, bool HALF = false>
__global__ __launch_bounds__(kNW * 64) void kquant_rows_kernel(const float* __restrict__ x, RowsArgs args,
                                                               float* __restrict__ y, int R) {
    constexpr int NM = EPI == kEpiSwiGLU ? 2 : 1;  // matrices read per output row
    extern __shared__ __align__(16) unsigned char lds[];
    const ActLds act = act_lds_layout(lds, R);
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    static_assert(!HALF || NWIN == 1, "HALF pairs rows of one window");
    constexpr int RPS = HALF ? 2 : 1;  // rows per wave step
    const int g = HALF ? ((lane >> 2) & 7) : (lane >> 2), k = lane & 3, hh = HALF ? lane >> 5 : 0;
    const int out_feat = EPI == kEpiSwiGLU ? args.rows[0] : args.rows[0] + args.rows[1] + args.rows[2];
    const float* xb = x + (size_t)blockIdx.y * (args.x_stride ? (size_t)args.x_stride : (size_t)R * 256);
    float* yb = y + (size_t)blockIdx.y * out_feat;
    const uint32_t row_bytes = args.row_stride ? args.row_stride : (uint32_t)R * Fmt::kBytes;
    static_assert(PREW == 0 || (PRE == 0 && PREW < NWIN && !POSTX), "PREW splits row 0 of a PRE = 0 ring");
    const int tw = gridDim.x * kNW;
    const int gw = 4 * ((int)blockIdx.x + (int)gridDim.x * (wave >> 2)) + (wave & 3);
    const int units = (out_feat + RPS - 1) / RPS;
    const int nrows = gw < units ? (units - 1 - gw) / tw + 1 : 0;  // steps of this wave, <= 64 (launcher)

    // R <= 16 * NWIN: each wave holds at most NWIN activation blocks
    float4 xv[NWIN], nw[NWIN];
    load_act(xv, xb, R, wave);
    if constexpr (NORM) load_act(nw, args.norm_w, R, wave);
    if constexpr (PREW > 0) __builtin_amdgcn_s_barrier();

    uint32_t boff[NWIN];
    bool valid[NWIN];
#pragma unroll
    for (int w = 0; w < NWIN; w++) {
        const int b = 16 * w + g;
        valid[w] = b < R;
        boff[w] = (uint32_t)(b < R ? b : R - 1) * Fmt::kBytes;
    }
    auto rsrc = [&](const uint8_t* w, int rows) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w), (short)0, (int)(row_bytes * (uint32_t)rows),
                                                 kBufferWord3);
    };
    const int c1 = args.rows[0], c2 = args.rows[0] + args.rows[1];
    typename Fmt::Regs buf[D][NM][NWIN];
    // windows [w0, w1) of the j-th row of this wave
    auto load_row = [&](typename Fmt::Regs (&rb)[NM][NWIN], int j, int w0 = 0, int w1 = NWIN) {
        const int rp = RPS * (gw + j * tw), r = rp + hh;  // rp: the step's first row (wave-uniform)
        const bool in = j < nrows && r < out_feat;
        if constexpr (EPI == kEpiSwiGLU) {
            const uint32_t ro = in ? (uint32_t)r * row_bytes : kOutOfRange;
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const __amdgpu_buffer_rsrc_t rs = rsrc(args.w[m], args.rows[m]);
#pragma unroll
                for (int w = 0; w < NWIN; w++)
                    if (w >= w0 && w < w1) Fmt::bload(rb[m][w], rs, ro + boff[w], k);
            }
        } else if constexpr (!MULTI) {
            const uint32_t ro = in ? (uint32_t)r * row_bytes : kOutOfRange;
            const __amdgpu_buffer_rsrc_t rs = rsrc(args.w[0], args.rows[0]);
#pragma unroll
            for (int w = 0; w < NWIN; w++)
                    if (w >= w0 && w < w1) Fmt::bload(rb[0][w], rs, ro + boff[w], k);
        } else {
            // segment of the step (wave-uniform; with HALF the launcher keeps
            // segment boundaries even, so both rows of a pair share it): the
            // matrix and the row inside it
            const int sg = (rp >= c1) + (rp >= c2);
            const int lr = r - (sg == 0 ? 0 : sg == 1 ? c1 : c2);
            const uint32_t ro = in ? (uint32_t)lr * row_bytes : kOutOfRange;
            const __amdgpu_buffer_rsrc_t rsel = rsrc(sg == 0 ? args.w[0] : sg == 1 ? args.w[1] : args.w[2],
                                                     sg == 0 ? args.rows[0] : sg == 1 ? args.rows[1] : args.rows[2]);
#pragma unroll
            for (int w = 0; w < NWIN; w++)
                    if (w >= w0 && w < w1) Fmt::bload(rb[0][w], rsel, ro + boff[w], k);
        }
    };
#pragma unroll
    for (int i = 0; i < PRE; i++) load_row(buf[i], i);
    if constexpr (PREW > 0) load_row(buf[0], 0, 0, PREW);
    // keep the x-dependent math (and its wait on the x loads) below the weight loads just issued
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (POSTX) {
        // an empty use of every activation register makes the compiler wait
        // for the activation loads here (vmcnt counts the loads issued after
        // them, so the wait is exact); then the rest of the ring is issued
#pragma unroll
        for (int j = 0; j < NWIN; j++) asm volatile("" ::"v"(xv[j].x), "v"(xv[j].y), "v"(xv[j].z), "v"(xv[j].w));
#pragma unroll
        for (int i = PRE; i < D; i++) load_row(buf[i], i);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (NORM) {
        // rms_norm_slice: x*x per element into LDS past the activation arrays
        // (in pass P, element 64L + k of the pass sits at float 4096P +
        // 256(k/4) + 4L + k%4, so lane L reads its 64 values as sixteen
        // conflict-free float4), the sum of squares in the reference's serial
        // order (by wave 0, with the walk of vtq_sumsq.h where it applies),
        // then x * scale * w
        float* prod = reinterpret_cast<float*>(lds + act_lds_end(R));
        const int npass = (R + 15) / 16;
        const int H = sumsq_walk_head(R * 256);  // 0: the plain chain only (uniform)
        SumsqWalk& walk = *reinterpret_cast<SumsqWalk*>(lds + norm_walk_off(R));
        float hpart = 0.0f, apart = 0.0f;
#pragma unroll
        for (int j = 0; j < NWIN; j++) {
            const int b = wave + kNW * j;
            const float4 v = xv[j];
            const float4 sq = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
            // elements 256b + 4 lane + c: pass b/16, segment 4(b%16) + lane/16, k = 4(lane%16) + c
            if (b < R) {
                reinterpret_cast<float4*>(prod + 4096 * (b >> 4) + 256 * (lane & 15) + 16 * (b & 15))[lane >> 4] = sq;
                const float s4 = (sq.x + sq.y) + (sq.z + sq.w);
                apart += s4;
                if (256 * b + 4 * lane < H) hpart += s4;  // H is a multiple of 64
            }
        }
        if (H) sumsq_walk_partials(hpart, apart, walk);
        __syncthreads();
        float sumsq = 0.0f;
        if (H) {
            if (wave == 0) {
                float r[64];
                sumsq_load_pass0(prod, r);
                sumsq = sumsq_chain(r, 0, H / 64, 0.0f);
            } else if (wave < 4) {
                sumsq_walk_helper(wave - 1, prod, R * 256, H, walk);  // waves 1-3: the other three SIMDs
            }
            __syncthreads();
            if (wave == 0) sumsq = sumsq_walk(sumsq, prod, R * 256, H, walk);
        } else if (wave == 0) {
            for (int ps = 0; ps < npass; ps++) {
                float r[64];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float4 t = reinterpret_cast<const float4*>(prod + 4096 * ps + 256 * i)[lane];
                    r[4 * i] = t.x, r[4 * i + 1] = t.y, r[4 * i + 2] = t.z, r[4 * i + 3] = t.w;
                }
                sumsq = serial_sum_lanes(r, 4 * min(16, R - 16 * ps), sumsq);
            }
        }
        if (wave == 0) {
            const float mean = sumsq / (float)(R * 256);
            if (lane == 0) prod[4096 * npass] = 1.0f / libm::sqrtf(mean + args.eps);
        }
        __syncthreads();
        const float scale = prod[4096 * npass];
#pragma unroll
        for (int j = 0; j < NWIN; j++) {
            const float4 v = xv[j], w = nw[j];
            xv[j] = make_float4(v.x * scale * w.x, v.y * scale * w.y, v.z * scale * w.z, v.w * scale * w.w);
        }
    }
    quantize_act(xv, xb, R, wave, act);
    __syncthreads();

    typename Fmt::X xr[NWIN];
    // the block slot once more from the thread index, through an opaque copy:
    // held from the top across the normalising chain, it was spilled to
    // scratch memory and reloaded here
    int tid_late = (int)threadIdx.x;
    asm volatile("" : "+v"(tid_late));
    const int gl = HALF ? ((tid_late >> 2) & 7) : ((tid_late & 63) >> 2);
#pragma unroll
    for (int w = 0; w < NWIN; w++) Fmt::load_x(xr[w], act, 16 * w + gl < R ? 16 * w + gl : R - 1, k);
    const typename Fmt::Lane lc = Fmt::lane_consts(k);
    if constexpr (PREW > 0) load_row(buf[0], 0, PREW, NWIN);
    if constexpr (!POSTX) {
#pragma unroll
        for (int i = PRE + (PREW > 0); i < D; i++) load_row(buf[i], i);
    }

    float yacc = 0.0f, yacc1 = 0.0f;  // results of the step's row (HALF: and of its second row)
    for (int j0 = 0; j0 < nrows; j0 += D) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            if (j0 + i < nrows) {
                float rv[NM], rv1[NM];
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    if constexpr (HALF) {
                        const float2 s2 = window8x2_tree(Fmt::part(buf[i][m][0], xr[0], lc, valid[0]));
                        rv[m] = s2.x;
                        rv1[m] = s2.y;
                    } else {
                        float wv[NWIN];
#pragma unroll
                        for (int w = 0; w < NWIN; w++)
                            wv[w] = window16_tree(Fmt::part(buf[i][m][w], xr[w], lc, valid[w]));
                        rv[m] = windows_tree<NWIN>(wv);
                    }
                }
                float v = rv[0], v1 = HALF ? rv1[0] : 0.0f;
                if constexpr (EPI == kEpiSwiGLU) {
                    if constexpr (HALF) {
                        // lanes 0..31 evaluate the first row's silu(g) * u, lanes
                        // 32..63 the second row's, in one pass
                        const float gs = hh ? rv1[0] : rv[0], us = hh ? rv1[1] : rv[1];
                        const float vs = (gs / (1.0f + libm::expf(-gs))) * us;
                        v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vs), 0));
                        v1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vs), 32));
                    } else {
                        v = (rv[0] / (1.0f + libm::expf(-rv[0]))) * rv[1];
                    }
                }
                yacc = (lane == j0 + i) ? v : yacc;
                if constexpr (HALF) yacc1 = (lane == j0 + i) ? v1 : yacc1;
            }
            load_row(buf[i], j0 + i + D);
        }
    }
    if (lane < nrows) {
        const int r0 = RPS * (gw + lane * tw);
        float* yp = yb + r0;
        if constexpr (EPI == kEpiAccumulate)
            yp[0] = yp[0] + yacc;
        else
            yp[0] = yacc;
        if constexpr (HALF) {
            if (r0 + 1 < out_feat) {
                if constexpr (EPI == kEpiAccumulate)
                    yp[1] = yp[1] + yacc1;
                else
                    yp[1] = yacc1;
            }
        }
    }
}

// ---------------------------------------------------------- windows kernel

// Every global load below is issued unconditionally (lanes of padded
// blocks and slots past a wave's last unit read a clamped, valid address and
// their results are masked).  vmcnt retires in issue order, so a load behind
// a branch would force the compiler to wait for all outstanding loads; with
// straight-line loads each wait covers exactly the data it needs.  Results
// are kept in registers and stored once at the end for the same reason.
// row_stride (bytes between weight rows) and x_stride (floats between batch
// rows of x) exceed R * block bytes and R * 256 when the launch is one
// segment of longer rows.
template <class Fmt, int D>
__global__ __launch_bounds__(kNW * 64) void kquant_windows_kernel(const float* __restrict__ x,
                                                                  const uint8_t* __restrict__ W,
                                                                  float* __restrict__ y, int R, int out_feat,
                                                                  size_t row_stride, size_t x_stride) {
    extern __shared__ __align__(16) unsigned char lds[];
    const ActLds act = act_lds_layout(lds, R);
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int g = lane >> 2, k = lane & 3;
    const float* xb = x + (size_t)blockIdx.y * x_stride;
    float* yb = y + (size_t)blockIdx.y * out_feat;
    const size_t row_bytes = row_stride;
    const int nwin = (R + 15) >> 4;

    // this wave's contiguous rows (at most 64: the launcher sizes the grid)
    const long tw = (long)gridDim.x * kNW, gw = (long)blockIdx.x * kNW + wave;
    const int r0 = (int)((long)out_feat * gw / tw), r1 = (int)((long)out_feat * (gw + 1) / tw);
    const int nunits = (r1 - r0) * nwin;
    // clamp target for loads past the wave's last unit; a wave without rows
    // still reads (and discards) one valid row so its loads stay straight-line
    const int last_row = r1 > r0 ? r1 - 1 : min(r0, out_feat - 1);

    // 1. activation loads first (older than every weight load)
    float4 xv[kXPerWave];
    load_act(xv, xb, R, wave);

    float yacc = 0.0f;  // lane i keeps the result of row r0 + i
    int crow = 0, cw = 0;
    // Unit u of this wave is (row r0 + u / nwin, window u % nwin); slots past
    // the last unit reload the last unit.  The clamp is arithmetic on the
    // index, so the compiler cannot prove two slots share an address and
    // fold a load into a register copy (which would have to wait for it).
    int unext = 0;
    typename Fmt::Regs buf[D];
    auto load_chunk = [&]() {
#pragma unroll
        for (int i = 0; i < D; i++) {
            const int u = max(min(unext + i, nunits - 1), 0);
            const int urow = nunits > 0 ? r0 + u / nwin : last_row;
            const int b = min(16 * (u % nwin) + g, R - 1);
            Fmt::load(buf[i], W + (size_t)urow * row_bytes + (size_t)b * Fmt::kBytes, k);
        }
        unext += D;
    };

    // 2. weight loads of the first D units
    load_chunk();
    // 3. quantize the activation into LDS while the weights stream in; the
    // scheduling barrier keeps the x-dependent math (and its wait on the x
    // loads) below the weight loads just issued.
    __builtin_amdgcn_sched_barrier(0);
    quantize_act(xv, xb, R, wave, act);
    __syncthreads();
    const typename Fmt::Lane lc = Fmt::lane_consts(k);

    // 4. compute each chunk of D units, then load the next one
    for (int u0 = 0;; u0 += D) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            if (u0 + i < nunits) {
                const int b = 16 * cw + g;
                typename Fmt::X xr;
                Fmt::load_x(xr, act, b < R ? b : R - 1, k);
                const float s = window16_tree(Fmt::part(buf[i], xr, lc, b < R));
                float rv = s;
                if (nwin > 1) {
                    float* ws = act.ws + wave * kMaxWindows;
                    if (lane == 0) ws[cw] = s;
                    if (cw == nwin - 1) {
                        float wv[kMaxWindows];
#pragma unroll
                        for (int t = 0; t < kMaxWindows; t++) wv[t] = ws[t];
                        rv = window_tree(wv, nwin);
                    }
                }
                if (cw == nwin - 1) yacc = (lane == crow) ? rv : yacc;
                if (++cw == nwin) {
                    cw = 0;
                    ++crow;
                }
            }
        }
        if (u0 + D >= nunits) break;
        load_chunk();
    }
    // 5. one coalesced store per wave
    if (lane < r1 - r0) yb[r0 + lane] = yacc;
}

// ------------------------------------------------------------- launchers

// Dynamic LDS above 64 KiB must be allowed per kernel; gfx950 has 160 KiB per CU.
template <class K>
static hipError_t allow_lds(K kernel, size_t bytes) {
    return allow_dynamic_lds(reinterpret_cast<const void*>(kernel), bytes);
}

template <class K, class... A>
static hipError_t launch_lds(K kern, int wgs, int batch, size_t lds, hipStream_t stream, A... a) {
    if (hipError_t e = allow_lds(kern, lds)) return e;
    hipLaunchKernelGGL(kern, dim3((unsigned)wgs, (unsigned)batch, 1), dim3(kNW * 64), lds, stream, a...);
    return hipGetLastError();
}
template <class K, class... A>
static hipError_t launch(K kern, int wgs, int batch, int R, hipStream_t stream, A... a) {
    return launch_lds(kern, wgs, batch, act_lds_bytes(R), stream, a...);
}
// the normalising prologue keeps the products (passes of 4096 floats), the
// scale and, where the walk applies, its tables past the activation arrays
static size_t norm_lds_bytes(int R) {
    return norm_walk_off(R) + (sumsq_walk_head(R * 256) ? sizeof(SumsqWalk) : 0);
}

// one 16-wave workgroup per CU; more if a wave would own over 64 rows
static int rows_grid(int out_feat, int num_cus) {
    const int need = (out_feat + kNW * 64 - 1) / (kNW * 64);
    return num_cus < need ? need : num_cus;
}

// Ring depth D and early loads of the rows kernel (measured on the config-2
// shapes): one-window rows keep two rows in flight, one issued before the
// activation reads and one as soon as they return; three-window rows keep a
// single row in flight whose first window is issued before the activation
// reads.  Two-window rows keep two (Q4_K) or one (Q6_K, SwiGLU) rows in
// flight; at most one Q4_K row per wave takes the three-window scheme.
// Deeper rings spill registers.
template <class Fmt, int EPI, bool MULTI, bool NORM = false>
static hipError_t launch_rows(int nwin, int wgs, int batch, int R, const float* x, const RowsArgs& a, float* y,
                              hipStream_t stream) {
    const size_t lds = NORM ? norm_lds_bytes(R) : act_lds_bytes(R);
    // rows of at most 8 super-blocks go two to a wave step (segment
    // boundaries of a multi-matrix launch must then be even)
    if (nwin == 1 && R <= 8 && (!MULTI || (a.rows[0] % 2 == 0 && a.rows[1] % 2 == 0)))
        return launch_lds(kquant_rows_kernel<Fmt, 1, 2, 1, 0, true, EPI, MULTI, NORM, true>, wgs, batch, lds, stream, x,
                          a, y, R);
    if (nwin == 1)
        return launch_lds(kquant_rows_kernel<Fmt, 1, 2, 1, 0, true, EPI, MULTI, NORM>, wgs, batch, lds, stream, x, a,
                          y, R);
    if constexpr (MULTI && Fmt::kRowsMaxWindows == 2) {
        return hipErrorInvalidValue;  // Q6_K segment selection at two windows would spill registers
    } else if constexpr (Fmt::kRowsMaxWindows == 2 || EPI == kEpiSwiGLU) {
        return launch_lds(kquant_rows_kernel<Fmt, 2, 1, 0, 0, false, EPI, MULTI, NORM>, wgs, batch, lds, stream, x,
                          a, y, R);
    } else {
        if (nwin == 2) {
            // at most one row per wave (2048 x 5632 W2 of the decode step:
            // 5.32 -> 4.62 us): a single ring slot whose first window is
            // issued before the activation loads return
            if (a.rows[0] + a.rows[1] + a.rows[2] <= wgs * kNW)
                return launch_lds(kquant_rows_kernel<Fmt, 2, 1, 0, 1, false, EPI, MULTI, NORM>, wgs, batch, lds,
                                  stream, x, a, y, R);
            return launch_lds(kquant_rows_kernel<Fmt, 2, 2, 1, 0, false, EPI, MULTI, NORM>, wgs, batch, lds, stream,
                              x, a, y, R);
        }
        return launch_lds(kquant_rows_kernel<Fmt, 3, 1, 0, 1, false, EPI, MULTI, NORM>, wgs, batch, lds, stream, x,
                          a, y, R);
    }
}

// row_stride / x_stride: 0 for a whole matrix, else the strides of a segment
template <class Fmt>
static hipError_t launch_kq(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                            int num_cus, hipStream_t stream, size_t row_stride = 0, int x_stride = 0) {
    const int R = in_feat / 256;
    const int nwin = (R + 15) / 16;
    const int wgs = rows_grid(out_feat, num_cus);
    const size_t rs = row_stride ? row_stride : (size_t)R * Fmt::kBytes;
    const size_t xs = x_stride ? (size_t)x_stride : (size_t)R * 256;
    const size_t bytes = (size_t)out_feat * rs;
    if (nwin <= Fmt::kRowsMaxWindows && bytes < (size_t)kOutOfRange) {
        RowsArgs a{{w, w, w}, {out_feat, 0, 0}, nullptr, 0.0f};
        a.row_stride = (uint32_t)rs;
        a.x_stride = (int)xs;
        return launch_rows<Fmt, kEpiStore, false>(nwin, wgs, batch, R, x, a, y, stream);
    }
    const long waves = (long)wgs * kNW;
    const long units = ((long)out_feat + waves - 1) / waves * nwin;  // per wave, upper bound
    // 16 waves per CU leave 128 VGPRs per wave: at most 4 (Q4_K) / 2 (Q6_K) units in flight
    constexpr int kMaxD = sizeof(typename Fmt::Regs) > 48 ? 2 : 4;
    if (units <= 1) return launch(kquant_windows_kernel<Fmt, 1>, wgs, batch, R, stream, x, w, y, R, out_feat, rs, xs);
    if constexpr (kMaxD == 2) {
        return launch(kquant_windows_kernel<Fmt, 2>, wgs, batch, R, stream, x, w, y, R, out_feat, rs, xs);
    } else {
        if (units <= 2)
            return launch(kquant_windows_kernel<Fmt, 2>, wgs, batch, R, stream, x, w, y, R, out_feat, rs, xs);
        return launch(kquant_windows_kernel<Fmt, 4>, wgs, batch, R, stream, x, w, y, R, out_feat, rs, xs);
    }
}

bool kquant_fused_supported(int ggml_type, int in_feat, int epi, const RowsArgs& a) {
    if ((ggml_type != 12 && ggml_type != 14) || in_feat <= 0 || in_feat % 256) return false;
    if (epi == kEpiSwiGLU && ggml_type != 12) return false;  // Q6_K pairs would spill registers
    const int R = in_feat / 256, nwin = (R + 15) / 16;
    const int maxw = ggml_type == 12 ? Q4K::kRowsMaxWindows : Q6K::kRowsMaxWindows;
    if (nwin > (epi == kEpiSwiGLU ? 2 : maxw)) return false;
    const size_t rb = (size_t)R * (ggml_type == 12 ? Q4K::kBytes : Q6K::kBytes);
    for (int m = 0; m < 3; m++) {
        if (a.rows[m] < 0 || (size_t)a.rows[m] * rb >= (size_t)kOutOfRange) return false;
        if (a.rows[m] > 0 && (reinterpret_cast<uintptr_t>(a.w[m]) & 15)) return false;
    }
    if (a.norm_w && (epi == kEpiAccumulate || (reinterpret_cast<uintptr_t>(a.norm_w) & 15))) return false;
    if (epi == kEpiSwiGLU) return a.rows[0] == a.rows[1] && a.rows[2] == 0;
    if (ggml_type == 14 && nwin > 1 && (a.rows[1] > 0 || a.rows[2] > 0)) return false;
    return (long)a.rows[0] + a.rows[1] + a.rows[2] < (1L << 30);
}

template <class Fmt>
static hipError_t launch_fused(int epi, const float* x, const RowsArgs& a, float* y, int R, int wgs,
                               hipStream_t stream) {
    const int nwin = (R + 15) / 16;
    const bool multi = a.rows[1] > 0 || a.rows[2] > 0, norm = a.norm_w != nullptr;
    if (epi == kEpiSwiGLU) {
        if constexpr (std::is_same<Fmt, Q4K>::value)
            return norm ? launch_rows<Fmt, kEpiSwiGLU, false, true>(nwin, wgs, 1, R, x, a, y, stream)
                        : launch_rows<Fmt, kEpiSwiGLU, false>(nwin, wgs, 1, R, x, a, y, stream);
        return hipErrorInvalidValue;
    }
    if (epi == kEpiAccumulate)
        return multi ? launch_rows<Fmt, kEpiAccumulate, true>(nwin, wgs, 1, R, x, a, y, stream)
                     : launch_rows<Fmt, kEpiAccumulate, false>(nwin, wgs, 1, R, x, a, y, stream);
    if (norm)
        return multi ? launch_rows<Fmt, kEpiStore, true, true>(nwin, wgs, 1, R, x, a, y, stream)
                     : launch_rows<Fmt, kEpiStore, false, true>(nwin, wgs, 1, R, x, a, y, stream);
    return multi ? launch_rows<Fmt, kEpiStore, true>(nwin, wgs, 1, R, x, a, y, stream)
                 : launch_rows<Fmt, kEpiStore, false>(nwin, wgs, 1, R, x, a, y, stream);
}

hipError_t launch_kquant_fused(int ggml_type, int epi, const float* x, const RowsArgs& a, float* y, int in_feat,
                               int num_cus, hipStream_t stream) {
    const int out = epi == kEpiSwiGLU ? a.rows[0] : a.rows[0] + a.rows[1] + a.rows[2];
    if (out == 0) return hipSuccess;
    const int wgs = rows_grid(out, num_cus);
    if (ggml_type == 12) return launch_fused<Q4K>(epi, x, a, y, in_feat / 256, wgs, stream);
    return launch_fused<Q6K>(epi, x, a, y, in_feat / 256, wgs, stream);
}

hipError_t launch_q4k_gemv(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           int num_cus, hipStream_t stream) {
    return launch_kq<Q4K>(x, w, y, batch, in_feat, out_feat, num_cus, stream);
}

hipError_t launch_q6k_gemv(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           int num_cus, hipStream_t stream) {
    return launch_kq<Q6K>(x, w, y, batch, in_feat, out_feat, num_cus, stream);
}

hipError_t launch_kquant_segment(int ggml_type, const float* x, int x_stride, const uint8_t* w, size_t row_stride,
                                 float* y, int batch, int seg_in, int out_feat, int num_cus, hipStream_t stream) {
    if (seg_in <= 0 || seg_in % 256 || seg_in > kquant_max_in_feat()) return hipErrorInvalidValue;
    if (ggml_type == 12)
        return launch_kq<Q4K>(x, w, y, batch, seg_in, out_feat, num_cus, stream, row_stride, x_stride);
    if (ggml_type == 14)
        return launch_kq<Q6K>(x, w, y, batch, seg_in, out_feat, num_cus, stream, row_stride, x_stride);
    return hipErrorInvalidValue;
}

int kquant_max_in_feat() { return kMaxWindows * 16 * 256; }

}  // namespace vtq
