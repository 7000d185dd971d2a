// kquant_gemv.hip -- exact-integer Q4_K / Q6_K decode GEMV for gfx950.
//
// Replaces linear_q4_k_integer[_parallel] (src/ops/quant.rs:936-980,
// :1149-1196) and linear_q6_k_integer[_parallel] (:1060-1146) for any batch;
// each batch row is one grid.y slice.
//
// Work unit = one 16-super-block window of one weight row.  Lane 4g+k of a
// wave handles quarter k of super-block 16w+g, so one unit is 2304
// contiguous bytes of Q4_K (3360 of Q6_K) read by the 64 lanes.  Each wave
// owns a contiguous range of rows and streams its units through a ring of D
// register buffers: the loads of D units are in flight before the activation
// is even quantized, and every computed unit immediately refills its slot.
//
// Per unit: integer sums with v_dot4_i32_i8 against the int8 activation held
// in LDS, reduced over the 4 lanes of a block with DPP (exact in any order);
// the per-block float epilogue evaluated exactly as the reference writes it;
// then the pinned fixed_tree over the window's 16 blocks and over the row's
// windows.  fixed_tree(p[0..R)) equals fixed_tree over 16-aligned windows of
// fixed_tree(window), because the first four levels of the reference's tree
// only pair blocks inside an aligned window; padded slots hold -0.0, the
// exact identity of +.
#include "vtq_device.h"
#include "vtq_kernels.h"

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
    float* ws;     // [NW*16] per-wave window sums
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
size_t act_lds_bytes(int R) { return act_off_ws(R) + kNW * kMaxWindows * 4; }

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

// fixed_tree over the 16 block slots of a window; slot g lives in lanes
// 4g..4g+3 and slots past the row's end hold -0.0.  The stride form pairs
// slot i with i+s for i a multiple of 2s; the sum is formed in the higher
// slot instead (IEEE addition is commutative, so a+b and b+a are the same
// bits and only the association has to match the reference):
//   stride 1, 2: row_shr:4, row_shr:8 inside each 16-lane row -> row sums at lane 15
//   stride 4:    row_bcast:15 adds row 0 into row 1 and row 2 into row 3
//   stride 8:    row_bcast:31 adds (row0+row1) into row 3
// The window sum ends in lane 63 and is read out once.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_add_f(float v) {
    const float t = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(-0.0f), __float_as_int(v), CTRL, ROWMASK, 0xF, false));
    return v + t;
}
__device__ __forceinline__ float window16_tree(float v) {
    v = dpp_add_f<0x114, 0xF>(v);  // row_shr:4  (lanes 0..3 of a row add -0.0)
    v = dpp_add_f<0x118, 0xF>(v);  // row_shr:8
    v = dpp_add_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add_f<0x143, 0x8>(v);  // row_bcast:31 into row 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ------------------------------------------------------------------ Q4_K

struct Q4K {
    static constexpr int kBytes = 144;
    static constexpr int kMaxD = 4;
    struct Regs {
        uint4 hdr, qa, qb;
    };
    __device__ static void load(Regs& r, const uint8_t* __restrict__ blk, int k) {
        r.hdr = *reinterpret_cast<const uint4*>(blk);
        r.qa = *reinterpret_cast<const uint4*>(blk + 16 + 32 * k);
        r.qb = *reinterpret_cast<const uint4*>(blk + 32 + 32 * k);
    }
    // dot_q4k_q8_block (src/ops/quant.rs:849-898) for quarter k = sub-blocks
    // 2k, 2k+1; returns this block's part (identical in the 4 lanes).
    __device__ static float part(const Regs& r, const ActLds& act, int b, int k, bool valid) {
        const uint4* xw4 = reinterpret_cast<const uint4*>(act.qs + b * 64 + 16 * k);
        const uint4 xl0 = xw4[0], xl1 = xw4[1], xh0 = xw4[2], xh1 = xw4[3];
        const uint32_t qw[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        const uint32_t xl[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
        const uint32_t xh[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
        int s_lo = 0, s_hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s_lo = __builtin_amdgcn_sdot4((int)(qw[i] & 0x0F0F0F0Fu), (int)xl[i], s_lo, false);
            s_hi = __builtin_amdgcn_sdot4((int)((qw[i] >> 4) & 0x0F0F0F0Fu), (int)xh[i], s_hi, false);
        }
        // get_scale_min_k4 (src/ops/quant.rs:267-276) for j = 2k, 2k+1, two
        // bytes at a time, without branching on the lane's k:
        //   j < 4:  sc = s[j] & 63,                       m = s[j+4] & 63
        //   j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4, m = (s[j+4] >> 4) | (s[j] >> 6) << 4
        const int sh = 16 * (k & 1);
        const bool hi = k >= 2;
        const uint32_t A = r.hdr.w >> sh, B = r.hdr.y >> sh, C = r.hdr.z >> sh;
        const uint32_t lowmask = hi ? 0x0F0Fu : 0x3F3Fu, topmask = hi ? 0x3030u : 0u;
        const uint32_t scp = ((hi ? A : B) & lowmask) | ((B >> 2) & topmask);
        const uint32_t mp = ((hi ? (A >> 4) : C) & lowmask) | ((C >> 2) & topmask);
        const int bs_lo = act.s32[b * 64 + 16 * k], bs_hi = act.s32[b * 64 + 16 * k + 8];
        // every factor fits 24 bits (sc, m <= 63; |s| <= 60960; |bsum| <= 4064): full-rate v_mad_i32_i24
        int acc = __mul24((int)(scp & 0xFFu), s_lo) + __mul24((int)(scp >> 8), s_hi);
        int accm = __mul24((int)(mp & 0xFFu), bs_lo) + __mul24((int)(mp >> 8), bs_hi);
        acc = quad_sum_i(acc);
        accm = quad_sum_i(accm);
        const float dx = act.d[b * 64];
        const float d = f16_hw(r.hdr.x & 0xFFFFu);
        const float dmin = f16_hw(r.hdr.x >> 16);
        const float t1 = (d * dx) * (float)acc;
        const float t2 = (dmin * dx) * (float)accm;
        return valid ? t1 - t2 : -0.0f;
    }
};

// ------------------------------------------------------------------ Q6_K

// 16 bytes from a 2-byte-aligned address p, as five aligned dwords from
// p & ~3 funnel-shifted by (p & 3) bytes.  Reads [p - (p&3), p - (p&3) + 20),
// which for the runs used below stays inside the 210-byte block.
__device__ __forceinline__ uint4 load16_a2(const uint8_t* p) {
    // pointer arithmetic (not an integer round trip) keeps the global address
    // space visible to the compiler: global_load, not flat_load
    const uint32_t off = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t* p4 = reinterpret_cast<const uint32_t*>(p - off);
    const u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p4);
    const uint32_t e = p4[4];
    return make_uint4(__builtin_amdgcn_alignbyte(v.y, v.x, off), __builtin_amdgcn_alignbyte(v.z, v.y, off),
                      __builtin_amdgcn_alignbyte(v.w, v.z, off), __builtin_amdgcn_alignbyte(e, v.w, off));
}

__device__ __forceinline__ int sext8(uint32_t v, int byte) { return (int)(int8_t)((v >> (8 * byte)) & 0xFFu); }

struct Q6K {
    static constexpr int kBytes = 210;
    static constexpr int kMaxD = 2;
    struct Regs {
        uint4 b0, b1, hh;
        uint4 sc;      // scale bytes 192..207 (funnel-shifted)
        uint32_t d;    // f16 bits of d
    };
    // Lane k: hf = k>>1 (128-element half), t = k&1 (positions l in [16t, 16t+16)).
    // Reads stay inside the block: ql/qh runs end by byte 196, the scale
    // dwords start at 192 - (blk&3) and two ushorts read bytes 206..209.
    __device__ static void load(Regs& r, const uint8_t* __restrict__ blk, int k) {
        const int hf = k >> 1, t = k & 1;
        r.b0 = load16_a2(blk + 64 * hf + 16 * t);
        r.b1 = load16_a2(blk + 64 * hf + 32 + 16 * t);
        r.hh = load16_a2(blk + 128 + 32 * hf + 16 * t);
        const uint32_t off = (uint32_t)(reinterpret_cast<uintptr_t>(blk + 192) & 3u);
        const u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(blk + 192 - off);
        const uint32_t tail = *reinterpret_cast<const uint16_t*>(blk + 206);  // bytes 206, 207
        r.sc = make_uint4(__builtin_amdgcn_alignbyte(v.y, v.x, off), __builtin_amdgcn_alignbyte(v.z, v.y, off),
                          __builtin_amdgcn_alignbyte(v.w, v.z, off), __builtin_amdgcn_alignbyte(tail, v.w, off));
        r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
    }
    // dot_q6k_q8_block (src/ops/quant.rs:995-1057): buckets 8hf+t+2q (q = 0..3)
    // are exactly one 16-element run each; (code - 32) is folded in as
    // sum(code*x) - 32*sum(x) with the run sums from the activation pass.
    __device__ static float part(const Regs& r, const ActLds& act, int b, int k, bool valid) {
        const int hf = k >> 1, t = k & 1;
        // activation words: element 128hf + 16t + 32q + 4i -> word 32hf + 4t + 8q + i
        const uint32_t* xw = act.qs + b * 64 + 32 * hf + 4 * t;
        const uint4 x1 = *reinterpret_cast<const uint4*>(xw);
        const uint4 x2 = *reinterpret_cast<const uint4*>(xw + 8);
        const uint4 x3 = *reinterpret_cast<const uint4*>(xw + 16);
        const uint4 x4 = *reinterpret_cast<const uint4*>(xw + 24);
        const uint32_t B0[4] = {r.b0.x, r.b0.y, r.b0.z, r.b0.w};
        const uint32_t B1[4] = {r.b1.x, r.b1.y, r.b1.z, r.b1.w};
        const uint32_t H[4] = {r.hh.x, r.hh.y, r.hh.z, r.hh.w};
        const uint32_t X1[4] = {x1.x, x1.y, x1.z, x1.w}, X2[4] = {x2.x, x2.y, x2.z, x2.w};
        const uint32_t X3[4] = {x3.x, x3.y, x3.z, x3.w}, X4[4] = {x4.x, x4.y, x4.z, x4.w};
        int S1 = 0, S2 = 0, S3 = 0, S4 = 0;
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
        // run (bucket) of q1 is 8hf + t, q2..q4 at +2, +4, +6; run r sits at lane 4r
        const int* s16 = act.s16 + b * 64 + 4 * (8 * hf + t);
        const int sum1 = S1 - 32 * s16[0];
        const int sum2 = S2 - 32 * s16[8];
        const int sum3 = S3 - 32 * s16[16];
        const int sum4 = S4 - 32 * s16[24];
        // scales: i8 at 192 + 8hf + t + 2q -> bytes t, t+2 of dwords 2hf and 2hf+1
        const uint32_t sa = hf ? r.sc.z : r.sc.x, sb = hf ? r.sc.w : r.sc.y;
        // |sc| <= 64 and |sum| <= 16*31*127: every product fits v_mad_i32_i24
        int acc = __mul24(sext8(sa, t), sum1) + __mul24(sext8(sa, t + 2), sum2) +
                  __mul24(sext8(sb, t), sum3) + __mul24(sext8(sb, t + 2), sum4);
        acc = quad_sum_i(acc);
        const float d = f16_hw(r.d);
        return valid ? (d * act.d[b * 64]) * (float)acc : -0.0f;
    }
};

// --------------------------------------------------------------- kernel

// Every global load below is issued unconditionally (lanes of padded
// blocks and slots past a wave's last unit read a clamped, valid address and
// their results are masked).  vmcnt retires in issue order, so a load behind
// a branch would force the compiler to wait for all outstanding loads; with
// straight-line loads each wait covers exactly the data it needs.  Results
// are kept in registers and stored once at the end for the same reason.
template <class Fmt, int D>
__global__ __launch_bounds__(kNW * 64) void kquant_gemv_kernel(const float* __restrict__ x,
                                                               const uint8_t* __restrict__ W,
                                                               float* __restrict__ y, int R, int out_feat) {
    extern __shared__ __align__(16) unsigned char lds[];
    const ActLds act = act_lds_layout(lds, R);
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int g = lane >> 2, k = lane & 3;
    const float* xb = x + (size_t)blockIdx.y * R * 256;
    float* yb = y + (size_t)blockIdx.y * out_feat;
    const size_t row_bytes = (size_t)R * Fmt::kBytes;
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
#pragma unroll
    for (int j = 0; j < kXPerWave; j++) {
        const int b = wave + kNW * j;
        if (b < R) xv[j] = reinterpret_cast<const float4*>(xb + (size_t)b * 256)[lane];
    }

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
#pragma unroll
    for (int j = 0; j < kXPerWave; j++) {
        const int b = wave + kNW * j;
        if (b < R) quantize_block_to_lds(xv[j], b, act);
    }
    for (int b = wave + kNW * kXPerWave; b < R; b += kNW)
        quantize_block_to_lds(reinterpret_cast<const float4*>(xb + (size_t)b * 256)[lane], b, act);
    __syncthreads();

    // 4. compute each chunk of D units, then load the next one
    for (int u0 = 0;; u0 += D) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            if (u0 + i < nunits) {
                const int b = 16 * cw + g;
                const float part = Fmt::part(buf[i], act, b < R ? b : R - 1, k, b < R);
                const float s = window16_tree(part);
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
    if (bytes <= 65536) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)bytes);
}

template <class Fmt, int D>
static hipError_t launch_kq_d(const float* x, const uint8_t* w, float* y, int batch, int R, int out_feat, int wgs,
                              hipStream_t stream) {
    auto kern = kquant_gemv_kernel<Fmt, D>;
    if (hipError_t e = allow_lds(kern, act_lds_bytes(R))) return e;
    hipLaunchKernelGGL(kern, dim3((unsigned)wgs, (unsigned)batch, 1), dim3(kNW * 64), act_lds_bytes(R), stream, x,
                       w, y, R, out_feat);
    return hipGetLastError();
}

template <class Fmt>
static hipError_t launch_kq(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                            int num_cus, hipStream_t stream) {
    const int R = in_feat / 256;
    const int nwin = (R + 15) / 16;
    // one 16-wave workgroup per CU; more if a wave would own over 64 rows
    int wgs = num_cus;
    const int need = (out_feat + kNW * 64 - 1) / (kNW * 64);
    if (wgs < need) wgs = need;
    const long waves = (long)wgs * kNW;
    const long units = ((long)out_feat + waves - 1) / waves * nwin;  // per wave, upper bound
    // 16 waves per CU leave 128 VGPRs per wave: at most kMaxD units in flight
    if (units <= 1 || Fmt::kMaxD == 1) return launch_kq_d<Fmt, 1>(x, w, y, batch, R, out_feat, wgs, stream);
    if (units <= 2 || Fmt::kMaxD == 2) return launch_kq_d<Fmt, 2>(x, w, y, batch, R, out_feat, wgs, stream);
    return launch_kq_d<Fmt, 4>(x, w, y, batch, R, out_feat, wgs, stream);
}

hipError_t launch_q4k_gemv(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           int num_cus, hipStream_t stream) {
    return launch_kq<Q4K>(x, w, y, batch, in_feat, out_feat, num_cus, stream);
}

hipError_t launch_q6k_gemv(const float* x, const uint8_t* w, float* y, int batch, int in_feat, int out_feat,
                           int num_cus, hipStream_t stream) {
    return launch_kq<Q6K>(x, w, y, batch, in_feat, out_feat, num_cus, stream);
}

int kquant_max_in_feat() { return kMaxWindows * 16 * 256; }

}  // namespace vtq
