// vtq_device.h -- gfx950 device primitives shared by the vtq kernels.
//
// Everything here is exact or is a single IEEE binary32 operation in source
// order: the library is compiled with -ffp-contract=off, fp32 division is
// the correctly rounded v_div_scale/v_div_fmas/v_div_fixup sequence, and the
// kernel descriptors keep fp32/fp16 denormals (float_denorm_mode 3).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vtq {

constexpr int kWave = 64;

// Index of the calling wave in its workgroup, as a uniform (scalar) value:
// without readfirstlane the compiler treats threadIdx.x >> 6 as divergent and
// turns every loop over a wave's work into an exec-masked vector loop.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// A 16-byte vector that only promises 4-byte alignment, so that the
// compiler may still emit one global_load_dwordx4 for it.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// IEEE binary16 bits -> binary32, exact, NaN payload kept unquieted
// (src/ops/quant.rs:40-66).  A subnormal half m*2^-24 is formed by an exact
// float product.
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0u) {
        bits = __float_as_uint((float)m * 0x1p-24f) | sign;
    } else if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    return __uint_as_float(bits);
}

// The same conversion with v_cvt_f32_f16: exact for every finite value and
// +-Inf (fp16 denormals are preserved by the kernel's float mode); a NaN
// comes out quieted, which only changes NaN payloads.
__device__ __forceinline__ float f16_hw(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// f16_to_f32's exact bits, branch-free: v_cvt_f32_f16 for every non-NaN
// code, and the payload-shifting formula selected for a NaN.
__device__ __forceinline__ float f16_to_f32_sel(uint32_t h) {
    const uint32_t nan_bits = ((h & 0x8000u) << 16) | 0x7F800000u | ((h & 0x3FFu) << 13);
    const uint32_t m = 0u - (uint32_t)((h & 0x7FFFu) > 0x7C00u);  // all ones for a NaN
    return __uint_as_float((__float_as_uint(f16_hw(h)) & ~m) | (nan_bits & m));
}

// Rust `(t as i32).clamp(-127, 127)` for the activation quantizer: NaN -> 0,
// truncation toward zero, saturation (src/ops/quant.rs:766).  Branch-free:
// clamp in float (exact), truncate (exact for |c| <= 127), and select 0
// for an unordered t.
__device__ __forceinline__ int quant_round_clamp(float t) {
    const float c = fminf(fmaxf(t, -127.0f), 127.0f);
    const int q = (int)c;
    return (t == t) ? q : 0;
}

// q = clamp(trunc(s + (s >= 0 ? 0.5 : -0.5))), s = x*inv (src/ops/quant.rs:764-766).
// copysign(0.5, s) differs from the reference's bias only at s = -0.0, where
// both -0.0 + 0.5 and -0.0 - 0.5 truncate to 0, so q is the same for every s.
__device__ __forceinline__ int quant_one(float v, float inv) {
    const float s = v * inv;
    const float t = s + copysignf(0.5f, s);
    return quant_round_clamp(t);
}

// |v| exactly as the reference forms it: (v < 0) ? -v : v (so -0.0 stays -0.0).
__device__ __forceinline__ float abs_ref(float v) { return v < 0.0f ? -v : v; }

// max in the reference's sense: keep m unless a > m (NaN never wins).
__device__ __forceinline__ float max_ref(float m, float a) { return a > m ? a : m; }

// ---- cross-lane helpers (DPP within quads/rows, bpermute across rows) ----

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
constexpr int kQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;  // lane i <-> 7-i within 8
constexpr int kRowMirror = 0x140;      // lane i <-> 15-i within 16

// Sum over the 4 lanes of a quad (integer: any order is exact).
__device__ __forceinline__ int quad_sum_i(int v) {
    v += dpp_i<kQuadXor1>(v);
    v += dpp_i<kQuadXor2>(v);
    return v;
}

__device__ __forceinline__ float shfl_down_f(float v, int delta) {
    return __shfl_down(v, delta, kWave);
}
__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, kWave); }

// Wave-wide maximum of per-lane values that are all non-NaN and >= +0.0
// (each lane's value came from max_ref starting at +0.0), so v_max_f32 is
// exact and order-free.  DPP inside each 16-lane row, readlane across rows.
__device__ __forceinline__ float wave_max_nonneg(float m) {
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), kQuadXor1, 0xF, 0xF, true)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), kQuadXor2, 0xF, 0xF, true)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), kRowHalfMirror, 0xF, 0xF, true)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), kRowMirror, 0xF, 0xF, true)));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Quantize one 256-element activation block with one wave: lane L holds
// elements 4L..4L+3 in v.  Produces (src/ops/quant.rs:750-771):
//   *packed : the lane's four int8 codes, element 4L in the low byte
//   *s16    : sum of the 16-element run containing the lane (lanes 4r..4r+3)
//   *s32    : sum of the 32-element sub-block containing the lane (bsums)
//   return  : d = amax / 127
__device__ __forceinline__ float quant_block_wave(float4 v, uint32_t* packed, int* s16, int* s32) {
    float m = 0.0f;
    m = max_ref(m, abs_ref(v.x));
    m = max_ref(m, abs_ref(v.y));
    m = max_ref(m, abs_ref(v.z));
    m = max_ref(m, abs_ref(v.w));
    const float amax = wave_max_nonneg(m);
    const float d = amax / 127.0f;
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    const int q0 = quant_one(v.x, inv), q1 = quant_one(v.y, inv);
    const int q2 = quant_one(v.z, inv), q3 = quant_one(v.w, inv);
    *packed = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
              ((uint32_t)(q3 & 0xFF) << 24);
    int s = q0 + q1 + q2 + q3;
    s = quad_sum_i(s);  // 16-element run
    *s16 = s;
    s += dpp_i<kRowHalfMirror>(s);  // lanes i and 7-i of each 8-lane group
    *s32 = s;
    return d;
}

// fixed_tree (src/ops/quant.rs:461-476) over values held in lane groups:
// group g of width W lanes (the value replicated or at least held in the
// group's first lane), G groups, n valid groups; slots >= n must hold -0.0f
// (x + -0.0 == x for every x, so padded slots never change a sum).
// Pairing at stride s: slot i (multiple of 2s) += slot i+s.  This equals the
// reference's level-by-level halving: level k pairs the 2^k-blocks starting
// at multiples of 2^(k+1), and an unpaired trailing block passes through.
// The result is in the first lane of group 0 (lane 0).
template <int W, int G>
__device__ __forceinline__ float group_tree(float v) {
#pragma unroll
    for (int s = 1; s < G; s <<= 1) v += shfl_down_f(v, s * W);
    return v;
}

// Serial left-to-right sum of v[0..n) held in LDS (16-byte aligned), by one
// lane.  Groups of 4G values alternate between two register sets: the loads
// of group g+1 are issued before the dependent adds of group g (the
// scheduling barriers keep the compiler from sinking them), so LDS latency
// hides behind the add chain.
template <int G>
__device__ __forceinline__ void add_group(float& s, const float4 (&r)[G]) {
#pragma unroll
    for (int j = 0; j < G; j++) {
        s += r[j].x;
        s += r[j].y;
        s += r[j].z;
        s += r[j].w;
    }
}
template <int G = 8>
__device__ inline float serial_sum_lds(const float* v, int n) {
    const float4* v4 = reinterpret_cast<const float4*>(v);
    const int ng = n / (4 * G);  // whole groups
    float s = 0.0f;
    float4 a[G], b[G];
    if (ng > 0) {
#pragma unroll
        for (int j = 0; j < G; j++) a[j] = v4[j];
    }
    int g = 0;
    for (; g + 1 < ng; g += 2) {
#pragma unroll
        for (int j = 0; j < G; j++) b[j] = v4[G * (g + 1) + j];
        __builtin_amdgcn_sched_barrier(0);
        add_group(s, a);
        __builtin_amdgcn_sched_barrier(0);
        const int gn = g + 2 < ng ? g + 2 : g + 1;  // a valid group; the last refill is unused
#pragma unroll
        for (int j = 0; j < G; j++) a[j] = v4[G * gn + j];
        __builtin_amdgcn_sched_barrier(0);
        add_group(s, b);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (g < ng) add_group(s, a);
    for (int i = 4 * G * ng; i < n; i++) s += v[i];
    return s;
}

// Serial left-to-right sum of 256*nchunks values, fed to the dependent add
// chain by DPP row broadcasts: one v_add_f32_dpp per element, no LDS read in
// the chain.  Layout: element 256c + 16i + l sits in LDS at 256c + 16l + i,
// so lane l (of every 16-lane row) loads its 16 values of chunk c as four
// float4.  Element order is kept: chunk by chunk, i outer, l inner; IEEE
// addition is commutative, so bcast(r) + acc equals acc + bcast(r).  Every
// lane of the calling wave ends with the same sum.
template <int L>
__device__ __forceinline__ void add_bcast(float& acc, float r) {
    asm volatile("v_add_f32_dpp %0, %1, %0 row_newbcast:%2 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(r), "i"(L));
}
__device__ __forceinline__ void add_bcast16(float& acc, float r) {
    add_bcast<0>(acc, r), add_bcast<1>(acc, r), add_bcast<2>(acc, r), add_bcast<3>(acc, r);
    add_bcast<4>(acc, r), add_bcast<5>(acc, r), add_bcast<6>(acc, r), add_bcast<7>(acc, r);
    add_bcast<8>(acc, r), add_bcast<9>(acc, r), add_bcast<10>(acc, r), add_bcast<11>(acc, r);
    add_bcast<12>(acc, r), add_bcast<13>(acc, r), add_bcast<14>(acc, r), add_bcast<15>(acc, r);
}
__device__ __forceinline__ void add_chunk(float& acc, const float4 (&r)[4]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        add_bcast16(acc, r[j].x);
        add_bcast16(acc, r[j].y);
        add_bcast16(acc, r[j].z);
        add_bcast16(acc, r[j].w);
    }
}
__device__ inline float serial_sum_bcast(const float* v, int nchunks) {
    const float4* v4 = reinterpret_cast<const float4*>(v) + 4 * (threadIdx.x & 15);
    float acc = 0.0f;
    float4 a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; j++) a[j] = v4[j];
    for (int c = 0; c < nchunks; c += 2) {
        const int c1 = c + 1 < nchunks ? c + 1 : c;
#pragma unroll
        for (int j = 0; j < 4; j++) b[j] = v4[64 * c1 + j];
        __builtin_amdgcn_sched_barrier(0);
        add_chunk(acc, a);
        __builtin_amdgcn_sched_barrier(0);
        const int c2 = c + 2 < nchunks ? c + 2 : c;
#pragma unroll
        for (int j = 0; j < 4; j++) a[j] = v4[64 * c2 + j];
        __builtin_amdgcn_sched_barrier(0);
        if (c + 1 < nchunks) add_chunk(acc, b);
        __builtin_amdgcn_sched_barrier(0);
    }
    return acc;
}

}  // namespace vtq
