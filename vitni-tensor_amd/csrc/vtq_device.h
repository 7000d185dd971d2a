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

// Serial left-to-right sum of v[0..n) held in LDS (16-byte aligned).  The
// chain walks chunks of 128 values; inside a chunk the four groups of 32 are
// straight-line code with the loads of group g+1 issued before the adds of
// group g, so LDS latency hides behind the add chain and the compiler's wait
// counts stay exact (a loop carrying loads across its back edge makes it wait
// for all of them at the top).  Every calling lane gets the sum; calling it
// from a whole wave costs no more than from one lane.
__device__ __forceinline__ void add_group32(float& s, const float4 (&r)[8]) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        s += r[j].x;
        s += r[j].y;
        s += r[j].z;
        s += r[j].w;
    }
}
__device__ inline float serial_sum_lds(const float* v, int n) {
    const float4* v4 = reinterpret_cast<const float4*>(v);
    float s = 0.0f;
    const int nc = n >> 7;
    for (int c = 0; c < nc; c++) {
        const float4* p = v4 + 32 * c;
        float4 a[8], b[8];
#pragma unroll
        for (int j = 0; j < 8; j++) a[j] = p[j];
#pragma unroll
        for (int j = 0; j < 8; j++) b[j] = p[8 + j];
        add_group32(s, a);
#pragma unroll
        for (int j = 0; j < 8; j++) a[j] = p[16 + j];
        add_group32(s, b);
#pragma unroll
        for (int j = 0; j < 8; j++) b[j] = p[24 + j];
        add_group32(s, a);
        add_group32(s, b);
    }
    for (int i = nc << 7; i < n; i++) s += v[i];
    return s;
}

// Serial left-to-right sum continued from `run`, over values held in
// registers, by a whole wave: lane L holds the V consecutive values of
// segment L in r[0..V), segments 0..nl-1 in order.  Every lane runs the
// same V dependent adds starting from the running sum, and readlane takes
// segment L's result from lane L, so the chain never waits on memory.  The
// result is the same in every lane.
template <int V>
__device__ inline float serial_sum_lanes(const float (&r)[V], int nl, float run) {
    // pin the values in registers: left alone, the compiler re-reads them
    // from LDS inside the loop and the chain waits on every segment's loads
    float v[V];
#pragma unroll
    for (int k = 0; k < V; k++) {
        v[k] = r[k];
        asm volatile("" : "+v"(v[k]));
    }
    for (int L = 0; L < nl; L++) {
        float s = run;
#pragma unroll
        for (int k = 0; k < V; k++) s = s + v[k];
        run = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), L));
    }
    return run;
}

// serial_sum_lanes over v[0..n) in LDS (16-byte aligned, allocated to a
// multiple of 4 floats), by a whole wave; slots past n read as -0.0, the
// exact identity of +.
__device__ inline float serial_sum_wave(const float* v, int n) {
    const int lane = threadIdx.x & 63;
    float run = 0.0f;
    for (int base = 0; base < n; base += 2048) {
        const int m = n - base < 2048 ? n - base : 2048;
        float r[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int idx = base + 32 * lane + 4 * i;
            float4 t = make_float4(-0.0f, -0.0f, -0.0f, -0.0f);
            if (idx < n) t = *reinterpret_cast<const float4*>(v + idx);
            r[4 * i] = idx < n ? t.x : -0.0f;
            r[4 * i + 1] = idx + 1 < n ? t.y : -0.0f;
            r[4 * i + 2] = idx + 2 < n ? t.z : -0.0f;
            r[4 * i + 3] = idx + 3 < n ? t.w : -0.0f;
        }
        run = serial_sum_lanes(r, (m + 31) / 32, run);
    }
    return run;
}

}  // namespace vtq
