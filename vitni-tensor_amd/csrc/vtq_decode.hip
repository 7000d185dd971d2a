// vtq_decode.hip -- device kernels of the decode step (libvtq_runtime).
//
// Restates, on the device and in the reference's operation order, the parts
// of forward_quantized::step (src/model/forward_quantized.rs:288-655) that
// are not linears: embedding_row, rms_norm_slice, RoPE, the KV-cache write,
// softmax attention, the residual adds, SwiGLU and argmax.  Reductions whose
// order the reference fixes (the RMSNorm sum of squares, the softmax
// denominator, each score's dot product, each output element's sum over
// positions) run serially in one lane; maxima, which no order changes, run as
// trees.  Transcendentals are the libm restatements of vtq_libm.h, so they
// round exactly as the reference's libm crate does.
#include "vtq_decode.h"
#include "vtq_device.h"
#include "vtq_kernels.h"
#include "vtq_libm.h"
#include "vtq_sumsq.h"

namespace vtq {
namespace decode {

namespace {

__device__ __forceinline__ uint32_t rd_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// one element of the table row (dequantize_* of src/ops/quant.rs)
__device__ float embed_elem(int type, const uint8_t* row, int i) {
    switch (type) {
    case 0:
        return reinterpret_cast<const float*>(row)[i];
    case 2: {  // dequantize_q4_0: element 2k low nibble, 2k+1 high
        const uint8_t* blk = row + 18 * (i / 32);
        const int e = i % 32, k = e / 2;
        const int q = (int)((blk[2 + k] >> (4 * (e & 1))) & 15) - 8;
        return f16_to_f32_sel(rd_u16(blk)) * (float)q;
    }
    case 6: {  // dequantize_q5_0: element j and j+16 share qs byte j
        const uint8_t* blk = row + 22 * (i / 32);
        const int e = i % 32;
        const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                            ((uint32_t)blk[5] << 24);
        int x;
        if (e < 16)
            x = (int)((blk[6 + e] & 15) | (((qh >> e) << 4) & 16)) - 16;
        else
            x = (int)((blk[6 + e - 16] >> 4) | ((qh >> (e - 16 + 12)) & 16)) - 16;
        return f16_to_f32_sel(rd_u16(blk)) * (float)x;
    }
    case 8: {  // dequantize_q8_0
        const uint8_t* blk = row + 34 * (i / 32);
        return f16_to_f32_sel(rd_u16(blk)) * (float)(int8_t)blk[2 + i % 32];
    }
    case 12: {  // dequantize_q4_k: d1 * q - m1 per 32-element sub-block
        const uint8_t* blk = row + 144 * (i / 256);
        const int e = i % 256, j = e / 32, l = e % 32;
        const uint8_t* s = blk + 4;
        uint32_t sc, mn;
        if (j < 4) {
            sc = s[j] & 63;
            mn = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
            mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const float d1 = f16_to_f32_sel(rd_u16(blk)) * (float)sc;
        const float m1 = f16_to_f32_sel(rd_u16(blk + 2)) * (float)mn;
        const uint8_t qb = blk[16 + 32 * (j / 2) + l];
        const uint32_t q = (j & 1) ? (qb >> 4) : (qb & 15);
        return d1 * (float)q - m1;
    }
    default: {  // 14, dequantize_q6_k: (d * sc) * q, q = 6-bit code - 32
        const uint8_t* blk = row + 210 * (i / 256);
        const int e = i % 256, hf = e / 128, r = e % 128, k = r / 32, l = r % 32;
        const uint8_t* ql = blk + 64 * hf;
        const uint8_t h = blk[128 + 32 * hf + l];
        const uint8_t lo = ql[l + 32 * (k & 1)];
        const int q = (int)(((k >= 2) ? (lo >> 4) : (lo & 15)) | (((h >> (2 * k)) & 3) << 4)) - 32;
        const float d = f16_to_f32_sel(rd_u16(blk + 208));
        return d * (float)(int8_t)blk[192 + 8 * hf + l / 16 + 2 * k] * (float)q;
    }
    }
}

size_t row_bytes(int type, int dim) {
    switch (type) {
    case 0: return (size_t)dim * 4;
    case 2: return (size_t)dim / 32 * 18;
    case 6: return (size_t)dim / 32 * 22;
    case 8: return (size_t)dim / 32 * 34;
    case 12: return (size_t)dim / 256 * 144;
    default: return (size_t)dim / 256 * 210;
    }
}

// RoPE angles of position q for pair m = 0..head_dim/2 - 1
// (forward_quantized.rs:417-456): e = (2m)/head_dim, freq = 1 / theta^e,
// val = q * freq; cs[2m] = cos(val), cs[2m+1] = sin(val).  The same for
// every head and layer, so computed once per step.
__device__ void rope_table(const RopeArgs& r, int q) {
    for (int m = threadIdx.x; m < r.head_dim / 2; m += blockDim.x) {
        const float e = (float)(2 * m) / (float)r.head_dim;
        const float freq = 1.0f / libm::powf(r.theta, e);
        const float val = (float)q * freq;
        r.cs[2 * m] = libm::cosf(val);
        r.cs[2 * m + 1] = libm::sinf(val);
    }
}

// the angle table's rows 0..rows-1: workgroup q writes position q's
__global__ __launch_bounds__(128) void rope_rows_kernel(RopeArgs r) {
    const int q = (int)blockIdx.x;
    RopeArgs rq = r;
    rq.cs = r.cs + (size_t)q * r.head_dim;
    rope_table(rq, q);
}

// a token past the table reads row 0 (the host reports the reference's error)
__global__ __launch_bounds__(256) void embed_kernel(int type, const uint8_t* __restrict__ table, uint32_t rows,
                                                    const uint32_t* __restrict__ tokens, const int* __restrict__ pos,
                                                    int dim, size_t rb, float* __restrict__ x) {
    const uint32_t tok = tokens[*pos];
    const uint8_t* row = table + (size_t)(tok < rows ? tok : 0u) * rb;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) x[i] = embed_elem(type, row, i);
}

// the prompt's rows at once: workgroup p embeds tokens[p] into x[p][..]
__global__ __launch_bounds__(256) void embed_rows_kernel(int type, const uint8_t* __restrict__ table, uint32_t rows,
                                                         const uint32_t* __restrict__ tokens, int dim, size_t rb,
                                                         float* __restrict__ x) {
    const int p = (int)blockIdx.x;
    const uint32_t tok = tokens[p];
    const uint8_t* row = table + (size_t)(tok < rows ? tok : 0u) * rb;
    float* xp = x + (size_t)p * dim;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) xp[i] = embed_elem(type, row, i);
}

// products in parallel, the sum of squares in the reference's serial order
// by wave 0: where the walk of vtq_sumsq.h applies (1024-4096 terms, a
// multiple of 64) with the products in its pass layout and waves 1-3 as its
// helpers, otherwise as one chain over the products in order
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* x, const float* __restrict__ add, float* xw,
                                                       const float* __restrict__ w, int n, float eps,
                                                       float* __restrict__ out) {
    // one row per workgroup (rows of n floats, row blockIdx.x); with add,
    // the row is x + add (a residual, x[i] + add[i] per element), written to
    // xw (which may be x) and normalised
    x += (size_t)blockIdx.x * n;
    out += (size_t)blockIdx.x * n;
    if (add) {
        add += (size_t)blockIdx.x * n;
        xw += (size_t)blockIdx.x * n;
    }
    auto elem = [&](int i) {
        float v = x[i];
        if (add) {
            v = v + add[i];
            xw[i] = v;
        }
        return v;
    };
    extern __shared__ float4 prod4[];
    float* prod = reinterpret_cast<float*>(prod4);
    __shared__ float scale_s;
    const int H = sumsq_walk_head(n);  // uniform
    if (H) {
        const int wave = threadIdx.x >> 6;
        SumsqWalk& walk = *reinterpret_cast<SumsqWalk*>(prod + 4096);
        float hpart = 0.0f, apart = 0.0f;
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const float v = elem(i);
            const float p = v * v;
            prod[sumsq_pass_index(i)] = p;
            apart += p;
            if (i < H) hpart += p;
        }
        if (threadIdx.x < 32 && (threadIdx.x & 15) >= 4) walk.part[threadIdx.x >> 4][threadIdx.x & 15] = 0.0f;  // no waves 4-15
        sumsq_walk_partials(hpart, apart, walk);
        __syncthreads();
        float sumsq = 0.0f;
        if (wave == 0) {
            float r[64];
            sumsq_load_pass0(prod, r);
            sumsq = sumsq_chain(r, 0, H / 64, 0.0f);
        } else {
            sumsq_walk_helper(wave - 1, prod, n, H, walk);
        }
        __syncthreads();
        if (wave == 0) {
            sumsq = sumsq_walk(sumsq, prod, n, H, walk);
            const float mean = sumsq / (float)n;
            if (threadIdx.x == 0) scale_s = 1.0f / libm::sqrtf(mean + eps);
        }
    } else {
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const float v = elem(i);
            prod[i] = v * v;
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            const float sumsq = serial_sum_wave(prod, n);
            const float mean = sumsq / (float)n;
            if (threadIdx.x == 0) scale_s = 1.0f / libm::sqrtf(mean + eps);
        }
    }
    __syncthreads();
    const float scale = scale_s;
    const float* xs = add ? xw : x;  // each thread reads back only what it wrote
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = xs[i] * scale * w[i];
}

// A prefetch workgroup: workgroup g of G streams its share of every range
// (16-byte loads, four in flight per thread).
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
__device__ void prefetch_ranges(const Prefetch& pf, int g, int G) {
    uint32_t acc = 0;
    const uint32_t step = (uint32_t)G * blockDim.x * 16u;
    const uint32_t rows = pf.pos ? (uint32_t)max(*pf.pos, 0) : 0u;
#pragma unroll
    for (int r = 0; r < Prefetch::kRanges; r++) {
        const uint32_t n = pf.row_bytes[r] ? min(pf.n[r], rows * pf.row_bytes[r]) : pf.n[r];
        if (!n) continue;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(pf.p[r]), (short)0, (int)n, 0x00020000);
        for (uint32_t off = ((uint32_t)g * blockDim.x + threadIdx.x) * 16u; off < n; off += 4 * step) {
            uint32_t o[4];
#pragma unroll
            for (int u = 0; u < 4; u++) o[u] = off + (uint32_t)u * step;  // out of range: zeros, no traffic
            v4u v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rs, o[u], 0, 0));
#pragma unroll
            for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        }
    }
    if (acc == pf.magic && pf.sink) pf.sink[0] = acc;
}

constexpr int kAttnThreads = 256;
constexpr int kAttnTile = 256;  // cached v positions per LDS tile at head_dim 64 (64 KiB)

// max in the reference's sense (strict >, NaN never wins), as a tree
// Largest of the threads' m (none is NaN, so the order of the comparisons
// is free): within each wave by DPP, then across the waves through red[].
// red[0..kAttnThreads/64) must not be rewritten before the next barrier.
__device__ float block_max(float m, float* red) {
    m = wave_max_nonneg(m);  // any non-NaN values: the DPP patterns stay inside each row
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kAttnThreads / 64; w++) r = red[w] > r ? red[w] : r;
    return r;
}

// One workgroup per query head h.  Shared: q (roped), this step's k (roped)
// and v of h's KV head, then the attention weights of positions 0..pos (in
// LDS, or for contexts too long for it in the head's row of a.att_g).
// HD > 0: the head dimension as a compile-time constant; with HD == 64 and
// pos < kAttnThreads the position is read first, every load that does not
// need it (q, k, v, the rope angles, thread t's cached k row) is issued
// with it, and the cached v rows 0..pos are issued as soon as it returns
// and stored to LDS only after the softmax, so they arrive behind the
// scores.
template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(AttnArgs a) {
    if ((int)blockIdx.x >= a.heads) {  // a prefetch workgroup
        prefetch_ranges(a.pf, (int)blockIdx.x - a.heads, a.pf.groups);
        return;
    }
    extern __shared__ float4 sh4[];
    float* sh = reinterpret_cast<float*>(sh4);
    const int hd = HD > 0 ? HD : a.head_dim, h = blockIdx.x, kv_mul = a.heads / a.kv_heads, hk = h / kv_mul;
    const int kv_dim = a.kv_heads * hd, dim = a.heads * hd;
    float* qs = sh;
    float* kp = qs + hd;
    float* vp = kp + hd;
    float* red = vp + hd;
    float* att_l = red + kAttnThreads + (4 - (3 * hd) % 4) % 4;  // 16-byte aligned for float4 reads
    const size_t seq4 = ((size_t)a.seq + 3) & ~(size_t)3;
    float* att = a.att_g ? a.att_g + (size_t)h * seq4 : att_l;
    float* vt = a.att_g ? att_l : att_l + seq4;
    const int t0 = threadIdx.x;
    constexpr bool kFast = HD == 64;
    // The position first, then every load that does not need it: q, k, v
    // (+ bias, forward_quantized.rs:390-404), this step's RoPE angles and
    // (head_dim 64) thread t's cached k row t into registers.  Rows at or
    // past the position hold older values and are never used; rows past the
    // cache are not read.
    const int p = *a.pos;
    const float* qkv = a.qkv;
    const float* cs = a.cs + (size_t)p * hd;
    float* out = a.out;
    float qv = 0.0f, kv = 0.0f, vv = 0.0f, rc = 0.0f, rs = 0.0f;
    if (t0 < hd) qv = qkv[h * hd + t0], kv = qkv[dim + hk * hd + t0], vv = qkv[dim + kv_dim + hk * hd + t0];
    if (t0 < hd / 2) rc = cs[2 * t0], rs = cs[2 * t0 + 1];
    constexpr int KPT = kFast ? HD / 4 : 1;
    float4 kr[KPT], vr[KPT];
    const bool fast = kFast && p < kAttnThreads;
    if constexpr (kFast) {
        // cached rows 0..pos-1 (fast path): float4 i = t0 + kAttnThreads*u
        // of the head's k rows and of its v rows (row i / 16, part i % 16:
        // each load instruction reads whole rows), as raw buffer loads whose
        // unneeded slots get an out-of-range offset (zeros, no memory
        // traffic), so every load is unconditional and the wait counts stay
        // exact.  The k rows then go through the v tile's LDS, so that thread
        // t can read row t for its score.
        const size_t cbytes = (size_t)a.seq * kv_dim * 4;
        const int nrec = (int)(cbytes < 0x7FFFFFF0u ? cbytes : 0x7FFFFFF0u);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(a.kc, (short)0, nrec, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(a.vc, (short)0, nrec, 0x00020000);
        const int nv = fast ? p * (HD / 4) : 0;
#pragma unroll
        for (int u = 0; u < KPT; u++) {
            const int i = t0 + kAttnThreads * u, t = i / (HD / 4);
            const uint32_t off = i < nv ? (uint32_t)(((size_t)t * kv_dim + hk * hd) * 4 + 16 * (i % (HD / 4)))
                                        : 0x80000000u;
            kr[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
            vr[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
        }
        // row t's part j at float4 16t + (j ^ (t % 16)) of the tile: a row's
        // sixteen writes and sixteen threads' reads of one part each cover
        // all banks
        if (fast) {
#pragma unroll
            for (int u = 0; u < KPT; u++) {
                const int i = t0 + kAttnThreads * u, t = i / (HD / 4);
                if (i < nv) reinterpret_cast<float4*>(vt)[16 * t + ((i % (HD / 4)) ^ (t & 15))] = kr[u];
            }
        }
    }
    for (int d = t0; d < hd; d += kAttnThreads) {
        float q = d == t0 ? qv : qkv[h * hd + d], k = d == t0 ? kv : qkv[dim + hk * hd + d],
              v = d == t0 ? vv : qkv[dim + kv_dim + hk * hd + d];
        if (a.bq) q = q + a.bq[h * hd + d];
        if (a.bk) k = k + a.bk[hk * hd + d];
        if (a.bv) v = v + a.bv[hk * hd + d];
        qs[d] = q;
        kp[d] = k;
        vp[d] = v;
    }
    __syncthreads();
    // RoPE with this step's angles (rope_table)
    for (int m = t0; m < hd / 2; m += kAttnThreads) {
        const float c = m == t0 ? rc : cs[2 * m], s = m == t0 ? rs : cs[2 * m + 1];
        const int i0 = a.neox ? m : 2 * m, i1 = a.neox ? m + hd / 2 : 2 * m + 1;
        const float q0 = qs[i0], q1 = qs[i1], k0 = kp[i0], k1 = kp[i1];
        qs[i0] = q0 * c - q1 * s;
        qs[i1] = q0 * s + q1 * c;
        kp[i0] = k0 * c - k1 * s;
        kp[i1] = k0 * s + k1 * c;
    }
    __syncthreads();
    // the cache write, once per KV head; other heads of the group read
    // positions < pos from the cache and this position from kp / vp
    if (h % kv_mul == 0) {
        for (int d = t0; d < hd; d += kAttnThreads) {
            a.kc[(size_t)p * kv_dim + hk * hd + d] = kp[d];
            a.vc[(size_t)p * kv_dim + hk * hd + d] = vp[d];
        }
    }
    // scores: sum over d in order, then / sqrt(head_dim)
    const float sq = libm::sqrtf((float)hd);
    float mx = -__builtin_inff();
    if (fast) {
        if (t0 <= p) {
            // position p's k is this step's roped k (LDS), the others' the
            // cached row (in the tile)
            if (t0 == p) {
#pragma unroll
                for (int j = 0; j < KPT; j++) kr[j] = reinterpret_cast<const float4*>(kp)[j];
            } else {
#pragma unroll
                for (int j = 0; j < KPT; j++) kr[j] = reinterpret_cast<const float4*>(vt)[16 * t0 + (j ^ (t0 & 15))];
            }
            float score = 0.0f;
#pragma unroll
            for (int j = 0; j < KPT; j++) {
                const float4 q4 = reinterpret_cast<const float4*>(qs)[j];
                score += q4.x * kr[j].x;
                score += q4.y * kr[j].y;
                score += q4.z * kr[j].z;
                score += q4.w * kr[j].w;
            }
            score /= sq;
            att[t0] = score;
            if (score > mx) mx = score;  // a NaN score never becomes the max
        }
    } else {
        for (int t = t0; t <= p; t += kAttnThreads) {
            const float* kt = t == p ? kp : a.kc + (size_t)t * kv_dim + hk * hd;
            float score = 0.0f;
            for (int d = 0; d < hd; d++) score += qs[d] * kt[d];
            score /= sq;
            att[t] = score;
            if (score > mx) mx = score;
        }
    }
    // softmax_inplace (forward_quantized.rs:925-941)
    mx = block_max(mx, red);
    for (int t = t0; t <= p; t += kAttnThreads) att[t] = libm::expf(att[t] - mx);
    __syncthreads();
    if (t0 < 64) {
        const float sum = serial_sum_wave(att, p + 1);
        if (t0 == 0) red[0] = 1.0f / sum;
    }
    __syncthreads();
    const float inv = red[0];
    for (int t = t0; t <= p; t += kAttnThreads) att[t] *= inv;
    // out[d] = sum over t in order of att[t] * v_t[d]: the cached v rows go
    // through LDS (in tiles of kAttnTile * 64 floats unless the fast path
    // already holds them all in registers), this position's v comes from vp
    auto accumulate = [&](float& acc, int c0, int nt) {
        if (t0 < hd) {
            int t = 0;
            // chunks of 32 positions: the loads of group g+1 are issued
            // before the adds of group g, in straight-line code
            auto ld = [&](float (&vb)[8], float (&ab)[8], int t1) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < 8; j++) vb[j] = vt[(t1 + j) * hd + t0];
                if (((c0 + t1) & 3) == 0) {  // the weights as two float4 (wave-uniform test)
                    const float4 w0 = *reinterpret_cast<const float4*>(att + c0 + t1);
                    const float4 w1 = *reinterpret_cast<const float4*>(att + c0 + t1 + 4);
                    ab[0] = w0.x, ab[1] = w0.y, ab[2] = w0.z, ab[3] = w0.w;
                    ab[4] = w1.x, ab[5] = w1.y, ab[6] = w1.z, ab[7] = w1.w;
                } else {
#pragma unroll
                    for (int j = 0; j < 8; j++) ab[j] = att[c0 + t1 + j];
                }
            };
            auto add = [&](const float (&vb)[8], const float (&ab)[8]) __attribute__((always_inline)) {
                float pr[8];
#pragma unroll
                for (int j = 0; j < 8; j++) pr[j] = ab[j] * vb[j];
#pragma unroll
                for (int j = 0; j < 8; j++) acc += pr[j];
            };
            for (; t + 32 <= nt; t += 32) {
                float va[8], aa[8], vb[8], ab[8];
                ld(va, aa, t);
                ld(vb, ab, t + 8);
                add(va, aa);
                ld(va, aa, t + 16);
                add(vb, ab);
                ld(vb, ab, t + 24);
                add(va, aa);
                add(vb, ab);
            }
            for (; t + 8 <= nt; t += 8) {
                float vb[8], ab[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    vb[j] = vt[(t + j) * hd + t0];
                    ab[j] = att[c0 + t + j];
                }
#pragma unroll
                for (int j = 0; j < 8; j++) acc += ab[j] * vb[j];
            }
            for (; t < nt; t++) acc += att[c0 + t] * vt[t * hd + t0];
        }
    };
    float acc = 0.0f;
    if (fast) {
#pragma unroll
        for (int u = 0; u < KPT; u++)
            if (t0 + kAttnThreads * u < p * (HD / 4)) reinterpret_cast<float4*>(vt)[t0 + kAttnThreads * u] = vr[u];
        __syncthreads();
        accumulate(acc, 0, p);
    } else {
        const int tile = kAttnTile * 64 / hd;
        for (int c0 = 0; c0 < p; c0 += tile) {
            const int nt = p - c0 < tile ? p - c0 : tile;
            for (int i = t0; i < nt * hd / 4; i += kAttnThreads) {
                const int t = i / (hd / 4), q4 = i % (hd / 4);
                reinterpret_cast<float4*>(vt)[i] =
                    *reinterpret_cast<const float4*>(a.vc + (size_t)(c0 + t) * kv_dim + hk * hd + 4 * q4);
            }
            __syncthreads();
            accumulate(acc, c0, nt);
            __syncthreads();
        }
    }
    __syncthreads();
    if (t0 < hd) out[h * hd + t0] = acc + att[p] * vp[t0];
}

// Orders one wave's LDS writes before its later LDS reads by other lanes:
// a wave's LDS operations complete in issue order, so only the compiler has
// to be kept from moving them across this point.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Attention of a prompt pass: one wave per (query head, position); a
// workgroup holds position blockIdx.y and G consecutive query heads of one KV
// group (heads G * blockIdx.x + wave), which share that KV head's cached rows.
// The arithmetic is attention_kernel's for its own position, step for step:
// q (+ bias) with RoPE at position p's angles, each score a dot over d in
// order, / sqrt(hd), the largest non-NaN score, expf, the serial sum over
// positions 0..p, its reciprocal, the weights scaled by it, then per output
// dim the weighted v rows summed over positions 0..p-1 in order, plus
// position p's term.  The cached rows (rope_cache_kernel has written position
// p's as well) go through one LDS tile of T rows, loaded by the whole
// workgroup with coalesced 16-byte loads: k rows 0..p (lane r of a wave
// scores row r of a tile, rows padded by 4 floats), then v rows 0..p-1 (lane
// d adds dim d).  Each tile's loads are issued before the tile ahead of it is
// used (the first k tile at the start, the first v tile before the softmax).
// LDS: per wave q (hd floats) and the scores (P rounded up to 4), then the
// tile.
constexpr int kRowsMaxWaves = 8;
constexpr int kRowsTileF4 = 4;  // float4 of a tile per thread
__host__ __device__ inline int rows_tile(int G, int hd) { return kRowsTileF4 * G * 64 * 4 / hd; }
__host__ __device__ inline int rows_tile_floats(int G, int hd) {
    const int k = rows_tile(G, hd) * (hd + 4), v = kRowsTileF4 * G * 64 * 4;
    return k > v ? k : v;
}

template <int HD>
__global__ __launch_bounds__(kRowsMaxWaves * 64) void attention_rows_kernel(AttnArgs a) {
    extern __shared__ float4 lds4[];
    const int hd = HD > 0 ? HD : a.head_dim, lane = threadIdx.x & 63, wave = (int)(threadIdx.x >> 6);
    const int G = (int)(blockDim.x >> 6), P = a.batched, nthr = (int)blockDim.x;
    const int p = (int)blockIdx.y;
    const int h = (int)blockIdx.x * G + wave, kv_mul = a.heads / a.kv_heads, hk = h / kv_mul;
    const int kv_dim = a.kv_heads * hd, dim = a.heads * hd;
    const int P4 = (P + 3) & ~3, T = rows_tile(G, hd), RS = hd + 4, H4 = hd / 4;
    float* qs = reinterpret_cast<float*>(lds4) + (size_t)wave * (hd + P4);
    float* att = qs + hd;
    float* tile = reinterpret_cast<float*>(lds4) + (size_t)G * (hd + P4);
    // rows c0 .. c0 + T - 1 below `end` of KV head hk of a cache: float4 i of
    // the tile is row c0 + i / (hd/4), part i % (hd/4); other slots get an
    // out-of-range offset (zeros, no memory traffic)
    const size_t cbytes = (size_t)a.seq * kv_dim * 4;
    const int nrec = (int)(cbytes < 0x7FFFFFF0u ? cbytes : 0x7FFFFFF0u);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(a.kc, (short)0, nrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(a.vc, (short)0, nrec, 0x00020000);
    float4 tr[kRowsTileF4];
    auto load_rows = [&](__amdgpu_buffer_rsrc_t rs, int c0, int end) {
#pragma unroll
        for (int u = 0; u < kRowsTileF4; u++) {
            const int i = (int)threadIdx.x + nthr * u, r = i / H4, t = c0 + r;
            const uint32_t off = r < T && t < end ? (uint32_t)(((size_t)t * kv_dim + hk * hd) * 4 + 16 * (i % H4))
                                                  : 0x80000000u;
            tr[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
        }
    };
    // the loaded rows into the tile, row stride `stride` floats
    auto store_rows = [&](int stride) {
#pragma unroll
        for (int u = 0; u < kRowsTileF4; u++) {
            const int i = (int)threadIdx.x + nthr * u, r = i / H4;
            if (r < T) reinterpret_cast<float4*>(tile + (size_t)r * stride)[i % H4] = tr[u];
        }
    };
    load_rows(rk, 0, p + 1);
    const float* qkv = a.qkv + (size_t)p * (dim + 2 * kv_dim);
    const float* cs = a.cs + (size_t)p * hd;
    for (int d = lane; d < hd; d += 64) {
        float q = qkv[h * hd + d];
        if (a.bq) q = q + a.bq[h * hd + d];
        qs[d] = q;
    }
    wave_lds_sync();
    for (int m = lane; m < hd / 2; m += 64) {
        const float c = cs[2 * m], sn = cs[2 * m + 1];
        const int i0 = a.neox ? m : 2 * m, i1 = a.neox ? m + hd / 2 : 2 * m + 1;
        const float q0 = qs[i0], q1 = qs[i1];
        qs[i0] = q0 * c - q1 * sn;
        qs[i1] = q0 * sn + q1 * c;
    }
    wave_lds_sync();
    const float sq = libm::sqrtf((float)hd);
    float mx = -__builtin_inff();
    for (int c0 = 0; c0 <= p; c0 += T) {  // uniform over the workgroup: every wave has this p
        store_rows(RS);
        __syncthreads();
        if (c0 + T <= p) load_rows(rk, c0 + T, p + 1);
        const int nt = p + 1 - c0 < T ? p + 1 - c0 : T;
        for (int r = lane; r < nt; r += 64) {
            const float4* kt = reinterpret_cast<const float4*>(tile + (size_t)r * RS);
            const float4* q4 = reinterpret_cast<const float4*>(qs);
            float score = 0.0f;
            if constexpr (HD > 0) {
#pragma unroll
                for (int j = 0; j < HD / 4; j++) {
                    const float4 qv = q4[j], kv = kt[j];
                    score += qv.x * kv.x;
                    score += qv.y * kv.y;
                    score += qv.z * kv.z;
                    score += qv.w * kv.w;
                }
            } else {
                for (int j = 0; j < H4; j++) {
                    const float4 qv = q4[j], kv = kt[j];
                    score += qv.x * kv.x;
                    score += qv.y * kv.y;
                    score += qv.z * kv.z;
                    score += qv.w * kv.w;
                }
            }
            score /= sq;
            att[c0 + r] = score;
            if (score > mx) mx = score;  // a NaN score never becomes the max
        }
        __syncthreads();
    }
    load_rows(rv, 0, p);  // the first v tile, in flight during the softmax
    mx = wave_max_nonneg(mx);  // exact for any non-NaN values
    for (int t = lane; t <= p; t += 64) att[t] = libm::expf(att[t] - mx);
    wave_lds_sync();
    const float inv = 1.0f / serial_sum_wave(att, p + 1);
    wave_lds_sync();
    for (int t = lane; t <= p; t += 64) att[t] *= inv;
    wave_lds_sync();
    // out[d] for d = lane + 64 s (s < hd/64 rounded up)
    constexpr int kS = HD > 0 ? (HD + 63) / 64 : 4;
    float acc[kS];
#pragma unroll
    for (int sl = 0; sl < kS; sl++) acc[sl] = 0.0f;
    for (int c0 = 0; c0 < p; c0 += T) {  // uniform over the workgroup
        store_rows(hd);
        __syncthreads();
        if (c0 + T < p) load_rows(rv, c0 + T, p);
        const int nt = p - c0 < T ? p - c0 : T;
#pragma unroll
        for (int sl = 0; sl < kS; sl++) {
            const int d = lane + 64 * sl;
            if (d < hd) {
                float s_acc = acc[sl];
                int t = 0;
                for (; t + 8 <= nt; t += 8) {
                    float vb[8], ab[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) vb[j] = tile[(t + j) * hd + d];
                    const float4 w0 = *reinterpret_cast<const float4*>(att + c0 + t);
                    const float4 w1 = *reinterpret_cast<const float4*>(att + c0 + t + 4);
                    ab[0] = w0.x, ab[1] = w0.y, ab[2] = w0.z, ab[3] = w0.w;
                    ab[4] = w1.x, ab[5] = w1.y, ab[6] = w1.z, ab[7] = w1.w;
                    float pr[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) pr[j] = ab[j] * vb[j];
#pragma unroll
                    for (int j = 0; j < 8; j++) s_acc += pr[j];
                }
                for (; t < nt; t++) s_acc += att[c0 + t] * tile[t * hd + d];
                acc[sl] = s_acc;
            }
        }
        __syncthreads();
    }
    const float* vrow = qkv + dim + kv_dim + hk * hd;
    float* out = a.out + (size_t)p * dim + h * hd;
#pragma unroll
    for (int sl = 0; sl < kS; sl++) {
        const int d = lane + 64 * sl;
        if (d < hd) {
            float v = vrow[d];
            if (a.bv) v = v + a.bv[hk * hd + d];
            out[d] = acc[sl] + att[p] * v;
        }
    }
}

// The cache write of a prompt pass: workgroup (p, hk) writes position p's
// roped k and its v of KV head hk, computed as attention_kernel does for its
// own position (bias, then the RoPE pairs with position p's angles).
__global__ __launch_bounds__(kAttnThreads) void rope_cache_kernel(AttnArgs a) {
    __shared__ float kp[kAttnThreads];
    const int p = (int)blockIdx.x, hk = (int)blockIdx.y, hd = a.head_dim, t0 = threadIdx.x;
    const int kv_dim = a.kv_heads * hd, dim = a.heads * hd;
    const float* qkv = a.qkv + (size_t)p * (dim + 2 * kv_dim);
    const float* cs = a.cs + (size_t)p * hd;
    float* kc = a.kc + (size_t)p * kv_dim + hk * hd;
    float* vc = a.vc + (size_t)p * kv_dim + hk * hd;
    for (int d = t0; d < hd; d += kAttnThreads) {
        float k = qkv[dim + hk * hd + d], v = qkv[dim + kv_dim + hk * hd + d];
        if (a.bk) k = k + a.bk[hk * hd + d];
        if (a.bv) v = v + a.bv[hk * hd + d];
        kp[d] = k;
        vc[d] = v;
    }
    __syncthreads();
    for (int m = t0; m < hd / 2; m += kAttnThreads) {
        const float c = cs[2 * m], s = cs[2 * m + 1];
        const int i0 = a.neox ? m : 2 * m, i1 = a.neox ? m + hd / 2 : 2 * m + 1;
        const float k0 = kp[i0], k1 = kp[i1];
        kc[i0] = k0 * c - k1 * s;
        kc[i1] = k0 * s + k1 * c;
    }
}

constexpr int kArgThreads = 1024;

// argmax of step p, then the embedding row of the token step p+1 consumes
// (the prompt's while p+1 < prompt_len, the pick after), into x
__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float* __restrict__ v, int n,
                                                             uint32_t* __restrict__ tokens, int* __restrict__ pos,
                                                             int prompt_len, int total, float* __restrict__ hist,
                                                             EmbedArgs e) {
    __shared__ float bv[kArgThreads];
    __shared__ int bi[kArgThreads];
    __shared__ uint32_t next_s;
    const int p = *pos;
    // first index of the largest non-NaN value (strict > in index order);
    // thread t scans float4 groups t, t + kArgThreads, ... in index order
    float b = 0.0f;
    int idx = -1;
    const int n4 = n / 4;
    constexpr int U = 8;
    for (int g0 = threadIdx.x; g0 < n4; g0 += U * kArgThreads) {
        float4 r[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int g = g0 + u * kArgThreads;
            r[u] = reinterpret_cast<const float4*>(v)[g < n4 ? g : 0];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int g = g0 + u * kArgThreads;
            if (g < n4) {
                const float xs[4] = {r[u].x, r[u].y, r[u].z, r[u].w};
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (xs[k] == xs[k] && (idx < 0 || xs[k] > b)) {
                        b = xs[k];
                        idx = 4 * g + k;
                    }
                if (hist) reinterpret_cast<float4*>(hist + (size_t)p * n)[g] = r[u];
            }
        }
    }
    for (int i = 4 * n4 + threadIdx.x; i < n; i += kArgThreads) {
        const float x = v[i];
        if (hist) hist[(size_t)p * n + i] = x;
        if (x == x && (idx < 0 || x > b)) {
            b = x;
            idx = i;
        }
    }
    bv[threadIdx.x] = b;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (int s = kArgThreads / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const int oi = bi[threadIdx.x + s], mi = bi[threadIdx.x];
            const float ov = bv[threadIdx.x + s], mv = bv[threadIdx.x];
            if (oi >= 0 && (mi < 0 || ov > mv || (ov == mv && oi < mi))) {
                bv[threadIdx.x] = ov;
                bi[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        // a NaN at index 0 is never beaten (argmax.rs: strict > against it)
        const uint32_t best = (v[0] != v[0] || bi[0] < 0) ? 0u : (uint32_t)bi[0];
        uint32_t next = best;
        if (p + 1 >= prompt_len && p + 1 <= total)
            tokens[p + 1] = best;
        else if (p + 1 < prompt_len)
            next = tokens[p + 1];
        next_s = next;
        *pos = p + 1;
    }
    __syncthreads();
    if (p + 1 < total && e.table) {
        const uint32_t tok = next_s;
        const uint8_t* row = e.table + (size_t)(tok < e.rows ? tok : 0u) * e.row_bytes;
        for (int i = threadIdx.x; i < e.dim; i += kArgThreads) e.x[i] = embed_elem(e.type, row, i);
    }
}

__global__ void add_kernel(float* __restrict__ x, const float* __restrict__ y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

__global__ void swiglu_kernel(const float* __restrict__ gate, const float* __restrict__ up, float* __restrict__ out,
                              int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float g = gate[i];
        const float silu = g / (1.0f + libm::expf(-g));
        out[i] = silu * up[i];
    }
}

// rows of gate | up (2 * hidden floats each): out[p][j] = silu(gate) * up
__global__ void swiglu_rows_kernel(const float* __restrict__ gu, int hidden, int rows, float* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * hidden) return;
    const size_t p = i / (size_t)hidden, j = i % (size_t)hidden;
    const float g = gu[p * 2 * hidden + j];
    const float silu = g / (1.0f + libm::expf(-g));
    out[i] = silu * gu[p * 2 * hidden + hidden + j];
}

}  // namespace

size_t embed_row_bytes(int ggml_type, int dim) {
    switch (ggml_type) {
    case 0: case 2: case 6: case 8: case 12: case 14: break;
    default: return 0;
    }
    const int blk = (ggml_type == 12 || ggml_type == 14) ? 256 : ggml_type == 0 ? 1 : 32;
    return dim > 0 && dim % blk == 0 ? row_bytes(ggml_type, dim) : 0;
}

hipError_t embed(int ggml_type, const uint8_t* table, uint32_t rows, const uint32_t* tokens, const int* pos, int dim,
                 float* x, hipStream_t stream) {
    hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(256), 0, stream, ggml_type, table, rows, tokens, pos, dim,
                       row_bytes(ggml_type, dim), x);
    return hipGetLastError();
}

hipError_t rms_norm(const float* x, const float* w, int n, float eps, float* out, hipStream_t stream) {
    // the walk: one 4096-float pass of products and its tables; else the
    // products in order (the serial sum reads whole float4s)
    const size_t lds = sumsq_walk_head(n) ? 4096 * 4 + sizeof(SumsqWalk) : (size_t)((n + 3) & ~3) * 4;
    if (hipError_t e = allow_dynamic_lds(reinterpret_cast<const void*>(rms_norm_kernel), lds)) return e;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(256), lds, stream, x, nullptr, nullptr, w, n, eps, out);
    return hipGetLastError();
}

hipError_t rms_norm_rows(const float* x, const float* w, int n, int rows, float eps, float* out, hipStream_t stream) {
    return add_rms_norm_rows(const_cast<float*>(x), nullptr, w, n, rows, eps, out, stream);
}

hipError_t add_rms_norm_rows(float* x, const float* add, const float* w, int n, int rows, float eps, float* out,
                             hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const size_t lds = sumsq_walk_head(n) ? 4096 * 4 + sizeof(SumsqWalk) : (size_t)((n + 3) & ~3) * 4;
    if (hipError_t e = allow_dynamic_lds(reinterpret_cast<const void*>(rms_norm_kernel), lds)) return e;
    hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)rows), dim3(256), lds, stream, x, add, add ? x : nullptr, w, n,
                       eps, out);
    return hipGetLastError();
}

template <int HD>
static hipError_t launch_attention(const AttnArgs& a, size_t lds, hipStream_t stream) {
    if (hipError_t e = allow_dynamic_lds(reinterpret_cast<const void*>(attention_kernel<HD>), lds)) return e;
    hipLaunchKernelGGL(attention_kernel<HD>, dim3((unsigned)(a.heads + a.pf.groups)), dim3(kAttnThreads), lds, stream,
                       a);
    return hipGetLastError();
}

// LDS bytes: q, k, v, the reduction slots, (the scores,) the v tiles
static size_t attention_lds(int head_dim, int seq, bool scores) {
    return ((size_t)3 * head_dim + kAttnThreads + 4 + (scores ? (((size_t)seq + 3) & ~(size_t)3) : 0) +
            kAttnTile * 64) * 4;
}

// a prompt pass: G query heads (waves) per workgroup, the largest divisor
// of the KV group size up to kRowsMaxWaves whose q and score rows fit in
// LDS; 0 if none does
static size_t attention_rows_lds(int head_dim, int P, int G) {
    return ((size_t)G * ((size_t)head_dim + (((size_t)P + 3) & ~(size_t)3)) + (size_t)rows_tile_floats(G, head_dim)) * 4;
}

static int attention_rows_waves(int head_dim, int P, int kv_mul) {
    for (int G = kv_mul < kRowsMaxWaves ? kv_mul : kRowsMaxWaves; G >= 1; G--)
        if (kv_mul % G == 0 && attention_rows_lds(head_dim, P, G) <= 160 * 1024 && rows_tile(G, head_dim) >= 1)
            return G;
    return 0;
}

template <int HD>
static hipError_t launch_attention_rows(const AttnArgs& a, int G, hipStream_t stream) {
    const size_t lds = attention_rows_lds(a.head_dim, a.batched, G);
    if (hipError_t e = allow_dynamic_lds(reinterpret_cast<const void*>(attention_rows_kernel<HD>), lds)) return e;
    hipLaunchKernelGGL(attention_rows_kernel<HD>, dim3((unsigned)(a.heads / G), (unsigned)a.batched),
                       dim3((unsigned)G * 64), lds, stream, a);
    return hipGetLastError();
}

bool attention_rows_supported(int head_dim, int P, int heads, int kv_heads) {
    return head_dim > 0 && head_dim <= 256 && head_dim % 4 == 0 && P > 0 && kv_heads > 0 && heads % kv_heads == 0 &&
           attention_rows_waves(head_dim, P, heads / kv_heads) > 0;
}

static hipError_t attention_rows(const AttnArgs& a, hipStream_t stream) {
    if (a.batched > a.seq || !attention_rows_supported(a.head_dim, a.batched, a.heads, a.kv_heads))
        return hipErrorInvalidValue;
    const int G = attention_rows_waves(a.head_dim, a.batched, a.heads / a.kv_heads);
    if (!G) return hipErrorInvalidValue;
    if (a.head_dim == 64) return launch_attention_rows<64>(a, G, stream);
    if (a.head_dim == 128) return launch_attention_rows<128>(a, G, stream);
    return launch_attention_rows<0>(a, G, stream);
}

bool attention_supported(int head_dim, int seq) {
    return head_dim > 0 && head_dim <= kAttnThreads && head_dim % 4 == 0 && (kAttnTile * 64) % head_dim == 0 &&
           seq > 0;
}

bool attention_scores_in_lds(int head_dim, int seq) {
    return attention_lds(head_dim, seq, true) <= 160 * 1024;
}

hipError_t attention(const AttnArgs& a, hipStream_t stream) {
    if (!attention_supported(a.head_dim, a.seq)) return hipErrorInvalidValue;
    if (a.batched) return attention_rows(a, stream);
    const bool in_lds = attention_scores_in_lds(a.head_dim, a.seq);
    if (!in_lds && !a.att_g) return hipErrorInvalidValue;
    const AttnArgs* ap = &a;
    AttnArgs lds_args;
    if (in_lds && a.att_g) {  // the scores fit: keep them in LDS
        lds_args = a;
        lds_args.att_g = nullptr;
        ap = &lds_args;
    }
    const size_t lds = attention_lds(a.head_dim, a.seq, in_lds);
    if (a.head_dim == 64) return launch_attention<64>(*ap, lds, stream);
    if (a.head_dim == 128) return launch_attention<128>(*ap, lds, stream);
    return launch_attention<0>(*ap, lds, stream);
}

hipError_t embed_rows(int ggml_type, const uint8_t* table, uint32_t rows, const uint32_t* tokens, int P, int dim,
                      float* x, hipStream_t stream) {
    if (P <= 0) return hipSuccess;
    hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)P), dim3(256), 0, stream, ggml_type, table, rows, tokens, dim,
                       row_bytes(ggml_type, dim), x);
    return hipGetLastError();
}

hipError_t rope_table_rows(const RopeArgs& r, int rows, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (!r.cs || r.head_dim <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_rows_kernel, dim3((unsigned)rows), dim3(128), 0, stream, r);
    return hipGetLastError();
}

hipError_t rope_cache_rows(const AttnArgs& a, hipStream_t stream) {
    if (a.batched <= 0 || a.batched > a.seq || !attention_supported(a.head_dim, a.seq)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_cache_kernel, dim3((unsigned)a.batched, (unsigned)a.kv_heads), dim3(kAttnThreads), 0,
                       stream, a);
    return hipGetLastError();
}

hipError_t argmax_advance(const float* logits, int vocab, uint32_t* tokens, int* pos, int prompt_len, int total,
                          float* hist, const EmbedArgs& e, hipStream_t stream) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgThreads), 0, stream, logits, vocab, tokens, pos, prompt_len,
                       total, hist, e);
    return hipGetLastError();
}

// The device libm of the decode step over an input array, in the order of
// the reference's transcendental sweep (tests/transcendental_determinism.rs:
// 34-42): expf, sqrtf(|x|), cosf, sinf, powf(1e4, x/64), powf(1e6, x/64),
// 1 / (1 + expf(-x)).
__global__ __launch_bounds__(256) void transcendentals_kernel(const float* __restrict__ x, int n,
                                                             float* __restrict__ y) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= n) return;
    const float v = x[i];
    float* o = y + (size_t)7 * i;
    o[0] = libm::expf(v);
    o[1] = libm::sqrtf(libm::fabsf_(v));
    o[2] = libm::cosf(v);
    o[3] = libm::sinf(v);
    o[4] = libm::powf(10000.0f, v / 64.0f);
    o[5] = libm::powf(1000000.0f, v / 64.0f);
    o[6] = 1.0f / (1.0f + libm::expf(-v));
}

hipError_t transcendentals(const float* x, int n, float* y, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(transcendentals_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, x, n, y);
    return hipGetLastError();
}

hipError_t add_inplace(float* x, const float* y, int n, hipStream_t stream) {
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, x, y, n);
    return hipGetLastError();
}

hipError_t swiglu_rows(const float* gu, int hidden, int rows, float* out, hipStream_t stream) {
    const size_t n = (size_t)hidden * rows;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, gu, hidden, rows,
                       out);
    return hipGetLastError();
}

hipError_t swiglu(const float* gate, const float* up, float* out, int n, hipStream_t stream) {
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, gate, up, out, n);
    return hipGetLastError();
}

}  // namespace decode
}  // namespace vtq
