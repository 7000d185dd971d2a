// vtq_sumsq.h -- the sum of squares of rms_norm_slice (src/ops/rms_norm.rs:
// 96-100: sumsq += v * v over the row, in order) for one workgroup, bit for
// bit, with a shortcut over the serial chain.
//
// The serial chain pays one dependent add per term.  The shortcut rests on
// how a rounded add behaves inside one binade: while the running sum s stays
// in [2^e, 2^(e+1)) its spacing is u = 2^(e-23), s is a multiple of u, and for
// a term p >= 0
//     fl(s + p) = s + u * rn(p / u)
// unless the result reaches 2^(e+1) (the spacing changes) or p / u is exactly
// halfway between two integers (then the parity of s / u decides).  So
// between such events the serial sum is an integer prefix sum of rn(p / u),
// which lanes can form in parallel.
//
//   1. wave 0 runs the plain chain over the first H terms (the head), where
//      the sum still changes binade often;
//   2. meanwhile three helper waves, one on each of the other SIMDs, build
//      for every binade the running sum can reach the prefix sums of
//      rn(p / u) over the remaining terms and a tie mask per 32 terms;
//   3. wave 0 then walks from event to event: a binade crossing or a tie is
//      the first term whose prefix passes the crossing threshold or whose
//      tie bit is set, found with two ballots; the sum up to that term is
//      exact integer arithmetic, and the term itself is one ordinary add.
// Non-finite or degenerate inputs, a binade outside the tabulated window and
// more than kWalkMaxStops events fall back to the plain chain from where the
// walk stands, so every result equals the serial chain's.
//
// The products sit in LDS in the "pass layout": element 64L + k of pass P
// (P = i / 4096) at float 4096P + 256(k/4) + 4L + k%4, so lane L of one wave
// reads its 64 consecutive elements as sixteen conflict-free float4.
#pragma once
#include "vtq_device.h"

namespace vtq {

__host__ __device__ constexpr int sumsq_pass_index(int i) {
    return 4096 * (i >> 12) + 256 * ((i & 63) >> 2) + 4 * ((i >> 6) & 63) + (i & 3);
}

constexpr int kWalkBinades = 5;      // binades the helpers tabulate
constexpr int kWalkMaxTerms = 1536;  // terms after the head: 3 helper waves x 64 lanes x 8
constexpr int kWalkMaxStops = 48;    // events walked before falling back to the chain
// Helper-lane totals are capped here.  Every threshold the walk compares with
// is below 2^25 (a sum in binade e is under 2^24 units of that binade, plus
// at most half a unit per term), so a capped prefix still compares right, and
// no sum of capped totals and offsets overflows 32 bits.
constexpr uint32_t kWalkCap = 1u << 25;

// Length of the serial head for n terms, or 0 where the walk does not apply
// (n not a multiple of 64, below 1024 or above 4096 terms).
__host__ __device__ constexpr int sumsq_walk_head(int n) {
    return (n % 64 == 0 && n >= 1024 && n <= 4096) ? (n - kWalkMaxTerms > 640 ? n - kWalkMaxTerms : 640) : 0;
}

struct SumsqWalk {
    uint32_t Q[kWalkBinades][kWalkMaxTerms];  // per helper wave: prefix of rn(p / u) over its terms
    uint32_t TM[kWalkBinades][64];             // tie bits of each 32-term segment
    uint32_t WT[kWalkBinades][4];              // helper wave totals, capped at kWalkCap
    float part[2][16];                         // per-wave partial sums: terms < H, all terms
    int elo, nb, fb;                           // binade window [elo, elo + nb); fb: plain chain only
};

#define VTQ_DPP_STEP(op, ctrl) "s_nop 1\n\t" op "_dpp %0, %0, %0 " ctrl " bank_mask:0xf\n\t"
// Inclusive prefix sum over the 64 lanes: row_shr inside each 16-lane row,
// then row_bcast across rows.  A lane whose source is outside the row is not
// written (bound_ctrl off) and keeps its value.
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
    asm volatile(VTQ_DPP_STEP("v_add_u32", "row_shr:1 row_mask:0xf") VTQ_DPP_STEP("v_add_u32", "row_shr:2 row_mask:0xf")
                 VTQ_DPP_STEP("v_add_u32", "row_shr:4 row_mask:0xf") VTQ_DPP_STEP("v_add_u32", "row_shr:8 row_mask:0xf")
                 VTQ_DPP_STEP("v_add_u32", "row_bcast:15 row_mask:0xa")
                 VTQ_DPP_STEP("v_add_u32", "row_bcast:31 row_mask:0xc") "s_nop 1"
                 : "+v"(v));
    return v;
}
// Sum over the 64 lanes in some fixed order (an estimate only: it picks the
// binade window, never a result).
__device__ __forceinline__ float wave_total_f32(float v) {
    asm volatile(VTQ_DPP_STEP("v_add_f32", "row_shr:1 row_mask:0xf") VTQ_DPP_STEP("v_add_f32", "row_shr:2 row_mask:0xf")
                 VTQ_DPP_STEP("v_add_f32", "row_shr:4 row_mask:0xf") VTQ_DPP_STEP("v_add_f32", "row_shr:8 row_mask:0xf")
                 VTQ_DPP_STEP("v_add_f32", "row_bcast:15 row_mask:0xa")
                 VTQ_DPP_STEP("v_add_f32", "row_bcast:31 row_mask:0xc") "s_nop 1"
                 : "+v"(v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
#undef VTQ_DPP_STEP

__device__ __forceinline__ uint32_t rdl(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ uint32_t rdf(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }

// Step 0, every wave before the workgroup barrier: this wave's sums of its
// products below H and of all its products (any order).
__device__ __forceinline__ void sumsq_walk_partials(float head_part, float all_part, SumsqWalk& w) {
    const float hs = wave_total_f32(head_part), ts = wave_total_f32(all_part);
    if ((threadIdx.x & 63) == 0) {
        w.part[0][threadIdx.x >> 6] = hs;
        w.part[1][threadIdx.x >> 6] = ts;
    }
}

// The plain chain over lanes l0 .. nl-1 of pass-0 registers r (lane L holds
// elements 64L .. 64L+63), continuing from run.
__device__ inline float sumsq_chain(const float (&r)[64], int l0, int nl, float run) {
    float v[64];
#pragma unroll
    for (int k = 0; k < 64; k++) {
        v[k] = r[k];
        asm volatile("" : "+v"(v[k]));  // keep the values in registers across the chain
    }
    for (int L = l0; L < nl; L++) {
        float s = run;
#pragma unroll
        for (int k = 0; k < 64; k++) s = s + v[k];
        run = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), L));
    }
    return run;
}

// The plain chain over terms from .. n-1 (n <= 4096) in 32-term segments:
// in each round of 2048 terms lane q holds terms 32q .. 32q+31 of the round
// (slots outside [from, n) hold -0.0, the identity of +).  Half the
// registers of sumsq_chain, for the walk's rare fallback.
__device__ inline float sumsq_chain32(const float* prod, int from, int n, float run) {
    const int lane = threadIdx.x & 63;
    for (int r0 = from & ~2047; r0 < n; r0 += 2048) {
        const int g0 = r0 + 32 * lane, L = g0 >> 6, hf = (g0 >> 5) & 1;
        float v[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 t = reinterpret_cast<const float4*>(prod + 256 * (8 * hf + i))[L & 63];
            const float tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int e = g0 + 4 * i + c;
                v[4 * i + c] = (e >= from && e < n) ? tv[c] : -0.0f;
                asm volatile("" : "+v"(v[4 * i + c]));  // keep the values in registers across the chain
            }
        }
        const int q0 = max(from - r0, 0) >> 5, q1 = min((n - r0 + 31) >> 5, 64);
        for (int q = q0; q < q1; q++) {
            float s = run;
#pragma unroll
            for (int k = 0; k < 32; k++) s = s + v[k];
            run = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), q));
        }
    }
    return run;
}

__device__ __forceinline__ void sumsq_load_pass0(const float* prod, float (&r)[64]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float4 q = reinterpret_cast<const float4*>(prod + 256 * i)[lane];
        r[4 * i] = q.x, r[4 * i + 1] = q.y, r[4 * i + 2] = q.z, r[4 * i + 3] = q.w;
    }
}

// Step 1, helper h (0..2), a wave on a SIMD other than wave 0's: for every
// binade of the window, the prefix sums of rn(p / u) over its 512 terms
// (terms H + 8q .. H + 8q + 7 for lane quarter q = 64h + lane) and its tie
// bits.  Helper 0 also publishes the window.
__device__ inline void sumsq_walk_helper(int h, const float* prod, int n, int H, SumsqWalk& w) {
    const int lane = threadIdx.x & 63;
    const int NQ = (n - H) >> 3;
    const int q = 64 * h + lane, qc = min(q, NQ - 1);
    const int g = H + 8 * qc, kk = g & 63, Lc = g >> 6;
    const float4 A = reinterpret_cast<const float4*>(prod + 256 * (kk >> 2))[Lc];
    const float4 B = reinterpret_cast<const float4*>(prod + 256 * ((kk >> 2) + 1))[Lc];
    const float pp = lane < 32 ? w.part[lane >> 4][lane & 15] : 0.0f;
    const float ah = wave_total_f32(lane < 16 ? pp : 0.0f), a = wave_total_f32(lane >= 16 ? pp : 0.0f);
    // window: from the head's binade to the total's, widened by one binade
    // only where an estimate is that close to a power of two (both estimates
    // are within n * 2^-24 relative of the exact sums, the serial chain too)
    const float lo = ah * (1.0f - 1.0f / 4096.0f), hi = a * (1.0f + 1.0f / 1024.0f);
    int elo = 0, nb = 0, fb = 0;
    const int flo = (int)(__float_as_uint(lo) >> 23) & 255, fhi = (int)(__float_as_uint(hi) >> 23) & 255;
    if (!(a < __builtin_inff()) || !(lo > 0.0f) || flo < 30) {
        fb = 1;  // non-finite, zero or tiny sums: the plain chain
    } else {
        elo = flo - 127;
        nb = min(fhi - flo + 1, kWalkBinades);
    }
    if (h == 0 && lane == 0) {
        w.elo = elo;
        w.nb = nb;
        w.fb = fb;
    }
    if (fb) return;
    const float pj[8] = {A.x, A.y, A.z, A.w, B.x, B.y, B.z, B.w};
    uint32_t rr[8];
    int tzm[8];
    const int efb0 = elo + 127;  // exponent field of the lowest binade
#pragma unroll
    for (int j = 0; j < 8; j++) {
        // p = mp * 2^(ep' - 150) with ep' = max(field, 1); in the lowest binade
        // p / u = mp >> d, d = efb0 - ep'; rr = floor(2 p / u), exact below
        // 2^28 (a term of 2^23 units or more is a crossing in every binade of
        // the window, so past that rr is capped)
        const uint32_t pb = __float_as_uint(pj[j]);
        const int ep = (int)(pb >> 23);
        const uint32_t mp = (pb & 0x7FFFFFu) | (ep ? 0x800000u : 0u);
        const int dm1 = efb0 - 1 - max(ep, 1);
        rr[j] = dm1 >= 0 ? mp >> min(dm1, 31) : min(mp << min(-dm1, 5), 1u << 28);
        // a tie in binade b: the half bit, bit (dm1 + b) of mp, is its lowest set bit
        const int tz = (int)__builtin_ctz(mp | 0x80000000u);
        tzm[j] = tz <= 23 ? tz - dm1 : -1000;
    }
#pragma unroll
    for (int b = 0; b < kWalkBinades; b++) {
        if (b < nb) {
            uint32_t acc = 0, tm = 0, loc[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (b > 0) rr[j] >>= 1;  // floor(2 p / 2u) = floor(floor(2 p / u) / 2)
                const bool tie = tzm[j] == b;
                acc += (rr[j] + (tie ? 0u : 1u)) >> 1;  // rn(p / u), a tie taken down (the walk stops there)
                loc[j] = acc;
                tm |= tie ? 1u << j : 0u;
            }
            const uint32_t tot = q < NQ ? min(acc, kWalkCap) : 0u;
            const uint32_t incl = wave_scan_u32(tot);
            const uint32_t ex = incl - tot;
            if (q < NQ) {
                uint4* dst = reinterpret_cast<uint4*>(&w.Q[b][8 * q]);
                dst[0] = make_uint4(ex + loc[0], ex + loc[1], ex + loc[2], ex + loc[3]);
                dst[1] = make_uint4(ex + loc[4], ex + loc[5], ex + loc[6], ex + loc[7]);
                reinterpret_cast<uint8_t*>(&w.TM[b][0])[q] = (uint8_t)tm;
            }
            if (lane == 63) w.WT[b][h] = min(incl, kWalkCap);
        }
    }
}

// Step 2, wave 0 after the barrier: the walk from the head's sum s to the sum
// of all n terms (every lane returns it).
__device__ inline float sumsq_walk(float s, const float* prod, int n, int H, const SumsqWalk& w) {
    const int lane = threadIdx.x & 63;
    const int M = n - H, NS = M >> 5;
    const int elo = w.elo, nb = w.nb;
    bool fb = w.fb != 0;
    int k = 0, stops = 0;  // terms H .. H+k-1 are summed into s
    uint32_t sb = rdf(__float_as_uint(s));
    int bi = (int)(sb >> 23) - 127 - elo;
    // per binade: the exact prefix at each segment end (helper offsets added), the tie words
    uint32_t base = 0, v1 = 0, tw = 0, o1 = 0, o2 = 0;
    const int pl = 256 * ((lane & 31) >> 2) + (lane & 3);                                // pass-layout part of term 32 seg + lane
    auto load_bin = [&](int b, uint32_t& v1o, uint32_t& two, uint32_t& a1, uint32_t& a2) {
        a1 = rdf(w.WT[b][0]);
        a2 = a1 + rdf(w.WT[b][1]);
        const uint32_t st = lane < NS ? w.Q[b][32 * lane + 31] : 0u;
        v1o = lane < NS ? st + (lane >= 32 ? a2 : lane >= 16 ? a1 : 0u) : 0u;
        two = lane < NS ? w.TM[b][lane] : 0u;
    };
    if (!fb) {
        if (bi < 0 || bi >= nb || (sb >> 23) < 30)
            fb = true;
        else
            load_bin(bi, v1, tw, o1, o2);
    }
    while (!fb && k < M) {
        if (stops >= kWalkMaxStops) {
            fb = true;
            break;
        }
        const int ef = (int)(sb >> 23);
        const uint32_t m = (sb & 0x7FFFFFu) | 0x800000u;  // s / u
        const uint32_t T = (1u << 24) - m + base;         // term i crosses when prefix(i) >= T
        const float u = __uint_as_float((uint32_t)(ef - 23) << 23);
        // tie words from term k on; segments that end before k have prefix <= base < T
        const int sh = min(max(k - 32 * lane, 0), 32);
        const uint32_t twm = tw & (uint32_t)(~0ull << sh);
        const uint64_t b1 = __builtin_amdgcn_ballot_w64(v1 >= T);
        const uint64_t bt = __builtin_amdgcn_ballot_w64(twm != 0u);
        const uint32_t seg = rdf(min(b1 ? (uint32_t)__builtin_ctzll(b1) : 64u, bt ? (uint32_t)__builtin_ctzll(bt) : 64u));
        if (seg >= 64) {  // no event: the rest is exact integer arithmetic
            sb = rdf(__float_as_uint(__uint_as_float(sb) + u * (float)(rdl(v1, NS - 1) - base)));
            k = M;
            break;
        }
        // one LDS round trip: the event segment's prefixes (this binade and the
        // next) and terms, and the next binade's segment ends and tie words
        const int bn = min(bi + 1, kWalkBinades - 1);  // (a clamped bn is never used: bi + 1 >= nb then)
        const uint32_t qv = w.Q[lane < 32 ? bi : bn][32 * seg + (lane & 31)];  // lanes 32..63: the next binade
        const float pv = prod[pl + 2048 * (seg & 1) + 4 * (H / 64 + (seg >> 1))];
        uint32_t v1n, twn, n1, n2;
        load_bin(bn, v1n, twn, n1, n2);
        const uint32_t wt = rdl(twm, seg);
        const int hs = seg >> 4;  // helper wave of the segment
        const uint32_t qt = qv + (lane < 32 ? (hs == 2 ? o2 : hs == 1 ? o1 : 0u) : (hs == 2 ? n2 : hs == 1 ? n1 : 0u));
        const int kr = k - 32 * (int)seg;
        const uint64_t b2 =
            __builtin_amdgcn_ballot_w64(lane < 32 && lane >= kr && (qt >= T || ((wt >> (lane & 31)) & 1u)));
        if (b2 == 0) {  // the segment holds the event by construction; if not, the chain (s, k unchanged here)
            fb = true;
            break;
        }
        const int el = (int)rdf((uint32_t)__builtin_ctzll(b2));
        const int ev = 32 * (int)seg + el;
        const uint32_t qa = rdl(qt, max(el - 1, 0)), qb = rdl(v1, max((int)seg - 1, 0));
        const uint32_t qprev = el > 0 ? qa : (seg > 0 ? qb : 0u);  // prefix of terms before the event
        const float pe = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), el));
        // s + u * (qprev - base) is exact (no crossing before the event); then the event's add
        const float snew = (__uint_as_float(sb) + u * (float)(qprev - base)) + pe;
        sb = rdf(__float_as_uint(snew));
        k = (int)rdf((uint32_t)(ev + 1));
        stops++;
        const int bi2 = (int)rdf((sb >> 23) - 127 - elo);
        if (bi2 == bi) {
            base = rdf(rdl(qt, el));
        } else if (bi2 == bi + 1 && bi2 < nb) {
            base = rdf(rdl(qt, 32 + el));
            v1 = v1n;
            tw = twn;
            o1 = n1;
            o2 = n2;
        } else if (bi2 > bi && bi2 < nb && (sb >> 23) < 255) {
            load_bin(bi2, v1, tw, o1, o2);
            const int hv = ev >> 9;
            base = rdf(w.Q[bi2][ev]) + (hv == 2 ? o2 : hv == 1 ? o1 : 0u);
        } else {
            fb = true;
        }
        bi = bi2;
    }
    s = __uint_as_float(sb);
    if (fb) {
        s = sumsq_chain32(prod, H + k, n, s);  // the plain chain from term H + k on
    }
    return s;
}

}  // namespace vtq
