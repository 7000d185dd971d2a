/*
 * vtq_synth.c -- seeded synthetic inputs for the benchmark configurations.
 * Stream and draw order are specified in vtq_synth.h.  The block encoders are
 * the inverses of the decoders of src/ops/quant.rs (get_scale_min_k4 :267-276,
 * Q6_K ql/qh split :352-383, Q5_0 qh bits :176-183, Q4_0 (2k, 2k+1) :102-108).
 */
#include "vtq_synth.h"

#include <math.h>
#include <string.h>

static inline uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint32_t uni(uint64_t *s, uint32_t range) { return (uint32_t)((splitmix64(s) >> 32) % range); }

static inline float normal(uint64_t *s, float sigma) {
    double u1 = ((double)(splitmix64(s) >> 11) + 1.0) * 0x1p-53; /* (0, 1] */
    double u2 = (double)(splitmix64(s) >> 11) * 0x1p-53;        /* [0, 1) */
    double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
    return (float)(z * (double)sigma);
}

uint16_t vtqs_f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    x &= 0x7FFFFFFFu;
    if (x >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (x > 0x7F800000u ? 0x200u : 0u));
    if (x >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to Inf */
    if (x < 0x38800000u) {                                    /* below 2^-14: subnormal half */
        float a;
        memcpy(&a, &x, 4);
        double m = nearbyint((double)a * 0x1p24); /* exact scale, RNE to integer */
        return (uint16_t)(sign | (uint16_t)m);
    }
    uint32_t h = (x >> 13) - (112u << 10);
    uint32_t rem = x & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static inline void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xFF);
    p[1] = (uint8_t)(v >> 8);
}

static inline uint16_t scale_f16(uint64_t *s, float sigma) { return vtqs_f32_to_f16_rne(fabsf(normal(s, sigma))); }

void vtqs_normal_f32(uint64_t seed, float *out, size_t n, float sigma) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i++) out[i] = normal(&s, sigma);
}

void vtqs_bytes(uint64_t seed, uint8_t *w, size_t n) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i++) w[i] = (uint8_t)(splitmix64(&s) >> 56);
}

void vtqs_q4_k(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma) {
    uint64_t s = seed;
    size_t nb = rows * (in_feat / 256);
    for (size_t b = 0; b < nb; b++) {
        uint8_t *blk = w + b * 144;
        put16(blk, scale_f16(&s, sigma));
        put16(blk + 2, scale_f16(&s, sigma));
        uint8_t sc[8], m[8];
        for (int j = 0; j < 8; j++) sc[j] = (uint8_t)uni(&s, 64);
        for (int j = 0; j < 8; j++) m[j] = (uint8_t)uni(&s, 64);
        uint8_t *k = blk + 4;
        for (int j = 0; j < 4; j++) {
            k[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            k[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
            k[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t *qs = blk + 16;
        memset(qs, 0, 128);
        for (int e = 0; e < 256; e++) {
            uint8_t q = (uint8_t)uni(&s, 16);
            int h = e / 64, l = e % 64;
            if (l < 32) qs[32 * h + l] |= q;
            else qs[32 * h + l - 32] |= (uint8_t)(q << 4);
        }
    }
}

void vtqs_q6_k(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma) {
    uint64_t s = seed;
    size_t nb = rows * (in_feat / 256);
    for (size_t b = 0; b < nb; b++) {
        uint8_t *blk = w + b * 210;
        uint16_t d = scale_f16(&s, sigma);
        for (int j = 0; j < 16; j++) blk[192 + j] = (uint8_t)(int8_t)((int)uni(&s, 128) - 64);
        memset(blk, 0, 192);
        for (int e = 0; e < 256; e++) {
            uint8_t q = (uint8_t)uni(&s, 64);
            int hf = e / 128, r = e % 128, k = r / 32, l = r % 32;
            uint8_t *ql = blk + 64 * hf, *qh = blk + 128 + 32 * hf;
            /* k = 0: ql[l] low, 1: ql[l+32] low, 2: ql[l] high, 3: ql[l+32] high */
            int qi = l + ((k & 1) ? 32 : 0);
            ql[qi] |= (uint8_t)((k & 2) ? (q & 15) << 4 : (q & 15));
            qh[l] |= (uint8_t)((q >> 4) << (2 * k));
        }
        put16(blk + 208, d);
    }
}

void vtqs_q8_0(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma) {
    uint64_t s = seed;
    size_t nb = rows * (in_feat / 32);
    for (size_t b = 0; b < nb; b++) {
        uint8_t *blk = w + b * 34;
        put16(blk, scale_f16(&s, sigma));
        for (int k = 0; k < 32; k++) blk[2 + k] = (uint8_t)(int8_t)((int)uni(&s, 255) - 127);
    }
}

void vtqs_q5_0(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma) {
    uint64_t s = seed;
    size_t nb = rows * (in_feat / 32);
    for (size_t b = 0; b < nb; b++) {
        uint8_t *blk = w + b * 22;
        put16(blk, scale_f16(&s, sigma));
        uint32_t qh = 0;
        uint8_t *qs = blk + 6;
        memset(qs, 0, 16);
        for (int e = 0; e < 32; e++) {
            uint32_t q = uni(&s, 32);
            int j = e % 16;
            if (e < 16) {
                qs[j] |= (uint8_t)(q & 15);
                qh |= ((q >> 4) & 1u) << j;
            } else {
                qs[j] |= (uint8_t)((q & 15) << 4);
                qh |= ((q >> 4) & 1u) << (j + 16);
            }
        }
        blk[2] = (uint8_t)qh;
        blk[3] = (uint8_t)(qh >> 8);
        blk[4] = (uint8_t)(qh >> 16);
        blk[5] = (uint8_t)(qh >> 24);
    }
}

void vtqs_q4_0(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma) {
    uint64_t s = seed;
    size_t nb = rows * (in_feat / 32);
    for (size_t b = 0; b < nb; b++) {
        uint8_t *blk = w + b * 18;
        put16(blk, scale_f16(&s, sigma));
        memset(blk + 2, 0, 16);
        for (int e = 0; e < 32; e++) {
            uint8_t q = (uint8_t)uni(&s, 16);
            blk[2 + e / 2] |= (uint8_t)((e & 1) ? q << 4 : q);
        }
    }
}
