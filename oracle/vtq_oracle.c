/*
 * vtq_oracle.c -- CPU restatement of vitni-tensor's quantized linear path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT: the checker for libvtq (see vtq_oracle.h).
 * Each function cites the reference function it restates (path:line relative
 * to the vitni-tensor 0.2.1 source root).  The code follows the reference's
 * evaluation order operation by operation; it is written in C from the
 * published algorithm, not translated mechanically.
 */
#include "vtq_oracle.h"

#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#define Q4_0_BYTES 18
#define Q5_0_BYTES 22
#define Q8_0_BYTES 34
#define QK 32
#define Q4_K_BYTES 144
#define Q6_K_BYTES 210
#define QK_K 256

#define FAIL(code, text)      \
    do {                      \
        if (msg) *msg = text; \
        return code;          \
    } while (0)

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* Rust `f as i32`: truncation toward zero, saturating, NaN -> 0. */
static inline int32_t rust_as_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

static inline int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* ---------------------------------------------------------------- f16 */

/* src/ops/quant.rs:40-66 */
float vtqo_f16_to_f32(uint16_t half) {
    uint32_t sign = (half >> 15) & 1u;
    uint32_t exp = (half >> 10) & 0x1Fu;
    uint32_t mant = half & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            uint32_t m = mant;
            int32_t e = 1;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                e -= 1;
            }
            m &= 0x3FFu;
            bits = (sign << 31) | ((uint32_t)(127 - 15 + e) << 23) | (m << 13);
        }
    } else if (exp == 0x1F) {
        bits = (sign << 31) | 0x7F800000u | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    return bits_f32(bits);
}

uint32_t vtqo_f16_to_f32_bits(uint16_t half) { return f32_bits(vtqo_f16_to_f32(half)); }

/* src/ops/quant.rs:68-83 */
uint16_t vtqo_f32_to_f16(float f) {
    uint32_t bits = f32_bits(f);
    uint16_t sign = (uint16_t)((bits >> 31) & 1u);
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu) - 127 + 15;
    uint32_t mant = (bits >> 13) & 0x3FFu;
    if (exp <= 0) return (uint16_t)(sign << 15);
    if (exp >= 0x1F) return (uint16_t)((sign << 15) | 0x7C00u);
    return (uint16_t)((sign << 15) | ((uint32_t)exp << 10) | mant);
}

/* ------------------------------------------------------ pinned reductions */

/* src/ops/quant.rs:461-476: halve the slice in place until one value is left;
 * pair (2t, 2t+1), an odd last element passes through unchanged. */
float vtqo_fixed_tree(float *part, size_t n) {
    size_t len = n;
    if (len == 0) return 0.0f;
    while (len > 1) {
        size_t half = (len + 1) / 2;
        for (size_t t = 0; t < half; t++) {
            size_t u = 2 * t;
            part[t] = (u + 1 < len) ? part[u] + part[u + 1] : part[u];
        }
        len = half;
    }
    return part[0];
}

/* src/ops/quant.rs:482-505: 8 lane chains from +0.0, element i -> lane i%8,
 * products rounded before the add, then the fixed tree over the 8 lanes. */
float vtqo_canonical_chunk(const float *x, const float *w, size_t n) {
    float lanes[VTQO_CANON_LANES] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    size_t full = n - (n % VTQO_CANON_LANES);
    size_t i = 0;
    while (i < full) {
        for (size_t j = 0; j < VTQO_CANON_LANES; j++) {
            float p = x[i + j] * w[i + j];
            lanes[j] = lanes[j] + p;
        }
        i += VTQO_CANON_LANES;
    }
    while (i < n) {
        size_t j = i % VTQO_CANON_LANES;
        float p = x[i] * w[i];
        lanes[j] = lanes[j] + p;
        i++;
    }
    return vtqo_fixed_tree(lanes, VTQO_CANON_LANES);
}

/* src/ops/quant.rs:551-566 */
float vtqo_canonical_dot(const float *x, const float *w, size_t n) {
    if (n == 0) return 0.0f;
    if (n <= VTQO_CANON_CHUNK) return vtqo_canonical_chunk(x, w, n);
    size_t nchunks = (n + VTQO_CANON_CHUNK - 1) / VTQO_CANON_CHUNK;
    float *sums = (float *)malloc(nchunks * sizeof(float));
    for (size_t c = 0; c < nchunks; c++) {
        size_t s = c * VTQO_CANON_CHUNK;
        size_t e = s + VTQO_CANON_CHUNK < n ? s + VTQO_CANON_CHUNK : n;
        sums[c] = vtqo_canonical_chunk(x + s, w + s, e - s);
    }
    float r = vtqo_fixed_tree(sums, nchunks);
    free(sums);
    return r;
}

/* src/ops/quant.rs:572-574 */
float vtqo_canonical_combine(float *chunk_sums, size_t n) { return vtqo_fixed_tree(chunk_sums, n); }

/* src/ops/quant.rs:579-608 */
float vtqo_canonical_dot_regime2(const float *x, const float *w, size_t n) {
    if (n == 0) return 0.0f;
    size_t nb = (n + 7) / 8;
    float *part = (float *)malloc(nb * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        size_t s = b * 8, e = s + 8 < n ? s + 8 : n;
        float acc = 0.0f;
        for (size_t i = s; i < e; i++) {
            float p = x[i] * w[i];
            acc = acc + p;
        }
        part[b] = acc;
    }
    float r = vtqo_fixed_tree(part, nb);
    free(part);
    return r;
}

/* ----------------------------------------------------------- decoders */

/* src/ops/quant.rs:91-111: reference order, element 2k = low nibble, 2k+1 = high. */
int vtqo_dequantize_q4_0(const uint8_t *w, size_t len, float *out, const char **msg) {
    if (len % Q4_0_BYTES != 0) FAIL(VTQO_E_INTERNAL, "Q4_0 byte length not a multiple of 18");
    size_t nb = len / Q4_0_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * Q4_0_BYTES;
        float scale = vtqo_f16_to_f32(rd16(blk));
        float *o = out + b * QK;
        for (int k = 0; k < 16; k++) {
            uint8_t byte = blk[2 + k];
            int32_t lo = (int32_t)(byte & 0x0F) - 8;
            int32_t hi = (int32_t)(byte >> 4) - 8;
            o[2 * k] = scale * (float)lo;
            o[2 * k + 1] = scale * (float)hi;
        }
    }
    return VTQO_OK;
}

/* src/ops/quant.rs:160-186: element j and j+16 share qs byte j (GGML order). */
int vtqo_dequantize_q5_0(const uint8_t *w, size_t len, float *out, const char **msg) {
    if (len % Q5_0_BYTES != 0) FAIL(VTQO_E_INTERNAL, "Q5_0 byte length not a multiple of 22");
    size_t nb = len / Q5_0_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * Q5_0_BYTES;
        float scale = vtqo_f16_to_f32(rd16(blk));
        uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                      ((uint32_t)blk[5] << 24);
        const uint8_t *qs = blk + 6;
        float *o = out + b * QK;
        for (int j = 0; j < 16; j++) {
            uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10u);
            uint8_t xh1 = (uint8_t)((qh >> (j + 12)) & 0x10u);
            int32_t x0 = (int32_t)((qs[j] & 0x0F) | xh0) - 16;
            int32_t x1 = (int32_t)((qs[j] >> 4) | xh1) - 16;
            o[j] = scale * (float)x0;
            o[j + 16] = scale * (float)x1;
        }
    }
    return VTQO_OK;
}

/* src/ops/quant.rs:193-210 */
int vtqo_dequantize_q8_0(const uint8_t *w, size_t len, float *out, const char **msg) {
    if (len % Q8_0_BYTES != 0) FAIL(VTQO_E_INTERNAL, "Q8_0 byte length not a multiple of 34");
    size_t nb = len / Q8_0_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * Q8_0_BYTES;
        float scale = vtqo_f16_to_f32(rd16(blk));
        for (int k = 0; k < 32; k++) out[b * QK + k] = scale * (float)(int8_t)blk[2 + k];
    }
    return VTQO_OK;
}

/* src/ops/quant.rs:267-276 */
static inline void get_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 0x3F;
        *m = s[j + 4] & 0x3F;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* src/ops/quant.rs:280-319 */
int vtqo_dequantize_q4_k(const uint8_t *w, size_t len, float *out, const char **msg) {
    if (len % Q4_K_BYTES != 0) FAIL(VTQO_E_INTERNAL, "Q4_K byte length not a multiple of 144");
    size_t nb = len / Q4_K_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * Q4_K_BYTES;
        float d = vtqo_f16_to_f32(rd16(blk));
        float dmin = vtqo_f16_to_f32(rd16(blk + 2));
        const uint8_t *scales = blk + 4;
        const uint8_t *qs = blk + 16;
        float *o = out + b * QK_K;
        for (int h = 0; h < 4; h++) {
            uint8_t sc1, m1, sc2, m2;
            get_scale_min_k4(2 * h, scales, &sc1, &m1);
            get_scale_min_k4(2 * h + 1, scales, &sc2, &m2);
            float d1 = d * (float)sc1, m1f = dmin * (float)m1;
            float d2 = d * (float)sc2, m2f = dmin * (float)m2;
            for (int l = 0; l < 32; l++) o[64 * h + l] = d1 * (float)(qs[32 * h + l] & 0x0F) - m1f;
            for (int l = 0; l < 32; l++) o[64 * h + 32 + l] = d2 * (float)(qs[32 * h + l] >> 4) - m2f;
        }
    }
    return VTQO_OK;
}

/* Decode one Q6_K block's element e into its signed 6-bit code and its scale
 * index, following the ql/qh/scale indexing of src/ops/quant.rs:352-383. */
static void q6k_block_decode(const uint8_t *blk, float d, float *o) {
    for (int hf = 0; hf < 2; hf++) {
        const uint8_t *ql = blk + 64 * hf;
        const uint8_t *qh = blk + 128 + 32 * hf;
        const uint8_t *sc = blk + 192 + 8 * hf;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            uint8_t h = qh[l];
            float q1 = (float)((int32_t)((ql[l] & 0x0F) | ((h & 3) << 4)) - 32);
            float q2 = (float)((int32_t)((ql[l + 32] & 0x0F) | (((h >> 2) & 3) << 4)) - 32);
            float q3 = (float)((int32_t)((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32);
            float q4 = (float)((int32_t)((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32);
            float s1 = (float)(int8_t)sc[is + 0];
            float s2 = (float)(int8_t)sc[is + 2];
            float s3 = (float)(int8_t)sc[is + 4];
            float s4 = (float)(int8_t)sc[is + 6];
            o[128 * hf + l] = d * s1 * q1;
            o[128 * hf + l + 32] = d * s2 * q2;
            o[128 * hf + l + 64] = d * s3 * q3;
            o[128 * hf + l + 96] = d * s4 * q4;
        }
    }
}

/* src/ops/quant.rs:337-386 */
int vtqo_dequantize_q6_k(const uint8_t *w, size_t len, float *out, const char **msg) {
    if (len % Q6_K_BYTES != 0) FAIL(VTQO_E_INTERNAL, "Q6_K byte length not a multiple of 210");
    size_t nb = len / Q6_K_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * Q6_K_BYTES;
        q6k_block_decode(blk, vtqo_f16_to_f32(rd16(blk + 208)), out + b * QK_K);
    }
    return VTQO_OK;
}

/* src/ops/quant.rs:115-150 */
int vtqo_quantize_q4_0(const float *x, size_t n, uint8_t *out, const char **msg) {
    if (n % QK != 0) FAIL(VTQO_E_INTERNAL, "Q4_0 quantize: input not a multiple of 32");
    for (size_t b = 0; b < n / QK; b++) {
        const float *blk = x + b * QK;
        float amax = 0.0f, max_val = 0.0f;
        for (int i = 0; i < QK; i++) {
            float a = blk[i] < 0.0f ? -blk[i] : blk[i];
            if (a > amax) {
                amax = a;
                max_val = blk[i];
            }
        }
        float scale = max_val / -8.0f;
        float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        uint16_t h = vtqo_f32_to_f16(scale);
        uint8_t *o = out + b * Q4_0_BYTES;
        o[0] = (uint8_t)(h & 0xFF);
        o[1] = (uint8_t)(h >> 8);
        for (int k = 0; k < 16; k++) {
            float x0 = blk[2 * k] * inv + 8.5f;
            float x1 = blk[2 * k + 1] * inv + 8.5f;
            uint8_t q0 = (uint8_t)clamp_i32(rust_as_i32(x0), 0, 15);
            uint8_t q1 = (uint8_t)clamp_i32(rust_as_i32(x1), 0, 15);
            o[2 + k] = (uint8_t)(q0 | (q1 << 4));
        }
    }
    return VTQO_OK;
}

/* src/ops/quant.rs:213-241 */
int vtqo_quantize_q8_0(const float *x, size_t n, uint8_t *out, const char **msg) {
    if (n % QK != 0) FAIL(VTQO_E_INTERNAL, "Q8_0 quantize: input not a multiple of 32");
    for (size_t b = 0; b < n / QK; b++) {
        const float *blk = x + b * QK;
        float amax = 0.0f;
        for (int i = 0; i < QK; i++) {
            float a = blk[i] < 0.0f ? -blk[i] : blk[i];
            if (a > amax) amax = a;
        }
        float scale = amax / 127.0f;
        float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        uint16_t h = vtqo_f32_to_f16(scale);
        uint8_t *o = out + b * Q8_0_BYTES;
        o[0] = (uint8_t)(h & 0xFF);
        o[1] = (uint8_t)(h >> 8);
        for (int k = 0; k < QK; k++) {
            float scaled = blk[k] * inv;
            float bias = scaled >= 0.0f ? 0.5f : -0.5f;
            o[2 + k] = (uint8_t)(int8_t)clamp_i32(rust_as_i32(scaled + bias), -127, 127);
        }
    }
    return VTQO_OK;
}

/* ------------------------------------------------- integer k-quant path */

/* src/ops/quant.rs:750-771 */
void vtqo_quantize_block_q8(const float *x, size_t n, vtqo_q8block *out) {
    float amax = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        float a = v < 0.0f ? -v : v;
        if (a > amax) amax = a;
    }
    float d = amax / 127.0f;
    float inv = d != 0.0f ? 1.0f / d : 0.0f;
    memset(out->qs, 0, sizeof out->qs);
    memset(out->bsums, 0, sizeof out->bsums);
    for (size_t i = 0; i < n; i++) {
        float scaled = x[i] * inv;
        float bias = scaled >= 0.0f ? 0.5f : -0.5f;
        int32_t q = clamp_i32(rust_as_i32(scaled + bias), -127, 127);
        out->qs[i] = (int8_t)q;
        out->bsums[i / 32] += q;
    }
    out->d = d;
}

/* src/ops/quant.rs:775-784 */
static inline void dot32_pair(const uint8_t *qsl, const int8_t *xlo, const int8_t *xhi,
                              int32_t *s_lo, int32_t *s_hi) {
    int32_t a = 0, b = 0;
    for (int l = 0; l < 32; l++) {
        a += (int32_t)(qsl[l] & 0x0F) * (int32_t)xlo[l];
        b += (int32_t)(qsl[l] >> 4) * (int32_t)xhi[l];
    }
    *s_lo = a;
    *s_hi = b;
}

/* src/ops/quant.rs:849-898: exact integer sums, then
 * part = (d*dx)*f32(acc) - (dmin*dx)*f32(acc_m). */
float vtqo_dot_q4k_q8_block(const uint8_t *w, const vtqo_q8block *xq, size_t n) {
    float d = vtqo_f16_to_f32(rd16(w));
    float dmin = vtqo_f16_to_f32(rd16(w + 2));
    const uint8_t *scales = w + 4;
    const uint8_t *qs = w + 16;
    int32_t acc = 0, acc_m = 0;
    for (int h = 0; h < 4; h++) {
        uint8_t sc_lo, m_lo, sc_hi, m_hi;
        get_scale_min_k4(2 * h, scales, &sc_lo, &m_lo);
        get_scale_min_k4(2 * h + 1, scales, &sc_hi, &m_hi);
        size_t q_off = 32 * (size_t)h, base = 64 * (size_t)h;
        int32_t s_lo = 0, s_hi = 0;
        if (base + 64 <= n) {
            dot32_pair(qs + q_off, xq->qs + base, xq->qs + base + 32, &s_lo, &s_hi);
        } else {
            for (size_t l = 0; l < 32; l++) {
                if (base + l < n) s_lo += (int32_t)(qs[q_off + l] & 0x0F) * (int32_t)xq->qs[base + l];
                if (base + 32 + l < n)
                    s_hi += (int32_t)(qs[q_off + l] >> 4) * (int32_t)xq->qs[base + 32 + l];
            }
        }
        acc += (int32_t)sc_lo * s_lo + (int32_t)sc_hi * s_hi;
        acc_m += (int32_t)m_lo * xq->bsums[2 * h] + (int32_t)m_hi * xq->bsums[2 * h + 1];
    }
    return d * xq->d * (float)acc - dmin * xq->d * (float)acc_m;
}

/* src/ops/quant.rs:995-1057: 16 scale buckets, bucket 8*hf + l/16 + 2k for
 * quant k of position l; part = (d*dx)*f32(sum_j sc_j * sums_j). */
float vtqo_dot_q6k_q8_block(const uint8_t *w, const vtqo_q8block *xq, size_t n) {
    float d = vtqo_f16_to_f32(rd16(w + 208));
    const uint8_t *ql = w, *qh = w + 128, *sc = w + 192;
    int32_t sums[16] = {0};
    for (int hf = 0; hf < 2; hf++) {
        size_t ql_p = 64 * (size_t)hf, qh_p = 32 * (size_t)hf, sc_p = 8 * (size_t)hf;
        size_t y = 128 * (size_t)hf;
        for (int is = 0; is < 2; is++) {
            size_t l0 = 16 * (size_t)is;
            for (size_t l = l0; l < l0 + 16; l++) {
                uint8_t h = qh[qh_p + l], b0 = ql[ql_p + l], b1 = ql[ql_p + l + 32];
                int32_t q1 = (int32_t)((b0 & 0x0F) | ((h & 3) << 4)) - 32;
                int32_t q2 = (int32_t)((b1 & 0x0F) | (((h >> 2) & 3) << 4)) - 32;
                int32_t q3 = (int32_t)((b0 >> 4) | (((h >> 4) & 3) << 4)) - 32;
                int32_t q4 = (int32_t)((b1 >> 4) | (((h >> 6) & 3) << 4)) - 32;
                if (y + l < n) sums[sc_p + is] += q1 * (int32_t)xq->qs[y + l];
                if (y + l + 32 < n) sums[sc_p + is + 2] += q2 * (int32_t)xq->qs[y + l + 32];
                if (y + l + 64 < n) sums[sc_p + is + 4] += q3 * (int32_t)xq->qs[y + l + 64];
                if (y + l + 96 < n) sums[sc_p + is + 6] += q4 * (int32_t)xq->qs[y + l + 96];
            }
        }
    }
    int32_t acc = 0;
    for (int j = 0; j < 16; j++) acc += (int32_t)(int8_t)sc[j] * sums[j];
    return d * xq->d * (float)acc;
}

/* src/ops/quant.rs:904-928 */
int vtqo_integer_dot_q4k(const float *x, const uint8_t *w, size_t w_len, size_t n, float *out,
                         const char **msg) {
    if (w_len % Q4_K_BYTES != 0) FAIL(VTQO_E_INTERNAL, "Q4_K byte length not a multiple of 144");
    if (n == 0) {
        *out = 0.0f;
        return VTQO_OK;
    }
    size_t n_super = w_len / Q4_K_BYTES;
    float *parts = (float *)malloc((n_super ? n_super : 1) * sizeof(float));
    size_t np = 0;
    vtqo_q8block xq;
    for (size_t b = 0; b < n_super; b++) {
        size_t base = b * QK_K;
        if (base >= n) break;
        size_t avail = n - base < QK_K ? n - base : QK_K;
        vtqo_quantize_block_q8(x + base, avail, &xq);
        parts[np++] = vtqo_dot_q4k_q8_block(w + b * Q4_K_BYTES, &xq, avail);
    }
    *out = vtqo_fixed_tree(parts, np);
    free(parts);
    return VTQO_OK;
}

/* ------------------------------------------------- float-fused k-quants */

/* src/ops/quant.rs:616-702 */
int vtqo_canonical_dot_q4k_fused(const float *x, const uint8_t *w, size_t w_len, size_t n,
                                 float *out, const char **msg) {
    if (w_len % Q4_K_BYTES != 0) FAIL(VTQO_E_INTERNAL, "Q4_K byte length not a multiple of 144");
    if (n == 0) {
        *out = 0.0f;
        return VTQO_OK;
    }
    size_t n_super = w_len / Q4_K_BYTES;
    float lanes[8] = {0};
    float buf[QK_K];
    const size_t per_chunk = VTQO_CANON_CHUNK / QK_K;
    float *chunk_sums = (float *)malloc((n_super / per_chunk + 2) * sizeof(float));
    size_t nc = 0;
    for (size_t b = 0; b < n_super; b++) {
        size_t base = b * QK_K;
        if (base >= n) break;
        const uint8_t *blk = w + b * Q4_K_BYTES;
        float d = vtqo_f16_to_f32(rd16(blk));
        float dmin = vtqo_f16_to_f32(rd16(blk + 2));
        const uint8_t *scales = blk + 4, *qs = blk + 16;
        for (int h = 0; h < 4; h++) {
            uint8_t sc1, m1, sc2, m2;
            get_scale_min_k4(2 * h, scales, &sc1, &m1);
            get_scale_min_k4(2 * h + 1, scales, &sc2, &m2);
            float d1 = d * (float)sc1, m1f = dmin * (float)m1;
            float d2 = d * (float)sc2, m2f = dmin * (float)m2;
            for (int l = 0; l < 32; l++) buf[64 * h + l] = d1 * (float)(qs[32 * h + l] & 0x0F) - m1f;
            for (int l = 0; l < 32; l++) buf[64 * h + 32 + l] = d2 * (float)(qs[32 * h + l] >> 4) - m2f;
        }
        size_t avail = n - base < QK_K ? n - base : QK_K;
        for (size_t t = 0; t < avail; t++) {
            float p = x[base + t] * buf[t];
            lanes[t % 8] = lanes[t % 8] + p;
        }
        int is_last = base + avail >= n;
        if ((b + 1) % per_chunk == 0 || is_last) {
            float l[8];
            memcpy(l, lanes, sizeof l);
            chunk_sums[nc++] = vtqo_fixed_tree(l, 8);
            memset(lanes, 0, sizeof lanes);
        }
    }
    *out = vtqo_fixed_tree(chunk_sums, nc);
    free(chunk_sums);
    return VTQO_OK;
}

/* src/ops/quant.rs:1212-1300 */
int vtqo_canonical_dot_q6k_fused(const float *x, const uint8_t *w, size_t w_len, size_t n,
                                 float *out, const char **msg) {
    if (w_len % Q6_K_BYTES != 0) FAIL(VTQO_E_INTERNAL, "Q6_K byte length not a multiple of 210");
    if (n == 0) {
        *out = 0.0f;
        return VTQO_OK;
    }
    size_t n_super = w_len / Q6_K_BYTES;
    if (n_super * QK_K < n) FAIL(VTQO_E_INTERNAL, "Q6_K row shorter than n");
    const size_t per_chunk = VTQO_CANON_CHUNK / QK_K;
    float *chunk_sums = (float *)malloc((n_super / per_chunk + 2) * sizeof(float));
    size_t nc = 0;
    float lanes[8] = {0};
    float buf[QK_K];
    for (size_t b = 0; b < n_super; b++) {
        size_t base = b * QK_K;
        if (base >= n) break;
        const uint8_t *blk = w + b * Q6_K_BYTES;
        q6k_block_decode(blk, vtqo_f16_to_f32(rd16(blk + 208)), buf);
        size_t avail = n - base < QK_K ? n - base : QK_K;
        for (size_t t = 0; t < avail; t++) {
            float p = x[base + t] * buf[t];
            lanes[t % 8] = lanes[t % 8] + p;
        }
        int is_last = base + avail >= n;
        if ((b + 1) % per_chunk == 0 || is_last) {
            float l[8];
            memcpy(l, lanes, sizeof l);
            chunk_sums[nc++] = vtqo_fixed_tree(l, 8);
            memset(lanes, 0, sizeof lanes);
        }
    }
    *out = vtqo_fixed_tree(chunk_sums, nc);
    free(chunk_sums);
    return VTQO_OK;
}

/* ------------------------------------------------------ row drivers */

typedef enum { ROW_Q4K_INT, ROW_Q6K_INT, ROW_Q4K_FUSED, ROW_Q6K_FUSED } row_kind;

typedef struct {
    row_kind kind;
    const float *x_row;            /* fused kinds */
    const vtqo_q8block *xq;        /* integer kinds */
    const uint8_t *w;
    float *out;                    /* y + b*out_feat */
    size_t row_bytes, n_super, in_feat, out_feat, grain, n_tasks;
    atomic_size_t next;
} row_job;

/* One output row: the per-row body of the serial functions
 * (src/ops/quant.rs:965-977, :1081-1093, :1447-1450, :1321-1324). */
static float row_value(const row_job *j, size_t r, float *parts) {
    const uint8_t *w_row = j->w + r * j->row_bytes;
    float v = 0.0f;
    switch (j->kind) {
    case ROW_Q4K_INT:
        for (size_t s = 0; s < j->n_super; s++)
            parts[s] = vtqo_dot_q4k_q8_block(w_row + s * Q4_K_BYTES, &j->xq[s], QK_K);
        return vtqo_fixed_tree(parts, j->n_super);
    case ROW_Q6K_INT:
        for (size_t s = 0; s < j->n_super; s++)
            parts[s] = vtqo_dot_q6k_q8_block(w_row + s * Q6_K_BYTES, &j->xq[s], QK_K);
        return vtqo_fixed_tree(parts, j->n_super);
    case ROW_Q4K_FUSED:
        /* errors cannot occur: shapes were validated (quant.rs:1423-1425) */
        if (vtqo_canonical_dot_q4k_fused(j->x_row, w_row, j->row_bytes, j->in_feat, &v, NULL)) v = 0.0f;
        return v;
    case ROW_Q6K_FUSED:
        if (vtqo_canonical_dot_q6k_fused(j->x_row, w_row, j->row_bytes, j->in_feat, &v, NULL)) v = 0.0f;
        return v;
    }
    return v;
}

/* Worker of the row-parallel twins: takes grains of `grain` consecutive
 * rows, as rayon's par_chunks_mut(grain) does (src/ops/quant.rs:1129-1143). */
static void *row_worker(void *arg) {
    row_job *j = (row_job *)arg;
    float *parts = (float *)malloc((j->n_super ? j->n_super : 1) * sizeof(float));
    for (;;) {
        size_t t = atomic_fetch_add(&j->next, 1);
        if (t >= j->n_tasks) break;
        size_t base = t * j->grain;
        size_t end = base + j->grain < j->out_feat ? base + j->grain : j->out_feat;
        for (size_t r = base; r < end; r++) j->out[r] = row_value(j, r, parts);
    }
    free(parts);
    return NULL;
}

static void run_rows(row_job *j, int threads) {
    if (threads <= 1) {
        j->grain = j->out_feat ? j->out_feat : 1;
        j->n_tasks = 1;
        atomic_store(&j->next, 0);
        row_worker(j);
        return;
    }
    size_t g = (j->out_feat + (size_t)threads * 4 - 1) / ((size_t)threads * 4);
    j->grain = g > 1 ? g : 1;
    j->n_tasks = (j->out_feat + j->grain - 1) / j->grain;
    atomic_store(&j->next, 0);
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
    int started = 0;
    for (int i = 1; i < threads; i++)
        if (pthread_create(&tid[started], NULL, row_worker, j) == 0) started++;
    row_worker(j);
    for (int i = 0; i < started; i++) pthread_join(tid[i], NULL);
    free(tid);
}

static int linear_kquant(row_kind kind, size_t block_bytes, const char *e_in, const char *e_w,
                         const float *x, const uint8_t *w, size_t w_len, float *y, size_t batch,
                         size_t in_feat, size_t out_feat, int threads, const char **msg) {
    if (in_feat % QK_K != 0) FAIL(VTQO_E_INTERNAL, e_in);
    size_t n_super = in_feat / QK_K;
    size_t row_bytes = n_super * block_bytes;
    if (w_len < out_feat * row_bytes) FAIL(VTQO_E_INTERNAL, e_w);
    int integer = (kind == ROW_Q4K_INT || kind == ROW_Q6K_INT);
    vtqo_q8block *xq = integer ? (vtqo_q8block *)malloc((n_super ? n_super : 1) * sizeof(vtqo_q8block)) : NULL;
    for (size_t b = 0; b < batch; b++) {
        const float *x_row = x + b * in_feat;
        if (integer)
            for (size_t s = 0; s < n_super; s++) vtqo_quantize_block_q8(x_row + s * QK_K, QK_K, &xq[s]);
        row_job j;
        j.kind = kind;
        j.x_row = x_row;
        j.xq = xq;
        j.w = w;
        j.out = y + b * out_feat;
        j.row_bytes = row_bytes;
        j.n_super = n_super;
        j.in_feat = in_feat;
        j.out_feat = out_feat;
        run_rows(&j, threads);
    }
    free(xq);
    return VTQO_OK;
}

/* src/ops/quant.rs:936-980 (serial), :1149-1196 (parallel) */
int vtqo_linear_q4_k_integer(const float *x, const uint8_t *w, size_t w_len, float *y, size_t batch,
                             size_t in_feat, size_t out_feat, int threads, const char **msg) {
    if (threads > 1)
        return linear_kquant(ROW_Q4K_INT, Q4_K_BYTES, "linear_q4_k_integer_parallel: in_feat % 256",
                             "linear_q4_k_integer_parallel: weight shape", x, w, w_len, y, batch,
                             in_feat, out_feat, threads, msg);
    return linear_kquant(ROW_Q4K_INT, Q4_K_BYTES, "linear_q4_k_integer: in_feat not a multiple of 256",
                         "linear_q4_k_integer: weight shape mismatch", x, w, w_len, y, batch, in_feat,
                         out_feat, 1, msg);
}

/* src/ops/quant.rs:1060-1096 (serial), :1099-1146 (parallel) */
int vtqo_linear_q6_k_integer(const float *x, const uint8_t *w, size_t w_len, float *y, size_t batch,
                             size_t in_feat, size_t out_feat, int threads, const char **msg) {
    if (threads > 1)
        return linear_kquant(ROW_Q6K_INT, Q6_K_BYTES, "linear_q6_k_integer_parallel: in_feat % 256",
                             "linear_q6_k_integer_parallel: weight shape", x, w, w_len, y, batch,
                             in_feat, out_feat, threads, msg);
    return linear_kquant(ROW_Q6K_INT, Q6_K_BYTES, "linear_q6_k_integer: in_feat not a multiple of 256",
                         "linear_q6_k_integer: weight shape mismatch", x, w, w_len, y, batch, in_feat,
                         out_feat, 1, msg);
}

/* src/ops/quant.rs:1433-1453 (serial, no blob-length check), :1386-1430 (parallel) */
int vtqo_linear_q4_k_fused(const float *x, const uint8_t *w, size_t w_len, float *y, size_t batch,
                           size_t in_feat, size_t out_feat, int threads, const char **msg) {
    if (threads > 1)
        return linear_kquant(ROW_Q4K_FUSED, Q4_K_BYTES,
                             "linear_q4_k_fused_parallel: in_feat not a multiple of 256",
                             "linear_q4_k_fused_parallel: weight shape mismatch", x, w, w_len, y,
                             batch, in_feat, out_feat, threads, msg);
    if (in_feat % QK_K != 0) FAIL(VTQO_E_INTERNAL, "linear_q4_k_fused: in_feat not a multiple of 256");
    size_t row_bytes = (in_feat / QK_K) * Q4_K_BYTES;
    /* The serial reference slices w[o*row_bytes..] and would panic on a short
     * blob; report it as an error instead. */
    if (w_len < out_feat * row_bytes) FAIL(VTQO_E_INTERNAL, "linear_q4_k_fused: weight shape mismatch");
    for (size_t b = 0; b < batch; b++)
        for (size_t o = 0; o < out_feat; o++) {
            int rc = vtqo_canonical_dot_q4k_fused(x + b * in_feat, w + o * row_bytes, row_bytes, in_feat,
                                                  &y[b * out_feat + o], msg);
            if (rc) return rc;
        }
    return VTQO_OK;
}

/* src/ops/quant.rs:1304-1327, :1331-1369 */
int vtqo_linear_q6_k_fused(const float *x, const uint8_t *w, size_t w_len, float *y, size_t batch,
                           size_t in_feat, size_t out_feat, int threads, const char **msg) {
    if (threads > 1)
        return linear_kquant(ROW_Q6K_FUSED, Q6_K_BYTES,
                             "linear_q6_k_fused_parallel: in_feat not a multiple of 256",
                             "linear_q6_k_fused_parallel: weight shape mismatch", x, w, w_len, y,
                             batch, in_feat, out_feat, threads, msg);
    return linear_kquant(ROW_Q6K_FUSED, Q6_K_BYTES, "linear_q6_k_fused: in_feat not a multiple of 256",
                         "linear_q6_k_fused: weight shape mismatch", x, w, w_len, y, batch, in_feat,
                         out_feat, 1, msg);
}

typedef int (*dequant_fn)(const uint8_t *, size_t, float *, const char **);

static int linear_dequant_then_dot(dequant_fn deq, size_t block_bytes, size_t block_numel,
                                   const char *ex, const char *ey, const char *ew, const float *x,
                                   size_t x_len, const uint8_t *w, size_t w_len, float *y, size_t y_len,
                                   size_t batch, size_t in_feat, size_t out_feat, const char **msg) {
    if (x_len != batch * in_feat) FAIL(VTQO_E_INTERNAL, ex);
    if (y_len != batch * out_feat) FAIL(VTQO_E_INTERNAL, ey);
    if (w_len % block_bytes != 0) return deq(w, w_len, NULL, msg);
    size_t numel = (w_len / block_bytes) * block_numel;
    if (numel != out_feat * in_feat) FAIL(VTQO_E_INTERNAL, ew);
    float *wf = (float *)malloc((numel ? numel : 1) * sizeof(float));
    deq(w, w_len, wf, msg);
    for (size_t b = 0; b < batch; b++)
        for (size_t o = 0; o < out_feat; o++)
            y[b * out_feat + o] = vtqo_canonical_dot(x + b * in_feat, wf + o * in_feat, in_feat);
    free(wf);
    return VTQO_OK;
}

/* src/ops/quant.rs:1456-1482 */
int vtqo_linear_q4_k_cpu(const float *x, size_t x_len, const uint8_t *w, size_t w_len, float *y,
                         size_t y_len, size_t batch, size_t in_feat, size_t out_feat, const char **msg) {
    return linear_dequant_then_dot(vtqo_dequantize_q4_k, Q4_K_BYTES, QK_K, "linear_q4_k_cpu: x shape mismatch",
                                   "linear_q4_k_cpu: y shape mismatch", "linear_q4_k_cpu: weight shape mismatch",
                                   x, x_len, w, w_len, y, y_len, batch, in_feat, out_feat, msg);
}

/* src/ops/quant.rs:1485-1511 */
int vtqo_linear_q6_k_cpu(const float *x, size_t x_len, const uint8_t *w, size_t w_len, float *y,
                         size_t y_len, size_t batch, size_t in_feat, size_t out_feat, const char **msg) {
    return linear_dequant_then_dot(vtqo_dequantize_q6_k, Q6_K_BYTES, QK_K, "linear_q6_k_cpu: x shape mismatch",
                                   "linear_q6_k_cpu: y shape mismatch", "linear_q6_k_cpu: weight shape mismatch",
                                   x, x_len, w, w_len, y, y_len, batch, in_feat, out_feat, msg);
}

/* src/ops/quant.rs:1529-1565 */
int vtqo_linear_q4_0_cpu(const float *x, size_t x_len, const uint8_t *w, size_t w_len, float *y,
                         size_t y_len, size_t batch, size_t in_feat, size_t out_feat, const char **msg) {
    if (in_feat % QK != 0) FAIL(VTQO_E_INTERNAL, "linear_q4_0: in_feat must be multiple of 32");
    if (w_len != out_feat * (in_feat / QK) * Q4_0_BYTES) FAIL(VTQO_E_INTERNAL, "linear_q4_0: weight blob length mismatch");
    if (x_len != batch * in_feat) FAIL(VTQO_E_INTERNAL, "linear_q4_0: x size mismatch");
    if (y_len != batch * out_feat) FAIL(VTQO_E_INTERNAL, "linear_q4_0: y_out size mismatch");
    size_t numel = out_feat * in_feat;
    float *wf = (float *)malloc((numel ? numel : 1) * sizeof(float));
    vtqo_dequantize_q4_0(w, w_len, wf, msg);
    for (size_t b = 0; b < batch; b++)
        for (size_t o = 0; o < out_feat; o++)
            y[b * out_feat + o] = vtqo_canonical_dot(x + b * in_feat, wf + o * in_feat, in_feat);
    free(wf);
    return VTQO_OK;
}

/* Per-row decode + canonical dot, the Q8_0 / Q5_0 arms of linear_dispatch
 * (src/model/forward_quantized.rs:751-776). */
static int dispatch_rowwise(dequant_fn deq, size_t block_bytes, const char *e_in, const char *e_w,
                            const float *x, const uint8_t *w, size_t w_len, float *y, size_t batch,
                            size_t in_feat, size_t out_feat, const char **msg) {
    if (in_feat % QK != 0) FAIL(VTQO_E_INTERNAL, e_in);
    size_t row_bytes = (in_feat / QK) * block_bytes;
    if (w_len < out_feat * row_bytes) FAIL(VTQO_E_INTERNAL, e_w);
    float *row = (float *)malloc((in_feat ? in_feat : 1) * sizeof(float));
    for (size_t b = 0; b < batch; b++)
        for (size_t o = 0; o < out_feat; o++) {
            deq(w + o * row_bytes, row_bytes, row, msg);
            y[b * out_feat + o] = vtqo_canonical_dot(x + b * in_feat, row, in_feat);
        }
    free(row);
    return VTQO_OK;
}

int vtqo_linear_dispatch(int ggml_type, int regime, const float *x, size_t x_len, const uint8_t *w,
                         size_t w_len, float *y, size_t y_len, size_t batch, size_t in_feat,
                         size_t out_feat, int threads, const char **msg) {
    int par = (threads > 1 && out_feat >= 512) ? threads : 1; /* PAR_MIN_ROWS, :710 */
    switch (ggml_type) {
    case 2: /* Q4_0, :671-673 */
        return vtqo_linear_q4_0_cpu(x, x_len, w, w_len, y, y_len, batch, in_feat, out_feat, msg);
    case 0: { /* F32, :674-697 */
        if (w_len != out_feat * in_feat * 4) FAIL(VTQO_E_INTERNAL, "linear_dispatch F32: weight size mismatch");
        const float *wf = (const float *)(const void *)w;
        for (size_t b = 0; b < batch; b++)
            for (size_t o = 0; o < out_feat; o++)
                y[b * out_feat + o] = vtqo_canonical_dot(x + b * in_feat, wf + o * in_feat, in_feat);
        return VTQO_OK;
    }
    case 12: /* Q4_K, :698-726: the std-parallel build calls the row-parallel
              * function (and reports its errors) for out_feat >= PAR_MIN_ROWS
              * whatever the thread count; the default build the fused one */
        if (regime == 1) return vtqo_linear_q4_k_fused(x, w, w_len, y, batch, in_feat, out_feat, 1, msg);
        if (out_feat >= 512)
            return linear_kquant(ROW_Q4K_INT, Q4_K_BYTES, "linear_q4_k_integer_parallel: in_feat % 256",
                                 "linear_q4_k_integer_parallel: weight shape", x, w, w_len, y, batch, in_feat,
                                 out_feat, par, msg);
        return vtqo_linear_q4_k_integer(x, w, w_len, y, batch, in_feat, out_feat, 1, msg);
    case 14: /* Q6_K, :727-750: the same; the default build always the serial function */
        if (regime == 0 && out_feat >= 512)
            return linear_kquant(ROW_Q6K_INT, Q6_K_BYTES, "linear_q6_k_integer_parallel: in_feat % 256",
                                 "linear_q6_k_integer_parallel: weight shape", x, w, w_len, y, batch, in_feat,
                                 out_feat, par, msg);
        return vtqo_linear_q6_k_integer(x, w, w_len, y, batch, in_feat, out_feat, regime == 0 ? par : 1, msg);
    case 8: /* Q8_0, :751-764 */
        return dispatch_rowwise(vtqo_dequantize_q8_0, Q8_0_BYTES, "Q8_0: in_feat must be a multiple of 32",
                                "linear_dispatch Q8_0: weight blob too small", x, w, w_len, y, batch,
                                in_feat, out_feat, msg);
    case 6: /* Q5_0, :765-776 */
        return dispatch_rowwise(vtqo_dequantize_q5_0, Q5_0_BYTES, "Q5_0: in_feat must be a multiple of 32",
                                "linear_dispatch Q5_0: weight blob too small", x, w, w_len, y, batch,
                                in_feat, out_feat, msg);
    default: /* F16 / Other, :777-782 */
        FAIL(VTQO_E_NOT_IMPLEMENTED, "weight dtype not Q4_0 / Q4_K / Q5_0 / Q6_K / Q8_0 / F32");
    }
}

/* src/ops/matmul.rs:108-127 */
void vtqo_matmul_f32(const float *a, const float *b, float *out, size_t m, size_t k, size_t n) {
    float *col = (float *)malloc((k ? k : 1) * sizeof(float));
    for (size_t j = 0; j < n; j++) {
        if (k == 0) {
            for (size_t i = 0; i < m; i++) out[i * n + j] = 0.0f;
            continue;
        }
        for (size_t kk = 0; kk < k; kk++) col[kk] = b[kk * n + j];
        for (size_t i = 0; i < m; i++) out[i * n + j] = vtqo_canonical_dot(a + i * k, col, k);
    }
    free(col);
}
