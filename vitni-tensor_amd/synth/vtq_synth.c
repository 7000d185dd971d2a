/*
 * vtq_synth.c -- seeded synthetic inputs for the benchmark configurations.
 * Stream and draw order are specified in vtq_synth.h.  The block encoders are
 * the inverses of the decoders of src/ops/quant.rs (get_scale_min_k4 :267-276,
 * Q6_K ql/qh split :352-383, Q5_0 qh bits :176-183, Q4_0 (2k, 2k+1) :102-108).
 */
#include "vtq_synth.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

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

void vtqs_tokens(uint64_t seed, uint32_t *out, size_t n, uint32_t vocab) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i++) out[i] = uni(&s, vocab);
}

/* ---- GGUF v3 writer ---- */
typedef struct {
    uint8_t *out;
    size_t pos;
} gw_t;

static void gw_bytes(gw_t *g, const void *p, size_t n) {
    if (g->out) memcpy(g->out + g->pos, p, n);
    g->pos += n;
}
static void gw_u32(gw_t *g, uint32_t v) {
    uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
    gw_bytes(g, b, 4);
}
static void gw_u64(gw_t *g, uint64_t v) {
    gw_u32(g, (uint32_t)v);
    gw_u32(g, (uint32_t)(v >> 32));
}
static void gw_str(gw_t *g, const char *s) {
    gw_u64(g, strlen(s));
    gw_bytes(g, s, strlen(s));
}
static void gw_kv_u32(gw_t *g, const char *k, uint32_t v) {
    gw_str(g, k);
    gw_u32(g, 4);
    gw_u32(g, v);
}
static void gw_kv_f32(gw_t *g, const char *k, float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    gw_str(g, k);
    gw_u32(g, 6);
    gw_u32(g, b);
}

typedef struct {
    char name[64];
    uint32_t type;           /* 0 F32, 12 Q4_K, 14 Q6_K */
    uint64_t ne0, ne1;       /* row length, rows (ne1 = 0: 1-D) */
    size_t nbytes, offset;
} gt_t;

static size_t gt_bytes(const gt_t *t) {
    const uint64_t rows = t->ne1 ? t->ne1 : 1;
    switch (t->type) {  /* 100: an F32 bias (written with type 0) */
    case 12: return (size_t)(rows * (t->ne0 / 256) * 144);
    case 14: return (size_t)(rows * (t->ne0 / 256) * 210);
    default: return (size_t)(rows * t->ne0 * 4);
    }
}

size_t vtqs_llama_gguf(const vtqs_llama *c, uint64_t seed, uint8_t *out) {
    const uint32_t head = c->dim / c->heads, kv_dim = c->kv_heads * head;
    const uint64_t align = c->alignment ? c->alignment : 32;
    const char *arch = c->arch == 1 ? "qwen2" : "llama";
    const size_t nt = 3 + 9 * (size_t)c->layers + (c->qkv_bias ? 3 * (size_t)c->layers : 0);
    gt_t *ts = (gt_t *)calloc(nt, sizeof(gt_t));
    size_t k = 0;
#define T(NAME, TYPE, NE0, NE1)                                              \
    do {                                                                     \
        snprintf(ts[k].name, sizeof ts[k].name, "%s", NAME);                 \
        ts[k].type = TYPE;                                                   \
        ts[k].ne0 = NE0;                                                     \
        ts[k].ne1 = NE1;                                                     \
        k++;                                                                 \
    } while (0)
    T("token_embd.weight", 12, c->dim, c->vocab);
    for (uint32_t l = 0; l < c->layers; l++) {
        char nm[64];
        snprintf(nm, sizeof nm, "blk.%u.attn_norm.weight", l); T(nm, 0, c->dim, 0);
        snprintf(nm, sizeof nm, "blk.%u.attn_q.weight", l); T(nm, 12, c->dim, c->dim);
        snprintf(nm, sizeof nm, "blk.%u.attn_k.weight", l); T(nm, 12, c->dim, kv_dim - (l == 0 ? c->short_rows : 0));
        snprintf(nm, sizeof nm, "blk.%u.attn_v.weight", l); T(nm, 12, c->dim, kv_dim);
        snprintf(nm, sizeof nm, "blk.%u.attn_output.weight", l); T(nm, 12, c->dim, c->dim);
        snprintf(nm, sizeof nm, "blk.%u.ffn_norm.weight", l); T(nm, 0, c->dim, 0);
        snprintf(nm, sizeof nm, "blk.%u.ffn_gate.weight", l); T(nm, 12, c->dim, c->hidden);
        snprintf(nm, sizeof nm, "blk.%u.ffn_up.weight", l); T(nm, 12, c->dim, c->hidden);
        snprintf(nm, sizeof nm, "blk.%u.ffn_down.weight", l); T(nm, 12, c->hidden, c->dim);
        if (c->qkv_bias) {
            /* the bias tensors: F32 with ne1 = 0, marked by type 100 until written */
            snprintf(nm, sizeof nm, "blk.%u.attn_q.bias", l); T(nm, 100, c->dim, 0);
            snprintf(nm, sizeof nm, "blk.%u.attn_k.bias", l); T(nm, 100, kv_dim, 0);
            snprintf(nm, sizeof nm, "blk.%u.attn_v.bias", l); T(nm, 100, kv_dim, 0);
        }
    }
    T("output_norm.weight", 0, c->dim, 0);
    if (!c->tied) T("output.weight", 14, c->dim, c->vocab);
#undef T
    const size_t n_used = k;
    size_t off = 0;
    for (size_t i = 0; i < n_used; i++) {
        ts[i].nbytes = gt_bytes(&ts[i]);
        ts[i].offset = off;
        off += (ts[i].nbytes + align - 1) / align * align;
    }
    gw_t g = {out, 0};
    char key[96];
    gw_bytes(&g, "GGUF", 4);
    gw_u32(&g, 3);
    gw_u64(&g, n_used);
    gw_u64(&g, 11);
    gw_str(&g, "general.architecture");
    gw_u32(&g, 8);
    gw_str(&g, arch);
    gw_kv_u32(&g, "general.alignment", (uint32_t)align);
#define KV_U32(SUFFIX, V) snprintf(key, sizeof key, "%s." SUFFIX, arch); gw_kv_u32(&g, key, V)
#define KV_F32(SUFFIX, V) snprintf(key, sizeof key, "%s." SUFFIX, arch); gw_kv_f32(&g, key, V)
    KV_U32("embedding_length", c->dim);
    KV_U32("feed_forward_length", c->hidden);
    KV_U32("block_count", c->layers);
    KV_U32("attention.head_count", c->heads);
    KV_U32("attention.head_count_kv", c->kv_heads);
    KV_U32("context_length", c->ctx);
    KV_U32("vocab_size", c->vocab);
    KV_F32("rope.freq_base", c->rope_theta);
    KV_F32("attention.layer_norm_rms_epsilon", c->rms_eps);
#undef KV_U32
#undef KV_F32
    for (size_t i = 0; i < n_used; i++) {
        gw_str(&g, ts[i].name);
        gw_u32(&g, ts[i].ne1 ? 2 : 1);
        gw_u64(&g, ts[i].ne0);
        if (ts[i].ne1) gw_u64(&g, ts[i].ne1);
        gw_u32(&g, ts[i].type == 100 ? 0 : ts[i].type);
        gw_u64(&g, ts[i].offset);
    }
    const size_t base = (g.pos + align - 1) / align * align;
    if (out) memset(out + g.pos, 0, base - g.pos);
    if (out) {
        for (size_t i = 0; i < n_used; i++) {
            uint8_t *p = out + base + ts[i].offset;
            const uint64_t ts_seed = seed + i;
            const size_t pad = (ts[i].nbytes + align - 1) / align * align - ts[i].nbytes;
            if (ts[i].type == 12) {
                vtqs_q4_k(ts_seed, p, ts[i].ne1, ts[i].ne0, 0.01f);
            } else if (ts[i].type == 14) {
                vtqs_q6_k(ts_seed, p, ts[i].ne1, ts[i].ne0, 0.01f);
            } else {
                /* F32 tensors may sit at any multiple of the alignment: write
                 * them through a staging buffer */
                float *v = (float *)malloc(ts[i].ne0 * sizeof(float));
                vtqs_normal_f32(ts_seed, v, ts[i].ne0, ts[i].type == 100 ? 0.5f : 0.05f);
                if (ts[i].type != 100)
                    for (uint64_t e = 0; e < ts[i].ne0; e++) v[e] = 1.0f + v[e];
                memcpy(p, v, ts[i].ne0 * sizeof(float));
                free(v);
            }
            memset(p + ts[i].nbytes, 0, pad);
        }
    }
    free(ts);
    return base + off;
}
