/*
 * vtq_oracle_e2e.c -- TEST INFRASTRUCTURE (the checker; never linked into
 * the product).
 *
 * CPU restatement of the reference's quantized decode around the linear
 * layer: GGUF parsing (src/model/gguf.rs:305-421), Config::from_gguf
 * (src/model/config.rs:156-213), QuantizedWeights::from_gguf
 * (src/model/quant_weights.rs:121-181), forward_quantized::step
 * (src/model/forward_quantized.rs:329-655, helpers :818-941) and
 * inference::run_quantized (src/model/inference.rs:274-345) with its
 * receipt (src/cert/builder.rs:458-471).  Linears go through
 * vtqo_linear_dispatch (forward_quantized.rs:663-785).
 *
 * Pins: the libm and BLAKE3 restatements and the v2 digest are pinned by the
 * reference's own constants (tests/test_oracle_e2e.py); rms_norm, softmax
 * and argmax by the reference's known answers (src/ops/rms_norm.rs:117-160,
 * src/ops/argmax.rs:74-125) and closed forms.  Parity unpinned: the
 * composition of the forward step and run_quantized's token loop -- the
 * reference's model tests need GGUF files that are not in the repository,
 * and no reference-produced logits exist for any model here.
 */
#include "vtq_oracle_e2e.h"
#include "vtq_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- GGUF */

enum { T_U8 = 0, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 };

typedef struct {
    const uint8_t* p;
    size_t len, pos;
    int bad;
} cur_t;

static int need(cur_t* c, size_t n) {
    if (c->bad || c->len - c->pos < n) {
        c->bad = 1;
        return 0;
    }
    return 1;
}
static uint64_t rd(cur_t* c, int bytes) {
    if (!need(c, (size_t)bytes)) return 0;
    uint64_t v = 0;
    for (int i = 0; i < bytes; i++) v |= (uint64_t)c->p[c->pos + i] << (8 * i);
    c->pos += (size_t)bytes;
    return v;
}
static int scalar_size(uint32_t t) {
    switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    }
    return 0;
}

typedef struct {
    char key[96];
    uint32_t type;
    uint64_t num;           /* integer value / f32 bits */
    const uint8_t* str;     /* string bytes */
    uint64_t str_len;       /* string length or array element count */
} kv_t;

typedef struct {
    char name[96];
    uint32_t type;
    uint64_t numel;
    const uint8_t* bytes;
    size_t nbytes;
} tinfo_t;

static int skip_value(cur_t* c, uint32_t t, kv_t* out) {
    if (t == T_STR) {
        uint64_t n = rd(c, 8);
        if (!need(c, n)) return 0;
        if (out) {
            out->str = c->p + c->pos;
            out->str_len = n;
        }
        c->pos += n;
        return 1;
    }
    if (t == T_ARR) {
        uint32_t et = (uint32_t)rd(c, 4);
        uint64_t n = rd(c, 8);
        if (out) out->str_len = n;
        for (uint64_t i = 0; i < n && !c->bad; i++)
            if (!skip_value(c, et, NULL)) return 0;
        return !c->bad;
    }
    int s = scalar_size(t);
    if (!s) {
        c->bad = 1;
        return 0;
    }
    uint64_t v = rd(c, s);
    if (out) out->num = v;
    return !c->bad;
}

static size_t bytes_for(uint32_t t, uint64_t numel, int* ok) {
    *ok = 1;
    switch (t) {
    case 0: return (size_t)numel * 4;
    case 1: return (size_t)numel * 2;
    case 2: if (numel % 32) break; return (size_t)(numel / 32) * 18;
    case 6: if (numel % 32) break; return (size_t)(numel / 32) * 22;
    case 8: if (numel % 32) break; return (size_t)(numel / 32) * 34;
    case 12: if (numel % 256) break; return (size_t)(numel / 256) * 144;
    case 14: if (numel % 256) break; return (size_t)(numel / 256) * 210;
    }
    *ok = 0;
    return 0;
}

/* ---------------------------------------------------------------- model */

typedef struct {
    int dtype;
    const uint8_t* w;
    size_t len;
} qt_t;

typedef struct {
    const float *rms_att, *rms_ffn;
    const float *bq, *bk, *bv;
    qt_t wq, wk, wv, wo, w1, w2, w3;
} layer_t;

struct vtqo_model {
    int dim, hidden, n_layers, n_heads, n_kv_heads, vocab, seq_len, shared;
    float rope_theta, rms_eps;
    int rope_neox;
    qt_t tok_embd, wcls;
    const float* rms_final;
    layer_t* layers;
    kv_t* kvs;
    size_t n_kv;
    tinfo_t* tensors;
    size_t n_tensors;
};

static const kv_t* find_kv(const vtqo_model* m, const char* key) {
    for (size_t i = 0; i < m->n_kv; i++)
        if (!strcmp(m->kvs[i].key, key)) return &m->kvs[i];
    return NULL;
}
static const tinfo_t* find_t(const vtqo_model* m, const char* name) {
    for (size_t i = 0; i < m->n_tensors; i++)
        if (!strcmp(m->tensors[i].name, name)) return &m->tensors[i];
    return NULL;
}
static int read_usize(const vtqo_model* m, const char* key, int* out) {
    const kv_t* v = find_kv(m, key);
    if (!v) return 0;
    switch (v->type) {
    case T_U32: case T_U64: *out = (int)v->num; return 1;
    case T_I32: if ((int32_t)v->num < 0) return 0; *out = (int)(int32_t)v->num; return 1;
    case T_I64: if ((int64_t)v->num < 0) return 0; *out = (int)(int64_t)v->num; return 1;
    }
    return 0;
}
static float read_f32_meta(const vtqo_model* m, const char* key, float def) {
    const kv_t* v = find_kv(m, key);
    if (!v || v->type != T_F32) return def;
    float f;
    uint32_t b = (uint32_t)v->num;
    memcpy(&f, &b, 4);
    return f;
}
static int get_qt(const vtqo_model* m, const char* name, qt_t* out) {
    const tinfo_t* t = find_t(m, name);
    if (!t) return 0;
    out->dtype = (int)t->type;
    out->w = t->bytes;
    out->len = t->nbytes;
    return 1;
}
static const float* get_f32(const vtqo_model* m, const char* name, size_t want) {
    const tinfo_t* t = find_t(m, name);
    if (!t || t->type != 0 || t->nbytes != want * 4) return NULL;
    return (const float*)t->bytes;
}

void vtqo_model_free(vtqo_model* m) {
    if (!m) return;
    free(m->layers);
    free(m->kvs);
    free(m->tensors);
    free(m);
}

int vtqo_model_load(const uint8_t* blob, size_t len, vtqo_model** out, const char** msg) {
    *out = NULL;
    cur_t c = {blob, len, 0, 0};
    if (!need(&c, 4) || memcmp(blob, "GGUF", 4)) {
        *msg = "gguf: bad magic (not 'GGUF')";
        return 1;
    }
    c.pos = 4;
    uint32_t version = (uint32_t)rd(&c, 4);
    if (version != 2 && version != 3) {
        *msg = "gguf: unsupported version (only v2/v3 supported)";
        return 1;
    }
    uint64_t n_t = rd(&c, 8), n_kv = rd(&c, 8);
    if (c.bad || n_kv > len || n_t > len) {
        *msg = "gguf: truncated header";
        return 1;
    }
    vtqo_model* m = (vtqo_model*)calloc(1, sizeof *m);
    m->kvs = (kv_t*)calloc(n_kv ? n_kv : 1, sizeof(kv_t));
    m->tensors = (tinfo_t*)calloc(n_t ? n_t : 1, sizeof(tinfo_t));
    for (uint64_t i = 0; i < n_kv; i++) {
        uint64_t kl = rd(&c, 8);
        if (!need(&c, kl) || kl >= sizeof m->kvs[i].key) goto bad;
        memcpy(m->kvs[i].key, c.p + c.pos, kl);
        c.pos += kl;
        m->kvs[i].type = (uint32_t)rd(&c, 4);
        if (!skip_value(&c, m->kvs[i].type, &m->kvs[i])) goto bad;
        m->n_kv++;
    }
    uint64_t* offs = (uint64_t*)calloc(n_t ? n_t : 1, 8);
    for (uint64_t i = 0; i < n_t; i++) {
        uint64_t nl = rd(&c, 8);
        if (!need(&c, nl) || nl >= sizeof m->tensors[i].name) {
            free(offs);
            goto bad;
        }
        memcpy(m->tensors[i].name, c.p + c.pos, nl);
        c.pos += nl;
        uint32_t nd = (uint32_t)rd(&c, 4);
        if (nd > 8) {
            free(offs);
            goto bad;
        }
        uint64_t numel = 1;
        for (uint32_t d = 0; d < nd; d++) numel *= rd(&c, 8);
        m->tensors[i].numel = numel;
        m->tensors[i].type = (uint32_t)rd(&c, 4);
        offs[i] = rd(&c, 8);
        if (c.bad) {
            free(offs);
            goto bad;
        }
        m->n_tensors++;
    }
    {
        const kv_t* al = find_kv(m, "general.alignment");
        uint64_t alignment = (al && al->type == T_U32) ? al->num : 32;
        if (alignment == 0) {
            free(offs);
            goto bad;
        }
        size_t base = (size_t)((c.pos + alignment - 1) / alignment * alignment);
        for (size_t i = 0; i < m->n_tensors; i++) {
            int ok;
            size_t nb = bytes_for(m->tensors[i].type, m->tensors[i].numel, &ok);
            if (!ok || base + offs[i] + nb > len) {
                free(offs);
                goto bad;
            }
            m->tensors[i].bytes = blob + base + offs[i];
            m->tensors[i].nbytes = nb;
        }
    }
    free(offs);

    {
        /* Config::from_gguf (src/model/config.rs:156-213) */
        const kv_t* a = find_kv(m, "general.architecture");
        char arch[64] = {0}, key[160];
        if (!a || a->type != T_STR || a->str_len >= sizeof arch) {
            *msg = "gguf: missing 'general.architecture' metadata";
            vtqo_model_free(m);
            return 1;
        }
        memcpy(arch, a->str, a->str_len);
#define META(suffix, dst)                                          \
    snprintf(key, sizeof key, "%s.%s", arch, suffix);              \
    if (!read_usize(m, key, dst)) {                                \
        *msg = "gguf: numeric metadata missing or wrong type";     \
        vtqo_model_free(m);                                        \
        return 1;                                                  \
    }
        META("embedding_length", &m->dim);
        META("feed_forward_length", &m->hidden);
        META("block_count", &m->n_layers);
        META("attention.head_count", &m->n_heads);
        snprintf(key, sizeof key, "%s.attention.head_count_kv", arch);
        if (!read_usize(m, key, &m->n_kv_heads)) m->n_kv_heads = m->n_heads;
        META("context_length", &m->seq_len);
        const kv_t* toks = find_kv(m, "tokenizer.ggml.tokens");
        if (toks && toks->type == T_ARR) {
            m->vocab = (int)toks->str_len;
        } else {
            META("vocab_size", &m->vocab);
        }
#undef META
        m->shared = find_t(m, "output.weight") == NULL;
        snprintf(key, sizeof key, "%s.rope.freq_base", arch);
        m->rope_theta = read_f32_meta(m, key, 10000.0f);
        snprintf(key, sizeof key, "%s.attention.layer_norm_rms_epsilon", arch);
        m->rms_eps = read_f32_meta(m, key, 1e-5f);
        m->rope_neox = !strcmp(arch, "qwen2");
    }
    if (!get_qt(m, "token_embd.weight", &m->tok_embd) ||
        !(m->rms_final = get_f32(m, "output_norm.weight", (size_t)m->dim))) {
        *msg = "gguf: required Llama tensor not found";
        vtqo_model_free(m);
        return 1;
    }
    if (!m->shared) get_qt(m, "output.weight", &m->wcls);
    m->layers = (layer_t*)calloc((size_t)m->n_layers, sizeof(layer_t));
    for (int l = 0; l < m->n_layers; l++) {
        char nm[96];
        layer_t* L = &m->layers[l];
#define QT(field, suffix)                                       \
    snprintf(nm, sizeof nm, "blk.%d.%s", l, suffix);            \
    if (!get_qt(m, nm, &L->field)) {                            \
        *msg = "gguf: required Llama tensor not found";         \
        vtqo_model_free(m);                                     \
        return 1;                                               \
    }
        QT(wq, "attn_q.weight");
        QT(wk, "attn_k.weight");
        QT(wv, "attn_v.weight");
        QT(wo, "attn_output.weight");
        QT(w1, "ffn_gate.weight");
        QT(w2, "ffn_down.weight");
        QT(w3, "ffn_up.weight");
#undef QT
        snprintf(nm, sizeof nm, "blk.%d.attn_norm.weight", l);
        L->rms_att = get_f32(m, nm, (size_t)m->dim);
        snprintf(nm, sizeof nm, "blk.%d.ffn_norm.weight", l);
        L->rms_ffn = get_f32(m, nm, (size_t)m->dim);
        if (!L->rms_att || !L->rms_ffn) {
            *msg = "gguf: expected F32 norm-weight tensor, got something else";
            vtqo_model_free(m);
            return 1;
        }
        const int kv_dim = m->n_kv_heads * (m->dim / m->n_heads);
        snprintf(nm, sizeof nm, "blk.%d.attn_q.bias", l);
        L->bq = get_f32(m, nm, (size_t)m->dim);
        snprintf(nm, sizeof nm, "blk.%d.attn_k.bias", l);
        L->bk = get_f32(m, nm, (size_t)kv_dim);
        snprintf(nm, sizeof nm, "blk.%d.attn_v.bias", l);
        L->bv = get_f32(m, nm, (size_t)kv_dim);
    }
    *out = m;
    return 0;
bad:
    *msg = "gguf: malformed or truncated file";
    vtqo_model_free(m);
    return 1;
}

void vtqo_model_dims(const vtqo_model* m, int dims[7]) {
    dims[0] = m->dim;
    dims[1] = m->hidden;
    dims[2] = m->n_layers;
    dims[3] = m->n_heads;
    dims[4] = m->n_kv_heads;
    dims[5] = m->vocab;
    dims[6] = m->seq_len;
}

/* ---------------------------------------------------------------- step */

/* ---------------------------------------------------------------- receipts */

/* PerOpRecorder / PerActivationRecorder (src/model/forward_quantized.rs:64-132,
 * :260-284).  params[l][k]: k = 0 rms_att, 1 wq, 2 wk, 3 wv, 4 wo, 5 rms_ffn,
 * 6 w1, 7 w2, 8 w3 -- BLAKE3 of the weight bytes, hash_f32_slice of norms. */
#define NO_LAYER 0xFFFFFFFFu
typedef struct {
    int flags;
    uint8_t (*params)[9][32];
    uint8_t tok[32], rms_final[32], wcls[32];
    vtqo_op_record* ops;
    vtqo_act_record* acts;
    size_t n_ops, cap_ops, n_acts, cap_acts;
    int oom;
} rec_t;

/* hash_f32_slice (forward_quantized.rs:275-284): BLAKE3 of the LE bytes */
static void hash_f32(const float* v, size_t n, uint8_t out[32]) { vtqo_blake3_hash(v, n * 4, out); }

static void rec_op(rec_t* rc, const char* name, uint32_t layer, const uint8_t* params, const float* in, size_t n_in,
                   const float* out, size_t n_out) {
    if (!rc || !(rc->flags & VTQO_RECORD_OPS) || rc->oom) return;
    if (rc->n_ops == rc->cap_ops) {
        const size_t cap = rc->cap_ops ? 2 * rc->cap_ops : 256;
        vtqo_op_record* p = (vtqo_op_record*)realloc(rc->ops, cap * sizeof *p);
        if (!p) {
            rc->oom = 1;
            return;
        }
        rc->ops = p;
        rc->cap_ops = cap;
    }
    vtqo_op_record* o = &rc->ops[rc->n_ops];
    memset(o, 0, sizeof *o);
    o->op_index = (uint32_t)rc->n_ops;
    o->layer = layer;
    strncpy(o->op_name, name, sizeof o->op_name - 1);
    hash_f32(in, n_in, o->input_hash);
    if (params) memcpy(o->params_hash, params, 32);
    hash_f32(out, n_out, o->output_hash);
    rc->n_ops++;
}

static void rec_act(rec_t* rc, uint32_t token, uint32_t layer, const char* checkpoint, const float* t, size_t n) {
    if (!rc || !(rc->flags & VTQO_RECORD_ACTIVATIONS) || rc->oom) return;
    if (rc->n_acts == rc->cap_acts) {
        const size_t cap = rc->cap_acts ? 2 * rc->cap_acts : 256;
        vtqo_act_record* p = (vtqo_act_record*)realloc(rc->acts, cap * sizeof *p);
        if (!p) {
            rc->oom = 1;
            return;
        }
        rc->acts = p;
        rc->cap_acts = cap;
    }
    vtqo_act_record* a = &rc->acts[rc->n_acts];
    memset(a, 0, sizeof *a);
    a->act_index = (uint32_t)rc->n_acts;
    a->token_index = token;
    a->layer = layer;
    strncpy(a->checkpoint, checkpoint, sizeof a->checkpoint - 1);
    hash_f32(t, n, a->tensor_hash);
    rc->n_acts++;
}

typedef struct {
    const vtqo_model* m;
    rec_t* rec;
    int regime, threads;
    float *key_cache, *value_cache;  /* [layers][seq][kv_dim] */
    float *x, *xb, *q, *k, *v, *att, *xb_out, *xb2, *gate, *up, *ffn, *logits;
    const char* msg;
} run_t;

static int linear(run_t* r, const qt_t* w, const float* x, int in_f, int out_f, float* y) {
    return vtqo_linear_dispatch(w->dtype, r->regime, x, (size_t)in_f, w->w, w->len, y, (size_t)out_f, 1,
                                (size_t)in_f, (size_t)out_f, out_f >= 512 ? r->threads : 1, &r->msg);
}

/* rms_norm_slice (src/ops/rms_norm.rs:60-110) */
void vtqo_rms_norm(const float* x, const float* w, int n, float eps, float* out) {
    float sumsq = 0.0f;
    for (int i = 0; i < n; i++) sumsq += x[i] * x[i];
    const float mean = sumsq / (float)n;
    const float scale = 1.0f / vtqo_sqrtf(mean + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* softmax_inplace (src/model/forward_quantized.rs:925-941) */
void vtqo_softmax(float* x, int n) {
    float max = -INFINITY;
    for (int i = 0; i < n; i++)
        if (x[i] > max) max = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = vtqo_expf(x[i] - max);
        sum += x[i];
    }
    const float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* embedding_row (src/model/forward_quantized.rs:818-923) */
static int embedding_row(run_t* r, const qt_t* t, int row, int dim, float* out) {
    size_t rb;
    int (*deq)(const uint8_t*, size_t, float*, const char**) = NULL;
    switch (t->dtype) {
    case 0:
        if (t->len < (size_t)(row + 1) * dim * 4) {
            r->msg = "embedding_row F32: table too small for token id";
            return 1;
        }
        memcpy(out, t->w + (size_t)row * dim * 4, (size_t)dim * 4);
        return 0;
    case 2: rb = (size_t)dim / 32 * 18; deq = vtqo_dequantize_q4_0; break;
    case 6: rb = (size_t)dim / 32 * 22; deq = vtqo_dequantize_q5_0; break;
    case 8: rb = (size_t)dim / 32 * 34; deq = vtqo_dequantize_q8_0; break;
    case 12: rb = (size_t)dim / 256 * 144; deq = vtqo_dequantize_q4_k; break;
    case 14: rb = (size_t)dim / 256 * 210; deq = vtqo_dequantize_q6_k; break;
    default:
        r->msg = "embedding_row: non-Q4_0 / Q4_K / Q6_K / Q8_0 / F32 embedding dtype";
        return 1;
    }
    if ((size_t)(row + 1) * rb > t->len) {
        r->msg = "embedding_row: row past end of table";
        return 1;
    }
    return deq(t->w + (size_t)row * rb, rb, out, &r->msg);
}

static int step(run_t* r, uint32_t token, int pos) {
    const vtqo_model* m = r->m;
    const int dim = m->dim, head = dim / m->n_heads, kv_dim = m->n_kv_heads * head;
    const int kv_mul = m->n_heads / m->n_kv_heads, hidden = m->hidden;
    rec_t* rc = r->rec;
    const uint32_t tk = (uint32_t)pos;
    if (embedding_row(r, &m->tok_embd, (int)token, dim, r->x)) return 1;
    rec_act(rc, tk, NO_LAYER, "post_embed", r->x, dim);
    for (int l = 0; l < m->n_layers; l++) {
        const layer_t* L = &m->layers[l];
        const uint8_t(*P)[32] = rc && rc->params ? rc->params[l] : NULL;
        vtqo_rms_norm(r->x, L->rms_att, dim, m->rms_eps, r->xb);
        rec_op(rc, "rms_norm", (uint32_t)l, P ? P[0] : NULL, r->x, dim, r->xb, dim);
        if (linear(r, &L->wq, r->xb, dim, m->n_heads * head, r->q)) return 1;
        rec_op(rc, "linear_q4_0", (uint32_t)l, P ? P[1] : NULL, r->xb, dim, r->q, (size_t)m->n_heads * head);
        if (L->bq) for (int i = 0; i < dim; i++) r->q[i] += L->bq[i];
        if (linear(r, &L->wk, r->xb, dim, kv_dim, r->k)) return 1;
        rec_op(rc, "linear_q4_0", (uint32_t)l, P ? P[2] : NULL, r->xb, dim, r->k, kv_dim);
        if (L->bk) for (int i = 0; i < kv_dim; i++) r->k[i] += L->bk[i];
        if (linear(r, &L->wv, r->xb, dim, kv_dim, r->v)) return 1;
        rec_op(rc, "linear_q4_0", (uint32_t)l, P ? P[3] : NULL, r->xb, dim, r->v, kv_dim);
        if (L->bv) for (int i = 0; i < kv_dim; i++) r->v[i] += L->bv[i];
        const size_t loff = (size_t)l * m->seq_len * kv_dim;
        float* kc = r->key_cache + loff + (size_t)pos * kv_dim;
        memcpy(kc, r->k, (size_t)kv_dim * 4);
        memcpy(r->value_cache + loff + (size_t)pos * kv_dim, r->v, (size_t)kv_dim * 4);
        const float theta = m->rope_theta;
        if (m->rope_neox) {
            const int half = head / 2;
            for (int h = 0; h < m->n_heads; h++)
                for (int j = 0; j < half; j++) {
                    const float freq = 1.0f / vtqo_powf(theta, (float)(2 * j) / (float)head);
                    const float val = (float)pos * freq, fcr = vtqo_cosf(val), fci = vtqo_sinf(val);
                    float* qb = r->q + h * head;
                    const float a = qb[j], b = qb[j + half];
                    qb[j] = a * fcr - b * fci;
                    qb[j + half] = a * fci + b * fcr;
                }
            for (int h = 0; h < kv_dim / head; h++)
                for (int j = 0; j < half; j++) {
                    const float freq = 1.0f / vtqo_powf(theta, (float)(2 * j) / (float)head);
                    const float val = (float)pos * freq, fcr = vtqo_cosf(val), fci = vtqo_sinf(val);
                    float* kb = kc + h * head;
                    const float a = kb[j], b = kb[j + half];
                    kb[j] = a * fcr - b * fci;
                    kb[j + half] = a * fci + b * fcr;
                }
        } else {
            for (int i = 0; i < dim; i += 2) {
                const int hd = i % head;
                const float freq = 1.0f / vtqo_powf(theta, (float)hd / (float)head);
                const float val = (float)pos * freq, fcr = vtqo_cosf(val), fci = vtqo_sinf(val);
                const float q0 = r->q[i], q1 = r->q[i + 1];
                r->q[i] = q0 * fcr - q1 * fci;
                r->q[i + 1] = q0 * fci + q1 * fcr;
                if (i < kv_dim) {
                    const float k0 = kc[i], k1 = kc[i + 1];
                    kc[i] = k0 * fcr - k1 * fci;
                    kc[i + 1] = k0 * fci + k1 * fcr;
                }
            }
        }
        memset(r->xb_out, 0, (size_t)dim * 4);
        const float sq = vtqo_sqrtf((float)head);
        for (int h = 0; h < m->n_heads; h++) {
            const float* qh = r->q + h * head;
            for (int t = 0; t <= pos; t++) {
                const float* kt = r->key_cache + loff + (size_t)t * kv_dim + (size_t)(h / kv_mul) * head;
                float score = 0.0f;
                for (int d = 0; d < head; d++) score += qh[d] * kt[d];
                score /= sq;
                r->att[t] = score;
            }
            vtqo_softmax(r->att, pos + 1);
            float* xo = r->xb_out + h * head;
            for (int t = 0; t <= pos; t++) {
                const float* vt = r->value_cache + loff + (size_t)t * kv_dim + (size_t)(h / kv_mul) * head;
                const float a = r->att[t];
                for (int d = 0; d < head; d++) xo[d] += a * vt[d];
            }
        }
        if (linear(r, &L->wo, r->xb_out, dim, dim, r->xb2)) return 1;
        rec_op(rc, "linear_q4_0", (uint32_t)l, P ? P[4] : NULL, r->xb_out, dim, r->xb2, dim);
        for (int i = 0; i < dim; i++) r->x[i] = r->x[i] + r->xb2[i];
        rec_act(rc, tk, (uint32_t)l, "post_attn", r->x, dim);
        vtqo_rms_norm(r->x, L->rms_ffn, dim, m->rms_eps, r->xb);
        rec_op(rc, "rms_norm", (uint32_t)l, P ? P[5] : NULL, r->x, dim, r->xb, dim);
        if (linear(r, &L->w1, r->xb, dim, hidden, r->gate)) return 1;
        rec_op(rc, "linear_q4_0", (uint32_t)l, P ? P[6] : NULL, r->xb, dim, r->gate, hidden);
        if (linear(r, &L->w3, r->xb, dim, hidden, r->up)) return 1;
        rec_op(rc, "linear_q4_0", (uint32_t)l, P ? P[8] : NULL, r->xb, dim, r->up, hidden);
        for (int i = 0; i < hidden; i++) {
            const float g = r->gate[i];
            const float silu = g / (1.0f + vtqo_expf(-g));
            r->ffn[i] = silu * r->up[i];
        }
        if (linear(r, &L->w2, r->ffn, hidden, dim, r->xb2)) return 1;
        rec_op(rc, "linear_q4_0", (uint32_t)l, P ? P[7] : NULL, r->ffn, hidden, r->xb2, dim);
        for (int i = 0; i < dim; i++) r->x[i] = r->x[i] + r->xb2[i];
        rec_act(rc, tk, (uint32_t)l, "post_ffn", r->x, dim);
    }
    vtqo_rms_norm(r->x, m->rms_final, dim, m->rms_eps, r->xb);
    rec_op(rc, "rms_norm", NO_LAYER, rc ? rc->rms_final : NULL, r->x, dim, r->xb, dim);
    rec_act(rc, tk, NO_LAYER, "pre_lm_head", r->xb, dim);
    if (linear(r, m->shared ? &m->tok_embd : &m->wcls, r->xb, dim, m->vocab, r->logits)) return 1;
    rec_op(rc, "linear_q4_0", NO_LAYER, rc ? (m->shared ? rc->tok : rc->wcls) : NULL, r->xb, dim, r->logits,
           m->vocab);
    rec_act(rc, tk, NO_LAYER, "post_lm_head", r->logits, m->vocab);
    return 0;
}

/* argmax_last_dim (src/ops/argmax.rs:21-68): first maximum, strict > */
uint32_t vtqo_argmax(const float* v, int n) {
    int best = 0;
    float bv = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > bv) {
            bv = v[i];
            best = i;
        }
    return (uint32_t)best;
}

static void le32(uint8_t* o, uint32_t v) {
    o[0] = (uint8_t)v;
    o[1] = (uint8_t)(v >> 8);
    o[2] = (uint8_t)(v >> 16);
    o[3] = (uint8_t)(v >> 24);
}

static int run_impl(const vtqo_model* m, int regime, const char* model_id, const uint8_t weights_hash[32],
                    const uint32_t* prompt, int prompt_len, int n_new, int threads, float* logits, uint32_t* tokens,
                    rec_t* rec, uint8_t digest[32], const char** msg) {
    if (prompt_len == 0) {
        *msg = "prompt_tokens must not be empty";
        return 1;
    }
    const int total = prompt_len + n_new;
    if (total > m->seq_len) {
        *msg = "prompt + n_new_tokens exceeds seq_len";
        return 1;
    }
    const int dim = m->dim, head = dim / m->n_heads, kv_dim = m->n_kv_heads * head;
    run_t r;
    memset(&r, 0, sizeof r);
    r.m = m;
    r.rec = rec;
    r.regime = regime;
    r.threads = threads < 1 ? 1 : threads;
    const size_t kv = (size_t)m->n_layers * m->seq_len * kv_dim;
    r.key_cache = (float*)calloc(kv, 4);
    r.value_cache = (float*)calloc(kv, 4);
    float* buf = (float*)calloc((size_t)6 * dim + 2 * (size_t)kv_dim + (size_t)m->seq_len + 3 * (size_t)m->hidden +
                                    (size_t)m->vocab,
                                4);
    float* p = buf;
    r.x = p; p += dim;
    r.xb = p; p += dim;
    r.q = p; p += dim;
    r.xb_out = p; p += dim;
    r.xb2 = p; p += dim;
    p += dim;
    r.k = p; p += kv_dim;
    r.v = p; p += kv_dim;
    r.att = p; p += m->seq_len;
    r.gate = p; p += m->hidden;
    r.up = p; p += m->hidden;
    r.ffn = p; p += m->hidden;
    r.logits = p;
    int rc = 0, n_gen = 0;
    uint32_t cur = prompt[0];
    for (int pos = 0; pos < total; pos++) {
        if ((rc = step(&r, cur, pos))) break;
        if (logits) memcpy(logits + (size_t)pos * m->vocab, r.logits, (size_t)m->vocab * 4);
        const uint32_t picked = vtqo_argmax(r.logits, m->vocab);
        const uint32_t next = pos + 1 < prompt_len ? prompt[pos + 1] : picked;
        if (pos >= prompt_len) tokens[n_gen++] = next;
        cur = next;
    }
    if (!rc) {
        /* inference.rs:300-312 (inputs) and :329-333 (outputs) */
        char arch[256];
        snprintf(arch, sizeof arch, "llama2c:dim=%d,hidden=%d,layers=%d,heads=%d,kv_heads=%d,vocab=%d,seq=%d,shared=%s",
                 m->dim, m->hidden, m->n_layers, m->n_heads, m->n_kv_heads, m->vocab, m->seq_len,
                 m->shared ? "true" : "false");
        uint8_t arch_hash[32], n_new_le[4], out_hash[32];
        vtqo_blake3_hash(arch, strlen(arch), arch_hash);
        uint8_t* pb = (uint8_t*)malloc((size_t)prompt_len * 4);
        uint8_t* ob = (uint8_t*)malloc((size_t)(n_new > 0 ? n_new : 1) * 4);
        for (int i = 0; i < prompt_len; i++) le32(pb + 4 * i, prompt[i]);
        for (int i = 0; i < n_new; i++) le32(ob + 4 * i, tokens[i]);
        le32(n_new_le, (uint32_t)n_new);
        vtqo_blake3_hash(ob, (size_t)n_new * 4, out_hash);
        const char* in_names[5] = {"model_id", "weights_hash", "arch_hash", "prompt_tokens", "n_new_tokens"};
        const uint8_t* in_data[5] = {(const uint8_t*)model_id, weights_hash, arch_hash, pb, n_new_le};
        const size_t in_lens[5] = {strlen(model_id), 32, 32, (size_t)prompt_len * 4, 4};
        const char* out_names[2] = {"output_tokens", "output_tokens_hash"};
        const uint8_t* out_data[2] = {ob, out_hash};
        const size_t out_lens[2] = {(size_t)n_new * 4, 32};
        if (rec && rec->oom) {
            *msg = "out of memory";
            rc = 1;
        } else {
            vtqo_digest_v2_full(5, in_names, in_data, in_lens, 2, out_names, out_data, out_lens, rec ? rec->n_ops : 0,
                                rec ? rec->ops : NULL, rec ? rec->n_acts : 0, rec ? rec->acts : NULL, digest);
        }
        free(pb);
        free(ob);
    } else {
        *msg = r.msg;
    }
    free(buf);
    free(r.key_cache);
    free(r.value_cache);
    return rc;
}

int vtqo_run_quantized(const vtqo_model* m, int regime, const char* model_id, const uint8_t weights_hash[32],
                       const uint32_t* prompt, int prompt_len, int n_new, int threads, float* logits,
                       uint32_t* tokens, uint8_t digest[32], const char** msg) {
    return run_impl(m, regime, model_id, weights_hash, prompt, prompt_len, n_new, threads, logits, tokens, NULL,
                    digest, msg);
}

/* PerOpRecorder::new (forward_quantized.rs:76-105): every weight hashed once */
static void params_cache(const vtqo_model* m, rec_t* rc) {
    vtqo_blake3_hash(m->tok_embd.w, m->tok_embd.len, rc->tok);
    hash_f32(m->rms_final, (size_t)m->dim, rc->rms_final);
    if (!m->shared) vtqo_blake3_hash(m->wcls.w, m->wcls.len, rc->wcls);
    for (int l = 0; l < m->n_layers; l++) {
        const layer_t* L = &m->layers[l];
        hash_f32(L->rms_att, (size_t)m->dim, rc->params[l][0]);
        vtqo_blake3_hash(L->wq.w, L->wq.len, rc->params[l][1]);
        vtqo_blake3_hash(L->wk.w, L->wk.len, rc->params[l][2]);
        vtqo_blake3_hash(L->wv.w, L->wv.len, rc->params[l][3]);
        vtqo_blake3_hash(L->wo.w, L->wo.len, rc->params[l][4]);
        hash_f32(L->rms_ffn, (size_t)m->dim, rc->params[l][5]);
        vtqo_blake3_hash(L->w1.w, L->w1.len, rc->params[l][6]);
        vtqo_blake3_hash(L->w2.w, L->w2.len, rc->params[l][7]);
        vtqo_blake3_hash(L->w3.w, L->w3.len, rc->params[l][8]);
    }
}

int vtqo_run_quantized_recorded(const vtqo_model* m, int regime, const char* model_id,
                                const uint8_t weights_hash[32], const uint32_t* prompt, int prompt_len, int n_new,
                                int threads, int flags, uint32_t* tokens, vtqo_op_record* ops, size_t ops_cap,
                                vtqo_act_record* acts, size_t acts_cap, size_t* n_ops, size_t* n_acts,
                                uint8_t digest[32], const char** msg) {
    rec_t rc;
    memset(&rc, 0, sizeof rc);
    rc.flags = flags;
    rc.params = (uint8_t(*)[9][32])calloc((size_t)(m->n_layers > 0 ? m->n_layers : 1), sizeof *rc.params);
    if (!rc.params) {
        *msg = "out of memory";
        return 1;
    }
    if (flags & VTQO_RECORD_OPS) params_cache(m, &rc);
    const int err = run_impl(m, regime, model_id, weights_hash, prompt, prompt_len, n_new, threads, NULL, tokens, &rc,
                             digest, msg);
    if (!err) {
        if (n_ops) *n_ops = rc.n_ops;
        if (n_acts) *n_acts = rc.n_acts;
        if (ops) memcpy(ops, rc.ops, (rc.n_ops < ops_cap ? rc.n_ops : ops_cap) * sizeof *ops);
        if (acts) memcpy(acts, rc.acts, (rc.n_acts < acts_cap ? rc.n_acts : acts_cap) * sizeof *acts);
    }
    free(rc.ops);
    free(rc.acts);
    free(rc.params);
    return err;
}
