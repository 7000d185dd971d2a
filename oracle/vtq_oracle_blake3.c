/*
 * vtq_oracle_blake3.c -- TEST INFRASTRUCTURE (the checker; never linked into
 * the product).
 *
 * BLAKE3 (crate `blake3 = "1"`, Cargo.toml:28; absent from /root/reference),
 * restated from the published BLAKE3 specification: 1024-byte chunks of
 * 64-byte blocks, 7-round compression, binary tree of parent nodes merged
 * as chunks complete, ROOT flag on the final compression, 32-byte output.
 * The reference hashes receipts with it (src/cert/builder.rs:465-486,
 * src/model/inference.rs:287-288, :330) and the whole GGUF blob
 * (src/bin/vitni-receipt.rs:31).  Pinned by the empty-input test vector,
 * the reference's v2 digest pin (src/cert/builder.rs:719-741) and its
 * transcendental hash (multi-chunk input).
 *
 * Also: the `vitnify-receipt v2` digest framing (src/cert/builder.rs:440-597)
 * and the transcendental sweep of tests/transcendental_determinism.rs.
 */
#include "vtq_oracle_e2e.h"

#include <math.h>
#include <string.h>

enum { CHUNK_START = 1, CHUNK_END = 2, PARENT = 4, ROOT = 8 };
static const uint32_t IV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                               0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
static const uint8_t PERM[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};

static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void g(uint32_t* s, int a, int b, int c, int d, uint32_t mx, uint32_t my) {
    s[a] = s[a] + s[b] + mx;
    s[d] = rotr(s[d] ^ s[a], 16);
    s[c] = s[c] + s[d];
    s[b] = rotr(s[b] ^ s[c], 12);
    s[a] = s[a] + s[b] + my;
    s[d] = rotr(s[d] ^ s[a], 8);
    s[c] = s[c] + s[d];
    s[b] = rotr(s[b] ^ s[c], 7);
}

/* full 16-word output of the compression function */
static void compress(const uint32_t cv[8], const uint8_t block[64], uint64_t counter, uint32_t block_len,
                     uint32_t flags, uint32_t out[16]) {
    uint32_t m[16], s[16], t[16];
    for (int i = 0; i < 16; i++)
        m[i] = (uint32_t)block[4 * i] | ((uint32_t)block[4 * i + 1] << 8) | ((uint32_t)block[4 * i + 2] << 16) |
               ((uint32_t)block[4 * i + 3] << 24);
    for (int i = 0; i < 8; i++) s[i] = cv[i];
    for (int i = 0; i < 4; i++) s[8 + i] = IV[i];
    s[12] = (uint32_t)counter;
    s[13] = (uint32_t)(counter >> 32);
    s[14] = block_len;
    s[15] = flags;
    for (int r = 0; r < 7; r++) {
        g(s, 0, 4, 8, 12, m[0], m[1]);
        g(s, 1, 5, 9, 13, m[2], m[3]);
        g(s, 2, 6, 10, 14, m[4], m[5]);
        g(s, 3, 7, 11, 15, m[6], m[7]);
        g(s, 0, 5, 10, 15, m[8], m[9]);
        g(s, 1, 6, 11, 12, m[10], m[11]);
        g(s, 2, 7, 8, 13, m[12], m[13]);
        g(s, 3, 4, 9, 14, m[14], m[15]);
        if (r < 6) {
            for (int i = 0; i < 16; i++) t[i] = m[PERM[i]];
            memcpy(m, t, sizeof m);
        }
    }
    for (int i = 0; i < 8; i++) {
        out[i] = s[i] ^ s[i + 8];
        out[i + 8] = s[i + 8] ^ cv[i];
    }
}

static void parent_cv(const uint32_t l[8], const uint32_t r[8], uint32_t out_cv[8]) {
    uint8_t block[64];
    for (int i = 0; i < 8; i++)
        for (int b = 0; b < 4; b++) {
            block[4 * i + b] = (uint8_t)(l[i] >> (8 * b));
            block[32 + 4 * i + b] = (uint8_t)(r[i] >> (8 * b));
        }
    uint32_t o[16];
    compress(IV, block, 0, 64, PARENT, o);
    memcpy(out_cv, o, 32);
}

void vtqo_blake3_init(vtqo_blake3* h) {
    memcpy(h->cv, IV, 32);
    h->chunk_counter = 0;
    memset(h->block, 0, 64);
    h->block_len = 0;
    h->blocks_compressed = 0;
    h->cv_stack_len = 0;
}

static size_t chunk_len(const vtqo_blake3* h) { return 64u * h->blocks_compressed + h->block_len; }
static uint32_t start_flag(const vtqo_blake3* h) { return h->blocks_compressed == 0 ? CHUNK_START : 0; }

void vtqo_blake3_update(vtqo_blake3* h, const void* data, size_t len) {
    const uint8_t* p = (const uint8_t*)data;
    while (len > 0) {
        if (chunk_len(h) == 1024) {
            /* the chunk is complete and more input follows: not the root */
            uint32_t o[16], cv[8];
            compress(h->cv, h->block, h->chunk_counter, h->block_len, start_flag(h) | CHUNK_END, o);
            memcpy(cv, o, 32);
            uint64_t total = h->chunk_counter + 1;
            while ((total & 1) == 0) {
                h->cv_stack_len--;
                parent_cv(h->cv_stack[h->cv_stack_len], cv, cv);
                total >>= 1;
            }
            memcpy(h->cv_stack[h->cv_stack_len++], cv, 32);
            memcpy(h->cv, IV, 32);
            h->chunk_counter++;
            memset(h->block, 0, 64);
            h->block_len = 0;
            h->blocks_compressed = 0;
        }
        if (h->block_len == 64) {  /* the block is full and more input follows */
            uint32_t o[16];
            compress(h->cv, h->block, h->chunk_counter, 64, start_flag(h), o);
            memcpy(h->cv, o, 32);
            h->blocks_compressed++;
            memset(h->block, 0, 64);
            h->block_len = 0;
        }
        size_t want = 64 - h->block_len;
        size_t take = want < len ? want : len;
        memcpy(h->block + h->block_len, p, take);
        h->block_len = (uint8_t)(h->block_len + take);
        p += take;
        len -= take;
    }
}

void vtqo_blake3_final(const vtqo_blake3* h, uint8_t out[32]) {
    /* the pending output node: the current chunk's last block */
    uint32_t in_cv[8];
    uint8_t block[64];
    uint64_t counter = h->chunk_counter;
    uint32_t block_len = h->block_len, flags = start_flag(h) | CHUNK_END;
    memcpy(in_cv, h->cv, 32);
    memcpy(block, h->block, 64);
    for (int i = h->cv_stack_len; i > 0; i--) {
        uint32_t o[16], cv[8];
        compress(in_cv, block, counter, block_len, flags, o);
        memcpy(cv, o, 32);
        const uint32_t* l = h->cv_stack[i - 1];
        for (int w = 0; w < 8; w++)
            for (int b = 0; b < 4; b++) {
                block[4 * w + b] = (uint8_t)(l[w] >> (8 * b));
                block[32 + 4 * w + b] = (uint8_t)(cv[w] >> (8 * b));
            }
        memcpy(in_cv, IV, 32);
        counter = 0;
        block_len = 64;
        flags = PARENT;
    }
    uint32_t o[16];
    compress(in_cv, block, 0, block_len, flags | ROOT, o);
    for (int i = 0; i < 8; i++)
        for (int b = 0; b < 4; b++) out[4 * i + b] = (uint8_t)(o[i] >> (8 * b));
}

void vtqo_blake3_hash(const void* data, size_t len, uint8_t out[32]) {
    vtqo_blake3 h;
    vtqo_blake3_init(&h);
    vtqo_blake3_update(&h, data, len);
    vtqo_blake3_final(&h, out);
}

/* ---- vitnify-receipt v2 digest (src/cert/builder.rs:458-471, :489-597) ---- */
static void leb128(vtqo_blake3* h, uint64_t v) {
    uint8_t buf[10];
    int i = 0;
    for (;;) {
        uint8_t byte = (uint8_t)(v & 0x7f);
        v >>= 7;
        if (v != 0) byte |= 0x80;
        buf[i++] = byte;
        if (v == 0) break;
    }
    vtqo_blake3_update(h, buf, (size_t)i);
}

static void field(vtqo_blake3* h, const char* name, const uint8_t* data, size_t len) {
    const size_t nl = strlen(name);
    leb128(h, nl);
    vtqo_blake3_update(h, name, nl);
    leb128(h, len);
    vtqo_blake3_update(h, data, len);
}

/* write_op / write_activation (src/cert/builder.rs:525-560) */
static void write_op(vtqo_blake3* h, const vtqo_op_record* op) {
    const size_t nl = strlen(op->op_name);
    leb128(h, op->op_index);
    leb128(h, nl);
    vtqo_blake3_update(h, op->op_name, nl);
    leb128(h, op->layer);
    vtqo_blake3_update(h, op->input_hash, 32);
    vtqo_blake3_update(h, op->params_hash, 32);
    vtqo_blake3_update(h, op->output_hash, 32);
}

static void write_activation(vtqo_blake3* h, const vtqo_act_record* a) {
    const size_t nl = strlen(a->checkpoint);
    leb128(h, a->act_index);
    leb128(h, a->token_index);
    leb128(h, a->layer);
    leb128(h, nl);
    vtqo_blake3_update(h, a->checkpoint, nl);
    vtqo_blake3_update(h, a->tensor_hash, 32);
}

/* write_sections (builder.rs:491-519): identical in v1 and v2 */
static void sections(vtqo_blake3* h, int n_in, const char* const* in_names, const uint8_t* const* in_data,
                     const size_t* in_lens, int n_out, const char* const* out_names, const uint8_t* const* out_data,
                     const size_t* out_lens, size_t n_ops, const vtqo_op_record* ops, size_t n_acts,
                     const vtqo_act_record* acts) {
    leb128(h, (uint64_t)n_in);
    for (int i = 0; i < n_in; i++) field(h, in_names[i], in_data[i], in_lens[i]);
    leb128(h, (uint64_t)n_out);
    for (int i = 0; i < n_out; i++) field(h, out_names[i], out_data[i], out_lens[i]);
    leb128(h, (uint64_t)n_ops);
    for (size_t i = 0; i < n_ops; i++) write_op(h, &ops[i]);
    leb128(h, (uint64_t)n_acts);
    for (size_t i = 0; i < n_acts; i++) write_activation(h, &acts[i]);
    leb128(h, 0);  /* interventions */
}

void vtqo_digest_v2_full(int n_in, const char* const* in_names, const uint8_t* const* in_data, const size_t* in_lens,
                         int n_out, const char* const* out_names, const uint8_t* const* out_data,
                         const size_t* out_lens, size_t n_ops, const vtqo_op_record* ops, size_t n_acts,
                         const vtqo_act_record* acts, uint8_t out[32]) {
    static const char kRegime[] = "vitni-regime-1";  /* src/cert/builder.rs:440 */
    vtqo_blake3 h;
    vtqo_blake3_init(&h);
    vtqo_blake3_update(&h, "vitnify-receipt v2\x00", 19);
    leb128(&h, sizeof kRegime - 1);
    vtqo_blake3_update(&h, kRegime, sizeof kRegime - 1);
    sections(&h, n_in, in_names, in_data, in_lens, n_out, out_names, out_data, out_lens, n_ops, ops, n_acts, acts);
    vtqo_blake3_final(&h, out);
}

/* compute_digest_v1 (builder.rs:476-487): the frozen domain, no regime */
void vtqo_digest_v1_full(int n_in, const char* const* in_names, const uint8_t* const* in_data, const size_t* in_lens,
                         int n_out, const char* const* out_names, const uint8_t* const* out_data,
                         const size_t* out_lens, size_t n_ops, const vtqo_op_record* ops, size_t n_acts,
                         const vtqo_act_record* acts, uint8_t out[32]) {
    vtqo_blake3 h;
    vtqo_blake3_init(&h);
    vtqo_blake3_update(&h, "vitnify-receipt v1\x00", 19);
    sections(&h, n_in, in_names, in_data, in_lens, n_out, out_names, out_data, out_lens, n_ops, ops, n_acts, acts);
    vtqo_blake3_final(&h, out);
}

void vtqo_digest_v2(int n_in, const char* const* in_names, const uint8_t* const* in_data, const size_t* in_lens,
                    int n_out, const char* const* out_names, const uint8_t* const* out_data,
                    const size_t* out_lens, uint8_t out[32]) {
    vtqo_digest_v2_full(n_in, in_names, in_data, in_lens, n_out, out_names, out_data, out_lens, 0, NULL, 0, NULL,
                        out);
}

/* ---- tests/transcendental_determinism.rs:14-60 ---- */
size_t vtqo_transcendental_hash(uint8_t out[32]) {
    vtqo_blake3 h;
    vtqo_blake3_init(&h);
    size_t count = 0;
    const float corners[] = {0.0f, -0.0f, 1.0f, -1.0f, 0.5f, -0.5f, 1.17549435e-38f, 1e-20f, 1e-10f, 1e10f,
                             1e20f, 87.0f, 88.0f, 88.7f, -87.0f, -88.0f, -104.0f, 3.14159265358979323846f,
                             2.71828182845904523536f};
    float x = -30.0f;
    const size_t n_corner = sizeof corners / sizeof corners[0];
    for (int phase = 0; phase < 2; phase++) {
        size_t idx = 0;
        for (;;) {
            float v;
            if (phase == 0) {
                if (!(x <= 30.0f)) break;
                v = x;
                x += 0.000123f;
            } else {
                if (idx >= n_corner) break;
                v = corners[idx++];
            }
            const float vals[7] = {vtqo_expf(v), vtqo_sqrtf(fabsf(v)), vtqo_cosf(v), vtqo_sinf(v),
                                   vtqo_powf(10000.0f, v / 64.0f), vtqo_powf(1000000.0f, v / 64.0f),
                                   1.0f / (1.0f + vtqo_expf(-v))};
            for (int k = 0; k < 7; k++) {
                uint32_t b;
                memcpy(&b, &vals[k], 4);
                const uint8_t le[4] = {(uint8_t)b, (uint8_t)(b >> 8), (uint8_t)(b >> 16), (uint8_t)(b >> 24)};
                vtqo_blake3_update(&h, le, 4);
            }
            count++;
        }
    }
    vtqo_blake3_final(&h, out);
    return count;
}
