// vtq_runtime.hip -- libvtq_runtime: the reference's quantized decode,
// device-resident, with every linear on the GPU through libvtq
// (include/vtq_runtime.h).
//
// Restates, in the reference's operation order:
//   GgufFile::parse          src/model/gguf.rs:305-421
//   Config::from_gguf        src/model/config.rs:156-213
//   QuantizedWeights         src/model/quant_weights.rs:121-181
//   forward_quantized::step  src/model/forward_quantized.rs:329-655
//   embedding_row            src/model/forward_quantized.rs:818-923
//   softmax_inplace          src/model/forward_quantized.rs:925-941
//   rms_norm_slice           src/ops/rms_norm.rs:60-110
//   argmax_last_dim          src/ops/argmax.rs:21-68
//   run_quantized            src/model/inference.rs:274-345
//   compute_digest (v2)      src/cert/builder.rs:458-597
// The GGUF blob is uploaded once; the activations, the KV cache, the token
// sequence and the step position live in device memory, so a decode step is
// a fixed sequence of kernel launches (vtq_decode.hip for the non-linear
// parts, libvtq for the linears) that is captured once per run in a HIP graph
// and replayed for every position.  The host only uploads the prompt and
// reads back the generated tokens (and the logits history, when asked for)
// once at the end.  In the integer regime the Q4_K / Q6_K linears of a layer
// are fused: q, k and v in one launch, the residual add into the Wo and W2
// launches, SwiGLU into the W1 / W3 launch.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <array>
#include <map>
#include <string>
#include <thread>
#include <vector>

#include "../../include/vtq.h"
#include "../../include/vtq_runtime.h"
#include "vtq_decode.h"
#include "vtq_kernels.h"

namespace {

// ---------------------------------------------------------------- BLAKE3
// Published BLAKE3: 1024-byte chunks of 64-byte blocks, 7-round compression,
// parent nodes merged as chunks complete, ROOT flag on the last compression.
struct Blake3 {
    static constexpr uint32_t kIV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                                        0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
    enum { kStart = 1, kEnd = 2, kParent = 4, kRoot = 8 };
    uint32_t cv[8];
    uint64_t chunk = 0;
    uint8_t block[64] = {};
    int block_len = 0, blocks = 0;
    uint32_t stack[54][8];
    int depth = 0;

    Blake3() { std::memcpy(cv, kIV, 32); }

    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    static void compress(const uint32_t in_cv[8], const uint8_t blk[64], uint64_t ctr, uint32_t len, uint32_t flags,
                         uint32_t out[16]) {
        static constexpr uint8_t perm[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
        uint32_t m[16], s[16];
        for (int i = 0; i < 16; i++) std::memcpy(&m[i], blk + 4 * i, 4);  // little-endian host
        for (int i = 0; i < 8; i++) s[i] = in_cv[i];
        for (int i = 0; i < 4; i++) s[8 + i] = kIV[i];
        s[12] = (uint32_t)ctr;
        s[13] = (uint32_t)(ctr >> 32);
        s[14] = len;
        s[15] = flags;
        auto g = [&](int a, int b, int c, int d, uint32_t x, uint32_t y) {
            s[a] += s[b] + x;
            s[d] = rotr(s[d] ^ s[a], 16);
            s[c] += s[d];
            s[b] = rotr(s[b] ^ s[c], 12);
            s[a] += s[b] + y;
            s[d] = rotr(s[d] ^ s[a], 8);
            s[c] += s[d];
            s[b] = rotr(s[b] ^ s[c], 7);
        };
        for (int r = 0; r < 7; r++) {
            g(0, 4, 8, 12, m[0], m[1]);
            g(1, 5, 9, 13, m[2], m[3]);
            g(2, 6, 10, 14, m[4], m[5]);
            g(3, 7, 11, 15, m[6], m[7]);
            g(0, 5, 10, 15, m[8], m[9]);
            g(1, 6, 11, 12, m[10], m[11]);
            g(2, 7, 8, 13, m[12], m[13]);
            g(3, 4, 9, 14, m[14], m[15]);
            if (r < 6) {
                uint32_t t[16];
                for (int i = 0; i < 16; i++) t[i] = m[perm[i]];
                std::memcpy(m, t, 64);
            }
        }
        for (int i = 0; i < 8; i++) {
            out[i] = s[i] ^ s[i + 8];
            out[i + 8] = s[i + 8] ^ in_cv[i];
        }
    }
    static void words_to_bytes(const uint32_t* w, uint8_t* b) { std::memcpy(b, w, 32); }
    uint32_t start() const { return blocks == 0 ? kStart : 0; }

    void update(const void* data, size_t len) {
        const uint8_t* p = static_cast<const uint8_t*>(data);
        while (len > 0) {
            if (blocks * 64 + block_len == 1024) {  // full chunk, more input follows
                uint32_t o[16], c[8];
                compress(cv, block, chunk, block_len, start() | kEnd, o);
                std::memcpy(c, o, 32);
                for (uint64_t total = chunk + 1; (total & 1) == 0; total >>= 1) {
                    uint8_t pb[64];
                    words_to_bytes(stack[--depth], pb);
                    words_to_bytes(c, pb + 32);
                    compress(kIV, pb, 0, 64, kParent, o);
                    std::memcpy(c, o, 32);
                }
                std::memcpy(stack[depth++], c, 32);
                std::memcpy(cv, kIV, 32);
                chunk++;
                std::memset(block, 0, 64);
                block_len = blocks = 0;
            }
            if (block_len == 64) {  // full block, more input follows
                uint32_t o[16];
                compress(cv, block, chunk, 64, start(), o);
                std::memcpy(cv, o, 32);
                blocks++;
                std::memset(block, 0, 64);
                block_len = 0;
            }
            const size_t take = std::min<size_t>(64 - block_len, len);
            std::memcpy(block + block_len, p, take);
            block_len += (int)take;
            p += take;
            len -= take;
        }
    }
    void final(uint8_t out[32]) const {
        uint32_t in_cv[8], o[16];
        uint8_t blk[64];
        uint64_t ctr = chunk;
        uint32_t len = block_len, flags = start() | kEnd;
        std::memcpy(in_cv, cv, 32);
        std::memcpy(blk, block, 64);
        for (int i = depth; i > 0; i--) {
            compress(in_cv, blk, ctr, len, flags, o);
            words_to_bytes(stack[i - 1], blk);
            words_to_bytes(o, blk + 32);
            std::memcpy(in_cv, kIV, 32);
            ctr = 0;
            len = 64;
            flags = kParent;
        }
        compress(in_cv, blk, 0, len, flags | kRoot, o);
        words_to_bytes(o, out);
    }
};

void leb128(Blake3& h, uint64_t v) {
    uint8_t b[10];
    int n = 0;
    do {
        uint8_t byte = v & 0x7f;
        v >>= 7;
        if (v) byte |= 0x80;
        b[n++] = byte;
    } while (v);
    h.update(b, (size_t)n);
}

// ---------------------------------------------------------------- GGUF
struct Tensor {
    uint32_t type = 0;
    uint64_t numel = 0;
    size_t offset = 0, nbytes = 0;  // within the blob
};

struct Meta {
    uint32_t type = 0;
    uint64_t num = 0;
    std::string str;
    uint64_t count = 0;  // array length
};

class Reader {
  public:
    Reader(const uint8_t* p, size_t n) : p_(p), n_(n) {}
    bool ok() const { return ok_; }
    size_t pos() const { return pos_; }
    uint64_t uint(int bytes) {
        if (!ok_ || n_ - pos_ < (size_t)bytes) return fail();
        uint64_t v = 0;
        for (int i = 0; i < bytes; i++) v |= (uint64_t)p_[pos_ + i] << (8 * i);
        pos_ += bytes;
        return v;
    }
    std::string str() {
        const uint64_t len = uint(8);
        if (!ok_ || n_ - pos_ < len) {
            fail();
            return {};
        }
        std::string s(reinterpret_cast<const char*>(p_ + pos_), len);
        pos_ += len;
        return s;
    }
    bool value(uint32_t t, Meta* m) {
        static const int kSize[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
        if (t == 8) {
            std::string s = str();
            if (m) m->str = s;
        } else if (t == 9) {
            const uint32_t et = (uint32_t)uint(4);
            const uint64_t n = uint(8);
            if (m) m->count = n;
            for (uint64_t i = 0; i < n && ok_; i++) value(et, nullptr);
        } else if (t < 13) {
            const uint64_t v = uint(kSize[t]);
            if (m) m->num = v;
        } else {
            fail();
        }
        return ok_;
    }

  private:
    uint64_t fail() {
        ok_ = false;
        return 0;
    }
    const uint8_t* p_;
    size_t n_, pos_ = 0;
    bool ok_ = true;
};

bool tensor_bytes(uint32_t type, uint64_t numel, size_t* out) {
    switch (type) {
    case 0: *out = numel * 4; return true;
    case 1: *out = numel * 2; return true;
    case 2: if (numel % 32) return false; *out = numel / 32 * 18; return true;
    case 6: if (numel % 32) return false; *out = numel / 32 * 22; return true;
    case 8: if (numel % 32) return false; *out = numel / 32 * 34; return true;
    case 12: if (numel % 256) return false; *out = numel / 256 * 144; return true;
    case 14: if (numel % 256) return false; *out = numel / 256 * 210; return true;
    }
    return false;
}

// exact f16 -> f32 (src/ops/quant.rs:40-66)
struct Lin {
    int type = 0;
    size_t offset = 0, nbytes = 0;
};

struct Layer {
    size_t rms_att = 0, rms_ffn = 0, bq = 0, bk = 0, bv = 0;  // blob offsets of F32 tensors (0: absent)
    Lin wq, wk, wv, wo, w1, w2, w3;
};

}  // namespace

struct vtqrt_model {
    std::vector<uint8_t> blob;  // host copy (metadata, shapes)
    uint8_t* dblob = nullptr;   // device copy: every tensor is read in place
    vtq_ctx* ctx = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    int device = 0, num_cus = 0;
    int dim = 0, hidden = 0, layers = 0, heads = 0, kv_heads = 0, vocab = 0, seq = 0;
    bool shared = false, neox = false;
    float theta = 10000.0f, eps = 1e-5f;
    Lin tok, wcls;
    size_t rms_final = 0;  // blob offsets of F32 tensors
    std::vector<Layer> L;
    // device state of a run: activations, KV cache, tokens, position
    float *x = nullptr, *xb = nullptr, *qkv = nullptr, *att = nullptr, *ffn = nullptr, *gate = nullptr,
          *up = nullptr, *tmp = nullptr, *logits = nullptr, *kc = nullptr, *vc = nullptr, *hist = nullptr,
          *rope = nullptr;
    size_t hist_cap = 0;
    uint32_t* tokens = nullptr;
    int* pos = nullptr;
    // receipts: one step's recorded tensors (device and pinned host copies),
    // and the weights' hashes (PerOpRecorder's params cache), built once
    float *rec_dev = nullptr, *rec_host = nullptr;
    size_t rec_cap = 0;
    bool params_ready = false;
    std::vector<std::array<uint8_t, 32>> params;  // [layer * 9 + k], k as in RecSlots
    uint8_t tok_hash[32] = {}, rms_final_hash[32] = {}, wcls_hash[32] = {};
};

namespace {

int fail(vtqrt_model* m, int code, const std::string& msg) {
    if (m) m->err = msg;
    return code;
}

int hip_check(vtqrt_model* m, hipError_t e, const char* where) {
    if (e == hipSuccess) return VTQ_OK;
    return fail(m, VTQ_E_GPU, std::string("GpuError: ") + where + ": " + hipGetErrorString(e));
}

const float* f32_at(const vtqrt_model* m, size_t off) {
    return off ? reinterpret_cast<const float*>(m->dblob + off) : nullptr;
}

// y = W x through the C ABI (any type, either regime)
int linear(vtqrt_model* m, int regime, const Lin& w, const float* x, int in_feat, int out_feat, float* y) {
    const int rc = vtq_linear_device(m->ctx, w.type, regime, x, m->dblob + w.offset, w.nbytes, y, 1, (size_t)in_feat,
                                     (size_t)out_feat, m->stream);
    return rc ? fail(m, rc, vtq_last_error(m->ctx)) : VTQ_OK;
}

// rows of the embedding table (embedding_row checks a row against the table's bytes)
uint32_t table_rows(const vtqrt_model* m) {
    const size_t rb = vtq::decode::embed_row_bytes(m->tok.type, m->dim);
    return rb ? (uint32_t)std::min<size_t>(m->tok.nbytes / rb, 0xFFFFFFFFu) : 0u;
}

// The fused integer k-quant GEMV applies when every matrix is Q4_K in the
// integer regime or Q6_K (always integer, linear_dispatch arm Q6_K), and the
// shapes fit the rows kernel.
bool fused_args(const vtqrt_model* m, int regime, int epi, std::initializer_list<const Lin*> ws,
                std::initializer_list<int> rows, size_t norm_off, int in_feat, vtq::RowsArgs* a, int* type) {
    *a = vtq::RowsArgs{{nullptr, nullptr, nullptr}, {0, 0, 0}, f32_at(m, norm_off), m->eps};
    *type = -1;
    int i = 0;
    for (const Lin* w : ws) {
        if ((*type >= 0 && w->type != *type) || !(w->type == 14 || (w->type == 12 && regime == 0))) return false;
        *type = w->type;
        a->w[i++] = m->dblob + w->offset;
    }
    i = 0;
    for (int r : rows) a->rows[i++] = r;
    for (int k = 0; k < 3; k++)
        if (!a->w[k]) a->w[k] = a->w[0];
    return vtq::kquant_fused_supported(*type, in_feat, epi, *a);
}

int launch_fused(vtqrt_model* m, int type, int epi, const float* x, const vtq::RowsArgs& a, int in_feat, float* y) {
    return hip_check(m, vtq::launch_kquant_fused(type, epi, x, a, y, in_feat, m->num_cus, m->stream), "fused linear");
}

// rms_norm(x, w) into xb for linears that do not normalise in their own prologue
int norm_to_xb(vtqrt_model* m, size_t w_off) {
    return hip_check(m, vtq::decode::rms_norm(m->x, f32_at(m, w_off), m->dim, m->eps, m->xb, m->stream), "rms_norm");
}

vtq::decode::RopeArgs rope_args(vtqrt_model* m) {
    return vtq::decode::RopeArgs{m->rope, m->dim / m->heads, m->theta};
}

vtq::decode::EmbedArgs embed_args(vtqrt_model* m) {
    return vtq::decode::EmbedArgs{m->tok.type, m->dblob + m->tok.offset, table_rows(m),
                                  vtq::decode::embed_row_bytes(m->tok.type, m->dim), m->dim, m->x, rope_args(m)};
}

// One decode step at position *m->pos (forward_quantized::step), enqueued
// on m->stream.  x holds the step's embedding row on entry (the previous
// step's argmax kernel, or the run's first embedding, wrote it).
int enqueue_step(vtqrt_model* m, int regime, int prompt_len, int total, float* hist) {
    namespace dec = vtq::decode;
    const int dim = m->dim, head = dim / m->heads, kv_dim = m->kv_heads * head, hidden = m->hidden;
    int rc = VTQ_OK, type;
    vtq::RowsArgs fa;
    for (int l = 0; !rc && l < m->layers; l++) {
        const Layer& Ly = m->L[l];
        // q | k | v = W (rms_norm(x, attn_norm))
        if (fused_args(m, regime, vtq::kEpiStore, {&Ly.wq, &Ly.wk, &Ly.wv}, {dim, kv_dim, kv_dim}, Ly.rms_att, dim, &fa,
                       &type)) {
            rc = launch_fused(m, type, vtq::kEpiStore, m->x, fa, dim, m->qkv);
        } else {
            rc = norm_to_xb(m, Ly.rms_att);
            if (!rc) rc = linear(m, regime, Ly.wq, m->xb, dim, dim, m->qkv);
            if (!rc) rc = linear(m, regime, Ly.wk, m->xb, dim, kv_dim, m->qkv + dim);
            if (!rc) rc = linear(m, regime, Ly.wv, m->xb, dim, kv_dim, m->qkv + dim + kv_dim);
        }
        if (rc) break;
        dec::AttnArgs a;
        a.qkv = m->qkv;
        a.bq = f32_at(m, Ly.bq);
        a.bk = f32_at(m, Ly.bk);
        a.bv = f32_at(m, Ly.bv);
        a.kc = m->kc + (size_t)l * m->seq * kv_dim;
        a.vc = m->vc + (size_t)l * m->seq * kv_dim;
        a.cs = m->rope;
        a.out = m->att;
        a.pos = m->pos;
        a.heads = m->heads;
        a.kv_heads = m->kv_heads;
        a.head_dim = head;
        a.seq = m->seq;
        a.theta = m->theta;
        a.neox = m->neox ? 1 : 0;
        if ((rc = hip_check(m, dec::attention(a, m->stream), "attention"))) break;
        // x = x + Wo att
        if (fused_args(m, regime, vtq::kEpiAccumulate, {&Ly.wo}, {dim}, 0, dim, &fa, &type)) {
            rc = launch_fused(m, type, vtq::kEpiAccumulate, m->att, fa, dim, m->x);
        } else {
            rc = linear(m, regime, Ly.wo, m->att, dim, dim, m->tmp);
            if (!rc) rc = hip_check(m, dec::add_inplace(m->x, m->tmp, dim, m->stream), "residual");
        }
        if (rc) break;
        // ffn = silu(W1 h) * (W3 h), h = rms_norm(x, ffn_norm)
        if (fused_args(m, regime, vtq::kEpiSwiGLU, {&Ly.w1, &Ly.w3}, {hidden, hidden}, Ly.rms_ffn, dim, &fa, &type)) {
            rc = launch_fused(m, type, vtq::kEpiSwiGLU, m->x, fa, dim, m->ffn);
        } else {
            rc = norm_to_xb(m, Ly.rms_ffn);
            if (!rc) rc = linear(m, regime, Ly.w1, m->xb, dim, hidden, m->gate);
            if (!rc) rc = linear(m, regime, Ly.w3, m->xb, dim, hidden, m->up);
            if (!rc) rc = hip_check(m, dec::swiglu(m->gate, m->up, m->ffn, hidden, m->stream), "swiglu");
        }
        if (rc) break;
        // x = x + W2 ffn
        if (fused_args(m, regime, vtq::kEpiAccumulate, {&Ly.w2}, {dim}, 0, hidden, &fa, &type)) {
            rc = launch_fused(m, type, vtq::kEpiAccumulate, m->ffn, fa, hidden, m->x);
        } else {
            rc = linear(m, regime, Ly.w2, m->ffn, hidden, dim, m->tmp);
            if (!rc) rc = hip_check(m, dec::add_inplace(m->x, m->tmp, dim, m->stream), "residual");
        }
    }
    if (rc) return rc;
    // logits = W_out (rms_norm(x, output_norm))
    const Lin& head_w = m->shared ? m->tok : m->wcls;
    if (fused_args(m, regime, vtq::kEpiStore, {&head_w}, {m->vocab}, m->rms_final, dim, &fa, &type)) {
        rc = launch_fused(m, type, vtq::kEpiStore, m->x, fa, dim, m->logits);
    } else {
        rc = norm_to_xb(m, m->rms_final);
        if (!rc) rc = linear(m, regime, head_w, m->xb, dim, m->vocab, m->logits);
    }
    if (rc) return rc;
    return hip_check(m, dec::argmax_advance(m->logits, m->vocab, m->tokens, m->pos, prompt_len, total, hist,
                                            embed_args(m), m->stream),
                     "argmax");
}

// ---- receipts (PerOpRecorder / PerActivationRecorder) ----

// Float offsets of one step's recorded tensors in the record arena: per
// layer the 14 tensors below, then the model-level ones.
struct RecSlots {
    enum { X_IN, XB, Q, K, V, ATT, XB2, POST_ATTN, XB_FFN, GATE, UP, FFN, XB_DOWN, POST_FFN, NL };
    size_t off[NL] = {}, len[NL] = {}, per_layer = 0;
    size_t post_embed = 0, x_pre_final = 0, x_final = 0, logits = 0, total = 0;
    int layers = 0, dim = 0, vocab = 0;
    explicit RecSlots(const vtqrt_model* m) {
        const size_t D = m->dim, Kd = (size_t)m->kv_heads * (m->dim / m->heads), H = m->hidden;
        const size_t lens[NL] = {D, D, D, Kd, Kd, D, D, D, D, H, H, H, D, D};
        size_t o = 0;
        for (int k = 0; k < NL; k++) {
            off[k] = o;
            len[k] = lens[k];
            o += (lens[k] + 3) / 4 * 4;  // 16-byte aligned slots (q|k|v stay contiguous: D, Kd are multiples of 4)
        }
        per_layer = o;
        layers = m->layers;
        dim = m->dim;
        vocab = m->vocab;
        post_embed = (size_t)layers * per_layer;
        x_pre_final = post_embed + (D + 3) / 4 * 4;
        x_final = x_pre_final + (D + 3) / 4 * 4;
        logits = x_final + (D + 3) / 4 * 4;
        total = logits + ((size_t)m->vocab + 3) / 4 * 4;
    }
    size_t at(int l, int k) const { return (size_t)l * per_layer + off[k]; }
};

int dcopy(vtqrt_model* m, float* dst, const float* src, int n) {
    return hip_check(m, hipMemcpyAsync(dst, src, (size_t)n * 4, hipMemcpyDeviceToDevice, m->stream), "record copy");
}

// step_with_recorders: the unfused step with every recorded tensor written
// to (or copied into) the record arena A
int enqueue_step_recorded(vtqrt_model* m, int regime, int prompt_len, int total, float* A) {
    namespace dec = vtq::decode;
    const RecSlots S(m);
    const int dim = m->dim, head = dim / m->heads, kv_dim = m->kv_heads * head, hidden = m->hidden;
    int rc = dcopy(m, A + S.post_embed, m->x, dim);
    for (int l = 0; !rc && l < m->layers; l++) {
        const Layer& Ly = m->L[l];
        float* R[RecSlots::NL];
        for (int k = 0; k < RecSlots::NL; k++) R[k] = A + S.at(l, k);
        if ((rc = dcopy(m, R[RecSlots::X_IN], m->x, dim))) break;
        if ((rc = hip_check(m, dec::rms_norm(m->x, f32_at(m, Ly.rms_att), dim, m->eps, R[RecSlots::XB], m->stream),
                            "rms_norm")))
            break;
        if ((rc = linear(m, regime, Ly.wq, R[RecSlots::XB], dim, dim, R[RecSlots::Q])) ||
            (rc = linear(m, regime, Ly.wk, R[RecSlots::XB], dim, kv_dim, R[RecSlots::K])) ||
            (rc = linear(m, regime, Ly.wv, R[RecSlots::XB], dim, kv_dim, R[RecSlots::V])))
            break;
        dec::AttnArgs a;
        a.qkv = R[RecSlots::Q];
        a.bq = f32_at(m, Ly.bq);
        a.bk = f32_at(m, Ly.bk);
        a.bv = f32_at(m, Ly.bv);
        a.kc = m->kc + (size_t)l * m->seq * kv_dim;
        a.vc = m->vc + (size_t)l * m->seq * kv_dim;
        a.cs = m->rope;
        a.out = R[RecSlots::ATT];
        a.pos = m->pos;
        a.heads = m->heads;
        a.kv_heads = m->kv_heads;
        a.head_dim = head;
        a.seq = m->seq;
        a.theta = m->theta;
        a.neox = m->neox ? 1 : 0;
        if ((rc = hip_check(m, dec::attention(a, m->stream), "attention"))) break;
        if ((rc = linear(m, regime, Ly.wo, R[RecSlots::ATT], dim, dim, R[RecSlots::XB2])) ||
            (rc = hip_check(m, dec::add_inplace(m->x, R[RecSlots::XB2], dim, m->stream), "residual")) ||
            (rc = dcopy(m, R[RecSlots::POST_ATTN], m->x, dim)))
            break;
        if ((rc = hip_check(m, dec::rms_norm(m->x, f32_at(m, Ly.rms_ffn), dim, m->eps, R[RecSlots::XB_FFN], m->stream),
                            "rms_norm")))
            break;
        if ((rc = linear(m, regime, Ly.w1, R[RecSlots::XB_FFN], dim, hidden, R[RecSlots::GATE])) ||
            (rc = linear(m, regime, Ly.w3, R[RecSlots::XB_FFN], dim, hidden, R[RecSlots::UP])) ||
            (rc = hip_check(m, dec::swiglu(R[RecSlots::GATE], R[RecSlots::UP], R[RecSlots::FFN], hidden, m->stream),
                            "swiglu")) ||
            (rc = linear(m, regime, Ly.w2, R[RecSlots::FFN], hidden, dim, R[RecSlots::XB_DOWN])) ||
            (rc = hip_check(m, dec::add_inplace(m->x, R[RecSlots::XB_DOWN], dim, m->stream), "residual")) ||
            (rc = dcopy(m, R[RecSlots::POST_FFN], m->x, dim)))
            break;
    }
    if (rc) return rc;
    const Lin& head_w = m->shared ? m->tok : m->wcls;
    if ((rc = dcopy(m, A + S.x_pre_final, m->x, dim)) ||
        (rc = hip_check(m, dec::rms_norm(m->x, f32_at(m, m->rms_final), dim, m->eps, A + S.x_final, m->stream),
                        "rms_norm")) ||
        (rc = linear(m, regime, head_w, A + S.x_final, dim, m->vocab, A + S.logits)))
        return rc;
    return hip_check(m, dec::argmax_advance(A + S.logits, m->vocab, m->tokens, m->pos, prompt_len, total, nullptr,
                                            embed_args(m), m->stream),
                     "argmax");
}

// fn(i) for i in [0, n) on up to 16 threads (the items are independent)
template <class F>
void parallel_for(int n, F fn) {
    const unsigned hw = std::thread::hardware_concurrency();
    const int t = std::max(1, std::min({n, 16, (int)(hw ? hw : 1)}));
    std::vector<std::thread> th;
    for (int w = 1; w < t; w++)
        th.emplace_back([&, w] {
            for (int i = w; i < n; i += t) fn(i);
        });
    for (int i = 0; i < n; i += t) fn(i);
    for (auto& x : th) x.join();
}

// PerOpRecorder::new (forward_quantized.rs:76-105): BLAKE3 of every weight
// tensor's bytes, hash_f32_slice of every norm
void build_params(vtqrt_model* m) {
    if (m->params_ready) return;
    const uint8_t* b = m->blob.data();
    m->params.assign((size_t)m->layers * 9, {});
    auto lin_hash = [&](const Lin& w, uint8_t* out) { vtqrt_blake3(b + w.offset, w.nbytes, out); };
    auto f32_hash = [&](size_t off, uint8_t* out) { vtqrt_blake3(b + off, (size_t)m->dim * 4, out); };
    parallel_for(m->layers * 9 + 3, [&](int i) {
        if (i == m->layers * 9) return lin_hash(m->tok, m->tok_hash);
        if (i == m->layers * 9 + 1) return f32_hash(m->rms_final, m->rms_final_hash);
        if (i == m->layers * 9 + 2) {
            if (!m->shared) lin_hash(m->wcls, m->wcls_hash);
            return;
        }
        const Layer& Ly = m->L[i / 9];
        uint8_t* o = m->params[i].data();
        switch (i % 9) {
        case 0: return f32_hash(Ly.rms_att, o);
        case 1: return lin_hash(Ly.wq, o);
        case 2: return lin_hash(Ly.wk, o);
        case 3: return lin_hash(Ly.wv, o);
        case 4: return lin_hash(Ly.wo, o);
        case 5: return f32_hash(Ly.rms_ffn, o);
        case 6: return lin_hash(Ly.w1, o);
        case 7: return lin_hash(Ly.w2, o);
        default: return lin_hash(Ly.w3, o);
        }
    });
    m->params_ready = true;
}

struct Recorder {
    int flags = 0;
    std::vector<vtqrt_op_record> ops;
    std::vector<vtqrt_act_record> acts;
};

// hash one step's recorded tensors (host copy H) and append the step's
// records in the reference's declaration order
void record_step(vtqrt_model* m, Recorder& rec, const float* H, uint32_t token) {
    const RecSlots S(m);
    const int NL = RecSlots::NL, L = m->layers;
    const uint32_t kNoLayer = 0xFFFFFFFFu;
    std::vector<std::array<uint8_t, 32>> h((size_t)L * NL + 4);
    parallel_for((int)h.size(), [&](int i) {
        size_t off, n;
        if (i < L * NL) {
            off = S.at(i / NL, i % NL);
            n = S.len[i % NL];
        } else {
            const int j = i - L * NL;
            off = j == 0 ? S.post_embed : j == 1 ? S.x_pre_final : j == 2 ? S.x_final : S.logits;
            n = j == 3 ? (size_t)m->vocab : (size_t)m->dim;
        }
        vtqrt_blake3(H + off, n * 4, h[i].data());
    });
    auto H_ = [&](int l, int k) { return h[(size_t)l * NL + k].data(); };
    const uint8_t *post_embed = h[(size_t)L * NL].data(), *pre_final = h[(size_t)L * NL + 1].data(),
                  *x_final = h[(size_t)L * NL + 2].data(), *logits = h[(size_t)L * NL + 3].data();
    auto op = [&](const char* name, uint32_t layer, const uint8_t* params, const uint8_t* in, const uint8_t* out) {
        if (!(rec.flags & VTQRT_RECORD_OPS)) return;
        vtqrt_op_record r{};
        r.op_index = (uint32_t)rec.ops.size();
        r.layer = layer;
        std::strncpy(r.op_name, name, sizeof r.op_name - 1);
        std::memcpy(r.input_hash, in, 32);
        if (params) std::memcpy(r.params_hash, params, 32);
        std::memcpy(r.output_hash, out, 32);
        rec.ops.push_back(r);
    };
    auto act = [&](uint32_t layer, const char* cp, const uint8_t* t) {
        if (!(rec.flags & VTQRT_RECORD_ACTIVATIONS)) return;
        vtqrt_act_record r{};
        r.act_index = (uint32_t)rec.acts.size();
        r.token_index = token;
        r.layer = layer;
        std::strncpy(r.checkpoint, cp, sizeof r.checkpoint - 1);
        std::memcpy(r.tensor_hash, t, 32);
        rec.acts.push_back(r);
    };
    act(kNoLayer, "post_embed", post_embed);
    for (int l = 0; l < L; l++) {
        const auto P = [&](int k) { return m->params[(size_t)l * 9 + k].data(); };
        using RS = RecSlots;
        op("rms_norm", l, P(0), H_(l, RS::X_IN), H_(l, RS::XB));
        op("linear_q4_0", l, P(1), H_(l, RS::XB), H_(l, RS::Q));
        op("linear_q4_0", l, P(2), H_(l, RS::XB), H_(l, RS::K));
        op("linear_q4_0", l, P(3), H_(l, RS::XB), H_(l, RS::V));
        op("linear_q4_0", l, P(4), H_(l, RS::ATT), H_(l, RS::XB2));
        act(l, "post_attn", H_(l, RS::POST_ATTN));
        op("rms_norm", l, P(5), H_(l, RS::POST_ATTN), H_(l, RS::XB_FFN));
        op("linear_q4_0", l, P(6), H_(l, RS::XB_FFN), H_(l, RS::GATE));
        op("linear_q4_0", l, P(8), H_(l, RS::XB_FFN), H_(l, RS::UP));
        op("linear_q4_0", l, P(7), H_(l, RS::FFN), H_(l, RS::XB_DOWN));
        act(l, "post_ffn", H_(l, RS::POST_FFN));
    }
    op("rms_norm", kNoLayer, m->rms_final_hash, pre_final, x_final);
    act(kNoLayer, "pre_lm_head", x_final);
    op("linear_q4_0", kNoLayer, m->shared ? m->tok_hash : m->wcls_hash, x_final, logits);
    act(kNoLayer, "post_lm_head", logits);
}

const Meta* meta(const std::map<std::string, Meta>& kv, const std::string& k) {
    auto it = kv.find(k);
    return it == kv.end() ? nullptr : &it->second;
}

bool read_usize(const std::map<std::string, Meta>& kv, const std::string& k, int* out) {
    const Meta* v = meta(kv, k);
    if (!v) return false;
    switch (v->type) {
    case 4: case 10: *out = (int)v->num; return true;
    case 5: if ((int32_t)v->num < 0) return false; *out = (int32_t)v->num; return true;
    case 11: if ((int64_t)v->num < 0) return false; *out = (int)(int64_t)v->num; return true;
    }
    return false;
}

float read_f32(const std::map<std::string, Meta>& kv, const std::string& k, float def) {
    const Meta* v = meta(kv, k);
    if (!v || v->type != 6) return def;
    return __builtin_bit_cast(float, (uint32_t)v->num);
}

}  // namespace

extern "C" {

void vtqrt_blake3(const void* data, size_t len, uint8_t out[32]) {
    Blake3 h;
    h.update(data, len);
    h.final(out);
}

const char* vtqrt_last_error(const vtqrt_model* m) { return m ? m->err.c_str() : "null model"; }

int vtqrt_dims(const vtqrt_model* m, int dims[7]) {
    if (!m || !dims) return VTQ_E_INVALID_ARGUMENT;
    const int d[7] = {m->dim, m->hidden, m->layers, m->heads, m->kv_heads, m->vocab, m->seq};
    std::memcpy(dims, d, sizeof d);
    return VTQ_OK;
}

int vtqrt_rms_norm_device(const float* d_x, const float* d_w, size_t n, float eps, float* d_y, void* stream) {
    if (!d_x || !d_w || !d_y) return VTQ_E_INVALID_ARGUMENT;
    if (n < 1 || n > 32768) return VTQ_E_NOT_IMPLEMENTED;
    return vtq::decode::rms_norm(d_x, d_w, (int)n, eps, d_y, static_cast<hipStream_t>(stream)) == hipSuccess
               ? VTQ_OK
               : VTQ_E_GPU;
}

void vtqrt_free(vtqrt_model* m) {
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    for (void* p : {(void*)m->dblob, (void*)m->x, (void*)m->xb, (void*)m->qkv, (void*)m->att, (void*)m->ffn,
                    (void*)m->gate, (void*)m->up, (void*)m->tmp, (void*)m->logits, (void*)m->kc, (void*)m->vc,
                    (void*)m->hist, (void*)m->tokens, (void*)m->pos, (void*)m->rope})
        if (p) (void)hipFree(p);
    if (m->rec_dev) (void)hipFree(m->rec_dev);
    if (m->rec_host) (void)hipHostFree(m->rec_host);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    if (m->ctx) vtq_destroy(m->ctx);
    delete m;
}

int vtqrt_load(int device, const uint8_t* gguf, size_t len, vtqrt_model** out) {
    if (!out || (!gguf && len)) return VTQ_E_INVALID_ARGUMENT;
    *out = nullptr;
    auto* m = new vtqrt_model();
    m->blob.assign(gguf, gguf + len);
    Reader r(m->blob.data(), len);
    if (len < 4 || std::memcmp(gguf, "GGUF", 4)) {
        int rc = fail(m, VTQ_E_INTERNAL, "gguf: bad magic (not 'GGUF')");
        *out = m;
        return rc;
    }
    r.uint(4);
    const uint32_t version = (uint32_t)r.uint(4);
    const uint64_t n_t = r.uint(8), n_kv = r.uint(8);
    std::map<std::string, Meta> kv;
    std::map<std::string, Tensor> ts;
    std::vector<std::pair<std::string, uint64_t>> offsets;
    if (version != 2 && version != 3) {
        *out = m;
        return fail(m, VTQ_E_INTERNAL, "gguf: unsupported version (only v2/v3 supported)");
    }
    for (uint64_t i = 0; i < n_kv && r.ok(); i++) {
        std::string key = r.str();
        Meta v;
        v.type = (uint32_t)r.uint(4);
        if (!r.value(v.type, &v)) break;
        kv[key] = v;
    }
    for (uint64_t i = 0; i < n_t && r.ok(); i++) {
        std::string name = r.str();
        const uint32_t nd = (uint32_t)r.uint(4);
        if (nd > 8) {
            *out = m;
            return fail(m, VTQ_E_INTERNAL, "gguf: tensor rank > 8 (sanity bound)");
        }
        Tensor t;
        t.numel = 1;
        for (uint32_t d = 0; d < nd; d++) t.numel *= r.uint(8);
        t.type = (uint32_t)r.uint(4);
        offsets.emplace_back(name, r.uint(8));
        ts[name] = t;
    }
    if (!r.ok()) {
        *out = m;
        return fail(m, VTQ_E_INTERNAL, "gguf: truncated");
    }
    const Meta* al = meta(kv, "general.alignment");
    const uint64_t align = (al && al->type == 4) ? al->num : 32;
    if (align == 0) {
        *out = m;
        return fail(m, VTQ_E_INTERNAL, "gguf: general.alignment is zero");
    }
    const size_t base = (r.pos() + align - 1) / align * align;
    for (auto& [name, off] : offsets) {
        Tensor& t = ts[name];
        if (!tensor_bytes(t.type, t.numel, &t.nbytes)) {
            *out = m;
            return fail(m, VTQ_E_INTERNAL, "gguf: tensor size not a whole number of blocks");
        }
        t.offset = base + off;
        if (t.offset + t.nbytes > len) {
            *out = m;
            return fail(m, VTQ_E_INTERNAL, "gguf: tensor extends past end of file");
        }
    }
    // Config::from_gguf
    const Meta* a = meta(kv, "general.architecture");
    if (!a || a->type != 8) {
        *out = m;
        return fail(m, VTQ_E_INTERNAL, "gguf: missing 'general.architecture' metadata");
    }
    const std::string arch = a->str;
    bool ok = read_usize(kv, arch + ".embedding_length", &m->dim) &&
              read_usize(kv, arch + ".feed_forward_length", &m->hidden) &&
              read_usize(kv, arch + ".block_count", &m->layers) &&
              read_usize(kv, arch + ".attention.head_count", &m->heads) &&
              read_usize(kv, arch + ".context_length", &m->seq);
    if (ok && !read_usize(kv, arch + ".attention.head_count_kv", &m->kv_heads)) m->kv_heads = m->heads;
    const Meta* toks = meta(kv, "tokenizer.ggml.tokens");
    if (ok) {
        if (toks && toks->type == 9)
            m->vocab = (int)toks->count;
        else
            ok = read_usize(kv, arch + ".vocab_size", &m->vocab);
    }
    if (!ok || m->heads <= 0 || m->kv_heads <= 0 || m->dim % m->heads || m->heads % m->kv_heads) {
        *out = m;
        return fail(m, VTQ_E_INTERNAL, "gguf: numeric metadata missing or wrong type");
    }
    m->theta = read_f32(kv, arch + ".rope.freq_base", 10000.0f);
    m->eps = read_f32(kv, arch + ".attention.layer_norm_rms_epsilon", 1e-5f);
    m->neox = arch == "qwen2";
    m->shared = ts.find("output.weight") == ts.end();
    auto lin = [&](const std::string& n, Lin* o) {
        auto it = ts.find(n);
        if (it == ts.end()) return false;
        o->type = (int)it->second.type;
        o->offset = it->second.offset;
        o->nbytes = it->second.nbytes;
        return true;
    };
    auto f32 = [&](const std::string& n, size_t want, bool required, size_t* o) {
        auto it = ts.find(n);
        if (it == ts.end()) return !required;
        if (it->second.type != 0 || it->second.nbytes != want * 4 || it->second.offset % 4) return false;
        *o = it->second.offset;
        return true;
    };
    const int head = m->dim / m->heads, kv_dim = m->kv_heads * head;
    ok = lin("token_embd.weight", &m->tok) && f32("output_norm.weight", m->dim, true, &m->rms_final);
    if (ok && !m->shared) ok = lin("output.weight", &m->wcls);
    m->L.resize(m->layers);
    for (int l = 0; ok && l < m->layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        Layer& Ly = m->L[l];
        ok = lin(p + "attn_q.weight", &Ly.wq) && lin(p + "attn_k.weight", &Ly.wk) && lin(p + "attn_v.weight", &Ly.wv) &&
             lin(p + "attn_output.weight", &Ly.wo) && lin(p + "ffn_gate.weight", &Ly.w1) &&
             lin(p + "ffn_down.weight", &Ly.w2) && lin(p + "ffn_up.weight", &Ly.w3) &&
             f32(p + "attn_norm.weight", m->dim, true, &Ly.rms_att) &&
             f32(p + "ffn_norm.weight", m->dim, true, &Ly.rms_ffn) && f32(p + "attn_q.bias", m->dim, false, &Ly.bq) &&
             f32(p + "attn_k.bias", kv_dim, false, &Ly.bk) && f32(p + "attn_v.bias", kv_dim, false, &Ly.bv);
    }
    if (!ok) {
        *out = m;
        return fail(m, VTQ_E_INTERNAL, "gguf: required Llama tensor not found");
    }
    int rc = vtq_create(device, &m->ctx);
    if (rc) {
        *out = m;
        return fail(m, rc, m->ctx ? vtq_last_error(m->ctx) : "vtq_create failed");
    }
    if ((rc = hip_check(m, hipSetDevice(device), "hipSetDevice")) ||
        (rc = hip_check(m, hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "hipStreamCreate")) ||
        (rc = hip_check(m, hipMalloc(&m->dblob, (len + 15) / 16 * 16 + 16), "hipMalloc(blob)")) ||
        (rc = hip_check(m, hipMemcpy(m->dblob, m->blob.data(), len, hipMemcpyHostToDevice), "hipMemcpy(blob)"))) {
        *out = m;
        return rc;
    }
    m->device = device;
    if ((rc = hip_check(m, hipDeviceGetAttribute(&m->num_cus, hipDeviceAttributeMultiprocessorCount, device),
                        "hipDeviceGetAttribute"))) {
        *out = m;
        return rc;
    }
    const size_t kv_elems = (size_t)m->layers * m->seq * kv_dim;
    auto dalloc = [&](auto** p, size_t n) {
        return hip_check(m, hipMalloc(reinterpret_cast<void**>(p), std::max<size_t>(n, 1) * 4), "hipMalloc(state)");
    };
    if ((rc = dalloc(&m->x, m->dim)) || (rc = dalloc(&m->xb, m->dim)) || (rc = dalloc(&m->qkv, m->dim + 2 * kv_dim)) ||
        (rc = dalloc(&m->att, m->dim)) || (rc = dalloc(&m->ffn, m->hidden)) || (rc = dalloc(&m->gate, m->hidden)) ||
        (rc = dalloc(&m->up, m->hidden)) || (rc = dalloc(&m->tmp, m->dim)) || (rc = dalloc(&m->logits, m->vocab)) ||
        (rc = dalloc(&m->kc, kv_elems)) || (rc = dalloc(&m->vc, kv_elems)) || (rc = dalloc(&m->tokens, m->seq + 1)) ||
        (rc = dalloc(&m->pos, 1)) || (rc = dalloc(&m->rope, head))) {
        *out = m;
        return rc;
    }
    *out = m;
    return VTQ_OK;
}

}  // extern "C"

namespace {

// run_quantized (inference.rs:274-345), optionally with the step recorders
int run_impl(vtqrt_model* m, int regime, const char* model_id, const uint8_t weights_hash[32], const uint32_t* prompt,
             int prompt_len, int n_new, float* logits, uint32_t* tokens, uint8_t digest[32], Recorder* rec) {
    if (!m || !m->ctx || !model_id || !weights_hash || !digest || (prompt_len > 0 && !prompt) ||
        (n_new > 0 && !tokens) || n_new < 0)
        return VTQ_E_INVALID_ARGUMENT;
    m->err.clear();
    if (prompt_len <= 0) return fail(m, VTQ_E_INTERNAL, "prompt_tokens must not be empty");
    const int total = prompt_len + n_new;
    if (total > m->seq) return fail(m, VTQ_E_INTERNAL, "prompt + n_new_tokens exceeds seq_len");
    if (!vtq::decode::embed_row_bytes(m->tok.type, m->dim))
        return fail(m, VTQ_E_NOT_IMPLEMENTED, "embedding_row: non-Q4_0 / Q4_K / Q6_K / Q8_0 / F32 embedding dtype");
    if ((m->dim / m->heads) % 2)
        return fail(m, VTQ_E_NOT_IMPLEMENTED, "RoPE: odd head dimension");
    const uint32_t rows = table_rows(m);
    for (int i = 0; i < prompt_len; i++)
        if (prompt[i] >= rows) return fail(m, VTQ_E_INTERNAL, "embedding_row: row past end of table");
    int rc = hip_check(m, hipSetDevice(m->device), "hipSetDevice");
    if (rc) return rc;
    if (logits && m->hist_cap < (size_t)total * m->vocab) {
        if (m->hist) (void)hipFree(m->hist);
        m->hist = nullptr;
        m->hist_cap = 0;
        if ((rc = hip_check(m, hipMalloc(&m->hist, (size_t)total * m->vocab * 4), "hipMalloc(logits)"))) return rc;
        m->hist_cap = (size_t)total * m->vocab;
    }
    float* hist = logits ? m->hist : nullptr;
    if (rec) {
        build_params(m);
        const RecSlots S(m);
        if (m->rec_cap < S.total) {
            if (m->rec_dev) (void)hipFree(m->rec_dev);
            if (m->rec_host) (void)hipHostFree(m->rec_host);
            m->rec_dev = m->rec_host = nullptr;
            m->rec_cap = 0;
            if ((rc = hip_check(m, hipMalloc(&m->rec_dev, S.total * 4), "hipMalloc(records)")) ||
                (rc = hip_check(m, hipHostMalloc(&m->rec_host, S.total * 4, hipHostMallocDefault),
                                "hipHostMalloc(records)")))
                return rc;
            m->rec_cap = S.total;
        }
    }
    auto enqueue = [&]() {
        return rec ? enqueue_step_recorded(m, regime, prompt_len, total, m->rec_dev)
                   : enqueue_step(m, regime, prompt_len, total, hist);
    };
    // tokens[0 .. prompt_len) = prompt; step p reads tokens[p] and its argmax
    // writes tokens[p + 1] once p + 1 >= prompt_len
    const int zero = 0;
    if ((rc = hip_check(m, hipMemcpyAsync(m->tokens, prompt, (size_t)prompt_len * 4, hipMemcpyHostToDevice, m->stream),
                        "hipMemcpyAsync(prompt)")) ||
        (rc = hip_check(m, hipMemcpyAsync(m->pos, &zero, 4, hipMemcpyHostToDevice, m->stream), "hipMemcpyAsync(pos)")) ||
        (rc = hip_check(m, hipStreamSynchronize(m->stream), "hipStreamSynchronize")))
        return rc;
    // capture one step and replay it per position; launch eagerly when the
    // graph cannot be built (or VTQRT_EAGER is set)
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    const char* eager_env = std::getenv("VTQRT_EAGER");
    if (!(eager_env && *eager_env && *eager_env != '0') &&
        hipStreamBeginCapture(m->stream, hipStreamCaptureModeRelaxed) == hipSuccess) {
        const int crc = enqueue();
        const hipError_t ce = hipStreamEndCapture(m->stream, &graph);
        if (crc || ce != hipSuccess || !graph || hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
            if (exec) (void)hipGraphExecDestroy(exec);
            exec = nullptr;
            (void)hipGetLastError();
            m->err.clear();
        }
        if (graph) (void)hipGraphDestroy(graph);
    }
    rc = hip_check(m, vtq::decode::embed(m->tok.type, m->dblob + m->tok.offset, table_rows(m), m->tokens, m->pos, m->dim,
                                         m->x, rope_args(m), m->stream),
                   "embedding_row");
    for (int pos = 0; pos < total && !rc; pos++) {
        rc = exec ? hip_check(m, hipGraphLaunch(exec, m->stream), "hipGraphLaunch") : enqueue();
        if (!rc && rec) {
            // this step's recorded tensors to the host, hashed there
            const RecSlots S(m);
            rc = hip_check(m, hipMemcpyAsync(m->rec_host, m->rec_dev, S.total * 4, hipMemcpyDeviceToHost, m->stream),
                           "hipMemcpyAsync(records)");
            if (!rc) rc = hip_check(m, hipStreamSynchronize(m->stream), "hipStreamSynchronize");
            if (!rc) record_step(m, *rec, m->rec_host, (uint32_t)pos);
        }
    }
    if (exec) (void)hipGraphExecDestroy(exec);
    if (rc) {
        (void)hipStreamSynchronize(m->stream);
        return rc;
    }
    // tokens[prompt_len .. total]: fed[i] was consumed by step prompt_len + i
    // (i < n_new); the generated tokens are fed[1 ..] (run_quantized pushes
    // the pick of steps prompt_len .. total-1)
    std::vector<uint32_t> fed((size_t)n_new + 1);
    if (n_new > 0 &&
        (rc = hip_check(m, hipMemcpyAsync(fed.data(), m->tokens + prompt_len, (size_t)(n_new + 1) * 4,
                                          hipMemcpyDeviceToHost, m->stream),
                        "hipMemcpyAsync(tokens)")))
        return rc;
    if (logits && (rc = hip_check(m, hipMemcpyAsync(logits, hist, (size_t)total * m->vocab * 4, hipMemcpyDeviceToHost,
                                                    m->stream),
                                  "hipMemcpyAsync(logits)")))
        return rc;
    if ((rc = hip_check(m, hipStreamSynchronize(m->stream), "hipStreamSynchronize"))) return rc;
    // a picked token that a step consumed must name a table row
    for (int i = 0; i < n_new; i++)
        if (fed[i] >= rows) return fail(m, VTQ_E_INTERNAL, "embedding_row: row past end of table");
    std::vector<uint32_t> gen(fed.begin() + 1, fed.end());
    std::memcpy(tokens, gen.data(), gen.size() * 4);
    // the receipt: inputs then outputs, length-prefixed (inference.rs:300-333)
    char arch[256];
    std::snprintf(arch, sizeof arch, "llama2c:dim=%d,hidden=%d,layers=%d,heads=%d,kv_heads=%d,vocab=%d,seq=%d,shared=%s",
                  m->dim, m->hidden, m->layers, m->heads, m->kv_heads, m->vocab, m->seq, m->shared ? "true" : "false");
    uint8_t arch_hash[32], out_hash[32];
    vtqrt_blake3(arch, std::strlen(arch), arch_hash);
    std::vector<uint8_t> pb((size_t)prompt_len * 4), ob(gen.size() * 4);
    std::memcpy(pb.data(), prompt, pb.size());  // little-endian host: u32::to_le_bytes
    std::memcpy(ob.data(), gen.data(), ob.size());
    vtqrt_blake3(ob.data(), ob.size(), out_hash);
    const uint32_t n_new_u32 = (uint32_t)n_new;
    static const char kRegime[] = "vitni-regime-1";
    Blake3 h;
    h.update("vitnify-receipt v2\x00", 19);
    leb128(h, sizeof kRegime - 1);
    h.update(kRegime, sizeof kRegime - 1);
    auto field = [&](const char* name, const void* data, size_t n) {
        leb128(h, std::strlen(name));
        h.update(name, std::strlen(name));
        leb128(h, n);
        h.update(data, n);
    };
    leb128(h, 5);
    field("model_id", model_id, std::strlen(model_id));
    field("weights_hash", weights_hash, 32);
    field("arch_hash", arch_hash, 32);
    field("prompt_tokens", pb.data(), pb.size());
    field("n_new_tokens", &n_new_u32, 4);
    leb128(h, 2);
    field("output_tokens", ob.data(), ob.size());
    field("output_tokens_hash", out_hash, 32);
    // ops and activations (write_op / write_activation, builder.rs:525-560); no interventions
    const size_t n_ops = rec ? rec->ops.size() : 0, n_acts = rec ? rec->acts.size() : 0;
    leb128(h, n_ops);
    for (size_t i = 0; i < n_ops; i++) {
        const vtqrt_op_record& o = rec->ops[i];
        const size_t nl = std::strlen(o.op_name);
        leb128(h, o.op_index);
        leb128(h, nl);
        h.update(o.op_name, nl);
        leb128(h, o.layer);
        h.update(o.input_hash, 32);
        h.update(o.params_hash, 32);
        h.update(o.output_hash, 32);
    }
    leb128(h, n_acts);
    for (size_t i = 0; i < n_acts; i++) {
        const vtqrt_act_record& a = rec->acts[i];
        const size_t nl = std::strlen(a.checkpoint);
        leb128(h, a.act_index);
        leb128(h, a.token_index);
        leb128(h, a.layer);
        leb128(h, nl);
        h.update(a.checkpoint, nl);
        h.update(a.tensor_hash, 32);
    }
    leb128(h, 0);
    h.final(digest);
    return VTQ_OK;
}

}  // namespace

extern "C" {

int vtqrt_run(vtqrt_model* m, int regime, const char* model_id, const uint8_t weights_hash[32],
              const uint32_t* prompt, int prompt_len, int n_new, float* logits, uint32_t* tokens,
              uint8_t digest[32]) {
    return run_impl(m, regime, model_id, weights_hash, prompt, prompt_len, n_new, logits, tokens, digest, nullptr);
}

int vtqrt_run_recorded(vtqrt_model* m, int regime, const char* model_id, const uint8_t weights_hash[32],
                       const uint32_t* prompt, int prompt_len, int n_new, int flags, uint32_t* tokens,
                       vtqrt_op_record* ops, size_t ops_cap, vtqrt_act_record* acts, size_t acts_cap,
                       size_t* n_ops, size_t* n_acts, uint8_t digest[32]) {
    if (flags & ~(VTQRT_RECORD_OPS | VTQRT_RECORD_ACTIVATIONS)) return VTQ_E_INVALID_ARGUMENT;
    Recorder rec;
    rec.flags = flags;
    const int rc = run_impl(m, regime, model_id, weights_hash, prompt, prompt_len, n_new, nullptr, tokens, digest,
                            &rec);
    if (rc) return rc;
    if (n_ops) *n_ops = rec.ops.size();
    if (n_acts) *n_acts = rec.acts.size();
    if (ops) std::memcpy(ops, rec.ops.data(), std::min(ops_cap, rec.ops.size()) * sizeof *ops);
    if (acts) std::memcpy(acts, rec.acts.data(), std::min(acts_cap, rec.acts.size()) * sizeof *acts);
    return VTQ_OK;
}

}  // extern "C"
