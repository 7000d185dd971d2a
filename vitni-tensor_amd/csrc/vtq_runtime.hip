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
// and replayed for every position past the prompt; the prompt's positions
// run before it as one batched pass (enqueue_prefill), or step by step like
// the rest (vtqrt_set_prompt_mode).  The host only uploads the prompt and
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
#include "vtq_gguf.h"
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

// ---------------------------------------------------------------- model
// A tensor as the step uses it: its bytes in the host copy of the blob (the
// op receipts hash weights there) and its copy in the device arena.  Every
// device copy starts 256-byte aligned, whatever general.alignment the file
// declares.
struct Lin {
    int type = -1;               // -1: absent (optional biases)
    size_t host = 0, nbytes = 0;  // byte range in the host blob
    size_t dev = 0;              // offset in the device arena
};

struct Layer {
    Lin rms_att, rms_ffn, bq, bk, bv, wq, wk, wv, wo, w1, w2, w3;
};

}  // namespace

struct vtqrt_model {
    std::vector<uint8_t> blob;  // host copy (the op receipts hash the weights there)
    uint8_t* dblob = nullptr;   // device arena: one aligned copy of every tensor the step reads
    vtq_ctx* ctx = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    int device = 0, num_cus = 0;
    int dim = 0, hidden = 0, layers = 0, heads = 0, kv_heads = 0, vocab = 0, seq = 0;
    bool shared = false, neox = false;
    float theta = 10000.0f, eps = 1e-5f;
    Lin tok, wcls, rms_final;
    std::vector<Layer> L;
    // device state of a run: activations, KV cache, tokens, position
    float *x = nullptr, *xb = nullptr, *qkv = nullptr, *att = nullptr, *ffn = nullptr, *gate = nullptr,
          *up = nullptr, *tmp = nullptr, *logits = nullptr, *kc = nullptr, *vc = nullptr, *hist = nullptr,
          *rope = nullptr, *att_g = nullptr;  // att_g: score rows of contexts too long for LDS
    size_t hist_cap = 0;
    // the prompt pass (all prompt positions at once): its activations, grown per run
    float* pf = nullptr;
    size_t pf_cap = 0;
    int prompt_mode = VTQRT_PROMPT_BATCHED;
    uint32_t* pf_sink = nullptr;  // the prefetch workgroups' never-taken store
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

const float* f32_at(const vtqrt_model* m, const Lin& t) {
    return t.type >= 0 ? reinterpret_cast<const float*>(m->dblob + t.dev) : nullptr;
}

// y = W x through the C ABI (any type, either regime); `rows` rows of x and y
int linear_rows(vtqrt_model* m, int regime, int type, const uint8_t* w, size_t w_len, const float* x, int rows,
                int in_feat, int out_feat, float* y) {
    const int rc = vtq_linear_device(m->ctx, type, regime, x, w, w_len, y, (size_t)rows, (size_t)in_feat,
                                     (size_t)out_feat, m->stream);
    return rc ? fail(m, rc, vtq_last_error(m->ctx)) : VTQ_OK;
}
int linear(vtqrt_model* m, int regime, const Lin& w, const float* x, int in_feat, int out_feat, float* y) {
    return linear_rows(m, regime, w.type, m->dblob + w.dev, w.nbytes, x, 1, in_feat, out_feat, y);
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
                std::initializer_list<int> rows, const Lin* norm, int in_feat, vtq::RowsArgs* a, int* type) {
    *a = vtq::RowsArgs{{nullptr, nullptr, nullptr}, {0, 0, 0}, norm ? f32_at(m, *norm) : nullptr, m->eps};
    *type = -1;
    int i = 0;
    for (const Lin* w : ws) {
        if ((*type >= 0 && w->type != *type) || !(w->type == 14 || (w->type == 12 && regime == 0))) return false;
        *type = w->type;
        a->w[i++] = m->dblob + w->dev;
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
int norm_to_xb(vtqrt_model* m, const Lin& w) {
    return hip_check(m, vtq::decode::rms_norm(m->x, f32_at(m, w), m->dim, m->eps, m->xb, m->stream), "rms_norm");
}

// the RoPE angle table, one row per position of the cache
vtq::decode::RopeArgs rope_args(vtqrt_model* m) {
    return vtq::decode::RopeArgs{m->rope, m->dim / m->heads, m->theta};
}

vtq::decode::EmbedArgs embed_args(vtqrt_model* m) {
    return vtq::decode::EmbedArgs{m->tok.type, m->dblob + m->tok.dev, table_rows(m),
                                  vtq::decode::embed_row_bytes(m->tok.type, m->dim), m->dim, m->x};
}

// a range for the attention launch's prefetch workgroups; row_bytes nonzero:
// cached rows, of which only 0 .. *pos - 1 are read
void pf_add(vtq::decode::Prefetch& pf, const uint8_t* p, size_t n, uint32_t row_bytes = 0) {
    for (int r = 0; r < vtq::decode::Prefetch::kRanges; r++)
        if (!pf.n[r]) {
            pf.p[r] = p;
            pf.n[r] = (uint32_t)std::min<size_t>(n, (size_t)1 << 31);
            pf.row_bytes[r] = row_bytes;
            return;
        }
}

int enqueue_step(vtqrt_model* m, int regime, int prompt_len, int total, float* hist) {
    namespace dec = vtq::decode;
    const int dim = m->dim, head = dim / m->heads, kv_dim = m->kv_heads * head, hidden = m->hidden;
    int rc = VTQ_OK, type;
    vtq::RowsArgs fa;
    for (int l = 0; !rc && l < m->layers; l++) {
        const Layer& Ly = m->L[l];
        // q | k | v = W (rms_norm(x, attn_norm))
        if (fused_args(m, regime, vtq::kEpiStore, {&Ly.wq, &Ly.wk, &Ly.wv}, {dim, kv_dim, kv_dim}, &Ly.rms_att, dim, &fa,
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
        a.att_g = m->att_g;
        {
            // The attention launch uses one workgroup per head and leaves the
            // other CUs idle: one extra workgroup on each streams what the
            // step reads next (Wo, W1 | W3, the next layer's q | k | v and its
            // cached k and v rows) through the memory-side cache, so the
            // kernels that follow find it there.
            dec::Prefetch& pf = a.pf;
            pf.magic = 0xA5A5A5A5u;
            pf.sink = m->pf_sink;
            pf_add(pf, m->dblob + Ly.wo.dev, Ly.wo.nbytes);
            if (Ly.w3.dev == Ly.w1.dev + Ly.w1.nbytes) {
                pf_add(pf, m->dblob + Ly.w1.dev, Ly.w1.nbytes + Ly.w3.nbytes);
            } else {
                pf_add(pf, m->dblob + Ly.w1.dev, Ly.w1.nbytes);
                pf_add(pf, m->dblob + Ly.w3.dev, Ly.w3.nbytes);
            }
            if (l + 1 < m->layers) {
                const Layer& Ln = m->L[l + 1];
                if (Ln.wk.dev == Ln.wq.dev + Ln.wq.nbytes && Ln.wv.dev == Ln.wk.dev + Ln.wk.nbytes)
                    pf_add(pf, m->dblob + Ln.wq.dev, Ln.wq.nbytes + Ln.wk.nbytes + Ln.wv.nbytes);
                else
                    pf_add(pf, m->dblob + Ln.wq.dev, Ln.wq.nbytes);
                // and the next layer's cached k and v rows 0 .. pos-1, which
                // its attention reads (the row count is read on the device)
                const size_t lay = (size_t)m->seq * kv_dim * 4;
                pf.pos = m->pos;
                pf_add(pf, reinterpret_cast<const uint8_t*>(m->kc) + (size_t)(l + 1) * lay, lay, (uint32_t)kv_dim * 4);
                pf_add(pf, reinterpret_cast<const uint8_t*>(m->vc) + (size_t)(l + 1) * lay, lay, (uint32_t)kv_dim * 4);
            }
            pf.groups = std::max(0, m->num_cus - m->heads);
        }
        if ((rc = hip_check(m, dec::attention(a, m->stream), "attention"))) break;
        // x = x + Wo att
        if (fused_args(m, regime, vtq::kEpiAccumulate, {&Ly.wo}, {dim}, nullptr, dim, &fa, &type)) {
            rc = launch_fused(m, type, vtq::kEpiAccumulate, m->att, fa, dim, m->x);
        } else {
            rc = linear(m, regime, Ly.wo, m->att, dim, dim, m->tmp);
            if (!rc) rc = hip_check(m, dec::add_inplace(m->x, m->tmp, dim, m->stream), "residual");
        }
        if (rc) break;
        // ffn = silu(W1 h) * (W3 h), h = rms_norm(x, ffn_norm)
        if (fused_args(m, regime, vtq::kEpiSwiGLU, {&Ly.w1, &Ly.w3}, {hidden, hidden}, &Ly.rms_ffn, dim, &fa, &type)) {
            rc = launch_fused(m, type, vtq::kEpiSwiGLU, m->x, fa, dim, m->ffn);
        } else {
            rc = norm_to_xb(m, Ly.rms_ffn);
            if (!rc) rc = linear(m, regime, Ly.w1, m->xb, dim, hidden, m->gate);
            if (!rc) rc = linear(m, regime, Ly.w3, m->xb, dim, hidden, m->up);
            if (!rc) rc = hip_check(m, dec::swiglu(m->gate, m->up, m->ffn, hidden, m->stream), "swiglu");
        }
        if (rc) break;
        // x = x + W2 ffn
        if (fused_args(m, regime, vtq::kEpiAccumulate, {&Ly.w2}, {dim}, nullptr, hidden, &fa, &type)) {
            rc = launch_fused(m, type, vtq::kEpiAccumulate, m->ffn, fa, hidden, m->x);
        } else {
            rc = linear(m, regime, Ly.w2, m->ffn, hidden, dim, m->tmp);
            if (!rc) rc = hip_check(m, dec::add_inplace(m->x, m->tmp, dim, m->stream), "residual");
        }
    }
    if (rc) return rc;
    // logits = W_out (rms_norm(x, output_norm))
    const Lin& head_w = m->shared ? m->tok : m->wcls;
    if (fused_args(m, regime, vtq::kEpiStore, {&head_w}, {m->vocab}, &m->rms_final, dim, &fa, &type)) {
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

// The prompt pass: positions 0 .. P-1 of forward_quantized::step at once,
// then step P-1's argmax (which writes tokens[P] and the next step's
// embedding row, and advances *pos to P).  Every linear takes the P rows as
// one batch (the prefill GEMM for Q4_K), and batch rows are independent, so
// each position's activations, cache rows and logits are those of its own
// step: the same kernels' arithmetic per row (RMSNorm per row, the cache
// write and attention of each position as the step computes them for its
// own), in the same order.  Only step P-1's logits feed the run; with hist
// every prompt position's logits are also computed, into hist.
int enqueue_prefill(vtqrt_model* m, int regime, int P, int total, float* hist) {
    namespace dec = vtq::decode;
    const int dim = m->dim, head = dim / m->heads, kv_dim = m->kv_heads * head, hidden = m->hidden;
    const int qw = dim + 2 * kv_dim;
    auto al = [](size_t n) { return (n + 63) / 64 * 64; };
    const size_t Pz = (size_t)P;
    const size_t nX = al(Pz * dim), nQKV = al(Pz * qw), nH = al(Pz * hidden), nK = al(Pz * kv_dim);
    const size_t need = 5 * nX + nQKV + 3 * nH + 2 * nK;
    int rc = VTQ_OK;
    if (m->pf_cap < need) {
        if (m->pf) (void)hipFree(m->pf);
        m->pf = nullptr;
        m->pf_cap = 0;
        if ((rc = hip_check(m, hipMalloc(&m->pf, need * 4), "hipMalloc(prompt pass)"))) return rc;
        m->pf_cap = need;
    }
    float* X = m->pf;
    float* XN = X + nX;
    float* ATT = XN + nX;
    float* TMP = ATT + nX;
    float* QB = TMP + nX;
    float* QKV = QB + nX;
    float* G = QKV + nQKV;
    float* U = G + nH;
    float* F = U + nH;
    float* KB = F + nH;
    float* VB = KB + nK;
    if ((rc = hip_check(m, dec::embed_rows(m->tok.type, m->dblob + m->tok.dev, table_rows(m), m->tokens, P, dim, X,
                                           m->stream),
                        "embedding_row")))
        return rc;
    auto cp_cols = [&](float* dst, const float* src, int width) {
        return hip_check(m, hipMemcpy2DAsync(dst, (size_t)qw * 4, src, (size_t)width * 4, (size_t)width * 4, Pz,
                                             hipMemcpyDeviceToDevice, m->stream),
                         "q|k|v rows");
    };
    // the previous layer's W2 rows, added to x by the next norm (residual)
    const float* pend = nullptr;
    for (int l = 0; !rc && l < m->layers; l++) {
        const Layer& Ly = m->L[l];
        // q | k | v = W (rms_norm(x + residual, attn_norm)), one row per position
        rc = hip_check(m, dec::add_rms_norm_rows(X, pend, f32_at(m, Ly.rms_att), dim, P, m->eps, XN, m->stream),
                       "rms_norm");
        if (rc) break;
        const bool joint = Ly.wk.type == Ly.wq.type && Ly.wv.type == Ly.wq.type &&
                           Ly.wk.dev == Ly.wq.dev + Ly.wq.nbytes && Ly.wv.dev == Ly.wk.dev + Ly.wk.nbytes;
        if (joint) {
            // the three matrices lie back to back in the arena: one linear of dim + 2 kv_dim rows
            rc = linear_rows(m, regime, Ly.wq.type, m->dblob + Ly.wq.dev, Ly.wq.nbytes + Ly.wk.nbytes + Ly.wv.nbytes,
                             XN, P, dim, qw, QKV);
        } else {
            rc = linear_rows(m, regime, Ly.wq.type, m->dblob + Ly.wq.dev, Ly.wq.nbytes, XN, P, dim, dim, QB);
            if (!rc) rc = linear_rows(m, regime, Ly.wk.type, m->dblob + Ly.wk.dev, Ly.wk.nbytes, XN, P, dim, kv_dim, KB);
            if (!rc) rc = linear_rows(m, regime, Ly.wv.type, m->dblob + Ly.wv.dev, Ly.wv.nbytes, XN, P, dim, kv_dim, VB);
            if (!rc) rc = cp_cols(QKV, QB, dim);
            if (!rc) rc = cp_cols(QKV + dim, KB, kv_dim);
            if (!rc) rc = cp_cols(QKV + dim + kv_dim, VB, kv_dim);
        }
        if (rc) break;
        dec::AttnArgs a;
        a.qkv = QKV;
        a.bq = f32_at(m, Ly.bq);
        a.bk = f32_at(m, Ly.bk);
        a.bv = f32_at(m, Ly.bv);
        a.kc = m->kc + (size_t)l * m->seq * kv_dim;
        a.vc = m->vc + (size_t)l * m->seq * kv_dim;
        a.cs = m->rope;
        a.out = ATT;
        a.pos = m->pos;
        a.heads = m->heads;
        a.kv_heads = m->kv_heads;
        a.head_dim = head;
        a.seq = m->seq;
        a.theta = m->theta;
        a.neox = m->neox ? 1 : 0;
        a.att_g = nullptr;
        a.batched = P;
        if ((rc = hip_check(m, dec::rope_cache_rows(a, m->stream), "kv cache")) ||
            (rc = hip_check(m, dec::attention(a, m->stream), "attention")))
            break;
        // x = x + Wo att
        rc = linear_rows(m, regime, Ly.wo.type, m->dblob + Ly.wo.dev, Ly.wo.nbytes, ATT, P, dim, dim, TMP);
        // ffn = silu(W1 h) * (W3 h), h = rms_norm(x, ffn_norm), with the residual
        if (!rc)
            rc = hip_check(m, dec::add_rms_norm_rows(X, TMP, f32_at(m, Ly.rms_ffn), dim, P, m->eps, XN, m->stream),
                           "rms_norm");
        if (!rc && Ly.w3.type == Ly.w1.type && Ly.w3.dev == Ly.w1.dev + Ly.w1.nbytes) {
            // gate | up rows from one linear of 2 * hidden rows (G and U back to back)
            rc = linear_rows(m, regime, Ly.w1.type, m->dblob + Ly.w1.dev, Ly.w1.nbytes + Ly.w3.nbytes, XN, P, dim,
                             2 * hidden, G);
            if (!rc) rc = hip_check(m, dec::swiglu_rows(G, hidden, P, F, m->stream), "swiglu");
        } else if (!rc) {
            rc = linear_rows(m, regime, Ly.w1.type, m->dblob + Ly.w1.dev, Ly.w1.nbytes, XN, P, dim, hidden, G);
            if (!rc) rc = linear_rows(m, regime, Ly.w3.type, m->dblob + Ly.w3.dev, Ly.w3.nbytes, XN, P, dim, hidden, U);
            if (!rc) rc = hip_check(m, dec::swiglu(G, U, F, P * hidden, m->stream), "swiglu");
        }
        // x = x + W2 ffn
        // (the residual add is the next norm's: the next layer's or the final one)
        if (!rc) rc = linear_rows(m, regime, Ly.w2.type, m->dblob + Ly.w2.dev, Ly.w2.nbytes, F, P, hidden, dim, TMP);
        pend = TMP;
    }
    if (rc) return rc;
    // logits = W_out (rms_norm(x, output_norm)): every position's into hist,
    // or position P-1's alone
    const Lin& head_w = m->shared ? m->tok : m->wcls;
    const float* lg = m->logits;
    if (hist) {
        rc = hip_check(m, dec::add_rms_norm_rows(X, pend, f32_at(m, m->rms_final), dim, P, m->eps, XN, m->stream),
                       "rms_norm");
        if (!rc) rc = linear_rows(m, regime, head_w.type, m->dblob + head_w.dev, head_w.nbytes, XN, P, dim, m->vocab, hist);
        lg = hist + (size_t)(P - 1) * m->vocab;
    } else {
        // position P-1's row alone (the other rows' last residual is not needed)
        const size_t r = (size_t)(P - 1) * dim;
        rc = hip_check(m, dec::add_rms_norm_rows(X + r, pend ? pend + r : nullptr, f32_at(m, m->rms_final), dim, 1,
                                                 m->eps, m->xb, m->stream),
                       "rms_norm");
        if (!rc) rc = linear(m, regime, head_w, m->xb, dim, m->vocab, m->logits);
    }
    if (rc) return rc;
    // step P-1's argmax: tokens[P], the next step's row, *pos = P
    if ((rc = hip_check(m, hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(m->pos), P - 1, 1, m->stream),
                        "position")))
        return rc;
    return hip_check(m, dec::argmax_advance(lg, m->vocab, m->tokens, m->pos, P, total, hist, embed_args(m), m->stream),
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
        a.att_g = m->att_g;
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
    // hash_f32_slice of a norm is BLAKE3 of its little-endian bytes: the same bytes
    auto lin_hash = [&](const Lin& w, uint8_t* out) { vtqrt_blake3(b + w.host, w.nbytes, out); };
    auto f32_hash = lin_hash;
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

int vtqrt_transcendentals_device(const float* d_x, size_t n, float* d_y, void* stream) {
    if (n && (!d_x || !d_y)) return VTQ_E_INVALID_ARGUMENT;
    if (n > (size_t)INT32_MAX / 7) return VTQ_E_NOT_IMPLEMENTED;
    return vtq::decode::transcendentals(d_x, (int)n, d_y, static_cast<hipStream_t>(stream)) == hipSuccess
               ? VTQ_OK
               : VTQ_E_GPU;
}

void vtqrt_free(vtqrt_model* m) {
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    for (void* p : {(void*)m->dblob, (void*)m->x, (void*)m->xb, (void*)m->qkv, (void*)m->att, (void*)m->ffn,
                    (void*)m->gate, (void*)m->up, (void*)m->tmp, (void*)m->logits, (void*)m->kc, (void*)m->vc,
                    (void*)m->hist, (void*)m->tokens, (void*)m->pos, (void*)m->rope, (void*)m->att_g,
                    (void*)m->pf, (void*)m->pf_sink})
        if (p) (void)hipFree(p);
    if (m->rec_dev) (void)hipFree(m->rec_dev);
    if (m->rec_host) (void)hipHostFree(m->rec_host);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    if (m->ctx) vtq_destroy(m->ctx);
    delete m;
}

int vtqrt_parse(const uint8_t* gguf, size_t len, int level, int dims[7], char* err, size_t err_cap) {
    if ((!gguf && len) || level < 0 || level > 1) return VTQ_E_INVALID_ARGUMENT;
    static const uint8_t kEmpty[1] = {0};
    vtq::gguf::File f;
    vtq::gguf::Model md;
    const char* msg = "";
    int rc = vtq::gguf::parse(gguf ? gguf : kEmpty, len, &f, &msg);
    if (!rc && level == 1) rc = vtq::gguf::describe(f, &md, &msg);
    if (!rc && level == 1 && dims) {
        const int d[7] = {md.dim, md.hidden, md.layers, md.heads, md.kv_heads, md.vocab, md.seq};
        std::memcpy(dims, d, sizeof d);
    }
    if (err && err_cap) {
        std::strncpy(err, msg, err_cap - 1);
        err[err_cap - 1] = 0;
    }
    return rc;
}

int vtqrt_load(int device, const uint8_t* gguf, size_t len, vtqrt_model** out) {
    if (!out || (!gguf && len)) return VTQ_E_INVALID_ARGUMENT;
    *out = nullptr;
    auto* m = new (std::nothrow) vtqrt_model();
    if (!m) return VTQ_E_GPU;
    *out = m;
    // GgufFile::parse, Config::from_gguf and QuantizedWeights::from_gguf on
    // the host: a file that fails any check never reaches the device
    static const uint8_t kEmpty[1] = {0};
    vtq::gguf::File f;
    vtq::gguf::Model md;
    const char* msg = "";
    int rc = vtq::gguf::parse(gguf ? gguf : kEmpty, len, &f, &msg);
    if (!rc) rc = vtq::gguf::describe(f, &md, &msg);
    if (rc) return fail(m, rc, msg);
    m->dim = md.dim;
    m->hidden = md.hidden;
    m->layers = md.layers;
    m->heads = md.heads;
    m->kv_heads = md.kv_heads;
    m->vocab = md.vocab;
    m->seq = md.seq;
    m->shared = md.shared;
    m->neox = md.neox;
    m->theta = md.theta;
    m->eps = md.eps;
    const int head = m->dim / m->heads, kv_dim = m->kv_heads * head;

    // device arena: every tensor the step reads, each copy 256-byte aligned;
    // a bias is stored at the length it is added to, past its own end padded
    // with -0.0 (add_bias zips the two slices, and v + -0.0 == v bit for bit)
    size_t arena = 0;
    auto place = [&](const vtq::gguf::View& v, size_t dev_bytes, Lin* o) {
        if (v.type < 0) return;
        o->type = v.type;
        o->host = (size_t)v.offset;
        o->nbytes = (size_t)v.nbytes;
        o->dev = arena;
        arena += (std::max<size_t>(dev_bytes, 1) + 255) / 256 * 256;
    };
    auto place_t = [&](const vtq::gguf::View& v, Lin* o) { place(v, (size_t)v.nbytes, o); };
    place_t(md.tok, &m->tok);
    place_t(md.rms_final, &m->rms_final);
    if (!m->shared) place_t(md.wcls, &m->wcls);
    m->L.resize((size_t)m->layers);
    for (int l = 0; l < m->layers; l++) {
        const vtq::gguf::LayerViews& V = md.L[(size_t)l];
        Layer& Ly = m->L[(size_t)l];
        place_t(V.rms_att, &Ly.rms_att);
        place_t(V.rms_ffn, &Ly.rms_ffn);
        place_t(V.wq, &Ly.wq);
        place_t(V.wk, &Ly.wk);
        place_t(V.wv, &Ly.wv);
        place_t(V.wo, &Ly.wo);
        // w1 then w3: back to back, the prompt pass runs them as one linear
        place_t(V.w1, &Ly.w1);
        place_t(V.w3, &Ly.w3);
        place_t(V.w2, &Ly.w2);
        place(V.bq, (size_t)m->dim * 4, &Ly.bq);
        place(V.bk, (size_t)kv_dim * 4, &Ly.bk);
        place(V.bv, (size_t)kv_dim * 4, &Ly.bv);
    }
    arena += 256;  // the kernels fetch whole 16-byte chunks past a tensor's end

    m->blob.assign(gguf, gguf + len);
    if ((rc = vtq_create(device, &m->ctx))) return fail(m, rc, "vtq_create failed");
    if ((rc = hip_check(m, hipSetDevice(device), "hipSetDevice")) ||
        (rc = hip_check(m, hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "hipStreamCreate")) ||
        (rc = hip_check(m, hipMalloc(&m->dblob, arena), "hipMalloc(weights)")))
        return rc;
    m->device = device;
    std::vector<float> pad;
    auto upload = [&](const Lin& t, size_t dev_floats) {
        if (t.type < 0) return VTQ_OK;
        if (!dev_floats)
            return hip_check(m, hipMemcpy(m->dblob + t.dev, m->blob.data() + t.host, t.nbytes, hipMemcpyHostToDevice),
                             "hipMemcpy(weights)");
        pad.assign(dev_floats, -0.0f);
        std::memcpy(pad.data(), m->blob.data() + t.host, std::min(t.nbytes, dev_floats * 4));
        return hip_check(m, hipMemcpy(m->dblob + t.dev, pad.data(), dev_floats * 4, hipMemcpyHostToDevice),
                         "hipMemcpy(bias)");
    };
    if ((rc = upload(m->tok, 0)) || (rc = upload(m->rms_final, 0)) || (rc = upload(m->wcls, 0))) return rc;
    for (const Layer& Ly : m->L) {
        for (const Lin* t : {&Ly.rms_att, &Ly.rms_ffn, &Ly.wq, &Ly.wk, &Ly.wv, &Ly.wo, &Ly.w1, &Ly.w2, &Ly.w3})
            if ((rc = upload(*t, 0))) return rc;
        if ((rc = upload(Ly.bq, (size_t)m->dim)) || (rc = upload(Ly.bk, (size_t)kv_dim)) ||
            (rc = upload(Ly.bv, (size_t)kv_dim)))
            return rc;
    }
    if ((rc = hip_check(m, hipDeviceGetAttribute(&m->num_cus, hipDeviceAttributeMultiprocessorCount, device),
                        "hipDeviceGetAttribute")))
        return rc;
    // RunState::new (forward.rs:28-34): k and v caches of layers * seq * kv_dim
    size_t kv_elems = 0;
    if (__builtin_mul_overflow((size_t)m->layers, (size_t)m->seq, &kv_elems) ||
        __builtin_mul_overflow(kv_elems, (size_t)kv_dim, &kv_elems) || kv_elems > ((size_t)1 << 60))
        return fail(m, VTQ_E_NOT_IMPLEMENTED, "vtq: KV cache size overflows");
    auto dalloc = [&](auto** p, size_t n) {
        return hip_check(m, hipMalloc(reinterpret_cast<void**>(p), std::max<size_t>(n, 1) * 4), "hipMalloc(state)");
    };
    if ((rc = dalloc(&m->x, m->dim)) || (rc = dalloc(&m->xb, m->dim)) ||
        (rc = dalloc(&m->qkv, (size_t)m->dim + 2 * (size_t)kv_dim)) ||
        (rc = dalloc(&m->att, m->dim)) || (rc = dalloc(&m->ffn, m->hidden)) || (rc = dalloc(&m->gate, m->hidden)) ||
        (rc = dalloc(&m->up, m->hidden)) || (rc = dalloc(&m->tmp, m->dim)) || (rc = dalloc(&m->logits, m->vocab)) ||
        (rc = dalloc(&m->kc, kv_elems)) || (rc = dalloc(&m->vc, kv_elems)) ||
        (rc = dalloc(&m->tokens, (size_t)m->seq + 1)) || (rc = dalloc(&m->pos, 1)) ||
        (rc = dalloc(&m->rope, (size_t)m->seq * (size_t)std::max(head, 1))) ||
        (rc = dalloc(&m->pf_sink, 64)))
        return rc;
    // the RoPE angles of every position, once (rope_table)
    if (head > 0 && (rc = hip_check(m, vtq::decode::rope_table_rows(rope_args(m), m->seq, m->stream), "rope table")))
        return rc;
    // a context too long for the attention kernel's LDS keeps each head's
    // scores in a row of HBM
    if (head > 0 && m->dim % m->heads == 0 && !vtq::decode::attention_scores_in_lds(head, m->seq) &&
        (rc = dalloc(&m->att_g, (size_t)m->heads * (((size_t)m->seq + 3) & ~(size_t)3))))
        return rc;
    return VTQ_OK;
}

}  // extern "C"

namespace {

// embedding_row's checks (forward_quantized.rs:818-919) for one token id
int embed_check(vtqrt_model* m, uint32_t token) {
    struct Fmt {
        int type;
        uint64_t elems, bytes;
        const char *dim_msg, *row_msg;
    };
    static const Fmt kFmt[] = {
        {2, 32, 18, "embedding_row Q4_0: dim must be a multiple of 32", "embedding_row Q4_0: row past end of table"},
        {12, 256, 144, "embedding_row Q4_K: dim must be a multiple of 256", "embedding_row Q4_K: row past end of table"},
        {14, 256, 210, "embedding_row Q6_K: dim must be a multiple of 256", "embedding_row Q6_K: row past end of table"},
        {6, 32, 22, "embedding_row Q5_0: dim must be a multiple of 32", "embedding_row Q5_0: row past end of table"},
        {8, 32, 34, "embedding_row Q8_0: dim must be a multiple of 32", "embedding_row Q8_0: row past end of table"},
    };
    // (row + 1) * row_bytes: below 2^33 * 2^33, so 128-bit arithmetic cannot wrap
    const unsigned __int128 row = token, dim = (uint64_t)m->dim, len = m->tok.nbytes;
    if (m->tok.type == 0)
        return (row + 1) * dim * 4 > len ? fail(m, VTQ_E_INTERNAL, "embedding_row F32: table too small for token id")
                                         : VTQ_OK;
    for (const Fmt& f : kFmt) {
        if (f.type != m->tok.type) continue;
        if (dim % f.elems) return fail(m, VTQ_E_INTERNAL, f.dim_msg);
        const unsigned __int128 row_bytes = dim / f.elems * f.bytes;
        return (row + 1) * row_bytes > len ? fail(m, VTQ_E_INTERNAL, f.row_msg) : VTQ_OK;
    }
    return fail(m, VTQ_E_NOT_IMPLEMENTED, "embedding_row: non-Q4_0 / Q4_K / Q6_K / Q8_0 / F32 embedding dtype");
}

// The checks one step makes before its arithmetic, in the step's order:
// rms_norm_slice's weight length (rms_norm.rs:80-85) and every
// linear_dispatch arm's shape checks (vtq_linear_device validates and, with
// batch 0, launches nothing).  Passing them is what makes the fused GEMVs'
// row counts safe to launch.
int step_check(vtqrt_model* m, int regime) {
    const int dim = m->dim, kv_dim = m->kv_heads * (m->dim / m->heads), hidden = m->hidden;
    auto norm = [&](const Lin& w) {
        return w.nbytes / 4 != (size_t)dim
                   ? fail(m, VTQ_E_SHAPE_MISMATCH, "expected weight length == last dim of x, got weight mismatch")
                   : VTQ_OK;
    };
    auto lin = [&](const Lin& w, int in_feat, int out_feat) {
        const int rc = vtq_linear_device(m->ctx, w.type, regime, nullptr, m->dblob + w.dev, w.nbytes, nullptr, 0,
                                         (size_t)in_feat, (size_t)out_feat, m->stream);
        return rc ? fail(m, rc, vtq_last_error(m->ctx)) : VTQ_OK;
    };
    int rc = VTQ_OK;
    for (const Layer& Ly : m->L) {
        if ((rc = norm(Ly.rms_att)) || (rc = lin(Ly.wq, dim, dim)) || (rc = lin(Ly.wk, dim, kv_dim)) ||
            (rc = lin(Ly.wv, dim, kv_dim)) || (rc = lin(Ly.wo, dim, dim)) || (rc = norm(Ly.rms_ffn)) ||
            (rc = lin(Ly.w1, dim, hidden)) || (rc = lin(Ly.w3, dim, hidden)) || (rc = lin(Ly.w2, hidden, dim)))
            return rc;
    }
    if ((rc = norm(m->rms_final))) return rc;
    return lin(m->shared ? m->tok : m->wcls, dim, m->vocab);
}

// run_quantized (inference.rs:274-345), optionally with the step recorders
int run_impl(vtqrt_model* m, int regime, const char* model_id, const uint8_t weights_hash[32], const uint32_t* prompt,
             int prompt_len, int n_new, float* logits, uint32_t* tokens, uint8_t digest[32], uint8_t* digest_v1,
             Recorder* rec) {
    if (!m || !m->ctx || !model_id || !weights_hash || !digest || (prompt_len > 0 && !prompt) ||
        (n_new > 0 && !tokens) || n_new < 0)
        return VTQ_E_INVALID_ARGUMENT;
    m->err.clear();
    // run_quantized_with_sink's checks (inference.rs:301-311), in usize there
    if (prompt_len <= 0) return fail(m, VTQ_E_INVALID_SHAPE, "prompt_tokens must not be empty");
    const int64_t total64 = (int64_t)prompt_len + (int64_t)n_new;
    if (total64 > (int64_t)m->seq) return fail(m, VTQ_E_INVALID_SHAPE, "prompt + n_new_tokens exceeds seq_len");
    const int total = (int)total64;
    // step 0 reports what any step would (embedding_row, then the step's
    // norms and linears in order); later prompt tokens fail at their own step
    int rc = embed_check(m, prompt[0]);
    if (!rc) rc = step_check(m, regime);
    for (int i = 1; !rc && i < prompt_len; i++) rc = embed_check(m, prompt[i]);
    if (rc) return rc;
    const int head = m->dim / m->heads;
    if (head % 2) return fail(m, VTQ_E_NOT_IMPLEMENTED, "vtq: odd head dimension (RoPE pairs)");
    if (!vtq::decode::attention_supported(head, m->seq))
        return fail(m, VTQ_E_NOT_IMPLEMENTED, "vtq: head dimension beyond the attention kernel");
    if (m->dim > 32768) return fail(m, VTQ_E_NOT_IMPLEMENTED, "vtq: model dimension above 32768 (rms_norm)");
    const uint32_t rows = table_rows(m);
    if ((rc = hip_check(m, hipSetDevice(m->device), "hipSetDevice"))) return rc;
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
    // the prompt at once where the recorders are off and its attention fits
    // the prompt-pass kernel; else step by step from position 0
    const bool batched = !rec && m->prompt_mode == VTQRT_PROMPT_BATCHED && prompt_len >= 2 &&
                         vtq::decode::attention_rows_supported(head, prompt_len, m->heads, m->kv_heads);
    int pos0 = 0;
    if (batched) {
        rc = enqueue_prefill(m, regime, prompt_len, total, hist);
        pos0 = prompt_len;
    } else {
        rc = hip_check(m, vtq::decode::embed(m->tok.type, m->dblob + m->tok.dev, table_rows(m), m->tokens, m->pos,
                                             m->dim, m->x, m->stream),
                       "embedding_row");
    }
    for (int pos = pos0; pos < total && !rc; pos++) {
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
        if (fed[i] >= rows) return embed_check(m, fed[i]);
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
    // write_sections (builder.rs:491-519): the part v1 and v2 share
    auto sections = [&](Blake3& h) {
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
    };
    // compute_digest (v2, builder.rs:458-471): the domain, then REGIME length-prefixed
    static const char kRegime[] = "vitni-regime-1";
    Blake3 h;
    h.update("vitnify-receipt v2\x00", 19);
    leb128(h, sizeof kRegime - 1);
    h.update(kRegime, sizeof kRegime - 1);
    sections(h);
    h.final(digest);
    // compute_digest_v1 (builder.rs:476-487): the frozen domain, no regime
    if (digest_v1) {
        Blake3 h1;
        h1.update("vitnify-receipt v1\x00", 19);
        sections(h1);
        h1.final(digest_v1);
    }
    return VTQ_OK;
}

}  // namespace

extern "C" {

int vtqrt_run(vtqrt_model* m, int regime, const char* model_id, const uint8_t weights_hash[32],
              const uint32_t* prompt, int prompt_len, int n_new, float* logits, uint32_t* tokens,
              uint8_t digest[32], uint8_t digest_v1[32]) {
    return run_impl(m, regime, model_id, weights_hash, prompt, prompt_len, n_new, logits, tokens, digest, digest_v1,
                    nullptr);
}

int vtqrt_set_prompt_mode(vtqrt_model* m, int mode) {
    if (!m || (mode != VTQRT_PROMPT_BATCHED && mode != VTQRT_PROMPT_STEPWISE)) return VTQ_E_INVALID_ARGUMENT;
    m->prompt_mode = mode;
    return VTQ_OK;
}

int vtqrt_run_recorded(vtqrt_model* m, int regime, const char* model_id, const uint8_t weights_hash[32],
                       const uint32_t* prompt, int prompt_len, int n_new, int flags, uint32_t* tokens,
                       vtqrt_op_record* ops, size_t ops_cap, vtqrt_act_record* acts, size_t acts_cap,
                       size_t* n_ops, size_t* n_acts, uint8_t digest[32]) {
    if (flags & ~(VTQRT_RECORD_OPS | VTQRT_RECORD_ACTIVATIONS)) return VTQ_E_INVALID_ARGUMENT;
    Recorder rec;
    rec.flags = flags;
    const int rc = run_impl(m, regime, model_id, weights_hash, prompt, prompt_len, n_new, nullptr, tokens, digest,
                            nullptr, &rec);
    if (rc) return rc;
    if (n_ops) *n_ops = rec.ops.size();
    if (n_acts) *n_acts = rec.acts.size();
    if (ops) std::memcpy(ops, rec.ops.data(), std::min(ops_cap, rec.ops.size()) * sizeof *ops);
    if (acts) std::memcpy(acts, rec.acts.data(), std::min(acts_cap, rec.acts.size()) * sizeof *acts);
    return VTQ_OK;
}

}  // extern "C"
