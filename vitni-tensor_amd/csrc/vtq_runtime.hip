// vtq_runtime.hip -- libvtq_runtime: the reference's quantized decode with
// every linear layer on the GPU through libvtq (include/vtq_runtime.h).
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
// The GGUF blob is uploaded once; linears read their weights in place on the
// device.  Host work per step: embedding row, RMSNorm, RoPE, attention over
// the KV cache (heads spread over a thread pool; each head's arithmetic is
// sequential exactly as in the reference), SwiGLU, residuals, argmax.
#include <hip/hip_runtime.h>

#include <atomic>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/vtq.h"
#include "../../include/vtq_runtime.h"
#include "vtq_libm.h"

namespace libm = vtq::libm;

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

// ---------------------------------------------------------------- thread pool
class Pool {
  public:
    explicit Pool(int n) {
        for (int i = 0; i < n; i++) workers_.emplace_back([this, i] { run(i); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> l(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : workers_) t.join();
    }
    int size() const { return (int)workers_.size() + 1; }
    // fn(i) for i in [0, n): items are independent, so the split is free
    void parallel_for(int n, const std::function<void(int)>& fn) {
        if (workers_.empty() || n <= 1) {
            for (int i = 0; i < n; i++) fn(i);
            return;
        }
        {
            std::lock_guard<std::mutex> l(mu_);
            fn_ = &fn;
            n_ = n;
            next_.store(0);
            pending_ = (int)workers_.size();
            gen_++;
        }
        cv_.notify_all();
        for (int i; (i = next_.fetch_add(1)) < n;) fn(i);
        std::unique_lock<std::mutex> l(mu_);
        done_.wait(l, [this] { return pending_ == 0; });
        fn_ = nullptr;
    }

  private:
    void run(int) {
        uint64_t seen = 0;
        for (;;) {
            const std::function<void(int)>* fn;
            int n;
            {
                std::unique_lock<std::mutex> l(mu_);
                cv_.wait(l, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
                fn = fn_;
                n = n_;
            }
            for (int i; (i = next_.fetch_add(1)) < n;) (*fn)(i);
            std::lock_guard<std::mutex> l(mu_);
            if (--pending_ == 0) done_.notify_one();
        }
    }
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    const std::function<void(int)>* fn_ = nullptr;
    int n_ = 0, pending_ = 0;
    std::atomic<int> next_{0};
    uint64_t gen_ = 0;
    bool stop_ = false;
};

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
float f16(const uint8_t* p) {
    const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
    const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        const float v = (float)m * 0x1p-24f;
        bits = __builtin_bit_cast(uint32_t, v) | sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    return __builtin_bit_cast(float, bits);
}

struct Lin {
    int type = 0;
    size_t offset = 0, nbytes = 0;
};

struct Layer {
    const float *rms_att = nullptr, *rms_ffn = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr;
    Lin wq, wk, wv, wo, w1, w2, w3;
};

}  // namespace

struct vtqrt_model {
    std::vector<uint8_t> blob;  // host copy (norms, embedding rows)
    uint8_t* dblob = nullptr;   // device copy (linear weights)
    vtq_ctx* ctx = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    int dim = 0, hidden = 0, layers = 0, heads = 0, kv_heads = 0, vocab = 0, seq = 0;
    bool shared = false, neox = false;
    float theta = 10000.0f, eps = 1e-5f;
    Lin tok, wcls;
    const float* rms_final = nullptr;
    std::vector<Layer> L;
    // device activations and pinned host staging
    float *dx = nullptr, *dy = nullptr, *hx = nullptr, *hy = nullptr;
    std::unique_ptr<Pool> pool;
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

// ---- one linear on the device: x (host) -> y (host), several outputs of
// the same input share one upload and one synchronisation.
struct LinCall {
    const Lin* w;
    int out_feat;
    float* y;
};

int linears(vtqrt_model* m, int regime, const float* x, int in_feat, std::initializer_list<LinCall> calls) {
    std::memcpy(m->hx, x, (size_t)in_feat * 4);
    int rc = hip_check(m, hipMemcpyAsync(m->dx, m->hx, (size_t)in_feat * 4, hipMemcpyHostToDevice, m->stream),
                       "hipMemcpyAsync(x)");
    if (rc) return rc;
    size_t off = 0;
    for (const LinCall& c : calls) {
        rc = vtq_linear_device(m->ctx, c.w->type, regime, m->dx, m->dblob + c.w->offset, c.w->nbytes, m->dy + off,
                               1, (size_t)in_feat, (size_t)c.out_feat, m->stream);
        if (rc) return fail(m, rc, vtq_last_error(m->ctx));
        off += ((size_t)c.out_feat + 63) / 64 * 64;
    }
    rc = hip_check(m, hipMemcpyAsync(m->hy, m->dy, off * 4, hipMemcpyDeviceToHost, m->stream), "hipMemcpyAsync(y)");
    if (rc) return rc;
    rc = hip_check(m, hipStreamSynchronize(m->stream), "hipStreamSynchronize");
    if (rc) return rc;
    off = 0;
    for (const LinCall& c : calls) {
        std::memcpy(c.y, m->hy + off, (size_t)c.out_feat * 4);
        off += ((size_t)c.out_feat + 63) / 64 * 64;
    }
    return VTQ_OK;
}

void rms_norm(const float* x, const float* w, int n, float eps, float* out) {
    float sumsq = 0.0f;
    for (int i = 0; i < n; i++) sumsq += x[i] * x[i];
    const float mean = sumsq / (float)n;
    const float scale = 1.0f / libm::sqrtf(mean + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

int embedding_row(vtqrt_model* m, int row, float* out) {
    const Lin& t = m->tok;
    const int dim = m->dim;
    const uint8_t* base = m->blob.data() + t.offset;
    size_t rb;
    switch (t.type) {
    case 0: rb = (size_t)dim * 4; break;
    case 2: rb = (size_t)dim / 32 * 18; break;
    case 6: rb = (size_t)dim / 32 * 22; break;
    case 8: rb = (size_t)dim / 32 * 34; break;
    case 12: rb = (size_t)dim / 256 * 144; break;
    case 14: rb = (size_t)dim / 256 * 210; break;
    default: return fail(m, VTQ_E_NOT_IMPLEMENTED, "embedding_row: non-Q4_0 / Q4_K / Q6_K / Q8_0 / F32 embedding dtype");
    }
    if ((size_t)(row + 1) * rb > t.nbytes) return fail(m, VTQ_E_INTERNAL, "embedding_row: row past end of table");
    const uint8_t* r = base + (size_t)row * rb;
    switch (t.type) {
    case 0:
        std::memcpy(out, r, rb);
        break;
    case 2:  // dequantize_q4_0: element 2k low nibble, 2k+1 high
        for (int b = 0; b < dim / 32; b++) {
            const uint8_t* blk = r + 18 * b;
            const float d = f16(blk);
            for (int k = 0; k < 16; k++) {
                out[32 * b + 2 * k] = d * (float)((int)(blk[2 + k] & 15) - 8);
                out[32 * b + 2 * k + 1] = d * (float)((int)(blk[2 + k] >> 4) - 8);
            }
        }
        break;
    case 6:  // dequantize_q5_0: element j and j+16 share qs byte j
        for (int b = 0; b < dim / 32; b++) {
            const uint8_t* blk = r + 22 * b;
            const float d = f16(blk);
            uint32_t qh;
            std::memcpy(&qh, blk + 2, 4);
            for (int j = 0; j < 16; j++) {
                const int x0 = (int)((blk[6 + j] & 15) | (((qh >> j) << 4) & 16)) - 16;
                const int x1 = (int)((blk[6 + j] >> 4) | ((qh >> (j + 12)) & 16)) - 16;
                out[32 * b + j] = d * (float)x0;
                out[32 * b + j + 16] = d * (float)x1;
            }
        }
        break;
    case 8:  // dequantize_q8_0
        for (int b = 0; b < dim / 32; b++) {
            const uint8_t* blk = r + 34 * b;
            const float d = f16(blk);
            for (int k = 0; k < 32; k++) out[32 * b + k] = d * (float)(int8_t)blk[2 + k];
        }
        break;
    case 12:  // dequantize_q4_k: d1*q - m1 per 32-element sub-block
        for (int b = 0; b < dim / 256; b++) {
            const uint8_t* blk = r + 144 * b;
            const float d = f16(blk), dmin = f16(blk + 2);
            const uint8_t* s = blk + 4;
            for (int j = 0; j < 8; j++) {
                uint32_t sc, mn;
                if (j < 4) {
                    sc = s[j] & 63;
                    mn = s[j + 4] & 63;
                } else {
                    sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
                    mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
                }
                const float d1 = d * (float)sc, m1 = dmin * (float)mn;
                const uint8_t* qs = blk + 16 + 32 * (j / 2);
                for (int l = 0; l < 32; l++) {
                    const uint32_t q = (j & 1) ? (qs[l] >> 4) : (qs[l] & 15);
                    out[256 * b + 32 * j + l] = d1 * (float)q - m1;
                }
            }
        }
        break;
    case 14:  // dequantize_q6_k: d * sc * q, q = 6-bit code - 32
        for (int b = 0; b < dim / 256; b++) {
            const uint8_t* blk = r + 210 * b;
            const float d = f16(blk + 208);
            for (int hf = 0; hf < 2; hf++) {
                const uint8_t *ql = blk + 64 * hf, *qh = blk + 128 + 32 * hf, *sc = blk + 192 + 8 * hf;
                float* o = out + 256 * b + 128 * hf;
                for (int l = 0; l < 32; l++) {
                    const int is = l / 16;
                    const uint8_t h = qh[l];
                    const int q[4] = {(int)((ql[l] & 15) | ((h & 3) << 4)) - 32,
                                      (int)((ql[l + 32] & 15) | (((h >> 2) & 3) << 4)) - 32,
                                      (int)((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32,
                                      (int)((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32};
                    for (int k = 0; k < 4; k++) o[l + 32 * k] = d * (float)(int8_t)sc[is + 2 * k] * (float)q[k];
                }
            }
        }
        break;
    }
    return VTQ_OK;
}

struct State {
    std::vector<float> kc, vc, x, xb, q, k, v, xo, x2, gate, up, ffn, logits, cosv, sinv, att;
};

int step(vtqrt_model* m, State& s, int regime, uint32_t token, int pos) {
    const int dim = m->dim, head = dim / m->heads, kv_dim = m->kv_heads * head, kv_mul = m->heads / m->kv_heads;
    const int hidden = m->hidden;
    int rc = embedding_row(m, (int)token, s.x.data());
    if (rc) return rc;
    // RoPE angles depend only on (pos, index): computed once per step with
    // the reference's expressions (forward_quantized.rs:417-456)
    const int nrot = m->neox ? head / 2 : dim / 2;
    for (int i = 0; i < nrot; i++) {
        const float e = m->neox ? (float)(2 * i) / (float)head : (float)((2 * i) % head) / (float)head;
        const float freq = 1.0f / libm::powf(m->theta, e);
        const float val = (float)pos * freq;
        s.cosv[i] = libm::cosf(val);
        s.sinv[i] = libm::sinf(val);
    }
    const float sq = libm::sqrtf((float)head);
    for (int l = 0; l < m->layers; l++) {
        const Layer& Ly = m->L[l];
        rms_norm(s.x.data(), Ly.rms_att, dim, m->eps, s.xb.data());
        rc = linears(m, regime, s.xb.data(), dim,
                     {{&Ly.wq, m->heads * head, s.q.data()}, {&Ly.wk, kv_dim, s.k.data()}, {&Ly.wv, kv_dim, s.v.data()}});
        if (rc) return rc;
        if (Ly.bq) for (int i = 0; i < dim; i++) s.q[i] += Ly.bq[i];
        if (Ly.bk) for (int i = 0; i < kv_dim; i++) s.k[i] += Ly.bk[i];
        if (Ly.bv) for (int i = 0; i < kv_dim; i++) s.v[i] += Ly.bv[i];
        const size_t loff = (size_t)l * m->seq * kv_dim;
        float* kc = s.kc.data() + loff + (size_t)pos * kv_dim;
        std::memcpy(kc, s.k.data(), (size_t)kv_dim * 4);
        std::memcpy(s.vc.data() + loff + (size_t)pos * kv_dim, s.v.data(), (size_t)kv_dim * 4);
        if (m->neox) {
            const int half = head / 2;
            for (int h = 0; h < m->heads; h++)
                for (int j = 0; j < half; j++) {
                    float* qb = s.q.data() + h * head;
                    const float a = qb[j], b = qb[j + half];
                    qb[j] = a * s.cosv[j] - b * s.sinv[j];
                    qb[j + half] = a * s.sinv[j] + b * s.cosv[j];
                }
            for (int h = 0; h < kv_dim / head; h++)
                for (int j = 0; j < half; j++) {
                    float* kb = kc + h * head;
                    const float a = kb[j], b = kb[j + half];
                    kb[j] = a * s.cosv[j] - b * s.sinv[j];
                    kb[j + half] = a * s.sinv[j] + b * s.cosv[j];
                }
        } else {
            for (int i = 0; i < dim; i += 2) {
                const float fcr = s.cosv[i / 2], fci = s.sinv[i / 2];
                const float q0 = s.q[i], q1 = s.q[i + 1];
                s.q[i] = q0 * fcr - q1 * fci;
                s.q[i + 1] = q0 * fci + q1 * fcr;
                if (i < kv_dim) {
                    const float k0 = kc[i], k1 = kc[i + 1];
                    kc[i] = k0 * fcr - k1 * fci;
                    kc[i + 1] = k0 * fci + k1 * fcr;
                }
            }
        }
        // attention, one head per pool item
        m->pool->parallel_for(m->heads, [&](int h) {
            float* att = s.att.data() + (size_t)h * m->seq;
            const float* qh = s.q.data() + h * head;
            for (int t = 0; t <= pos; t++) {
                const float* kt = s.kc.data() + loff + (size_t)t * kv_dim + (size_t)(h / kv_mul) * head;
                float score = 0.0f;
                for (int d = 0; d < head; d++) score += qh[d] * kt[d];
                score /= sq;
                att[t] = score;
            }
            float mx = -__builtin_inff();
            for (int t = 0; t <= pos; t++)
                if (att[t] > mx) mx = att[t];
            float sum = 0.0f;
            for (int t = 0; t <= pos; t++) {
                att[t] = libm::expf(att[t] - mx);
                sum += att[t];
            }
            const float inv = 1.0f / sum;
            for (int t = 0; t <= pos; t++) att[t] *= inv;
            float* xo = s.xo.data() + h * head;
            for (int d = 0; d < head; d++) xo[d] = 0.0f;
            for (int t = 0; t <= pos; t++) {
                const float* vt = s.vc.data() + loff + (size_t)t * kv_dim + (size_t)(h / kv_mul) * head;
                const float a = att[t];
                for (int d = 0; d < head; d++) xo[d] += a * vt[d];
            }
        });
        rc = linears(m, regime, s.xo.data(), dim, {{&Ly.wo, dim, s.x2.data()}});
        if (rc) return rc;
        for (int i = 0; i < dim; i++) s.x[i] = s.x[i] + s.x2[i];
        rms_norm(s.x.data(), Ly.rms_ffn, dim, m->eps, s.xb.data());
        rc = linears(m, regime, s.xb.data(), dim, {{&Ly.w1, hidden, s.gate.data()}, {&Ly.w3, hidden, s.up.data()}});
        if (rc) return rc;
        for (int i = 0; i < hidden; i++) {
            const float g = s.gate[i];
            const float silu = g / (1.0f + libm::expf(-g));
            s.ffn[i] = silu * s.up[i];
        }
        rc = linears(m, regime, s.ffn.data(), hidden, {{&Ly.w2, dim, s.x2.data()}});
        if (rc) return rc;
        for (int i = 0; i < dim; i++) s.x[i] = s.x[i] + s.x2[i];
    }
    rms_norm(s.x.data(), m->rms_final, dim, m->eps, s.xb.data());
    return linears(m, regime, s.xb.data(), dim, {{m->shared ? &m->tok : &m->wcls, m->vocab, s.logits.data()}});
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

void vtqrt_free(vtqrt_model* m) {
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->dblob) (void)hipFree(m->dblob);
    if (m->dx) (void)hipFree(m->dx);
    if (m->dy) (void)hipFree(m->dy);
    if (m->hx) (void)hipHostFree(m->hx);
    if (m->hy) (void)hipHostFree(m->hy);
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
    auto f32 = [&](const std::string& n, size_t want, bool required, const float** o) {
        auto it = ts.find(n);
        if (it == ts.end()) return !required;
        if (it->second.type != 0 || it->second.nbytes != want * 4) return false;
        *o = reinterpret_cast<const float*>(m->blob.data() + it->second.offset);
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
    const size_t act = 3 * (size_t)std::max({m->dim, m->hidden, m->vocab}) + 256;  // up to 3 outputs per upload
    if ((rc = hip_check(m, hipMalloc(&m->dx, act * 4), "hipMalloc(x)")) ||
        (rc = hip_check(m, hipMalloc(&m->dy, act * 4), "hipMalloc(y)")) ||
        (rc = hip_check(m, hipHostMalloc(&m->hx, act * 4, hipHostMallocDefault), "hipHostMalloc(x)")) ||
        (rc = hip_check(m, hipHostMalloc(&m->hy, act * 4, hipHostMallocDefault), "hipHostMalloc(y)"))) {
        *out = m;
        return rc;
    }
    const unsigned hw = std::thread::hardware_concurrency();
    const int threads = (int)std::min<unsigned>(hw ? hw : 1, 16);
    m->pool.reset(new Pool(std::max(0, threads - 1)));
    *out = m;
    return VTQ_OK;
}

int vtqrt_run(vtqrt_model* m, int regime, const char* model_id, const uint8_t weights_hash[32],
              const uint32_t* prompt, int prompt_len, int n_new, float* logits, uint32_t* tokens,
              uint8_t digest[32]) {
    if (!m || !m->ctx || !model_id || !weights_hash || !digest || (prompt_len > 0 && !prompt) ||
        (n_new > 0 && !tokens) || n_new < 0)
        return VTQ_E_INVALID_ARGUMENT;
    m->err.clear();
    if (prompt_len <= 0) return fail(m, VTQ_E_INTERNAL, "prompt_tokens must not be empty");
    const int total = prompt_len + n_new;
    if (total > m->seq) return fail(m, VTQ_E_INTERNAL, "prompt + n_new_tokens exceeds seq_len");
    const int head = m->dim / m->heads, kv_dim = m->kv_heads * head;
    State s;
    const size_t kv = (size_t)m->layers * m->seq * kv_dim;
    s.kc.assign(kv, 0.0f);
    s.vc.assign(kv, 0.0f);
    s.x.resize(m->dim);
    s.xb.resize(m->dim);
    s.q.resize(m->dim);
    s.k.resize(kv_dim);
    s.v.resize(kv_dim);
    s.xo.resize(m->dim);
    s.x2.resize(m->dim);
    s.gate.resize(m->hidden);
    s.up.resize(m->hidden);
    s.ffn.resize(m->hidden);
    s.logits.resize(m->vocab);
    s.cosv.resize(m->dim);
    s.sinv.resize(m->dim);
    s.att.resize((size_t)m->heads * m->seq);
    std::vector<uint32_t> gen;
    uint32_t cur = prompt[0];
    for (int pos = 0; pos < total; pos++) {
        if (cur >= (uint32_t)m->vocab) return fail(m, VTQ_E_INTERNAL, "embedding_row: row past end of table");
        int rc = step(m, s, regime, cur, pos);
        if (rc) return rc;
        if (logits) std::memcpy(logits + (size_t)pos * m->vocab, s.logits.data(), (size_t)m->vocab * 4);
        uint32_t best = 0;
        float bv = s.logits[0];
        for (int i = 1; i < m->vocab; i++)
            if (s.logits[i] > bv) {
                bv = s.logits[i];
                best = (uint32_t)i;
            }
        const uint32_t next = pos + 1 < prompt_len ? prompt[pos + 1] : best;
        if (pos >= prompt_len) gen.push_back(next);
        cur = next;
    }
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
    leb128(h, 0);
    leb128(h, 0);
    leb128(h, 0);
    h.final(digest);
    return VTQ_OK;
}

}  // extern "C"
