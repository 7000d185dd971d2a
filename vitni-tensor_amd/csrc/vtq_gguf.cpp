// vtq_gguf.cpp -- GGUF parsing and the model tables of libvtq_runtime (see
// vtq_gguf.h).  Every length, count and offset in the file is untrusted: each
// arithmetic step on them is checked, and the error is the one the reference
// returns at the same point (src/model/gguf.rs).
#include "vtq_gguf.h"

#include <climits>
#include <cstring>

#include "../../include/vtq.h"

namespace vtq {
namespace gguf {

namespace {

enum : uint32_t {
    kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64,
};

constexpr uint64_t kDefaultAlignment = 32;  // gguf.rs:53
constexpr uint64_t kMaxString = 1u << 20;   // Cursor::read_string's sanity cap

// Cursor (gguf.rs:483-617).  The first failure is kept; later reads fail too.
class Cursor {
  public:
    Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
    int code() const { return code_; }
    const char* msg() const { return msg_; }
    size_t pos() const { return pos_; }
    bool ok() const { return code_ == VTQ_OK; }
    bool fail(int code, const char* msg) {
        if (code_ == VTQ_OK) {
            code_ = code;
            msg_ = msg;
        }
        return false;
    }

    // read_n: pos + n overflowing is Overflow, past the end Truncated
    bool read_n(uint64_t n, const uint8_t** out) {
        if (!ok()) return false;
        if (n > SIZE_MAX - pos_) return fail(VTQ_E_OVERFLOW, "gguf: read past end (overflow)");
        if (pos_ + n > n_) return fail(VTQ_E_TRUNCATED, "gguf: read past end");
        *out = p_ + pos_;
        pos_ += n;
        return true;
    }
    bool u(int bytes, uint64_t* v) {
        const uint8_t* s;
        if (!read_n((uint64_t)bytes, &s)) return false;
        uint64_t r = 0;
        for (int i = 0; i < bytes; i++) r |= (uint64_t)s[i] << (8 * i);
        *v = r;
        return true;
    }
    bool u32(uint32_t* v) {
        uint64_t t = 0;
        if (!u(4, &t)) return false;
        *v = (uint32_t)t;
        return true;
    }
    bool u64(uint64_t* v) { return u(8, v); }

    // read_string: u64 length (capped at 1 MiB), then UTF-8 bytes
    bool string(std::string* s) {
        uint64_t n;
        if (!u64(&n)) return false;
        if (n > kMaxString) return fail(VTQ_E_MALFORMED, "gguf: string length > 1 MiB");
        const uint8_t* b;
        if (!read_n(n, &b)) return false;
        if (!utf8_ok(b, (size_t)n)) return fail(VTQ_E_MALFORMED, "gguf: non-UTF8 string");
        s->assign(reinterpret_cast<const char*>(b), (size_t)n);
        return true;
    }

    // read_value (gguf.rs:528-615)
    bool value(uint32_t type, Value* v) {
        v->type = type;
        static const int kSize[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
        if (type == kString) return string(&v->str);
        if (type != kArray) return u(kSize[type], &v->num);
        uint32_t et;
        if (!u32(&et)) return false;
        if (et > kF64) return fail(VTQ_E_MALFORMED, "gguf: bad array elem type");
        if (et == kArray) return fail(VTQ_E_MALFORMED, "gguf: nested arrays not supported");
        uint64_t len;
        if (!u64(&len)) return false;
        v->elem_type = et;
        v->count = len;
        if (et == kString) {
            // each element is a u64 length plus bytes (no UTF-8 check, no
            // cap); every element consumes at least 8 bytes, so a huge count
            // ends at the end of the buffer
            for (uint64_t i = 0; i < len; i++) {
                uint64_t n;
                if (!u64(&n)) return false;
                if (n > SIZE_MAX - pos_) return fail(VTQ_E_OVERFLOW, "gguf: array string overflow");
                if (pos_ + n > n_) return fail(VTQ_E_TRUNCATED, "gguf: array string past end");
                pos_ += n;
            }
            return true;
        }
        uint64_t total;
        if (__builtin_mul_overflow(len, (uint64_t)kSize[et], &total))
            return fail(VTQ_E_OVERFLOW, "gguf: array byte total overflow");
        if (total > SIZE_MAX - pos_) return fail(VTQ_E_OVERFLOW, "gguf: array end overflow");
        if (pos_ + total > n_) return fail(VTQ_E_TRUNCATED, "gguf: array past end of buffer");
        pos_ += total;
        return true;
    }

  private:
    // core::str::from_utf8: well-formed UTF-8 (no overlongs, surrogates or
    // code points past U+10FFFF)
    static bool utf8_ok(const uint8_t* s, size_t n) {
        size_t i = 0;
        while (i < n) {
            const uint8_t c = s[i];
            if (c < 0x80) {
                i++;
                continue;
            }
            int len;
            uint8_t lo = 0x80, hi = 0xBF;
            if (c >= 0xC2 && c <= 0xDF) {
                len = 2;
            } else if (c >= 0xE0 && c <= 0xEF) {
                len = 3;
                if (c == 0xE0) lo = 0xA0;
                if (c == 0xED) hi = 0x9F;
            } else if (c >= 0xF0 && c <= 0xF4) {
                len = 4;
                if (c == 0xF0) lo = 0x90;
                if (c == 0xF4) hi = 0x8F;
            } else {
                return false;
            }
            if (n - i < (size_t)len) return false;
            if (s[i + 1] < lo || s[i + 1] > hi) return false;
            for (int k = 2; k < len; k++)
                if ((s[i + k] & 0xC0) != 0x80) return false;
            i += (size_t)len;
        }
        return true;
    }

    const uint8_t* p_;
    size_t n_, pos_ = 0;
    int code_ = VTQ_OK;
    const char* msg_ = "";
};

// GgufTensorType::bytes_for_numel (gguf.rs:144-214)
bool bytes_for_numel(uint32_t type, uint64_t numel, uint64_t* out, int* code, const char** msg) {
    struct Blk {
        uint32_t type;
        uint64_t elems, bytes;
        const char *not_multiple, *overflow;
    };
    static const Blk kBlk[] = {
        {0, 1, 4, nullptr, "gguf: F32 byte size overflow"},
        {1, 1, 2, nullptr, "gguf: F16 byte size overflow"},
        {2, 32, 18, "gguf: Q4_0 tensor numel not a multiple of 32", "gguf: Q4_0 byte size overflow"},
        {8, 32, 34, "gguf: Q8_0 tensor numel not a multiple of 32", "gguf: Q8_0 byte size overflow"},
        {6, 32, 22, "gguf: Q5_0 tensor numel not a multiple of 32", "gguf: Q5_0 byte size overflow"},
        {12, 256, 144, "gguf: Q4_K tensor numel not a multiple of 256", "gguf: Q4_K byte size overflow"},
        {14, 256, 210, "gguf: Q6_K tensor numel not a multiple of 256", "gguf: Q6_K byte size overflow"},
    };
    for (const Blk& b : kBlk) {
        if (b.type != type) continue;
        if (numel % b.elems) {
            *code = VTQ_E_MALFORMED;
            *msg = b.not_multiple;
            return false;
        }
        if (__builtin_mul_overflow(numel / b.elems, b.bytes, out)) {
            *code = VTQ_E_OVERFLOW;
            *msg = b.overflow;
            return false;
        }
        return true;
    }
    *code = VTQ_E_MALFORMED;
    *msg = "gguf: byte size unknown for unsupported ggml_type";
    return false;
}

}  // namespace

const Tensor* File::tensor(const std::string& name) const {
    auto it = by_name.find(name);
    return it == by_name.end() ? nullptr : &tensors[it->second];
}

int parse(const uint8_t* blob, size_t len, File* f, const char** msg) {
    *f = File();
    Cursor c(blob, len);
    auto bad = [&]() {
        *msg = c.msg();
        return c.code();
    };
    const uint8_t* magic;
    if (!c.read_n(4, &magic)) return bad();
    if (std::memcmp(magic, "GGUF", 4)) {
        *msg = "gguf: bad magic (not 'GGUF')";
        return VTQ_E_MALFORMED;
    }
    uint64_t tensor_count, kv_count;
    if (!c.u32(&f->version)) return bad();
    if (f->version != 2 && f->version != 3) {
        *msg = "gguf: unsupported version (only v2/v3 supported)";
        return VTQ_E_MALFORMED;
    }
    if (!c.u64(&tensor_count) || !c.u64(&kv_count)) return bad();

    // metadata: every pair consumes at least 12 bytes, so the loop ends at
    // the end of the buffer whatever the count claims
    for (uint64_t i = 0; i < kv_count; i++) {
        std::string key;
        uint32_t vt;
        if (!c.string(&key) || !c.u32(&vt)) return bad();
        if (vt > kF64) {
            *msg = "gguf: unknown value type";
            return VTQ_E_MALFORMED;
        }
        Value v;
        if (!c.value(vt, &v)) return bad();
        f->meta[key] = std::move(v);
    }

    // tensor infos (name, n_dims <= 8, dims, type, offset); each record is at
    // least 24 bytes, so the vector grows with the bytes actually present
    struct Info {
        std::string name;
        std::vector<uint64_t> shape;
        uint32_t type;
        uint64_t offset;
    };
    std::vector<Info> infos;
    for (uint64_t i = 0; i < tensor_count; i++) {
        Info t;
        uint32_t nd;
        if (!c.string(&t.name) || !c.u32(&nd)) return bad();
        if (nd > 8) {
            *msg = "gguf: tensor rank > 8 (sanity bound)";
            return VTQ_E_MALFORMED;
        }
        t.shape.resize(nd);
        for (uint32_t d = 0; d < nd; d++)
            if (!c.u64(&t.shape[d])) return bad();
        if (!c.u32(&t.type) || !c.u64(&t.offset)) return bad();
        infos.push_back(std::move(t));
    }

    // alignment: general.alignment when it is a U32, else 32
    uint64_t alignment = kDefaultAlignment;
    auto al = f->meta.find("general.alignment");
    if (al != f->meta.end() && al->second.type == kU32) alignment = al->second.num;
    if (alignment == 0) {
        *msg = "gguf: general.alignment is zero";
        return VTQ_E_MALFORMED;
    }
    const uint64_t unaligned = c.pos();
    uint64_t base;
    if (__builtin_mul_overflow(unaligned / alignment + (unaligned % alignment != 0), alignment, &base)) {
        *msg = "gguf: alignment padding overflow";
        return VTQ_E_OVERFLOW;
    }

    f->tensors.reserve(infos.size());
    for (Info& t : infos) {
        uint64_t numel = 1;
        for (uint64_t d : t.shape) {
            if (__builtin_mul_overflow(numel, d, &numel)) {
                *msg = "gguf: shape product overflows u64";
                return VTQ_E_OVERFLOW;
            }
        }
        uint64_t nbytes, start, end;
        int code;
        if (!bytes_for_numel(t.type, numel, &nbytes, &code, msg)) return code;
        if (__builtin_add_overflow(base, t.offset, &start)) {
            *msg = "gguf: tensor offset overflow";
            return VTQ_E_OVERFLOW;
        }
        if (__builtin_add_overflow(start, nbytes, &end)) {
            *msg = "gguf: tensor end overflow";
            return VTQ_E_OVERFLOW;
        }
        if (end > len) {
            *msg = "gguf: tensor extends past end of file";
            return VTQ_E_TRUNCATED;
        }
        Tensor out;
        out.name = std::move(t.name);
        out.shape = std::move(t.shape);
        out.type = t.type;
        out.offset = start;
        out.nbytes = nbytes;
        f->by_name[out.name] = f->tensors.size();
        f->tensors.push_back(std::move(out));
    }
    *msg = "";
    return VTQ_OK;
}

namespace {

// read_u32_loose (config.rs:171-181): U32, U64, or a non-negative I32 / I64.
bool read_usize(const File& f, const std::string& key, uint64_t* out) {
    auto it = f.meta.find(key);
    if (it == f.meta.end()) return false;
    const Value& v = it->second;
    switch (v.type) {
    case kU32: case kU64: *out = v.num; return true;
    case kI32: if ((int32_t)(uint32_t)v.num < 0) return false; *out = (uint64_t)(int32_t)(uint32_t)v.num; return true;
    case kI64: if ((int64_t)v.num < 0) return false; *out = v.num; return true;
    }
    return false;
}

float read_f32(const File& f, const std::string& key, float def) {
    auto it = f.meta.find(key);
    if (it == f.meta.end() || it->second.type != kF32) return def;
    float r;
    const uint32_t b = (uint32_t)it->second.num;
    std::memcpy(&r, &b, 4);
    return r;
}

View view_of(const Tensor* t) {
    View v;
    if (t) {
        v.type = (int)t->type;
        v.offset = t->offset;
        v.nbytes = t->nbytes;
    }
    return v;
}

}  // namespace

int describe(const File& f, Model* m, const char** msg) {
    *m = Model();
    // Config::from_gguf
    auto a = f.meta.find("general.architecture");
    if (a == f.meta.end() || a->second.type != kString) {
        *msg = "gguf: missing 'general.architecture' metadata";
        return VTQ_E_INTERNAL;
    }
    const std::string arch = a->second.str;
    uint64_t dim, hidden, layers, heads, kv_heads, seq, vocab;
    auto need = [&](const char* suffix, uint64_t* out) {
        if (read_usize(f, arch + "." + suffix, out)) return VTQ_OK;
        *msg = "gguf: numeric metadata missing or wrong type";
        return VTQ_E_INTERNAL;
    };
    int rc;
    if ((rc = need("embedding_length", &dim)) || (rc = need("feed_forward_length", &hidden)) ||
        (rc = need("block_count", &layers)) || (rc = need("attention.head_count", &heads)))
        return rc;
    // head_count_kv is optional: missing or unusable falls back to n_heads
    if (!read_usize(f, arch + ".attention.head_count_kv", &kv_heads)) kv_heads = heads;
    if ((rc = need("context_length", &seq))) return rc;
    auto toks = f.meta.find("tokenizer.ggml.tokens");
    if (toks != f.meta.end() && toks->second.type == kArray)
        vocab = toks->second.count;
    else if ((rc = need("vocab_size", &vocab)))
        return rc;
    // usize in the reference; the sizes that follow are refused here above
    // INT_MAX, where the reference would abort on an allocation
    for (uint64_t v : {dim, hidden, layers, heads, kv_heads, seq, vocab}) {
        if (v > (uint64_t)INT_MAX) {
            *msg = "vtq: model dimension above INT_MAX";
            return VTQ_E_NOT_IMPLEMENTED;
        }
    }
    m->dim = (int)dim;
    m->hidden = (int)hidden;
    m->layers = (int)layers;
    m->heads = (int)heads;
    m->kv_heads = (int)kv_heads;
    m->seq = (int)seq;
    m->vocab = (int)vocab;
    m->shared = f.tensor("output.weight") == nullptr;

    // QuantizedWeights::from_gguf: tensors in the order the reference reads them
    auto get = [&](const std::string& name, View* v) {
        const Tensor* t = f.tensor(name);
        if (!t) {
            *msg = "gguf: required Llama tensor not found";
            return VTQ_E_INTERNAL;
        }
        *v = view_of(t);
        return VTQ_OK;
    };
    auto get_f32 = [&](const std::string& name, View* v) {
        if (int r = get(name, v)) return r;
        if (v->type != 0) {
            *msg = "gguf: expected F32 norm-weight tensor, got something else";
            return VTQ_E_INTERNAL;
        }
        return VTQ_OK;
    };
    auto get_bias = [&](const std::string& name, View* v) {
        const Tensor* t = f.tensor(name);
        if (!t) return VTQ_OK;  // absent: no bias (Llama)
        if (t->type != 0) {
            *msg = "gguf: expected F32 bias tensor";
            return VTQ_E_INTERNAL;
        }
        *v = view_of(t);
        return VTQ_OK;
    };
    if ((rc = get("token_embd.weight", &m->tok)) || (rc = get_f32("output_norm.weight", &m->rms_final))) return rc;
    if (!m->shared) m->wcls = view_of(f.tensor("output.weight"));
    m->theta = read_f32(f, arch + ".rope.freq_base", 10000.0f);
    m->eps = read_f32(f, arch + ".attention.layer_norm_rms_epsilon", 1e-5f);
    m->neox = arch == "qwen2";
    // one entry per layer only while the tensors exist: a huge block_count
    // fails at the first missing name, not at an allocation
    for (int l = 0; l < m->layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        LayerViews Ly;
        if ((rc = get_f32(p + "attn_norm.weight", &Ly.rms_att)) || (rc = get(p + "attn_q.weight", &Ly.wq)) ||
            (rc = get(p + "attn_k.weight", &Ly.wk)) || (rc = get(p + "attn_v.weight", &Ly.wv)) ||
            (rc = get(p + "attn_output.weight", &Ly.wo)) || (rc = get_f32(p + "ffn_norm.weight", &Ly.rms_ffn)) ||
            (rc = get(p + "ffn_gate.weight", &Ly.w1)) || (rc = get(p + "ffn_down.weight", &Ly.w2)) ||
            (rc = get(p + "ffn_up.weight", &Ly.w3)) || (rc = get_bias(p + "attn_q.bias", &Ly.bq)) ||
            (rc = get_bias(p + "attn_k.bias", &Ly.bk)) || (rc = get_bias(p + "attn_v.bias", &Ly.bv)))
            return rc;
        m->L.push_back(Ly);
    }
    // Shapes the reference would only trip over while stepping (a division by
    // a zero head count, a head that does not tile dim): refused here.
    if (m->dim <= 0 || m->heads <= 0 || m->kv_heads <= 0 || m->dim % m->heads || m->heads % m->kv_heads) {
        *msg = "vtq: unsupported head layout (heads and kv_heads must tile dim)";
        return VTQ_E_NOT_IMPLEMENTED;
    }
    *msg = "";
    return VTQ_OK;
}

}  // namespace gguf
}  // namespace vtq
