// vtq_gguf.h -- host-side model description of libvtq_runtime: GGUF v2/v3
// parsing, Config and the tensor table of a quantized Llama-family model.
// Plain C++ with no device code, so it builds and is tested without a GPU
// (including under AddressSanitizer).
//
// Restates, with the reference's checks in the reference's order and its
// error texts verbatim:
//   GgufFile::parse            src/model/gguf.rs:305-421 (Cursor :483-617,
//                              bytes_for_numel :144-214, checked_numel :470-478)
//   Config::from_gguf          src/model/config.rs:156-213
//   QuantizedWeights::from_gguf src/model/quant_weights.rs:121-181 (get_tensor,
//                              read_f32_tensor[_opt] :222-272)
// Status codes are include/vtq.h's (VTQ_E_MALFORMED, VTQ_E_TRUNCATED,
// VTQ_E_OVERFLOW for the parse; VTQ_E_INTERNAL for the model tables, as the
// reference's Error variants).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace vtq {
namespace gguf {

struct Value {
    uint32_t type = 0;      // GGUF value type tag (0..12)
    uint64_t num = 0;       // integer value, or the f32 / f64 bits
    std::string str;        // STRING
    uint32_t elem_type = 0; // ARRAY: element type
    uint64_t count = 0;     // ARRAY: element count
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> shape;  // GGML order: shape[0] is the row length
    uint32_t type = 0;
    uint64_t offset = 0, nbytes = 0;  // absolute byte range in the blob
};

struct File {
    uint32_t version = 0;
    std::map<std::string, Value> meta;       // a repeated key keeps its last value
    std::vector<Tensor> tensors;             // in file order
    std::map<std::string, size_t> by_name;   // a repeated name maps to its last tensor
    const Tensor* tensor(const std::string& name) const;
};

// GgufFile::parse.  Returns VTQ_OK or an error status with *msg set to the
// reference's text.  Never reads outside blob[0, len), never allocates more
// than O(len) and never throws.
int parse(const uint8_t* blob, size_t len, File* out, const char** msg);

// One weight or norm tensor as the model uses it (QuantTensor / &[f32]).
struct View {
    int type = -1;  // -1: absent (optional tensors)
    uint64_t offset = 0, nbytes = 0;
};

struct LayerViews {
    View rms_att, wq, wk, wv, wo, rms_ffn, w1, w2, w3, bq, bk, bv;
};

// Config::from_gguf + QuantizedWeights::from_gguf of a parsed file.  The
// dimensions are usize in the reference; values above INT_MAX are refused
// here (VTQ_E_NOT_IMPLEMENTED) where the reference would abort on the
// allocation that follows.
struct Model {
    int dim = 0, hidden = 0, layers = 0, heads = 0, kv_heads = 0, vocab = 0, seq = 0;
    bool shared = false, neox = false;
    float theta = 10000.0f, eps = 1e-5f;
    View tok, rms_final, wcls;
    std::vector<LayerViews> L;
};
int describe(const File& f, Model* out, const char** msg);

}  // namespace gguf
}  // namespace vtq
