// vtq_decode.h -- internal interface of the device-resident decode step
// (libvtq_runtime).  All pointers are device memory; launches are
// asynchronous on `stream`.  The position of the step being computed is read
// from device memory (*pos), so one step's launches can be captured once in a
// HIP graph and replayed for every position; the argmax kernel, the last of
// the step, advances *pos.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vtq {
namespace decode {

// The RoPE angle table: position q's (cos, sin) of pair m < head_dim/2 at
// cs[q * head_dim + 2m], +1 (rope_table, forward_quantized.rs:417-456).  It
// depends on the position alone, so rope_table_rows fills it once per model
// for every position of the cache; attention reads row *pos.
struct RopeArgs {
    float* cs;
    int head_dim;
    float theta;
};
hipError_t rope_table_rows(const RopeArgs& r, int rows, hipStream_t stream);

// embedding_row (src/model/forward_quantized.rs:818-923): row tokens[*pos]
// of the table (ggml type 0, 2, 6, 8, 12 or 14, `rows` rows) into x[0..dim);
// a token >= rows reads row 0 instead, and the caller reports the error.
// embed_row_bytes: bytes per table row, 0 for an unsupported type or a dim
// that is not a whole number of blocks.
size_t embed_row_bytes(int ggml_type, int dim);
hipError_t embed(int ggml_type, const uint8_t* table, uint32_t rows, const uint32_t* tokens, const int* pos, int dim,
                 float* x, hipStream_t stream);

// rms_norm_slice (src/ops/rms_norm.rs:60-110): out = x * scale * w with the
// sum of squares accumulated serially, as the reference does.
hipError_t rms_norm(const float* x, const float* w, int n, float eps, float* out, hipStream_t stream);
// the same for `rows` rows of n floats (row r of x into row r of out)
hipError_t rms_norm_rows(const float* x, const float* w, int n, int rows, float eps, float* out, hipStream_t stream);
// the residual first: x[i] = x[i] + add[i] over the rows (as add_inplace),
// then rms_norm_rows of the updated x; add == nullptr: rms_norm_rows
hipError_t add_rms_norm_rows(float* x, const float* add, const float* w, int n, int rows, float eps, float* out,
                             hipStream_t stream);

// Byte ranges later kernels of the step read, streamed through the
// memory-side cache by `groups` extra workgroups of the attention launch
// (which leaves most CUs idle), so that those kernels read them from the
// cache.  A range of cached k or v rows gives its row size: only the rows
// before the step's position (*pos) are streamed.  The loaded bytes are folded into one value, stored to sink only if
// it equals magic, so the loads are kept and nothing is written in practice.
struct Prefetch {
    static constexpr int kRanges = 6;
    const uint8_t* p[kRanges] = {};
    uint32_t n[kRanges] = {};
    // nonzero: the range holds cached rows, and only rows 0 .. *pos - 1 of
    // row_bytes each (at most n) are streamed
    uint32_t row_bytes[kRanges] = {};
    const int* pos = nullptr;
    int groups = 0;
    uint32_t magic = 0;
    uint32_t* sink = nullptr;
};

struct AttnArgs {
    const float* qkv;            // q[dim] | k[kv_dim] | v[kv_dim] of this step
    const float *bq, *bk, *bv;   // optional biases (added before RoPE / the cache write)
    float *kc, *vc;              // this layer's caches, [seq][kv_dim]
    const float* cs;             // the RoPE angle table (RopeArgs): row p is position p's
    float* out;                  // [dim] attention output (the Wo input)
    const int* pos;
    int heads, kv_heads, head_dim, seq;
    float theta;
    int neox;                    // 1: RoPE on (j, j + head/2) pairs, 0: on (2j, 2j+1)
    // the heads' score rows in HBM, [heads][seq rounded up to 4], where
    // attention_scores_in_lds is false; nullptr otherwise
    float* att_g = nullptr;
    // 0: one decode step at *pos.  P > 0: a prompt pass over positions
    // 0..P-1 at once (qkv, cs and out hold P rows; rope_cache_rows has
    // written every position's k and v; see attention_rows_supported)
    int batched = 0;
    Prefetch pf;  // extra workgroups (one-step launches only)
};
// RoPE of q and of this step's k, the cache write of k and v at *pos, and
// per-head softmax attention (src/model/forward_quantized.rs:405-560).
// attention_supported: whether the kernel takes this head dimension (a
// multiple of 4 up to 256 that divides 16384); any cache length is taken.
// attention_scores_in_lds: whether a head's seq scores fit in LDS beside the
// cached-v tiles; else they go to the caller's att_g rows.
bool attention_supported(int head_dim, int seq);
bool attention_scores_in_lds(int head_dim, int seq);
hipError_t attention(const AttnArgs& a, hipStream_t stream);
// Whether a prompt pass of P positions can run its attention: one wave per
// (query head, position), the waves of a workgroup on one KV group, each
// wave's q and P scores and one tile of cached rows in LDS.
bool attention_rows_supported(int head_dim, int P, int heads, int kv_heads);
// The prompt pass's cache write: position p's k (bias, RoPE) and v for
// p < a.batched, as attention computes them for its own position.
hipError_t rope_cache_rows(const AttnArgs& a, hipStream_t stream);
// embedding_row of tokens[0..P) into x[P][dim]
hipError_t embed_rows(int ggml_type, const uint8_t* table, uint32_t rows, const uint32_t* tokens, int P, int dim,
                      float* x, hipStream_t stream);

// The embedding table, for the next step's row (see embed).
struct EmbedArgs {
    int type;
    const uint8_t* table;  // nullptr: no embedding
    uint32_t rows;
    size_t row_bytes;
    int dim;
    float* x;
};

// argmax_last_dim (src/ops/argmax.rs:21-68) of logits[0..vocab): the next
// token tokens[*pos + 1] when *pos + 1 >= prompt_len (a prompt token is
// forced otherwise) and *pos + 1 <= total.  With hist, the logits are also
// copied to hist[*pos * vocab ..].  Then, when *pos + 1 < total, the
// embedding row of tokens[*pos + 1] goes to e.x (the next step's input), and
// *pos += 1.
hipError_t argmax_advance(const float* logits, int vocab, uint32_t* tokens, int* pos, int prompt_len, int total,
                          float* hist, const EmbedArgs& e, hipStream_t stream);

// Element-wise epilogues for linears that are not fused into the GEMV:
// x[i] = x[i] + y[i] (residual), v[i] = v[i] + b[i] (bias),
// out[i] = silu(gate[i]) * up[i] with silu(g) = g / (1 + expf(-g)).
hipError_t add_inplace(float* x, const float* y, int n, hipStream_t stream);

// y[7i + k] = f_k(x[i]) for the seven functions of the reference's
// transcendental sweep, evaluated by the device libm the step uses.
hipError_t transcendentals(const float* x, int n, float* y, hipStream_t stream);
hipError_t swiglu(const float* gate, const float* up, float* out, int n, hipStream_t stream);
// the same over rows of gate | up (2 * hidden floats each) into rows of hidden
hipError_t swiglu_rows(const float* gu, int hidden, int rows, float* out, hipStream_t stream);

}  // namespace decode
}  // namespace vtq
