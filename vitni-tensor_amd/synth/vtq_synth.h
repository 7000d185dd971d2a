/*
 * vtq_synth.h -- seeded synthetic GGUF blocks and activations for the
 * benchmark configurations (not part of the C ABI; used by tests and
 * bench.py on both sides of a parity check).
 *
 * Stream: SplitMix64.  Uniform integers in [0, range): (u >> 32) % range.
 * Gaussian: Box-Muller in double (cos branch only), cast to float.
 * fp16 scales: IEEE round-to-nearest-even encode, subnormals kept.
 *
 * Per block, draws are taken in this order:
 *   Q4_K: d, dmin, sc[0..8], m[0..8], nibble[0..256] (element order)
 *   Q6_K: d, sc[0..16] (U[-64,63]), code[0..256] (U[0,63], element order)
 *   Q8_0: d, code[0..32] (U[-127,127])
 *   Q5_0: d, code[0..32] (U[0,31], element order)
 *   Q4_0: d, code[0..32] (U[0,15], element order)
 * with d, dmin = f16(|N(0, sigma)|).
 */
#ifndef VTQ_SYNTH_H
#define VTQ_SYNTH_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

uint16_t vtqs_f32_to_f16_rne(float f);
void vtqs_normal_f32(uint64_t seed, float *out, size_t n, float sigma);
void vtqs_q4_k(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma);
void vtqs_q6_k(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma);
void vtqs_q8_0(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma);
void vtqs_q5_0(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma);
void vtqs_q4_0(uint64_t seed, uint8_t *w, size_t rows, size_t in_feat, float sigma);
void vtqs_bytes(uint64_t seed, uint8_t *w, size_t n);

/* Token ids U[0, vocab). */
void vtqs_tokens(uint64_t seed, uint32_t *out, size_t n, uint32_t vocab);

/* A random-init Llama model as a GGUF v3 blob (the file format the
 * reference loads, src/model/gguf.rs:305-421): general.architecture
 * "llama", the llama.* hyper-parameters (u32; rope.freq_base and
 * attention.layer_norm_rms_epsilon f32), general.alignment 32, and tensors
 *   token_embd.weight            Q4_K [dim, vocab]
 *   blk.L.attn_norm.weight       F32  [dim]        1 + N(0, 0.05)
 *   blk.L.attn_q/attn_output     Q4_K [dim, dim]
 *   blk.L.attn_k/attn_v          Q4_K [dim, kv_dim]
 *   blk.L.ffn_norm.weight        F32  [dim]
 *   blk.L.ffn_gate/ffn_up        Q4_K [dim, hidden]
 *   blk.L.ffn_down               Q4_K [hidden, dim]
 *   output_norm.weight           F32  [dim]
 *   output.weight                Q6_K [dim, vocab]
 * (GGML order: the first dimension is the row length).  Blocks come from
 * the generators above with sigma 0.01; tensor i uses seed + i.  Options:
 *   arch 1        general.architecture "qwen2" (qwen2.* keys; the loader
 *                 then rotates NeoX split halves), 0 "llama"
 *   tied 1        no output.weight: the head is token_embd (shared weights)
 *   qkv_bias 1    blk.L.attn_q.bias [dim], attn_k.bias / attn_v.bias
 *                 [kv_dim], F32 N(0, 0.5)
 *   alignment     general.alignment (0: 32); tensor offsets are multiples
 *                 of it, so a value below 16 places tensors off 16 bytes
 *   short_rows    that many rows fewer in blk.0.attn_k.weight (a tensor
 *                 shorter than its configured shape)
 * Returns the blob size; writes it to out when out is not NULL. */
typedef struct {
    uint32_t dim, hidden, layers, heads, kv_heads, vocab, ctx;
    float rope_theta, rms_eps;
    uint32_t arch, tied, qkv_bias, alignment, short_rows;
} vtqs_llama;
size_t vtqs_llama_gguf(const vtqs_llama *cfg, uint64_t seed, uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
