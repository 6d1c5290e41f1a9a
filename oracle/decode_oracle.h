/* decode_oracle.h - CPU restatement of the reference's decode step (test infrastructure only; see decode_oracle.c).
 *
 * How each function is pinned (tests/test_oracle_decode.py; nothing here is checked only against itself):
 *   vxo_ggml_dot_f16   bit for bit against the reference test's dot_f16_model (quintrit-runtime/src/ops.rs:2008-2060)
 *   vxo_ggml_dot_bf16  bit for bit against the reference's portable ggml_vec_dot_bf16_scalar (ops.rs:686-713)
 *   vxo_vec_mad_f16, vxo_vec_scale_f16  element by element against the rounding the reference's AVX2 code performs
 *   vxo_f32_to_bf16, vxo_bf16_to_f32, f16 conversions  against torch / numpy round-to-nearest-even
 *   vxo_rope_cache     position 0 is exact; the theta recurrence in f32; cos/sin within 2 ulps of float64
 *   vxo_rope_neox, vxo_rope_normal  exact one-hot rotations (pairing, signs) and float64 closeness
 *   vxo_ggml_expf      exact at 0 and in the overflow / underflow branches, within 2 ulps of float64 exp elsewhere,
 *                      and a few values worked by hand through the reference's steps; vxo_swiglu against float64
 *                      silu(g) * u, its scalar tail against the host expf formula
 *   vxo_attend_head    bit for bit against hand-computable closed forms in which every softmax weight is exactly 0 or
 *                      1 (padded length, split threshold, chunk size, FP16 chain, in-order f32 combine), with negative
 *                      controls (seq_len-based chunks, an f32 accumulator, no padding, 8 chunks, a reversed combine);
 *                      float64 softmax attention for general scores
 *   vxo_model_forward  a float64 model written from model.rs / attention.rs (logits within 6 % of the largest; the
 *                      structural mistakes tried land at 57-190 %), plus a negative control
 *   quantizer, RMSNorm (velurex_oracle.c)  the reference's known answers (ops.rs:1968-1991); the reference text
 * Only the bits of libm-dependent values (expf, cosf, sinf, powf) rest on the host glibc being the reference's libm:
 * the reference computes them with Rust's f32 methods, which call the same C library on Linux. */
#ifndef DECODE_ORACLE_H
#define DECODE_ORACLE_H

#include "velurex_oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

#define VXO_MAX_LAYERS 64

typedef struct vxo_model_config {
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx;
    float rms_eps, rope_theta;
    /* The architecture switches of ModelConfig (config.rs:155-227); all zero is BASELINE.json configs[3]'s BitNet. */
    uint32_t act;       /* VXO_ACT_RELU2: relu2(gate) * up; VXO_ACT_SILU: swiglu(gate, up) (model.rs:155-170) */
    uint32_t rope_mode; /* VXO_ROPE_NEOX or VXO_ROPE_NORMAL (ops.rs:199-221) */
    uint32_t no_sub_norm; /* 1: no attention / FFN sub-norms (has_sub_norm = false, model.rs:172-190) */
    uint32_t emb_f16;   /* 0: bf16 embedding, head by ggml_vec_dot_bf16; 1: f16 embedding, head by ggml_vec_dot_f16 */
    uint32_t untied;    /* 1: a separate head matrix of the embedding's type (lm_head_f16, model.rs:355) */
} vxo_model_config;

enum { VXO_ACT_RELU2 = 0, VXO_ACT_SILU = 1 };
enum { VXO_ROPE_NEOX = 0, VXO_ROPE_NORMAL = 1 };

typedef struct vxo_model vxo_model;

float vxo_bf16_to_f32(uint16_t h);                                        /* ops.rs:652-655 */
uint16_t vxo_f32_to_bf16(float f);                                        /* ops.rs:658-665 */
float vxo_ggml_dot_bf16(const uint16_t* x, const uint16_t* y, size_t n);  /* ops.rs:669-713 */
float vxo_ggml_dot_f16(const uint16_t* x, const uint16_t* y, size_t n);   /* ops.rs:960-1015, 1078-1093 */
void vxo_vec_mad_f16(uint16_t* y, const uint16_t* x, float v, size_t n);  /* ops.rs:1254-1300 */
void vxo_vec_scale_f16(uint16_t* y, float v, size_t n);                   /* ops.rs:1304-1345 */
void vxo_expf_batch(const float* x, size_t n, float* out);                /* the host libm expf */
void vxo_rope_cache(size_t pos, size_t n_dims, float freq_base, float* cache);            /* ops.rs:121-140 */
void vxo_rope_neox(float* x, size_t heads, size_t head_dim, const float* cache, size_t n_dims); /* ops.rs:199-221 */
void vxo_rope_normal(float* x, size_t heads, size_t head_dim, const float* cache, size_t n_dims); /* ops.rs:199-221 */
float vxo_ggml_expf(float x);                                             /* ops.rs:314-377, one lane */
void vxo_ggml_expf_batch(const float* x, size_t n, float* out);
void vxo_swiglu(const float* gate, const float* up, size_t n, float* out); /* ops.rs:430-464 (AVX2 path) */
void vxo_attend_head(const uint16_t* q_f16, const uint16_t* kbase, const uint16_t* vbase, size_t stride,
                     size_t head_dim, size_t seq_len, size_t max_ctx, float scale, float* out); /* attention.rs:436-542 */
void vxo_projection(const uint8_t* planar, size_t rows, size_t cols, float ws, const int8_t* q, float as, float* out);

/* The model of BASELINE.json configs[3] with weights generated from `seed` (projections: kind 0..6 = q, k, v, o, gate,
 * up, down; norms: kind 0..3 = attn, attn_sub, ffn, ffn_sub, layer n_layers kind 0 = output norm). */
void vxo_projection_shape(const vxo_model_config* c, int kind, size_t* rows, size_t* cols);
vxo_model* vxo_model_create(const vxo_model_config* cfg, uint64_t seed);
void vxo_model_free(vxo_model* m);
const uint8_t* vxo_model_projection(const vxo_model* m, size_t layer, int kind, float* weight_scale);
const float* vxo_model_norm(const vxo_model* m, size_t layer, int kind);
const uint16_t* vxo_model_embedding(const vxo_model* m);
const uint16_t* vxo_model_head(const vxo_model* m); /* the untied head, or the embedding when tied */
const float* vxo_model_rope_table(const vxo_model* m);
void vxo_model_reset(vxo_model* m);
void vxo_model_kv_get(const vxo_model* m, size_t layer, size_t pos, size_t kv_head, uint16_t* k, uint16_t* v);
void vxo_model_kv_set(vxo_model* m, size_t layer, size_t pos, size_t kv_head, const uint16_t* k, const uint16_t* v);
uint32_t vxo_model_forward(vxo_model* m, uint32_t token, size_t pos, float* logits);
void vxo_model_generate(vxo_model* m, const uint32_t* prompt, size_t n_prompt, size_t n_new, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif
