/*
 * decode_oracle.c - CPU restatement of the reference's decode step (TEST INFRASTRUCTURE ONLY).
 *
 * The token loop of BASELINE.json configs[3] (a BitNet-b1.58-2B-shaped model with random weights): RMSNorm, per-token
 * int8 quantization, ternary projections with the layer epilogue, NEOX RoPE, an F16 KV cache, the FP16-accumulator
 * flash attention of bitnet.cpp with its 4-chunk split, sub-norms, ReLU^2, a tied bf16 head and greedy argmax; and the
 * Falcon3 variant of the same loop (Normal RoPE, no sub-norms, SwiGLU with ggml's vector expf, an f16 embedding and
 * an untied f16 head, ModelConfig::falcon3_*_default, config.rs:179-227). Each
 * function names the reference file:line it restates; the FP operations, their order and their fused multiply-adds
 * are the reference's. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline load this code; the product
 * (quintrit_amd/) never calls it. OpenMP splits rows of independent outputs only, so results do not depend on the
 * thread count.
 */
#include "decode_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- bf16 / f16 vector primitives ------------------------------------------------------------------------------- */

/* ops.rs:652-665 */
float vxo_bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t vxo_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 64u);
    return (uint16_t)((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

/* ops.rs:669-713 (ggml_vec_dot_bf16): four accumulators of eight lanes, acc + x*y rounded separately, reduced as
 * (a0 + a2) + (a1 + a3) and ((l0+l4) + (l2+l6)) + ((l1+l5) + (l3+l7)); the tail in double. */
float vxo_ggml_dot_bf16(const uint16_t* x, const uint16_t* y, size_t n) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l) {
                const size_t k = i + 8 * (size_t)j + (size_t)l;
                const float p = vxo_bf16_to_f32(x[k]) * vxo_bf16_to_f32(y[k]);
                acc[j][l] = acc[j][l] + p;
            }
    float a[8];
    for (int l = 0; l < 8; ++l) a[l] = (acc[0][l] + acc[2][l]) + (acc[1][l] + acc[3][l]);
    const float g0 = a[4] + a[0], g1 = a[5] + a[1], g2 = a[6] + a[2], g3 = a[7] + a[3];
    double sum = (double)((g0 + g2) + (g1 + g3));
    for (; i < n; ++i) sum += (double)(vxo_bf16_to_f32(x[i]) * vxo_bf16_to_f32(y[i]));
    return (float)sum;
}

/* ops.rs:960-1015 (ggml_vec_dot_f16, AVX2 + F16C + FMA): four accumulators of eight lanes take fma(x, y, acc) per 32
 * values, red = (s0 + s2) + (s1 + s3), t[k] = red[k] + red[k + 4], result (t0 + t1) + (t2 + t3); tail sequential. */
float vxo_ggml_dot_f16(const uint16_t* x, const uint16_t* y, size_t n) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l) {
                const size_t k = i + 8 * (size_t)j + (size_t)l;
                acc[j][l] = fmaf(vxo_f16_to_f32(x[k]), vxo_f16_to_f32(y[k]), acc[j][l]);
            }
    float red[8];
    for (int l = 0; l < 8; ++l) red[l] = (acc[0][l] + acc[2][l]) + (acc[1][l] + acc[3][l]);
    float t[4];
    for (int k = 0; k < 4; ++k) t[k] = red[k] + red[k + 4];
    float sum = (t[0] + t[1]) + (t[2] + t[3]);
    for (; i < n; ++i) {
        const float p = vxo_f16_to_f32(x[i]) * vxo_f16_to_f32(y[i]);
        sum = sum + p;
    }
    return sum;
}

/* ops.rs:1254-1300 (the AVX2 path): the first n & ~31 values are y = f16(fma(x, v, y)) (_mm256_fmadd_ps), the rest
 * y = f16(y + x * v) with a separate multiply and add (Rust does not contract; this file is built with
 * -ffp-contract=off). */
void vxo_vec_mad_f16(uint16_t* y, const uint16_t* x, float v, size_t n) {
    const size_t np = n & ~(size_t)31;
    size_t i = 0;
    for (; i < np; ++i) y[i] = vxo_f32_to_f16(fmaf(vxo_f16_to_f32(x[i]), v, vxo_f16_to_f32(y[i])));
    for (; i < n; ++i) {
        const float fy = vxo_f16_to_f32(y[i]), fx = vxo_f16_to_f32(x[i]);
        const float p = fx * v;
        y[i] = vxo_f32_to_f16(fy + p);
    }
}

/* ops.rs:1304-1345: y = f16(y * v). */
void vxo_vec_scale_f16(uint16_t* y, float v, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = vxo_f32_to_f16(vxo_f16_to_f32(y[i]) * v);
}

void vxo_expf_batch(const float* x, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = expf(x[i]);
}

/* ---- RoPE ---------------------------------------------------------------------------------------------------------- */

/* ops.rs:121-140 with freq_scale = 1, ext_factor = 0, attn_factor = 1 (RopeConfig::plain): theta_scale =
 * freq_base^(-2 / n_dims); theta_k = pos * theta_scale^k accumulated by repeated multiplication; cache = (cos, sin). */
void vxo_rope_cache(size_t pos, size_t n_dims, float freq_base, float* cache) {
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    float theta = (float)pos;
    for (size_t i = 0; i < n_dims / 2; ++i) {
        cache[2 * i] = cosf(theta) * 1.0f;
        cache[2 * i + 1] = sinf(theta) * 1.0f;
        theta *= theta_scale;
    }
}

/* ops.rs:199-221: NEOX pairing (offset n_dims / 2, stride 1); x0' = fma(x0, c, -(x1 s)), x1' = fma(x0, s, x1 c). */
void vxo_rope_neox(float* x, size_t heads, size_t head_dim, const float* cache, size_t n_dims) {
    const size_t half = n_dims / 2;
    for (size_t h = 0; h < heads; ++h) {
        float* head = x + h * head_dim;
        for (size_t i = 0; i < half; ++i) {
            const float c = cache[2 * i], s = cache[2 * i + 1];
            const float x0 = head[i], x1 = head[i + half];
            const float x1s = x1 * s, x1c = x1 * c;
            head[i] = fmaf(x0, c, -x1s);
            head[i + half] = fmaf(x0, s, x1c);
        }
    }
}

/* ops.rs:199-221: Normal pairing (offset 1, stride 2): pair i rotates (x[2i], x[2i + 1]) with the same fused
 * multiply-adds. */
void vxo_rope_normal(float* x, size_t heads, size_t head_dim, const float* cache, size_t n_dims) {
    for (size_t h = 0; h < heads; ++h) {
        float* head = x + h * head_dim;
        for (size_t i = 0; i < n_dims / 2; ++i) {
            const float c = cache[2 * i], s = cache[2 * i + 1];
            const float x0 = head[2 * i], x1 = head[2 * i + 1];
            const float x1s = x1 * s, x1c = x1 * c;
            head[2 * i] = fmaf(x0, c, -x1s);
            head[2 * i + 1] = fmaf(x0, s, x1c);
        }
    }
}

/* ---- SiLU / SwiGLU ------------------------------------------------------------------------------------------------ */

static float f32_of(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t bits_of(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* ops.rs:314-377 (ggml_v_expf_avx2) for one lane. n = round(x log2 e) by the 1.5 * 2^23 shift; b = x - n ln 2 in two
 * parts (fnmadd = fma with the product negated); j = the degree-5 polynomial of b without its constant term;
 * k = 2^n built in the exponent field. |n| <= 126: k + k j. Beyond, 2^n is split into s1 s2 (s1 = 2^+-127 by the sign
 * of n) to reach the subnormal / overflow ranges, and |n| > 192 gives s1 * s1 (0 or inf). A lane's result does not
 * depend on the other lanes: the whole-vector shortcut returns the same fma(j, k, k). */
float vxo_ggml_expf(float x) {
    const float r = f32_of(0x4b400000u);
    const float z = fmaf(x, f32_of(0x3fb8aa3bu), r);
    const float n = z - r;
    const float b = fmaf(-n, f32_of(0x35bfbe8eu), fmaf(-n, f32_of(0x3f317200u), x));
    const uint32_t e = bits_of(z) << 23;
    const float k = f32_of(e + bits_of(1.0f));
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(f32_of(0x3c072010u), b, f32_of(0x3d2b9f17u)), u,
                              fmaf(f32_of(0x3e2aaf33u), b, f32_of(0x3efffedbu))),
                         u, f32_of(0x3f7ffff6u) * b);
    if (!(fabsf(n) > 126.0f)) return fmaf(k, j, k);
    const uint32_t g = n <= 0.0f ? 0x82000000u : 0u;
    const float s1 = f32_of(g + 0x7f000000u);
    const float s2 = f32_of(e - g);
    if (fabsf(n) > 192.0f) return s1 * s1;
    return fmaf(s2, j, s2) * s1;
}

void vxo_ggml_expf_batch(const float* x, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = vxo_ggml_expf(x[i]);
}

/* ops.rs:430-464 (swiglu, AVX2 + FMA path): blocks of 8 take ggml_v_silu = x / (1 + ggml_v_expf(0 - x)) times up; the
 * last n % 8 values take v / (1 + expf(-v)) * up with the libm exponential. */
void vxo_swiglu(const float* gate, const float* up, size_t n, float* out) {
    const size_t n8 = n / 8 * 8;
    for (size_t i = 0; i < n8; ++i) {
        const float v = gate[i];
        const float den = 1.0f + vxo_ggml_expf(0.0f - v);
        const float s = v / den;
        out[i] = s * up[i];
    }
    for (size_t i = n8; i < n; ++i) {
        const float v = gate[i];
        const float den = 1.0f + expf(-v);
        const float s = v / den;
        out[i] = s * up[i];
    }
}

/* ---- attention --------------------------------------------------------------------------------------------------- */

/* attention.rs:436-468 (attend_range): online softmax over positions [start, end) with an FP16 value accumulator. */
static void attend_range(const uint16_t* q_f16, const uint16_t* kbase, const uint16_t* vbase, size_t stride,
                         size_t head_dim, size_t start, size_t end, float scale, uint16_t* vkq, float* m_out,
                         float* s_out) {
    float s_sum = 0.0f, max_score = -INFINITY;
    memset(vkq, 0, head_dim * 2);
    for (size_t p = start; p < end; ++p) {
        const float score = vxo_ggml_dot_f16(q_f16, kbase + p * stride, head_dim) * scale;
        const float m_old = max_score;
        float ms = 1.0f, vs = 1.0f;
        if (score > max_score) {
            max_score = score;
            ms = expf(m_old - max_score);
            vxo_vec_scale_f16(vkq, ms, head_dim);
        } else {
            vs = expf(score - max_score);
        }
        vxo_vec_mad_f16(vkq, vbase + p * stride, vs, head_dim);
        s_sum = fmaf(s_sum, ms, vs);
    }
    *m_out = max_score;
    *s_out = s_sum;
}

/* attention.rs:483-542 (attend_head, FP16 values): n_kv = min(max_ctx, max(roundup(seq, 256), 256)); one online
 * softmax below a padded length of 512, otherwise 4 chunks of ceil(n_kv / 4) combined in order. kbase/vbase point at
 * position 0 of this layer and KV head; stride = elements between positions. */
void vxo_attend_head(const uint16_t* q_f16, const uint16_t* kbase, const uint16_t* vbase, size_t stride,
                     size_t head_dim, size_t seq_len, size_t max_ctx, float scale, float* out) {
    uint16_t vkq[512];
    float acc[512];
    size_t n_kv = (seq_len + 255) / 256 * 256;
    if (n_kv < 256) n_kv = 256;
    if (n_kv > max_ctx) n_kv = max_ctx;
    if (n_kv < 512) {
        float m, s;
        attend_range(q_f16, kbase, vbase, stride, head_dim, 0, seq_len, scale, vkq, &m, &s);
        const float s_inv = s == 0.0f ? 0.0f : 1.0f / s;
        for (size_t d = 0; d < head_dim; ++d) out[d] = vxo_f16_to_f32(vkq[d]) * s_inv;
        return;
    }
    const size_t chunk = (n_kv + 3) / 4;
    float m_final = -INFINITY, s_final = 0.0f;
    for (size_t d = 0; d < head_dim; ++d) acc[d] = 0.0f;
    for (size_t c = 0; c < 4; ++c) {
        const size_t start = c * chunk;
        size_t end = start + chunk;
        if (end > n_kv) end = n_kv;
        if (end > seq_len) end = seq_len;
        if (start >= end) continue;
        float m_chunk, s_chunk;
        attend_range(q_f16, kbase, vbase, stride, head_dim, start, end, scale, vkq, &m_chunk, &s_chunk);
        if (s_chunk == 0.0f) continue;
        const float m_new = fmaxf(m_final, m_chunk);
        const float scale_old = expf(m_final - m_new);
        const float scale_new = expf(m_chunk - m_new);
        for (size_t d = 0; d < head_dim; ++d) {
            const float vn = vxo_f16_to_f32(vkq[d]) * scale_new;
            acc[d] = fmaf(acc[d], scale_old, vn);
        }
        const float sn = s_chunk * scale_new;
        s_final = fmaf(s_final, scale_old, sn);
        m_final = m_new;
    }
    if (s_final != 0.0f) {
        const float s_inv = 1.0f / s_final;
        for (size_t d = 0; d < head_dim; ++d) out[d] = acc[d] * s_inv;
    } else {
        for (size_t d = 0; d < head_dim; ++d) out[d] = acc[d];
    }
}

/* ---- ternary projection ------------------------------------------------------------------------------------------ */

/* The exact int32 product of a planar velurex matrix with int8 activations (the quantity every kernel of
 * quintrit-core/src/simd computes), then the layer epilogue of layer.rs:246-253: y = float(acc) * (ws / as), zeros
 * when as <= 0. Rows are independent, so they are split between threads. */
void vxo_projection(const uint8_t* planar, size_t rows, size_t cols, float ws, const int8_t* q, float as, float* out) {
    const size_t rb = vxo_planar_row_bytes(cols);
    if (!(as > 0.0f)) {
        for (size_t r = 0; r < rows; ++r) out[r] = 0.0f;
        return;
    }
    int8_t tt[256][5];
    for (int b = 0; b < 256; ++b) vxo_byte_to_trits((uint8_t)b, tt[b]);
    const float post = ws / as;
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        const uint8_t* row = planar + r * rb;
        int32_t acc = 0;
        for (size_t b = 0; b < rb / 32; ++b)
            for (size_t j = 0; j < 32; ++j) {
                const int8_t* t = tt[row[b * 32 + j]];
                for (size_t p = 0; p < 5; ++p) {
                    const size_t c = b * 160 + p * 32 + j;
                    if (c < cols) acc += (int32_t)t[p] * (int32_t)q[c];
                }
            }
        out[r] = (float)acc * post;
    }
}

/* ---- the model ---------------------------------------------------------------------------------------------------- */

enum { Q, K, V, O, GATE, UP, DOWN, NPROJ };

struct vxo_model {
    vxo_model_config cfg;
    uint8_t* w[VXO_MAX_LAYERS][NPROJ];
    float ws[VXO_MAX_LAYERS][NPROJ];
    float* norm[VXO_MAX_LAYERS][4]; /* attn_norm, attn_sub_norm, ffn_norm, ffn_sub_norm */
    float* out_norm;
    uint16_t* emb;  /* bf16 or f16 [vocab][hidden], also the head when tied */
    uint16_t* head; /* the untied head (same type), or NULL */
    uint16_t* kc;  /* f16 [layer][pos][kv_head][head_dim] (kv_cache.rs:32-35) */
    uint16_t* vc;
    float* rope; /* [max_ctx][head_dim] cos/sin pairs */
};

void vxo_projection_shape(const vxo_model_config* c, int kind, size_t* rows, size_t* cols) {
    const size_t qd = (size_t)c->n_heads * c->head_dim, kvd = (size_t)c->n_kv_heads * c->head_dim;
    switch (kind) {
        case Q: *rows = qd; *cols = c->hidden; break;
        case K:
        case V: *rows = kvd; *cols = c->hidden; break;
        case O: *rows = c->hidden; *cols = qd; break;
        case GATE:
        case UP: *rows = c->ffn; *cols = c->hidden; break;
        default: *rows = c->hidden; *cols = c->ffn; break;
    }
}

static uint64_t mix_seed(uint64_t seed, uint64_t a, uint64_t b) {
    uint64_t s = seed ^ (a * 0x9e3779b97f4a7c15ull) ^ (b * 0xc2b2ae3d27d4eb4full);
    return vxo_splitmix64(&s);
}

/* Normal(0, sigma) from splitmix64 with Box-Muller (glibc log, cos, sin in double), rounded to float. */
static void gen_normal(uint64_t seed, size_t n, float sigma, float* out) {
    uint64_t st = seed;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = 1.0 - (double)(vxo_splitmix64(&st) >> 11) * 0x1.0p-53;
        const double u2 = (double)(vxo_splitmix64(&st) >> 11) * 0x1.0p-53;
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(6.283185307179586 * u2) * sigma);
        if (i + 1 < n) out[i + 1] = (float)(r * sin(6.283185307179586 * u2) * sigma);
    }
}

vxo_model* vxo_model_create(const vxo_model_config* cfg, uint64_t seed) {
    if (cfg->n_layers > VXO_MAX_LAYERS || cfg->head_dim > 512 || cfg->n_heads % cfg->n_kv_heads) return NULL;
    vxo_model* m = (vxo_model*)calloc(1, sizeof(vxo_model));
    m->cfg = *cfg;
    const size_t L = cfg->n_layers;
#pragma omp parallel for schedule(dynamic)
    for (size_t t = 0; t < L * NPROJ; ++t) {
        const size_t l = t / NPROJ;
        const int kind = (int)(t % NPROJ);
        size_t rows, cols;
        vxo_projection_shape(cfg, kind, &rows, &cols);
        int8_t* trits = (int8_t*)malloc(rows * cols);
        vxo_gen_trits(mix_seed(seed, 1 + l, (uint64_t)kind), rows * cols, 35, 30, trits);
        m->w[l][kind] = (uint8_t*)malloc(rows * vxo_planar_row_bytes(cols));
        vxo_pack_matrix(trits, rows, cols, m->w[l][kind]);
        free(trits);
        m->ws[l][kind] = 1.0f / sqrtf((float)cols);
    }
    for (size_t l = 0; l <= L; ++l) {
        for (int k = 0; k < 4; ++k) {
            if (l == L && k > 0) break;
            if (cfg->no_sub_norm && (k == 1 || k == 3)) continue;
            const size_t n = (k == 3) ? cfg->ffn : (k == 1 ? (size_t)cfg->n_heads * cfg->head_dim : cfg->hidden);
            float* w = (float*)malloc(n * sizeof(float));
            uint64_t st = mix_seed(seed, 1000 + l, (uint64_t)k);
            for (size_t i = 0; i < n; ++i) w[i] = 0.75f + (float)(vxo_splitmix64(&st) >> 40) * 0x1.0p-24f * 0.5f;
            if (l == L) m->out_norm = w;
            else m->norm[l][k] = w;
        }
    }
    const size_t ne = (size_t)cfg->vocab * cfg->hidden;
    const size_t rows_per = 1024;
    for (int t = 0; t < (cfg->untied ? 2 : 1); ++t) {
        uint16_t* dst = (uint16_t*)malloc(ne * 2);
        if (t == 0) m->emb = dst;
        else m->head = dst;
#pragma omp parallel for schedule(dynamic)
        for (size_t r0 = 0; r0 < cfg->vocab; r0 += rows_per) {
            const size_t r1 = r0 + rows_per < cfg->vocab ? r0 + rows_per : cfg->vocab;
            float* tmp = (float*)malloc((r1 - r0) * cfg->hidden * sizeof(float));
            gen_normal(mix_seed(seed, 5000 + r0, (uint64_t)t), (r1 - r0) * cfg->hidden, 0.02f, tmp);
            for (size_t i = 0; i < (r1 - r0) * cfg->hidden; ++i)
                dst[r0 * cfg->hidden + i] = cfg->emb_f16 ? vxo_f32_to_f16(tmp[i]) : vxo_f32_to_bf16(tmp[i]);
            free(tmp);
        }
    }
    const size_t kvn = L * cfg->max_ctx * cfg->n_kv_heads * cfg->head_dim;
    m->kc = (uint16_t*)calloc(kvn, 2);
    m->vc = (uint16_t*)calloc(kvn, 2);
    m->rope = (float*)malloc((size_t)cfg->max_ctx * cfg->head_dim * sizeof(float));
    for (size_t p = 0; p < cfg->max_ctx; ++p) vxo_rope_cache(p, cfg->head_dim, cfg->rope_theta, m->rope + p * cfg->head_dim);
    return m;
}

void vxo_model_free(vxo_model* m) {
    if (!m) return;
    for (size_t l = 0; l < m->cfg.n_layers; ++l) {
        for (int k = 0; k < NPROJ; ++k) free(m->w[l][k]);
        for (int k = 0; k < 4; ++k) free(m->norm[l][k]);
    }
    free(m->out_norm);
    free(m->emb);
    free(m->head);
    free(m->kc);
    free(m->vc);
    free(m->rope);
    free(m);
}

const uint8_t* vxo_model_projection(const vxo_model* m, size_t layer, int kind, float* weight_scale) {
    *weight_scale = m->ws[layer][kind];
    return m->w[layer][kind];
}
const float* vxo_model_norm(const vxo_model* m, size_t layer, int kind) {
    return layer == m->cfg.n_layers ? m->out_norm : m->norm[layer][kind];
}
const uint16_t* vxo_model_embedding(const vxo_model* m) { return m->emb; }
const uint16_t* vxo_model_head(const vxo_model* m) { return m->head ? m->head : m->emb; }
const float* vxo_model_rope_table(const vxo_model* m) { return m->rope; }

/* Test access to the KV cache (KVCache::get_key / get_val and append, kv_cache.rs:124-155): the head_dim f16 key and
 * value of (layer, pos, kv_head). With them a test can give the oracle a long cache and run single steps at its end. */
void vxo_model_kv_get(const vxo_model* m, size_t layer, size_t pos, size_t kv_head, uint16_t* k, uint16_t* v) {
    const vxo_model_config* c = &m->cfg;
    const size_t off = (layer * c->max_ctx + pos) * c->n_kv_heads * c->head_dim + kv_head * c->head_dim;
    memcpy(k, m->kc + off, c->head_dim * 2);
    memcpy(v, m->vc + off, c->head_dim * 2);
}

void vxo_model_kv_set(vxo_model* m, size_t layer, size_t pos, size_t kv_head, const uint16_t* k, const uint16_t* v) {
    const vxo_model_config* c = &m->cfg;
    const size_t off = (layer * c->max_ctx + pos) * c->n_kv_heads * c->head_dim + kv_head * c->head_dim;
    memcpy(m->kc + off, k, c->head_dim * 2);
    memcpy(m->vc + off, v, c->head_dim * 2);
}

void vxo_model_reset(vxo_model* m) {
    const size_t kvn = m->cfg.n_layers * m->cfg.max_ctx * m->cfg.n_kv_heads * m->cfg.head_dim;
    memset(m->kc, 0, kvn * 2);
    memset(m->vc, 0, kvn * 2);
}

/* model.rs:282-377 + model.rs:64-203 + attention.rs:115-260 for one token at `pos`; logits (vocab) and the greedy
 * token (sampler.rs:73-83: the first maximum). */
uint32_t vxo_model_forward(vxo_model* m, uint32_t token, size_t pos, float* logits) {
    const vxo_model_config* c = &m->cfg;
    const size_t H = c->hidden, F = c->ffn, hd = c->head_dim;
    const size_t qd = (size_t)c->n_heads * hd, kvd = (size_t)c->n_kv_heads * hd;
    const size_t big = F > qd ? F : qd;
    float* x = (float*)malloc(H * 4);
    float* xn = (float*)malloc((big > H ? big : H) * 4);
    int8_t* qi = (int8_t*)malloc(big > H ? big : H);
    float* q = (float*)malloc(qd * 4);
    float* k = (float*)malloc(kvd * 4);
    float* v = (float*)malloc(kvd * 4);
    float* att = (float*)malloc(qd * 4);
    float* proj = (float*)malloc(H * 4);
    float* gate = (float*)malloc(F * 4);
    float* up = (float*)malloc(F * 4);
    float* inter = (float*)malloc(F * 4);
    uint16_t* qh = (uint16_t*)malloc(qd * 2);

    for (size_t i = 0; i < H; ++i) {  /* model.rs:309-316 */
        const uint16_t e = m->emb[(size_t)token * H + i];
        x[i] = c->emb_f16 ? vxo_f16_to_f32(e) : vxo_bf16_to_f32(e);
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const size_t pos_stride = (size_t)c->n_kv_heads * hd;
    for (size_t l = 0; l < c->n_layers; ++l) {
        /* attention block (attention.rs:115-260) */
        vxo_rms_norm(x, m->norm[l][0], H, c->rms_eps, xn);
        float as = vxo_quantize_i8(xn, H, 127.0f, qi);
        vxo_projection(m->w[l][Q], qd, H, m->ws[l][Q], qi, as, q);
        vxo_projection(m->w[l][K], kvd, H, m->ws[l][K], qi, as, k);
        vxo_projection(m->w[l][V], kvd, H, m->ws[l][V], qi, as, v);
        const float* cache = m->rope + pos * hd;
        if (c->rope_mode == VXO_ROPE_NORMAL) {
            vxo_rope_normal(q, c->n_heads, hd, cache, hd);
            vxo_rope_normal(k, c->n_kv_heads, hd, cache, hd);
        } else {
            vxo_rope_neox(q, c->n_heads, hd, cache, hd);
            vxo_rope_neox(k, c->n_kv_heads, hd, cache, hd);
        }
        uint16_t* kl = m->kc + l * c->max_ctx * pos_stride;
        uint16_t* vl = m->vc + l * c->max_ctx * pos_stride;
        for (size_t i = 0; i < kvd; ++i) {
            kl[pos * pos_stride + i] = vxo_f32_to_f16(k[i]);
            vl[pos * pos_stride + i] = vxo_f32_to_f16(v[i]);
        }
        for (size_t i = 0; i < qd; ++i) qh[i] = vxo_f32_to_f16(q[i]);
        const size_t gqa = c->n_heads / c->n_kv_heads;
#pragma omp parallel for schedule(static)
        for (size_t h = 0; h < c->n_heads; ++h) {
            const size_t kvh = h / gqa;
            vxo_attend_head(qh + h * hd, kl + kvh * hd, vl + kvh * hd, pos_stride, hd, pos + 1, c->max_ctx, scale,
                            att + h * hd);
        }
        if (c->no_sub_norm) { /* attention.rs:232-254 */
            as = vxo_quantize_i8(att, qd, 127.0f, qi);
        } else {
            vxo_rms_norm(att, m->norm[l][1], qd, c->rms_eps, xn);
            as = vxo_quantize_i8(xn, qd, 127.0f, qi);
        }
        vxo_projection(m->w[l][O], H, qd, m->ws[l][O], qi, as, proj);
        for (size_t i = 0; i < H; ++i) x[i] = x[i] + proj[i];
        /* feed-forward block (model.rs:101-199) */
        vxo_rms_norm(x, m->norm[l][2], H, c->rms_eps, xn);
        as = vxo_quantize_i8(xn, H, 127.0f, qi);
        vxo_projection(m->w[l][GATE], F, H, m->ws[l][GATE], qi, as, gate);
        vxo_projection(m->w[l][UP], F, H, m->ws[l][UP], qi, as, up);
        if (c->act == VXO_ACT_SILU) {
            vxo_swiglu(gate, up, F, inter);
        } else {
            for (size_t i = 0; i < F; ++i) { /* relu2 then elementwise_mul (ops.rs:301-308, 467-473) */
                const float p = gate[i] > 0.0f ? gate[i] : 0.0f;
                const float a = p * p;
                inter[i] = a * up[i];
            }
        }
        if (c->no_sub_norm) { /* model.rs:172-190 */
            as = vxo_quantize_i8(inter, F, 127.0f, qi);
        } else {
            vxo_rms_norm(inter, m->norm[l][3], F, c->rms_eps, xn);
            as = vxo_quantize_i8(xn, F, 127.0f, qi);
        }
        vxo_projection(m->w[l][DOWN], H, F, m->ws[l][DOWN], qi, as, proj);
        for (size_t i = 0; i < H; ++i) x[i] = x[i] + proj[i];
    }
    /* final norm and the head (model.rs:326-376): x_final rounded to the head's type, then ggml_vec_dot_f16 (f16) or
     * ggml_vec_dot_bf16 (bf16) against every row of the head (the embedding when tied) */
    vxo_rms_norm(x, m->out_norm, H, c->rms_eps, xn);
    uint16_t* xb = (uint16_t*)malloc(H * 2);
    for (size_t i = 0; i < H; ++i) xb[i] = c->emb_f16 ? vxo_f32_to_f16(xn[i]) : vxo_f32_to_bf16(xn[i]);
    const uint16_t* hw = m->head ? m->head : m->emb;
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < c->vocab; ++r)
        logits[r] = c->emb_f16 ? vxo_ggml_dot_f16(xb, hw + r * H, H) : vxo_ggml_dot_bf16(xb, hw + r * H, H);
    uint32_t best = 0;
    float bv = logits[0];
    for (size_t r = 1; r < c->vocab; ++r)
        if (logits[r] > bv) {
            bv = logits[r];
            best = (uint32_t)r;
        }
    free(xb);
    free(x); free(xn); free(qi); free(q); free(k); free(v); free(att); free(proj); free(gate); free(up); free(inter);
    free(qh);
    return best;
}

/* engine.rs:590-686 (greedy, prompt fed one token at a time): n_new tokens after the prompt. */
void vxo_model_generate(vxo_model* m, const uint32_t* prompt, size_t n_prompt, size_t n_new, uint32_t* out) {
    float* logits = (float*)malloc(m->cfg.vocab * sizeof(float));
    vxo_model_reset(m);
    uint32_t next = 0;
    size_t pos = 0;
    for (; pos < n_prompt; ++pos) next = vxo_model_forward(m, prompt[pos], pos, logits);
    for (size_t t = 0; t < n_new; ++t) {
        out[t] = next;
        if (t + 1 < n_new) next = vxo_model_forward(m, next, pos++, logits);
    }
    free(logits);
}
