// Decode step of a ternary decoder on gfx950: the token loop around the velurex GEMV.
//
// One step follows the reference's CPU runtime operation by operation (quintrit-runtime/src/model.rs:64-377,
// attention.rs:115-542, ops.rs), so that logits and greedy tokens are bit-identical to it:
//   embed (bf16 row -> f32)
//   per layer: [residual add +] RMSNorm + int8 quantization -> staged activations (one kernel)
//              q, k, v projections (one plan, the fp32 layer epilogue)           -> NEOX RoPE, f16 KV append
//              FP16-accumulator flash attention with bitnet.cpp's 4-chunk split  -> sub-norm + quantization
//              o projection -> residual add + RMSNorm + quantization -> gate, up (one plan)
//              ReLU^2(gate) * up + sub-norm + quantization -> down projection
//   residual add + final RMSNorm -> bf16 -> tied bf16 head (ggml_vec_dot_bf16 order) -> greedy argmax (first maximum)
// The position, the token and the generated ids live in device memory, so the whole step is one HIP graph replayed per
// token (the reference's CUDA graph is position-independent the same way, quintrit-runtime/src/gpu.rs:459-493).
//
// RMSNorm (ops.rs:43-57) sums the f32 squares sequentially in f64 and rounds sum / n to f32. Here the squares are
// summed as a tree; both sums differ from the exact one by at most (n - 1) 2^-53 sum, so when the f32 mean is the same
// at both ends of that interval the tree's mean is the reference's; otherwise (rare) one lane redoes the sum in the
// reference's order. The exponentials are glibc's expf (vx_expf.h).
#include "vx_expf.h"
#include "vx_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

namespace vx {

// ---- small helpers --------------------------------------------------------------------------------------------------------

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_f32(uint16_t h) { return bits_f32(static_cast<uint32_t>(h) << 16); }

__device__ __forceinline__ uint16_t f32_bf16(float f) {  // ops.rs:658-665
    const uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 64u);
    return static_cast<uint16_t>((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

// f32 -> f16, round to nearest even (the F16C conversion). The reference rounds every f16 result twice: the
// arithmetic to f32, then the f32 to f16. The empty asm keeps the f32 value opaque, so the compiler cannot fold the
// producing fma or multiply and the conversion into one v_fma_mixlo_f16, which rounds once.
__device__ __forceinline__ float keep_f32(float f) {
    asm volatile("" : "+v"(f));
    return f;
}
__device__ __forceinline__ uint16_t f32_f16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(keep_f32(f)));
}
__device__ __forceinline__ float f16_f32(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

// ---- RMSNorm + quantization ------------------------------------------------------------------------------------------------

enum NormInput : uint32_t {
    kInPlain = 0,     // v = a[i]
    kInResidual = 1,  // v = a[i] + b[i], written back to a (add_residual, ops.rs:476-481)
    kInRelu2Mul = 2,  // v = relu2(a[i]) * b[i] (ops.rs:301-308, 467-473)
};

struct NormArgs {
    float* a;
    const float* b;
    const float* gamma;
    uint32_t n;
    float eps;
    uint32_t input;
    uint32_t quantize;      // 1: int8 codes into `staged` + scale into act_scale; 0: bf16 of y into out_bf16
    uint8_t* staged;        // GEMV staging (kStageHeader + dbr * 8 bytes)
    float* act_scale;
    uint16_t* out_bf16;
    uint32_t tbr, dbr;      // tile and device row bytes of n columns
};

constexpr int kNormThreads = 1024;
constexpr uint32_t kNormMax = 8192;  // largest vector

__global__ __launch_bounds__(kNormThreads) void norm_quant_kernel(NormArgs p) {
    __shared__ float ys[kNormMax];
    __shared__ int8_t qs[kNormMax];
    __shared__ double red_d[16];
    __shared__ float red_f[16];
    __shared__ int red_i[16];
    __shared__ float s_mean;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n = p.n;

    double ss = 0.0;
    for (uint32_t i = tid; i < n; i += kNormThreads) {
        float v;
        if (p.input == kInPlain) {
            v = p.a[i];
        } else if (p.input == kInResidual) {
            v = p.a[i] + p.b[i];
            p.a[i] = v;
        } else {
            const float g = p.a[i];
            const float pos = g > 0.0f ? g : 0.0f;
            const float sq = pos * pos;
            v = sq * p.b[i];
        }
        ys[i] = v;
        const float sqv = v * v;
        ss += static_cast<double>(sqv);
    }
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if (lane == 0) red_d[wave] = ss;
    __syncthreads();
    if (tid == 0) {
        double t = 0.0;
        for (int w = 0; w < kNormThreads / 64; ++w) t += red_d[w];
        // the sequential f64 sum of the reference lies within d of t (both within (n-1) 2^-53 t of the exact sum)
        const double d = 2.0 * static_cast<double>(n) * 0x1.0p-53 * t;
        float mean = static_cast<float>(t / static_cast<double>(n));
        const float lo = static_cast<float>((t - d) / static_cast<double>(n));
        const float hi = static_cast<float>((t + d) / static_cast<double>(n));
        if (lo != hi) {  // too close to an f32 rounding boundary: redo the sum in the reference's order
            double seq = 0.0;
            for (uint32_t i = 0; i < n; ++i) {
                const float sqv = ys[i] * ys[i];
                seq += static_cast<double>(sqv);
            }
            mean = static_cast<float>(seq / static_cast<double>(n));
        }
        s_mean = mean;
    }
    __syncthreads();
    const float scale = 1.0f / __builtin_sqrtf(s_mean + p.eps);
    float mx = 0.0f;
    for (uint32_t i = tid; i < n; i += kNormThreads) {
        const float t = ys[i] * scale;
        const float y = t * p.gamma[i];
        ys[i] = y;
        const float ay = __builtin_fabsf(y);
        if (ay > mx) mx = ay;
        if (!p.quantize) p.out_bf16[i] = f32_bf16(y);
    }
    if (!p.quantize) return;
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(mx, off);
        if (o > mx) mx = o;
    }
    if (lane == 0) red_f[wave] = mx;
    __syncthreads();
    float m = 0.0f;
    for (int w = 0; w < kNormThreads / 64; ++w)
        if (red_f[w] > m) m = red_f[w];
    // quantize_activations_int8_with_range (ops.rs:241-267), levels 127
    const float s = m > 0.0f ? 127.0f / m : 0.0f;
    for (uint32_t i = tid; i < n; i += kNormThreads) {
        int q = 0;
        if (m > 0.0f) {
            float r = __builtin_roundf(ys[i] * s);
            r = r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r);
            q = static_cast<int>(r);
        }
        qs[i] = static_cast<int8_t>(q);
    }
    __syncthreads();
    // GEMV staging (vx_stage_acts_dev's format): nibbles of the five activations of each device byte-column
    const uint32_t full = n / 160u * 32u;
    uint2* ent = reinterpret_cast<uint2*>(p.staged + kStageHeader);
    int sum = 0;
    for (uint32_t c = tid; c < p.dbr; c += kNormThreads) {  // the entries of vx_stage_acts_dev
        uint32_t lo = 0, hi = 0;
        for (uint32_t k = 0; k < 5; ++k) {
            const uint32_t idx = c < full ? (c / 32u) * 160u + k * 32u + (c % 32u) : (n / 160u) * 160u + 5u * (c - full) + k;
            const int x = c < p.tbr && idx < n ? qs[idx] : 0;
            lo |= ((static_cast<uint32_t>(x) & 15u) ^ 8u) << (4 * k);
            hi |= (static_cast<uint32_t>(x >> 4) & 15u) << (4 * k);
            sum += x;
        }
        ent[c] = make_uint2(lo, hi);
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if (lane == 0) red_i[wave] = sum;
    __syncthreads();
    if (tid < 16) {
        int t = 0;
        if (tid == 0)
            for (int w = 0; w < kNormThreads / 64; ++w) t += red_i[w];
        reinterpret_cast<int*>(p.staged)[tid] = t;
        if (tid == 0) *p.act_scale = s;
    }
}

// ---- embedding, RoPE + KV append ---------------------------------------------------------------------------------------------

struct Ctl {          // device-resident loop state
    uint32_t pos;     // position of the step
    uint32_t token;   // token generated by the previous step
    uint32_t n_prompt;
    uint32_t n_out;   // capacity of the generated-token array
};

__global__ void embed_kernel(const Ctl* __restrict__ ctl, const uint32_t* __restrict__ prompt,
                             const uint16_t* __restrict__ emb, uint32_t hidden, float* __restrict__ x) {
    const uint32_t pos = ctl->pos;
    const uint32_t tok = pos < ctl->n_prompt ? prompt[pos] : ctl->token;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        x[i] = bf16_f32(emb[static_cast<size_t>(tok) * hidden + i]);
}

struct RopeArgs {
    const Ctl* ctl;
    const float* q;
    const float* k;
    const float* v;
    const float* rope;  // [max_ctx][head_dim]: (cos, sin) of pair i at 2i, 2i + 1
    uint16_t* qh;       // f16 queries
    uint16_t* kc;       // f16 [kv_head][max_ctx][head_dim] of this layer
    uint16_t* vc;
    uint32_t n_heads, n_kv_heads, head_dim, max_ctx;
};

// NEOX pairing over all head_dim coordinates (ops.rs:199-221): x0' = fma(x0, c, -(x1 s)), x1' = fma(x0, s, x1 c).
__global__ void rope_kv_kernel(RopeArgs a) {
    const uint32_t half = a.head_dim / 2u;
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t pos = a.ctl->pos;
    const float* cache = a.rope + static_cast<size_t>(pos) * a.head_dim;
    const uint32_t nq = a.n_heads * half, nk = a.n_kv_heads * half;
    if (t < nq + nk) {
        const bool isq = t < nq;
        const uint32_t u = isq ? t : t - nq;
        const uint32_t h = u / half, i = u - h * half;
        const float* src = (isq ? a.q : a.k) + static_cast<size_t>(h) * a.head_dim;
        const float c = cache[2 * i], s = cache[2 * i + 1];
        const float x0 = src[i], x1 = src[i + half];
        const float x1s = x1 * s, x1c = x1 * c;
        const float y0 = __builtin_fmaf(x0, c, -x1s);
        const float y1 = __builtin_fmaf(x0, s, x1c);
        if (isq) {
            a.qh[h * a.head_dim + i] = f32_f16(y0);
            a.qh[h * a.head_dim + i + half] = f32_f16(y1);
        } else {
            uint16_t* dst = a.kc + (static_cast<size_t>(h) * a.max_ctx + pos) * a.head_dim;
            dst[i] = f32_f16(y0);
            dst[i + half] = f32_f16(y1);
        }
    }
    const uint32_t kvd = a.n_kv_heads * a.head_dim;
    if (t < kvd) {
        const uint32_t h = t / a.head_dim, d = t - h * a.head_dim;
        a.vc[(static_cast<size_t>(h) * a.max_ctx + pos) * a.head_dim + d] = f32_f16(a.v[t]);
    }
}

// ---- attention ------------------------------------------------------------------------------------------------------------

struct AttnArgs {
    const Ctl* ctl;
    const uint16_t* qh;  // f16 queries, n_heads x kAttnHd
    const uint16_t* kc;  // this layer: [kv_head][max_ctx][kAttnHd]
    const uint16_t* vc;
    float* out;          // n_heads x kAttnHd
    uint32_t n_heads, gqa, max_ctx;
    float scale;
};

constexpr uint32_t kAttnHd = 128;       // head_dim of the attention kernel
constexpr uint32_t kAttnMaxCtx = 4096;  // KV positions held in LDS (scores, running maxima)
constexpr uint32_t kAttnWaves = 8;      // 4 chunks x 2 halves of the head
constexpr uint32_t kAttnWin = 64;       // positions of V staged per wave at a time

// ggml_vec_dot_f16 of 128 values (ops.rs:960-1015): four accumulators of eight lanes take fma per 32 values,
// red = (s0 + s2) + (s1 + s3), t[k] = red[k] + red[k + 4], (t0 + t1) + (t2 + t3).
__device__ float dot_f16_128(const uint16_t* q, const uint16_t* __restrict__ k) {
    float acc[4][8];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[j][l] = 0.0f;
#pragma unroll 1
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 kv = *reinterpret_cast<const uint4*>(k + 32 * i + 8 * j);
            const uint4 qv = *reinterpret_cast<const uint4*>(q + 32 * i + 8 * j);
            const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w}, qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const uint16_t kb = static_cast<uint16_t>(kw[l >> 1] >> ((l & 1) * 16));
                const uint16_t qb = static_cast<uint16_t>(qw[l >> 1] >> ((l & 1) * 16));
                acc[j][l] = __builtin_fmaf(f16_f32(qb), f16_f32(kb), acc[j][l]);
            }
        }
    }
    float red[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) red[l] = (acc[0][l] + acc[2][l]) + (acc[1][l] + acc[3][l]);
    const float t0 = red[0] + red[4], t1 = red[1] + red[5], t2 = red[2] + red[6], t3 = red[3] + red[7];
    return (t0 + t1) + (t2 + t3);
}

// f16 value of an f32 (round to nearest even, after the f32 rounding of x), kept in an f32
__device__ __forceinline__ float r16(float x) { return static_cast<float>(static_cast<_Float16>(keep_f32(x))); }

// One workgroup per query head; the reference's attend_head (attention.rs:483-542) over the positions 0..pos.
// Below a padded KV length of 512 one online softmax covers all positions; from 512 on, 4 chunks of ceil(n_kv / 4)
// positions run one each and are combined in order. The online softmax of a chunk (attend_range,
// attention.rs:436-468) is rebuilt without its serial dependences except the FP16 accumulator itself:
//   scores        every position in parallel: ggml_vec_dot_f16(q, k) * scale
//   running max   a scan per chunk; the reference's max moves only on score > max, the scan combines the same way
//   factors       every position in parallel: a new maximum gives ms = expf(m_old - score), vs = 1; otherwise ms = 1,
//                 vs = expf(score - max); stored as -ms or vs (the sign marks the case)
//   accumulator   per coordinate, in position order: y = f16(y * ms), y = f16(fma(v, vs, y)), s = fma(s, ms, vs)
// Wave w accumulates chunk w / 2, coordinates 64 (w % 2) .. + 63, one per lane, with V streamed through LDS in
// windows of 64 positions, the next window loaded while the current one is consumed.
__global__ __launch_bounds__(kAttnWaves * 64) void attention_kernel(AttnArgs a) {
    __shared__ float sc[kAttnMaxCtx];
    __shared__ float pm[kAttnMaxCtx];
    __shared__ __align__(16) uint16_t vbuf[kAttnWaves][kAttnWin * 64];
    __shared__ __align__(16) uint16_t qs[kAttnHd];
    __shared__ float cm[4], cs[4];
    __shared__ uint16_t cv[4][kAttnHd];
    const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t kvh = h / a.gqa;
    const uint32_t seq = a.ctl->pos + 1;
    uint32_t n_kv = (seq + 255u) / 256u * 256u;
    if (n_kv > a.max_ctx) n_kv = a.max_ctx;
    const bool split = n_kv >= 512u;
    const uint32_t chunk = split ? (n_kv + 3u) / 4u : seq;
    const uint32_t n_chunks = split ? 4u : 1u;
    const uint16_t* kb = a.kc + static_cast<size_t>(kvh) * a.max_ctx * kAttnHd;
    const uint16_t* vb = a.vc + static_cast<size_t>(kvh) * a.max_ctx * kAttnHd;
    if (tid < kAttnHd) qs[tid] = a.qh[h * kAttnHd + tid];
    __syncthreads();

    for (uint32_t p = tid; p < seq; p += kAttnWaves * 64u) sc[p] = dot_f16_128(qs, kb + static_cast<size_t>(p) * kAttnHd) * a.scale;
    __syncthreads();

    if (wave < n_chunks) {
        const uint32_t st = wave * chunk, en = min(min(st + chunk, n_kv), seq);
        float carry = -__builtin_inff();
        for (uint32_t base = st; base < en; base += 64u) {
            const uint32_t p = base + lane;
            float v = p < en ? sc[p] : -__builtin_inff();
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const float o = __shfl_up(v, off);
                if (lane >= static_cast<uint32_t>(off)) v = v > o ? v : o;
            }
            v = v > carry ? v : carry;
            if (p < en) pm[p] = v;
            carry = __shfl(v, 63);
        }
    }
    __syncthreads();

    for (uint32_t p = tid; p < seq; p += kAttnWaves * 64u) {
        const uint32_t st = split ? p / chunk * chunk : 0u;
        const float prev = p == st ? -__builtin_inff() : pm[p - 1];
        const float s = sc[p];
        sc[p] = s > prev ? -glibc_expf(prev - s) : glibc_expf(s - prev);
    }
    __syncthreads();

    const uint32_t c = wave >> 1, half = wave & 1u, d = half * 64u + lane;
    uint32_t st = 0, en = 0;
    if (c < n_chunks) {
        st = c * chunk;
        en = min(min(st + chunk, n_kv), seq);
    }
    float y = 0.0f, ssum = 0.0f;
    if (st < en) {
        uint16_t* buf = vbuf[wave];
        const uint16_t* vsrc = vb + half * 64u + (lane & 7u) * 8u;
        u32x4 r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t p = min(st + 8u * j + (lane >> 3), en - 1u);
            r[j] = *reinterpret_cast<const u32x4*>(vsrc + static_cast<size_t>(p) * kAttnHd);
        }
        for (uint32_t base = st; base < en; base += kAttnWin) {
#pragma unroll
            for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x4*>(buf + (8u * j + (lane >> 3)) * 64u + (lane & 7u) * 8u) = r[j];
            if (base + kAttnWin < en) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t p = min(base + kAttnWin + 8u * j + (lane >> 3), en - 1u);
                    r[j] = *reinterpret_cast<const u32x4*>(vsrc + static_cast<size_t>(p) * kAttnHd);
                }
            }
            const uint32_t n = min(kAttnWin, en - base);
            const float f = lane < n ? sc[base + lane] : 0.0f;
            if (__ballot(__builtin_signbit(f)) == 0) {  // no new maximum in the window: ms = 1
                for (uint32_t i = 0; i < n; ++i) {
                    const float e = sc[base + i];
                    const float v = f16_f32(buf[i * 64u + lane]);
                    y = r16(__builtin_fmaf(v, e, y));
                    ssum = ssum + e;
                }
            } else {
                for (uint32_t i = 0; i < n; ++i) {
                    const float fi = sc[base + i];
                    const bool nm = __builtin_signbit(fi);
                    const float e = __builtin_fabsf(fi);
                    const float ms = nm ? e : 1.0f, vs = nm ? 1.0f : e;
                    const float v = f16_f32(buf[i * 64u + lane]);
                    y = r16(y * ms);
                    y = r16(__builtin_fmaf(v, vs, y));
                    ssum = __builtin_fmaf(ssum, ms, vs);
                }
            }
        }
    }
    float* out = a.out + static_cast<size_t>(h) * kAttnHd;
    if (!split) {
        if (c == 0) {
            const float s_inv = ssum == 0.0f ? 0.0f : 1.0f / ssum;
            out[d] = y * s_inv;
        }
        return;
    }
    if (c < 4) {
        cv[c][d] = f32_f16(y);
        if (half == 0 && lane == 0) {
            cm[c] = st < en ? pm[en - 1] : -__builtin_inff();
            cs[c] = ssum;
        }
    }
    __syncthreads();
    if (c != 0) return;
    float mf = -__builtin_inff(), sf = 0.0f, acc = 0.0f;
    for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t ks = k * chunk, ke = min(min(ks + chunk, n_kv), seq);
        if (ks >= ke) continue;
        const float sk = cs[k];
        if (sk == 0.0f) continue;
        const float mk = cm[k];
        const float mn = __builtin_fmaxf(mf, mk);
        const float so = glibc_expf(mf - mn);
        const float sn = glibc_expf(mk - mn);
        const float vn = f16_f32(cv[k][d]) * sn;
        acc = __builtin_fmaf(acc, so, vn);
        const float ssn = sk * sn;
        sf = __builtin_fmaf(sf, so, ssn);
        mf = mn;
    }
    out[d] = sf != 0.0f ? acc * (1.0f / sf) : acc;
}

// ---- head and greedy argmax ----------------------------------------------------------------------------------------------

// logits[r] = ggml_vec_dot_bf16(x, emb[r]) (ops.rs:669-713): lane (r, j) of four per row holds the eight lanes of
// accumulator j, acc + x*y rounded separately, then (a0 + a2) + (a1 + a3) across the four lanes and
// ((l0+l4) + (l2+l6)) + ((l1+l5) + (l3+l7)) inside one. hidden must be a multiple of 32.
__global__ __launch_bounds__(256) void head_kernel(const uint16_t* __restrict__ xb, const uint16_t* __restrict__ emb,
                                                   uint32_t hidden, uint32_t vocab, float* __restrict__ logits) {
    __shared__ uint4 xs[kNormMax / 8];
    for (uint32_t i = threadIdx.x; i < hidden / 8u; i += 256u) xs[i] = reinterpret_cast<const uint4*>(xb)[i];
    __syncthreads();
    const uint32_t r = blockIdx.x * 64u + (threadIdx.x >> 2), j = threadIdx.x & 3u;
    if (r >= vocab) return;
    const u32x4* row = reinterpret_cast<const u32x4*>(emb + static_cast<size_t>(r) * hidden);
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t i = 0; i < hidden / 32u; ++i) {
        const u32x4 w = __builtin_nontemporal_load(row + 4u * i + j);
        const uint4 x = xs[4u * i + j];
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w}, xx[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const float wf = bits_f32((ww[l >> 1] >> ((l & 1) * 16)) << 16);
            const float xf = bits_f32((xx[l >> 1] >> ((l & 1) * 16)) << 16);
            const float p = xf * wf;
            acc[l] = acc[l] + p;
        }
    }
    // (a0 + a2) + (a1 + a3): lanes j and j ^ 2, then j and j ^ 1
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        acc[l] = acc[l] + __shfl_xor(acc[l], 2);
        acc[l] = acc[l] + __shfl_xor(acc[l], 1);
    }
    if (j == 0) {
        const float g0 = acc[4] + acc[0], g1 = acc[5] + acc[1], g2 = acc[6] + acc[2], g3 = acc[7] + acc[3];
        logits[r] = (g0 + g2) + (g1 + g3);
    }
}

// Greedy sampling (sampler.rs:73-83): the first index of the maximum; NaN never replaces (a NaN first logit wins).
// Then the loop state advances: the token is recorded once the prompt is consumed and the position moves on.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ logits, uint32_t vocab, Ctl* ctl,
                                                      uint32_t* __restrict__ out_tokens) {
    __shared__ float bv[16];
    __shared__ uint32_t bi[16];
    const uint32_t tid = threadIdx.x;
    float v = -__builtin_inff();
    uint32_t idx = 0xffffffffu;
    for (uint32_t i = tid; i < vocab; i += 1024u) {
        const float x = logits[i];
        if (x > v || (idx == 0xffffffffu && x == v)) {
            v = x;
            idx = i;
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off);
        const uint32_t oi = __shfl_xor(idx, off);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    if ((tid & 63u) == 0) {
        bv[tid >> 6] = v;
        bi[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; ++w)
            if (bv[w] > v || (bv[w] == v && bi[w] < idx)) {
                v = bv[w];
                idx = bi[w];
            }
        if (logits[0] != logits[0] || idx == 0xffffffffu) idx = 0;
        const uint32_t pos = ctl->pos;
        ctl->token = idx;
        if (pos + 1 >= ctl->n_prompt) {
            const uint32_t k = pos + 1 - ctl->n_prompt;
            if (k < ctl->n_out) out_tokens[k] = idx;
        }
        ctl->pos = pos + 1;
    }
}

// ---- launches ----------------------------------------------------------------------------------------------------------------

int launch_norm(const NormArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(norm_quant_kernel, dim3(1), dim3(kNormThreads), 0, s, a);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_embed(const void* ctl, const uint32_t* prompt, const uint16_t* emb, uint32_t hidden, float* x, hipStream_t s) {
    hipLaunchKernelGGL(embed_kernel, dim3((hidden + 255u) / 256u), dim3(256), 0, s, static_cast<const Ctl*>(ctl), prompt,
                       emb, hidden, x);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_rope_kv(const RopeArgs& a, hipStream_t s) {
    const uint32_t n = std::max(a.n_heads * a.head_dim / 2u + a.n_kv_heads * a.head_dim / 2u, a.n_kv_heads * a.head_dim);
    hipLaunchKernelGGL(rope_kv_kernel, dim3((n + 255u) / 256u), dim3(256), 0, s, a);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_attention(const AttnArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(attention_kernel, dim3(a.n_heads), dim3(kAttnWaves * 64), 0, s, a);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_head(const uint16_t* xb, const uint16_t* emb, uint32_t hidden, uint32_t vocab, float* logits, hipStream_t s) {
    hipLaunchKernelGGL(head_kernel, dim3((vocab + 63u) / 64u), dim3(256), 0, s, xb, emb, hidden, vocab, logits);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_argmax(const float* logits, uint32_t vocab, void* ctl, uint32_t* out_tokens, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, logits, vocab, static_cast<Ctl*>(ctl), out_tokens);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

__global__ void expf_kernel(const float* __restrict__ x, uint32_t n, float* __restrict__ out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = glibc_expf(x[i]);
}

int launch_expf(const float* x, size_t n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(expf_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s, x,
                       static_cast<uint32_t>(n), out);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

// ---- the decoder handle ----------------------------------------------------------------------------------------------------

constexpr uint32_t kDecoderMagic = 0x56584431u;  // "VXD1"
constexpr int kProjKinds = 7;
constexpr int kNormKinds = 4;

// The GEMV launches of one layer stage (q/k/v, o, gate/up, down) with their K-split finish.
struct StageLaunch {
    LaunchArgs a;
    uint32_t max_rows;
    const uint32_t* split;
    uint32_t n_split;
};

}  // namespace vx

struct vx_decoder {
    uint32_t magic;
    int device, num_cus;
    vx_decoder_config_t cfg;
    size_t qd, kvd;
    std::vector<vx_matrix_t*> proj;   // [layer * 7 + kind]
    std::vector<float*> norms;        // [layer * 4 + kind]; the output norm at [n_layers * 4]
    std::vector<uint8_t> norm_set, emb_set;
    uint16_t* d_emb;
    float* d_rope;
    uint16_t *d_kc, *d_vc;            // [layer][kv_head][max_ctx][head_dim]
    float *d_x, *d_q, *d_k, *d_v, *d_att, *d_o, *d_gate, *d_up, *d_down, *d_logits;
    uint16_t *d_qh, *d_xb;
    uint8_t* d_stage[4];              // staged activations of the q/k/v, o, gate/up and down inputs
    float* d_as;                      // their activation scales
    vx::Ctl* d_ctl;
    uint32_t* d_prompt;
    uint32_t* d_tokens;
    vx::Job* d_jobs;
    int32_t* d_part;
    uint32_t* d_split;
    std::vector<vx::StageLaunch> stages;  // [layer * 4 + stage]
    vx::Ctl* h_ctl;                   // pinned
    hipStream_t stream;
    hipGraph_t graph;
    hipGraphExec_t exec;
    bool ready;
    size_t bytes;
    std::mutex mu;
};

namespace vx {

static int check_decoder(const vx_decoder_t* d) {
    if (d == nullptr) VX_FAIL(VX_ERR_INVALID_HANDLE, "decoder handle is NULL");
    if (d->magic != kDecoderMagic) VX_FAIL(VX_ERR_INVALID_HANDLE, "decoder handle is not valid (freed or foreign)");
    return VX_OK;
}

static int set_device(int dev) {
    int cur = -1;
    VX_HIP(hipGetDevice(&cur));
    if (cur != dev) VX_HIP(hipSetDevice(dev));
    return VX_OK;
}

static void drop_graph(vx_decoder* d) {
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    d->exec = nullptr;
    d->graph = nullptr;
    d->ready = false;
}

static void destroy_decoder(vx_decoder* d) {
    drop_graph(d);
    for (auto* m : d->proj)
        if (m) (void)vx_matrix_free(m);
    for (auto* p : d->norms)
        if (p) (void)hipFree(p);
    void* bufs[] = {d->d_emb,  d->d_rope, d->d_kc,    d->d_vc,     d->d_x,      d->d_q,      d->d_k,      d->d_v,
                    d->d_att,  d->d_o,    d->d_gate,  d->d_up,     d->d_down,   d->d_logits, d->d_qh,     d->d_xb,
                    d->d_as,   d->d_ctl,  d->d_prompt, d->d_tokens, d->d_jobs,  d->d_part,   d->d_split,  d->d_stage[0],
                    d->d_stage[1], d->d_stage[2], d->d_stage[3]};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (d->h_ctl) (void)hipHostFree(d->h_ctl);
    if (d->stream) (void)hipStreamDestroy(d->stream);
    d->magic = 0;
    delete d;
}

static size_t proj_rows(const vx_decoder* d, int kind) {
    switch (kind) {
        case VX_PROJ_Q: return d->qd;
        case VX_PROJ_K:
        case VX_PROJ_V: return d->kvd;
        case VX_PROJ_GATE:
        case VX_PROJ_UP: return d->cfg.ffn;
        default: return d->cfg.hidden;
    }
}

static size_t proj_cols(const vx_decoder* d, int kind) {
    switch (kind) {
        case VX_PROJ_O: return d->qd;
        case VX_PROJ_DOWN: return d->cfg.ffn;
        default: return d->cfg.hidden;
    }
}

static size_t norm_len(const vx_decoder* d, uint32_t layer, uint32_t kind) {
    if (layer == d->cfg.n_layers) return d->cfg.hidden;
    if (kind == VX_NORM_ATTN_SUB) return d->qd;
    if (kind == VX_NORM_FFN_SUB) return d->cfg.ffn;
    return d->cfg.hidden;
}

// RoPE cache (ops.rs:121-140, RopeConfig::plain): theta_scale = theta^(-2 / head_dim); theta_i = pos * theta_scale^i
// by repeated multiplication; (cos, sin) in f32 from the host's libm, the functions Rust's f32::powf/cos/sin call.
static void rope_table(const vx_decoder_config_t& c, std::vector<float>& t) {
    t.assign(static_cast<size_t>(c.max_ctx) * c.head_dim, 0.0f);
    const float theta_scale = powf(c.rope_theta, -2.0f / static_cast<float>(c.head_dim));
    for (size_t p = 0; p < c.max_ctx; ++p) {
        float theta = static_cast<float>(p);
        float* row = t.data() + p * c.head_dim;
        for (size_t i = 0; i < c.head_dim / 2; ++i) {
            row[2 * i] = cosf(theta) * 1.0f;
            row[2 * i + 1] = sinf(theta) * 1.0f;
            theta *= theta_scale;
        }
    }
}

template <class T>
static hipError_t dalloc(vx_decoder* d, T** p, size_t bytes) {
    d->bytes += bytes;
    return hipMalloc(reinterpret_cast<void**>(p), bytes);
}

static int create_decoder(const vx_decoder_config_t* c, vx_decoder_t** out) {
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_decoder is NULL");
    *out = nullptr;
    if (c == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "config is NULL");
    if (c->struct_size != sizeof(vx_decoder_config_t))
        VX_FAIL(VX_ERR_INVALID_ARGUMENT, "config.struct_size is %u, expected %zu", c->struct_size, sizeof(vx_decoder_config_t));
    if (c->n_layers == 0 || c->n_layers > 1024) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "n_layers must be in 1..=1024");
    if (c->head_dim != kAttnHd) VX_FAIL(VX_ERR_UNSUPPORTED, "head_dim %u is not supported (128 only)", c->head_dim);
    if (c->n_heads == 0 || c->n_kv_heads == 0 || c->n_heads % c->n_kv_heads)
        VX_FAIL(VX_ERR_INVALID_ARGUMENT, "n_heads (%u) must be a positive multiple of n_kv_heads (%u)", c->n_heads, c->n_kv_heads);
    if (c->max_ctx == 0 || c->max_ctx > kAttnMaxCtx) VX_FAIL(VX_ERR_UNSUPPORTED, "max_ctx must be in 1..=%u", kAttnMaxCtx);
    if (c->hidden == 0 || c->hidden % 32 || c->hidden > kNormMax)
        VX_FAIL(VX_ERR_UNSUPPORTED, "hidden must be a positive multiple of 32 up to %u", kNormMax);
    if (static_cast<size_t>(c->n_heads) * c->head_dim > kNormMax || c->ffn == 0 || c->ffn > kNormMax)
        VX_FAIL(VX_ERR_UNSUPPORTED, "n_heads * head_dim and ffn must be in 1..=%u", kNormMax);
    if (c->vocab == 0 || c->vocab > (1u << 24)) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "vocab must be in 1..=2^24");
    if (!(c->rms_eps >= 0.0f) || !(c->rope_theta > 0.0f)) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "rms_eps must be >= 0 and rope_theta > 0");
    DeviceInfo di;
    VX_TRY(device_info(&di));
    vx_decoder* d = new vx_decoder();
    d->magic = kDecoderMagic;
    d->device = di.device;
    d->num_cus = di.num_cus;
    d->cfg = *c;
    d->qd = static_cast<size_t>(c->n_heads) * c->head_dim;
    d->kvd = static_cast<size_t>(c->n_kv_heads) * c->head_dim;
    d->proj.assign(static_cast<size_t>(c->n_layers) * kProjKinds, nullptr);
    d->norms.assign(static_cast<size_t>(c->n_layers + 1) * kNormKinds, nullptr);
    d->norm_set.assign(d->norms.size(), 0);
    d->emb_set.assign(1, 0);
    const size_t L = c->n_layers, H = c->hidden, F = c->ffn;
    const size_t kv_elems = L * d->kvd * c->max_ctx;
    hipError_t e = dalloc(d, &d->d_emb, static_cast<size_t>(c->vocab) * H * 2);
    if (e == hipSuccess) e = dalloc(d, &d->d_rope, static_cast<size_t>(c->max_ctx) * c->head_dim * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_kc, kv_elems * 2);
    if (e == hipSuccess) e = dalloc(d, &d->d_vc, kv_elems * 2);
    if (e == hipSuccess) e = dalloc(d, &d->d_x, H * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_q, d->qd * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_k, d->kvd * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_v, d->kvd * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_att, d->qd * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_o, H * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_gate, F * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_up, F * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_down, H * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_logits, static_cast<size_t>(c->vocab) * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_qh, d->qd * 2);
    if (e == hipSuccess) e = dalloc(d, &d->d_xb, H * 2);
    const size_t stage_cols[4] = {H, d->qd, H, F};
    for (int s = 0; s < 4 && e == hipSuccess; ++s) e = dalloc(d, &d->d_stage[s], staged_bytes(stage_cols[s]));
    if (e == hipSuccess) e = dalloc(d, &d->d_as, 4 * sizeof(float));
    if (e == hipSuccess) e = dalloc(d, &d->d_ctl, sizeof(Ctl));
    if (e == hipSuccess) e = dalloc(d, &d->d_prompt, static_cast<size_t>(c->max_ctx) * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_tokens, static_cast<size_t>(c->max_ctx) * 4);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&d->h_ctl), sizeof(Ctl), hipHostMallocDefault);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking);
    if (e == hipSuccess) {
        std::vector<float> rope;
        rope_table(*c, rope);
        e = hipMemcpy(d->d_rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        destroy_decoder(d);
        VX_FAIL(VX_ERR_DEVICE, "decoder allocation failed: %s", hipGetErrorString(e));
    }
    *out = d;
    return VX_OK;
}

// The GEMV plans of every stage: each job's K slices are chosen so that a stage offers about one work item per CU in
// proportion to its weight bytes (bs = 1 matrices are small: one tile group per K slice would leave most CUs idle).
static int build_plans(vx_decoder* d) {
    const size_t L = d->cfg.n_layers;
    static const int kStageKinds[4][3] = {{VX_PROJ_Q, VX_PROJ_K, VX_PROJ_V}, {VX_PROJ_O, -1, -1},
                                          {VX_PROJ_GATE, VX_PROJ_UP, -1}, {VX_PROJ_DOWN, -1, -1}};
    float* outs[kProjKinds] = {d->d_q, d->d_k, d->d_v, d->d_o, d->d_gate, d->d_up, d->d_down};
    std::vector<Job> jobs;
    std::vector<uint32_t> split;
    std::vector<size_t> job_first(L * 4), split_first(L * 4);
    std::vector<uint32_t> stage_jobs(L * 4), stage_items(L * 4), stage_rows(L * 4), stage_split(L * 4);
    size_t part_ints = 0;
    for (size_t l = 0; l < L; ++l)
        for (int s = 0; s < 4; ++s) {
            const size_t si = l * 4 + s;
            size_t stage_bytes = 0;
            for (int k : kStageKinds[s])
                if (k >= 0) stage_bytes += d->proj[l * kProjKinds + k]->g.device_bytes;
            job_first[si] = jobs.size();
            split_first[si] = split.size();
            uint32_t items = 0, max_rows = 0;
            size_t part = 0;
            for (int k : kStageKinds[s]) {
                if (k < 0) continue;
                const vx_matrix* m = d->proj[l * kProjKinds + k];
                const uint32_t target = static_cast<uint32_t>(
                    (static_cast<uint64_t>(d->num_cus) * m->g.device_bytes + stage_bytes - 1) / stage_bytes);
                Job j{};
                plan_job(j, m->g, target);
                j.w = m->d_w;
                j.dsum = m->d_dsum;
                j.staged = d->d_stage[s];
                j.out = outs[k];
                j.act_scale = d->d_as + s;
                j.weight_scale = m->weight_scale;
                j.out_kind = kOutF32Dev;
                j.item_begin = items;
                items += job_items(j);
                if (j.kslices > 1) {
                    j.part = reinterpret_cast<int32_t*>(part);  // offset into the shared partial buffer, rebased below
                    part += static_cast<size_t>(j.kslices) * j.padded_rows;
                    split.push_back(static_cast<uint32_t>(jobs.size() - job_first[si]));
                    max_rows = std::max(max_rows, j.rows);
                }
                jobs.push_back(j);
            }
            stage_jobs[si] = static_cast<uint32_t>(jobs.size() - job_first[si]);
            stage_items[si] = items;
            stage_rows[si] = max_rows;
            stage_split[si] = static_cast<uint32_t>(split.size() - split_first[si]);
            part_ints = std::max(part_ints, part);
        }
    if (d->d_jobs) (void)hipFree(d->d_jobs);
    if (d->d_part) (void)hipFree(d->d_part);
    if (d->d_split) (void)hipFree(d->d_split);
    d->d_jobs = nullptr;
    d->d_part = nullptr;
    d->d_split = nullptr;
    VX_HIP(hipMalloc(&d->d_jobs, jobs.size() * sizeof(Job)));
    VX_HIP(hipMalloc(&d->d_part, std::max<size_t>(part_ints, 1) * 4));
    VX_HIP(hipMalloc(&d->d_split, std::max<size_t>(split.size(), 1) * 4));
    for (auto& j : jobs)
        if (j.kslices > 1) j.part = d->d_part + reinterpret_cast<size_t>(j.part);
    VX_HIP(hipMemcpy(d->d_jobs, jobs.data(), jobs.size() * sizeof(Job), hipMemcpyHostToDevice));
    if (!split.empty()) VX_HIP(hipMemcpy(d->d_split, split.data(), split.size() * 4, hipMemcpyHostToDevice));
    d->stages.assign(L * 4, StageLaunch{});
    for (size_t si = 0; si < L * 4; ++si) {
        StageLaunch& st = d->stages[si];
        st.a.jobs = d->d_jobs + job_first[si];
        st.a.n_jobs = stage_jobs[si];
        st.a.total_items = stage_items[si];
        st.max_rows = stage_rows[si];
        st.split = d->d_split + split_first[si];
        st.n_split = stage_split[si];
    }
    return VX_OK;
}

static int run_stage(const vx_decoder* d, size_t layer, int s, hipStream_t st) {
    const StageLaunch& sl = d->stages[layer * 4 + s];
    return launch_gemv(sl.a, sl.max_rows, sl.split, sl.n_split, d->num_cus, st);
}

static NormArgs norm_args(const vx_decoder* d, float* a, const float* b, uint32_t input, const float* gamma, size_t n,
                          int stage) {
    NormArgs p{};
    p.a = a;
    p.b = b;
    p.gamma = gamma;
    p.n = static_cast<uint32_t>(n);
    p.eps = d->cfg.rms_eps;
    p.input = input;
    p.quantize = stage >= 0 ? 1u : 0u;
    p.staged = stage >= 0 ? d->d_stage[stage] : nullptr;
    p.act_scale = stage >= 0 ? d->d_as + stage : nullptr;
    p.out_bf16 = stage >= 0 ? nullptr : d->d_xb;
    p.tbr = static_cast<uint32_t>(tile_row_bytes(n));
    p.dbr = static_cast<uint32_t>(device_row_bytes(n));
    return p;
}

// Enqueues one decode step on `st` (also the sequence captured into the step graph).
static int record_step(const vx_decoder* d, hipStream_t st) {
    const vx_decoder_config_t& c = d->cfg;
    const size_t L = c.n_layers, H = c.hidden;
    VX_TRY(launch_embed(d->d_ctl, d->d_prompt, d->d_emb, c.hidden, d->d_x, st));
    const size_t layer_kv = d->kvd * c.max_ctx;
    for (size_t l = 0; l < L; ++l) {
        float* const* nw = d->norms.data() + l * kNormKinds;
        VX_TRY(launch_norm(norm_args(d, d->d_x, d->d_down, l == 0 ? kInPlain : kInResidual, nw[VX_NORM_ATTN], H, 0), st));
        VX_TRY(run_stage(d, l, 0, st));
        RopeArgs r{};
        r.ctl = d->d_ctl;
        r.q = d->d_q;
        r.k = d->d_k;
        r.v = d->d_v;
        r.rope = d->d_rope;
        r.qh = d->d_qh;
        r.kc = d->d_kc + l * layer_kv;
        r.vc = d->d_vc + l * layer_kv;
        r.n_heads = c.n_heads;
        r.n_kv_heads = c.n_kv_heads;
        r.head_dim = c.head_dim;
        r.max_ctx = c.max_ctx;
        VX_TRY(launch_rope_kv(r, st));
        AttnArgs at{};
        at.ctl = d->d_ctl;
        at.qh = d->d_qh;
        at.kc = r.kc;
        at.vc = r.vc;
        at.out = d->d_att;
        at.n_heads = c.n_heads;
        at.gqa = c.n_heads / c.n_kv_heads;
        at.max_ctx = c.max_ctx;
        at.scale = 1.0f / sqrtf(static_cast<float>(c.head_dim));
        VX_TRY(launch_attention(at, st));
        VX_TRY(launch_norm(norm_args(d, d->d_att, nullptr, kInPlain, nw[VX_NORM_ATTN_SUB], d->qd, 1), st));
        VX_TRY(run_stage(d, l, 1, st));
        VX_TRY(launch_norm(norm_args(d, d->d_x, d->d_o, kInResidual, nw[VX_NORM_FFN], H, 2), st));
        VX_TRY(run_stage(d, l, 2, st));
        VX_TRY(launch_norm(norm_args(d, d->d_gate, d->d_up, kInRelu2Mul, nw[VX_NORM_FFN_SUB], c.ffn, 3), st));
        VX_TRY(run_stage(d, l, 3, st));
    }
    VX_TRY(launch_norm(norm_args(d, d->d_x, d->d_down, kInResidual, d->norms[L * kNormKinds], H, -1), st));
    VX_TRY(launch_head(d->d_xb, d->d_emb, c.hidden, c.vocab, d->d_logits, st));
    return launch_argmax(d->d_logits, c.vocab, d->d_ctl, d->d_tokens, st);
}

// Builds the plans and captures the step graph once every weight is set.
static int prepare(vx_decoder* d) {
    if (d->ready) return VX_OK;
    const size_t L = d->cfg.n_layers;
    for (size_t i = 0; i < L * kProjKinds; ++i)
        if (!d->proj[i]) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "projection %zu of layer %zu is not set", i % kProjKinds, i / kProjKinds);
    for (size_t l = 0; l <= L; ++l)
        for (int k = 0; k < (l == L ? 1 : kNormKinds); ++k)
            if (!d->norm_set[l * kNormKinds + k]) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "norm %d of layer %zu is not set", k, l);
    if (!d->emb_set[0]) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the embedding is not set");
    drop_graph(d);
    VX_TRY(build_plans(d));
    VX_HIP(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
    const int st = record_step(d, d->stream);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(d->stream, &g);
    if (st != VX_OK) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    VX_HIP(e);
    d->graph = g;
    VX_HIP(hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0));
    d->ready = true;
    return VX_OK;
}

static int put_ctl(vx_decoder* d, uint32_t pos, uint32_t token, uint32_t n_prompt, uint32_t n_out) {
    d->h_ctl->pos = pos;
    d->h_ctl->token = token;
    d->h_ctl->n_prompt = n_prompt;
    d->h_ctl->n_out = n_out;
    VX_HIP(hipMemcpyAsync(d->d_ctl, d->h_ctl, sizeof(Ctl), hipMemcpyHostToDevice, d->stream));
    return VX_OK;
}

}  // namespace vx

extern "C" {

using namespace vx;

int vx_decoder_create(const vx_decoder_config_t* config, vx_decoder_t** out_decoder) {
    return guard([&]() -> int { return create_decoder(config, out_decoder); });
}

int vx_decoder_set_projection(vx_decoder_t* d, uint32_t layer, uint32_t kind, const uint8_t* planar, size_t planar_len,
                              float weight_scale) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        std::lock_guard<std::mutex> lk(d->mu);
        if (layer >= d->cfg.n_layers) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "layer %u out of range (n_layers %u)", layer, d->cfg.n_layers);
        if (kind >= static_cast<uint32_t>(kProjKinds)) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "projection kind %u is not 0..6", kind);
        VX_TRY(set_device(d->device));
        vx_matrix_t* m = nullptr;
        VX_TRY(vx_matrix_create(planar, planar_len, proj_rows(d, kind), proj_cols(d, kind), weight_scale, &m));
        vx_matrix_t*& slot = d->proj[static_cast<size_t>(layer) * kProjKinds + kind];
        if (slot) (void)vx_matrix_free(slot);
        slot = m;
        drop_graph(d);
        return VX_OK;
    });
}

int vx_decoder_set_norm(vx_decoder_t* d, uint32_t layer, uint32_t kind, const float* weights, size_t n) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        std::lock_guard<std::mutex> lk(d->mu);
        if (layer > d->cfg.n_layers) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "layer %u out of range (n_layers %u)", layer, d->cfg.n_layers);
        if (kind >= static_cast<uint32_t>(kNormKinds) || (layer == d->cfg.n_layers && kind != 0))
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "norm kind %u is not valid for layer %u", kind, layer);
        if (weights == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "weights is NULL");
        const size_t need = norm_len(d, layer, kind);
        if (n != need) VX_FAIL(VX_ERR_INVALID_SHAPE, "norm %u of layer %u has %zu weights, expected %zu", kind, layer, n, need);
        VX_TRY(set_device(d->device));
        float*& slot = d->norms[static_cast<size_t>(layer) * kNormKinds + kind];
        if (!slot) VX_HIP(dalloc(d, &slot, need * 4));
        VX_HIP(hipMemcpy(slot, weights, need * 4, hipMemcpyHostToDevice));
        d->norm_set[static_cast<size_t>(layer) * kNormKinds + kind] = 1;
        return VX_OK;
    });
}

int vx_decoder_set_embedding_bf16(vx_decoder_t* d, const uint16_t* embedding, size_t n) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        std::lock_guard<std::mutex> lk(d->mu);
        if (embedding == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "embedding is NULL");
        const size_t need = static_cast<size_t>(d->cfg.vocab) * d->cfg.hidden;
        if (n != need) VX_FAIL(VX_ERR_INVALID_SHAPE, "the embedding has %zu values, expected vocab * hidden = %zu", n, need);
        VX_TRY(set_device(d->device));
        VX_HIP(hipMemcpy(d->d_emb, embedding, need * 2, hipMemcpyHostToDevice));
        d->emb_set[0] = 1;
        return VX_OK;
    });
}

int vx_decoder_step(vx_decoder_t* d, uint32_t token, uint32_t pos, float* logits, size_t logits_capacity,
                    uint32_t* out_next) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        std::lock_guard<std::mutex> lk(d->mu);
        if (token >= d->cfg.vocab) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "token %u out of range (vocab %u)", token, d->cfg.vocab);
        if (pos >= d->cfg.max_ctx) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "pos %u out of range (max_ctx %u)", pos, d->cfg.max_ctx);
        if (logits && logits_capacity < d->cfg.vocab)
            VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "logits hold %zu values but vocab = %u", logits_capacity, d->cfg.vocab);
        VX_TRY(set_device(d->device));
        VX_TRY(prepare(d));
        VX_TRY(put_ctl(d, pos, token, 0, 0));
        VX_HIP(hipGraphLaunch(d->exec, d->stream));
        VX_HIP(hipStreamSynchronize(d->stream));
        if (logits) VX_HIP(hipMemcpy(logits, d->d_logits, static_cast<size_t>(d->cfg.vocab) * 4, hipMemcpyDeviceToHost));
        if (out_next) {
            Ctl c{};
            VX_HIP(hipMemcpy(&c, d->d_ctl, sizeof c, hipMemcpyDeviceToHost));
            *out_next = c.token;
        }
        return VX_OK;
    });
}

int vx_decoder_generate(vx_decoder_t* d, const uint32_t* prompt, size_t n_prompt, size_t n_new, uint32_t* out_tokens,
                        size_t out_capacity) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        std::lock_guard<std::mutex> lk(d->mu);
        if (n_prompt == 0) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the prompt is empty");
        if (prompt == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "prompt is NULL");
        if (n_new > 0 && out_tokens == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_tokens is NULL");
        if (out_capacity < n_new) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "out_tokens holds %zu values, %zu requested", out_capacity, n_new);
        const size_t steps = n_new ? n_prompt + n_new - 1 : n_prompt;
        if (steps > d->cfg.max_ctx)
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "prompt (%zu) + new tokens (%zu) exceed the context of %u", n_prompt, n_new, d->cfg.max_ctx);
        for (size_t i = 0; i < n_prompt; ++i)
            if (prompt[i] >= d->cfg.vocab) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "prompt[%zu] = %u out of range (vocab %u)", i, prompt[i], d->cfg.vocab);
        VX_TRY(set_device(d->device));
        VX_TRY(prepare(d));
        VX_HIP(hipMemcpy(d->d_prompt, prompt, n_prompt * 4, hipMemcpyHostToDevice));
        VX_TRY(put_ctl(d, 0, 0, static_cast<uint32_t>(n_prompt), static_cast<uint32_t>(n_new)));
        for (size_t i = 0; i < steps; ++i) VX_HIP(hipGraphLaunch(d->exec, d->stream));
        VX_HIP(hipStreamSynchronize(d->stream));
        if (n_new) VX_HIP(hipMemcpy(out_tokens, d->d_tokens, n_new * 4, hipMemcpyDeviceToHost));
        return VX_OK;
    });
}

int vx_decoder_memory_bytes(const vx_decoder_t* d, size_t* out_bytes) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        if (out_bytes == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_bytes is NULL");
        size_t b = d->bytes;
        for (auto* m : d->proj)
            if (m) b += m->g.device_bytes;
        *out_bytes = b;
        return VX_OK;
    });
}

int vx_decoder_free(vx_decoder_t* d) {
    return guard([&]() -> int {
        if (d == nullptr) return VX_OK;
        VX_TRY(check_decoder(d));
        (void)set_device(d->device);
        (void)hipStreamSynchronize(d->stream);
        destroy_decoder(d);
        return VX_OK;
    });
}

int vx_expf_dev(const float* x, size_t n, float* out, void* stream) {
    return guard([&]() -> int {
        if (n == 0) return VX_OK;
        if (x == nullptr || out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "x or out is NULL");
        if (n > 0xffffffffu) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "n must be below 2^32");
        return launch_expf(x, n, out, static_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
