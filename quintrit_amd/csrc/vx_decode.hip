// Decode step of a ternary decoder on gfx950: the token loop around the velurex GEMV.
//
// One step follows the reference's CPU runtime operation by operation (quintrit-runtime/src/model.rs:64-377,
// attention.rs:115-542, ops.rs), so that logits and greedy tokens are bit-identical to it:
//   embed (bf16 row -> f32)
//   per layer: [residual add +] RMSNorm + int8 quantization -> q, k, v projections (the fp32 layer epilogue)
//              NEOX RoPE, f16 KV append, FP16-accumulator attention with bitnet.cpp's 4-chunk split
//              sub-norm + quantization -> o projection
//              residual add + RMSNorm + quantization -> gate, up projections
//              ReLU^2(gate) * up + sub-norm + quantization -> down projection
//   residual add + final RMSNorm -> bf16 -> tied bf16 head (ggml_vec_dot_bf16 order) -> greedy argmax (first maximum)
//
// Kernels. A step is 1 + 5 per layer launches, replayed as one HIP graph per token with the position, the token and the
// generated ids in device memory (the reference's CUDA graph is position-independent the same way,
// quintrit-runtime/src/gpu.rs:459-493):
//   dgemv_kernel x4   per layer and projection stage, one workgroup per 64-row tile: every workgroup first computes
//                     the stage input itself (the embedding row or a residual add or ReLU^2 gating of the previous
//                     projections' outputs, RMSNorm, int8 quantization, GEMV staging, all in LDS) while its weights
//                     are in flight, then its 16 waves split the row's chunks and add their exact int32 sums in LDS;
//                     one wave applies the layer epilogue and stores the tile's fp32 outputs
//   attention_kernel  per query head: RoPE of q and k, the KV append, attention
//   head_kernel       final residual + RMSNorm, the bf16 head, and the greedy argmax across workgroups
// Computing a stage input in every workgroup repeats a few microseconds of work that one workgroup would do alone, but
// it runs in parallel with the weight loads and saves a launch and a wait on a single-CU kernel.
//
// RMSNorm (ops.rs:43-57) sums the f32 squares sequentially in f64 and rounds sum / n to f32. Here the squares are
// summed as a tree; both sums differ from the exact one by at most (n - 1) 2^-53 sum, so when the f32 mean is the same
// at both ends of that interval the tree's mean is the reference's; otherwise (rare) one lane redoes the sum in the
// reference's order. The exponentials are glibc's expf (vx_expf.h).
#include "vx_expf.h"
#include "vx_gemv_core.h"
#include "vx_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <type_traits>
#include <vector>

namespace vx {

// ---- small helpers --------------------------------------------------------------------------------------------------------

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 g_u4;

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

// f(std::integral_constant<uint32_t, k>) for k = 0 .. N - 1: a loop body with its index as a compile-time constant, so that
// arrays indexed by it stay in fixed registers (a counted loop may be kept rolled, with the registers rotated).
template <uint32_t N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<uint32_t, N - 1>{});
    }
}

// ---- wave reductions (DPP within rows of 16 lanes, then the four row results) ------------------------------------------------

template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror: lane i of 8 reads lane 7 - i
constexpr int kDppMirror = 0x140;     // row_mirror: lane i of 16 reads lane 15 - i

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double x) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint64_t lo = dpp32<CTRL>(static_cast<uint32_t>(u)), hi = dpp32<CTRL>(static_cast<uint32_t>(u >> 32));
    return __builtin_bit_cast(double, (hi << 32) | lo);
}
__device__ __forceinline__ double readlane_f64(double x, int l) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), l));
    const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), l));
    return __builtin_bit_cast(double, (hi << 32) | lo);
}

// After the four DPP steps every lane holds the result of its row of 16; the wave's is combined from lanes 0, 16, 32, 48.
__device__ __forceinline__ double wave_sum_f64(double x) {
    x += dpp_f64<kDppXor1>(x);
    x += dpp_f64<kDppXor2>(x);
    x += dpp_f64<kDppHalfMirror>(x);
    x += dpp_f64<kDppMirror>(x);
    return (readlane_f64(x, 0) + readlane_f64(x, 16)) + (readlane_f64(x, 32) + readlane_f64(x, 48));
}

__device__ __forceinline__ int wave_sum_i32(int x) {
    x += static_cast<int>(dpp32<kDppXor1>(static_cast<uint32_t>(x)));
    x += static_cast<int>(dpp32<kDppXor2>(static_cast<uint32_t>(x)));
    x += static_cast<int>(dpp32<kDppHalfMirror>(static_cast<uint32_t>(x)));
    x += static_cast<int>(dpp32<kDppMirror>(static_cast<uint32_t>(x)));
    return (__builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16)) +
           (__builtin_amdgcn_readlane(x, 32) + __builtin_amdgcn_readlane(x, 48));
}

// Largest of non-negative, non-NaN values.
__device__ __forceinline__ float fmax_nn(float a, float b) { return b > a ? b : a; }
__device__ __forceinline__ float wave_max_f32(float x) {
    x = fmax_nn(x, bits_f32(dpp32<kDppXor1>(f32_bits(x))));
    x = fmax_nn(x, bits_f32(dpp32<kDppXor2>(f32_bits(x))));
    x = fmax_nn(x, bits_f32(dpp32<kDppHalfMirror>(f32_bits(x))));
    x = fmax_nn(x, bits_f32(dpp32<kDppMirror>(f32_bits(x))));
    const float a = bits_f32(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(f32_bits(x)), 0)));
    const float b = bits_f32(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(f32_bits(x)), 16)));
    const float c = bits_f32(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(f32_bits(x)), 32)));
    const float d = bits_f32(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(f32_bits(x)), 48)));
    return fmax_nn(fmax_nn(a, b), fmax_nn(c, d));
}

// ---- the stage input: embedding / residual add / gating, RMSNorm, int8 quantization --------------------------------------

constexpr int kNT = 1024;            // threads of the kernels that compute a stage input
constexpr uint32_t kNormMax = 8192;  // longest normed input, and the LDS window of a staged input slice (floats)
constexpr uint32_t kPlainMax = 24576;  // longest input without a norm (6 float4 groups per thread)
constexpr uint32_t kStChunks = 112;  // 16-byte chunks of a staged input slice in LDS (16 waves x kDPer)
constexpr int kMaxSlicesA = 6;       // K slices of a q/k/v, o or down projection at most
constexpr int kMaxSlicesB = 2;       // K slices of a separate gate and up projection at most

struct Ctl {          // device-resident loop state
    uint32_t pos;     // position of the step
    uint32_t token;   // token generated by the previous step
    uint32_t n_prompt;
    uint32_t n_out;   // capacity of the generated-token array
};

// *p if c, else zero (a branch, not a select between a load and a zero held in memory).
template <class T>
__device__ __forceinline__ T load_if(const T* p, bool c) {
    T v{};
    if (c) v = *p;
    return v;
}

// A projection output as its consumers read it: row i is float(part[i]) * (ws / as), zero when as is not > 0 (the layer
// epilogue, layer.rs:246-253). A projection split into K slices adds their exact int32 sums atomically into part, so
// their order does not matter; a prefill's outputs are token rows stride apart (kslices 1 in both).
struct ProjOut {
    const int32_t* part;  // [stride]; the row corrections are added by the producer's slice 0
    const float* as;      // activation scale of the producing stage
    float ws;             // weight scale
    uint32_t kslices, stride;
};

__device__ __forceinline__ float proj_post(const ProjOut& o, bool* zero) {
    const float as = *o.as;
    *zero = !(as > 0.0f);
    return *zero ? 0.0f : o.ws / as;
}
// The same with the activation scale already loaded.
__device__ __forceinline__ float proj_post(const ProjOut& o, float as, bool* zero) {
    *zero = !(as > 0.0f);
    return *zero ? 0.0f : o.ws / as;
}
__device__ __forceinline__ float proj_value(int32_t acc, float post, bool zero) {
    return zero ? 0.0f : static_cast<float>(acc) * post;
}
// Row i of o (attention inputs: a few values per thread).
__device__ __forceinline__ float proj_at(const ProjOut& o, uint32_t i, float post, bool zero) {
    return proj_value(o.part[i], post, zero);
}

enum InputKind : uint32_t {
    kInEmbed = 0,     // v = the token's embedding row (bf16 or f16 -> f32, model.rs:309-316); the token from the loop state
    kInResidual = 1,  // v = x_in[i] + a[i] (add_residual, ops.rs:476-481)
    kInPlain = 2,     // v = x_in[i]
    kInRelu2Mul = 3,  // v = relu2(a[i]) * b[i] (ops.rs:301-308, 467-473)
};

struct StageInput {
    uint32_t kind, n;     // n: a multiple of 4
    const float* x_in;
    ProjOut a, b;         // the previous projections (residual: o or down; ReLU^2: gate and up)
    float* x_out;         // kInEmbed, kInResidual: v, the residual stream (workgroup 0 writes it), or null
    const float* gamma;   // RMSNorm weights (n <= kNormMax), or null: no norm, y = v (a model without sub-norms)
    float eps;
    const Ctl* ctl;       // kInEmbed
    const uint32_t* prompt;
    const uint16_t* emb;
    uint32_t emb_f16;     // kInEmbed: the embedding holds f16 (else bf16)
    // kInPlain without a norm: the largest |v| as float bits, accumulated by the producing gated pair; each workgroup
    // then reads only the elements of its own K slice
    const uint32_t* amax;
    // kInEmbed in a prefill: the token of this row (the decode step takes it from the loop state instead)
    const uint32_t* token_at;
};

// The loaded inputs of a thread: element e of float4 group k is 4 (tid + k kNT) + e. P4 groups cover P4 * 4 kNT
// elements; SA and SB K slices of the projections a and b (0: the kernel variant reads none).
template <int P4, int SA, int SB>
struct InputRegs {
    uint4 x[P4];                         // embedding bits (x, y) or x_in
    int4 pa[SA > 0 ? SA : 1][P4];        // K-slice partials of a
    int4 pb[SB > 0 ? SB : 1][P4];        // K-slice partials of b
    float4 g[P4];                        // gamma
    float as_a, as_b;                    // activation scales of a and b
    uint32_t amax;                       // StageInput::amax's value
};

struct __align__(16) InputLds {  // ys is accessed 16 bytes at a time
    float ys[kNormMax];          // v (a normed input, for the reference-order fallback), then this workgroup's y window
    double red_d[kNT / 64];
    float red_f[kNT / 64];
    int red_i[kNT / 64];
    float mean;
};

// Elements 4 (tid + k NI) .. + 3 of a stage input belong to thread tid < NI; the threads from NI on hold none (an index
// past every input).
template <uint32_t NI = kNT>
__device__ __forceinline__ uint32_t elem4(uint32_t tid, int k) {
    return tid < NI ? 4u * (tid + static_cast<uint32_t>(k) * NI) : 0xfffffff0u;
}

// Issues every load of the thread's inputs (16 bytes each, and the producers' activation scales) without using any, so
// that the loads a kernel issues after it (weights) do not delay them: vector-memory loads complete in issue order, so
// a load issued after the weights would wait for all of them.
template <int P4, int SA, int SB, uint32_t NI = kNT>
__device__ __forceinline__ void stage_load(const StageInput& p, InputRegs<P4, SA, SB>& r, uint32_t wlo, uint32_t whi) {
    const uint32_t tid = threadIdx.x, n = p.n;
    if (p.kind == kInEmbed) {
        uint32_t tok;
        if (p.token_at != nullptr) {
            tok = *p.token_at;
        } else {
            const uint32_t pos = p.ctl->pos;
            tok = pos < p.ctl->n_prompt ? p.prompt[pos] : p.ctl->token;
        }
        const uint2* row = reinterpret_cast<const uint2*>(p.emb + static_cast<size_t>(tok) * n);
#pragma unroll
        for (int k = 0; k < P4; ++k) {
            const uint32_t i = elem4<NI>(tid, k);
            const uint2 e = load_if(row + i / 4u, i < n);
            r.x[k] = make_uint4(e.x, e.y, 0u, 0u);
        }
    } else if (p.kind != kInRelu2Mul) {
        // with a precomputed maximum only the window [wlo, whi) is read (the elements outside stay 0)
        const bool all = p.amax == nullptr;
        if (!all) r.amax = *p.amax;
#pragma unroll
        for (int k = 0; k < P4; ++k) {
            const uint32_t i = elem4<NI>(tid, k);
            r.x[k] = load_if(reinterpret_cast<const uint4*>(p.x_in + i), i < n && (all || (i >= wlo && i < whi)));
        }
    }
    if constexpr (SA > 0) {
        if (p.kind == kInResidual || p.kind == kInRelu2Mul) {
            r.as_a = *p.a.as;
#pragma unroll
            for (int s = 0; s < SA; ++s)
#pragma unroll
                for (int k = 0; k < P4; ++k) {
                    const uint32_t i = elem4<NI>(tid, k);
                    r.pa[s][k] = load_if(reinterpret_cast<const int4*>(p.a.part + static_cast<size_t>(s) * p.a.stride + i),
                                         i < n && static_cast<uint32_t>(s) < p.a.kslices);
                }
        }
    }
    if constexpr (SB > 0) {
        if (p.kind == kInRelu2Mul) {
            r.as_b = *p.b.as;
#pragma unroll
            for (int s = 0; s < SB; ++s)
#pragma unroll
                for (int k = 0; k < P4; ++k) {
                    const uint32_t i = elem4<NI>(tid, k);
                    r.pb[s][k] = load_if(reinterpret_cast<const int4*>(p.b.part + static_cast<size_t>(s) * p.b.stride + i),
                                         i < n && static_cast<uint32_t>(s) < p.b.kslices);
                }
        }
    }
    if (p.gamma != nullptr) {
#pragma unroll
        for (int k = 0; k < P4; ++k) {
            const uint32_t i = elem4<NI>(tid, k);
            r.g[k] = load_if(reinterpret_cast<const float4*>(p.gamma + i), i < n);
        }
    }
}

// Waits until the thread's input loads (and `extra`) have arrived: an empty asm reads one word folded from every loaded
// register. (An asm that takes the registers themselves as in-out operands would pin them, and each conditional load
// would then be copied into them under its own wait.)
template <int P4, int SA, int SB>
__device__ __forceinline__ void input_arrived(const InputRegs<P4, SA, SB>& r, uint32_t extra) {
    uint32_t t = extra ^ f32_bits(r.as_a) ^ f32_bits(r.as_b);
#pragma unroll
    for (int k = 0; k < P4; ++k) {
        t ^= r.x[k].x ^ r.x[k].y ^ r.x[k].z ^ r.x[k].w;
        t ^= f32_bits(r.g[k].x) ^ f32_bits(r.g[k].y) ^ f32_bits(r.g[k].z) ^ f32_bits(r.g[k].w);
        if constexpr (SA > 0) {
#pragma unroll
            for (int s = 0; s < SA; ++s) t ^= r.pa[s][k].x ^ r.pa[s][k].y ^ r.pa[s][k].z ^ r.pa[s][k].w;
        }
        if constexpr (SB > 0) {
#pragma unroll
            for (int s = 0; s < SB; ++s) t ^= r.pb[s][k].x ^ r.pb[s][k].y ^ r.pb[s][k].z ^ r.pb[s][k].w;
        }
    }
    asm volatile("" : : "v"(t) : "memory");
}

template <int P4, int SA>
__device__ __forceinline__ void slice_sums(const int4 (&pa)[SA > 0 ? SA : 1][P4], int k, int32_t (&sa)[4]) {
    sa[0] = pa[0][k].x;
    sa[1] = pa[0][k].y;
    sa[2] = pa[0][k].z;
    sa[3] = pa[0][k].w;
#pragma unroll
    for (int s2 = 1; s2 < SA; ++s2) {
        sa[0] += pa[s2][k].x;
        sa[1] += pa[s2][k].y;
        sa[2] += pa[s2][k].z;
        sa[3] += pa[s2][k].w;
    }
}

// Times an RMSNorm took the reference's sequential order because its tree-summed mean lay too close to an f32 rounding
// boundary (one count per workgroup that computed such a norm). Diagnostic only: read by vx_decoder_norm_fallbacks.
__device__ unsigned int g_norm_fallbacks;

// y of the thread's elements: v by kind, then (with gamma) its RMSNorm y = (v * inv) * gamma (rms_norm, ops.rs:19-96).
// Every thread derives the mean from the per-wave sums itself, so the common path has one barrier; without gamma none.
// With write_x, an input that has an x_out also stores v there.
template <int P4, int SA, int SB, uint32_t NI = kNT>
__device__ __forceinline__ void stage_y(const StageInput& p, const InputRegs<P4, SA, SB>& r, InputLds& s, bool write_x,
                                        float (&y)[P4][4]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n = p.n;
    float v[P4][4];
    if (p.kind == kInEmbed) {
#pragma unroll
        for (int k = 0; k < P4; ++k) {
            const uint32_t h[4] = {r.x[k].x & 0xffffu, r.x[k].x >> 16, r.x[k].y & 0xffffu, r.x[k].y >> 16};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[k][e] = p.emb_f16 ? f16_f32(static_cast<uint16_t>(h[e])) : bits_f32(h[e] << 16);
        }
    } else if (SA > 0 && SB > 0 && p.kind == kInRelu2Mul) {
        bool za, zb;
        const float pa = proj_post(p.a, r.as_a, &za), pb = proj_post(p.b, r.as_b, &zb);
#pragma unroll
        for (int k = 0; k < P4; ++k) {
            int32_t sa[4], sb[4];
            slice_sums<P4, SA>(r.pa, k, sa);
            slice_sums<P4, SB>(r.pb, k, sb);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float g = proj_value(sa[e], pa, za), u = proj_value(sb[e], pb, zb);
                const float pos = g > 0.0f ? g : 0.0f;
                const float sq = pos * pos;
                v[k][e] = sq * u;
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < P4; ++k) {
            v[k][0] = bits_f32(r.x[k].x);
            v[k][1] = bits_f32(r.x[k].y);
            v[k][2] = bits_f32(r.x[k].z);
            v[k][3] = bits_f32(r.x[k].w);
        }
        if (SA > 0 && p.kind == kInResidual) {
            bool za;
            const float pa = proj_post(p.a, r.as_a, &za);
#pragma unroll
            for (int k = 0; k < P4; ++k) {
                int32_t sa[4];
                slice_sums<P4, SA>(r.pa, k, sa);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[k][e] = v[k][e] + proj_value(sa[e], pa, za);
            }
        }
    }
    if (write_x && (p.kind == kInEmbed || p.kind == kInResidual) && p.x_out != nullptr) {
#pragma unroll
        for (int k = 0; k < P4; ++k)
            if (elem4<NI>(tid, k) < n)
                *reinterpret_cast<float4*>(p.x_out + elem4<NI>(tid, k)) = make_float4(v[k][0], v[k][1], v[k][2], v[k][3]);
    }
    if (p.gamma == nullptr) {
#pragma unroll
        for (int k = 0; k < P4; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) y[k][e] = v[k][e];
        return;
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < P4; ++k) {
        const uint32_t i = elem4<NI>(tid, k);
        if (i < n) {
            *reinterpret_cast<float4*>(s.ys + i) = make_float4(v[k][0], v[k][1], v[k][2], v[k][3]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sqv = v[k][e] * v[k][e];
                ss += static_cast<double>(sqv);
            }
        }
    }
    constexpr uint32_t kW = NI / 64;  // waves that hold elements
    if (wave < kW) {
        ss = wave_sum_f64(ss);
        if (lane == 0) s.red_d[wave] = ss;
    }
    __syncthreads();
    // Wave 0 alone turns the sums into the scale (the other waves would only repeat it) and hands it over in LDS.
    if (wave == 0) {
        double t = 0.0;
        for (uint32_t w = 0; w < kW; ++w) t += s.red_d[w];
        // The reference's sequential f64 sum and t (any order of the same additions) both lie within (n - 1) 2^-53 S of
        // the exact sum S of the nonnegative squares, so the reference's quotient by n (rounded) lies within
        // (2 (n - 1) + 3) 2^-53 q of q = t / n and of the rounded ends of [q - e, q + e] for e = (2 n + 8) 2^-53 q;
        // when both ends round to the same f32, so does it.
        const double q = t / static_cast<double>(n);
        const double e = (2.0 * static_cast<double>(n) + 8.0) * 0x1.0p-53 * q;
        float mean = static_cast<float>(q);
        const float lo = static_cast<float>(q - e);
        const float hi = static_cast<float>(q + e);
        if (lane == 0) {
            if (lo != hi) {  // too close to an f32 rounding boundary: the reference's order
                atomicAdd(&g_norm_fallbacks, 1u);
                double seq = 0.0;
                for (uint32_t i = 0; i < n; ++i) {
                    const float sqv = s.ys[i] * s.ys[i];
                    seq += static_cast<double>(sqv);
                }
                mean = static_cast<float>(seq / static_cast<double>(n));
            }
            s.mean = 1.0f / __builtin_sqrtf(mean + p.eps);
        }
    }
    __syncthreads();
    const float scale = s.mean;
#pragma unroll
    for (int k = 0; k < P4; ++k) {
        const float gm[4] = {r.g[k].x, r.g[k].y, r.g[k].z, r.g[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float tt = v[k][e] * scale;
            y[k][e] = tt * gm[e];
        }
    }
}

// The elements [lo, hi) of a staged slice: byte-columns [c0, c1) of a row of n columns (pack.rs:230-237: column c of a
// full 160-trit block holds elements (c / 32) 160 + c % 32 + 32 k, the packed tail 5 per column), widened to whole
// float4 groups.
__device__ __forceinline__ void slice_window(uint32_t n, uint32_t c0, uint32_t c1, uint32_t* lo, uint32_t* hi) {
    const uint32_t full = n / 160u * 32u, tail0 = n / 160u * 160u;
    if (c1 <= c0) {
        *lo = *hi = 0;
        return;
    }
    const uint32_t a = c0 < full ? c0 / 32u * 160u + c0 % 32u : tail0 + 5u * (c0 - full);
    const uint32_t l = c1 - 1u;
    uint32_t b = l < full ? l / 32u * 160u + l % 32u + 129u : tail0 + 5u * (l - full) + 5u;
    b = b < n ? b : n;
    *lo = a & ~3u;
    *hi = (b + 3u) & ~3u;
}

// Writes the thread's y of elements [lo, hi) to s.ys[i - lo] and returns its largest |y| over all elements (NaN never
// counts). The window must be at most kNormMax long; it is readable after the next barrier.
template <int P4, uint32_t NI = kNT>
__device__ __forceinline__ float stage_window(const float (&y)[P4][4], uint32_t n, uint32_t lo, uint32_t hi, InputLds& s) {
    const uint32_t tid = threadIdx.x;
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < P4; ++k) {
        const uint32_t i = elem4<NI>(tid, k);
        if (i < n) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ay = __builtin_fabsf(y[k][e]);
                if (ay > mx) mx = ay;
            }
            if (i >= lo && i < hi)
                *reinterpret_cast<float4*>(s.ys + (i - lo)) = make_float4(y[k][0], y[k][1], y[k][2], y[k][3]);
        }
    }
    return mx;
}

__device__ __forceinline__ int quant_code(float y, float sc) {
    float rr = __builtin_roundf(y * sc);
    rr = rr < -128.0f ? -128.0f : (rr > 127.0f ? 127.0f : rr);
    return static_cast<int>(rr);
}

// Per-token absmax int8 quantization (quantize_activations_int8_with_range, ops.rs:241-267, levels 127) and the GEMV
// staging of the codes of byte-columns [c0, c1) into st[c - c0]: entry c holds the low nibbles ((x & 15) ^ 8) and the
// high nibbles (x >> 4) of its five activations (column_activation_index, pack.rs:230-237; zero past the row), read
// from the window s.ys[i - lo]. The sum of all n codes comes from the thread's own y. Two barriers; afterwards the
// entries are complete, *scale is the activation scale and *act_sum the sum of the codes, in every thread.
template <int P4, uint32_t NI = kNT>
__device__ __forceinline__ void stage_quant(const float (&y)[P4][4], InputLds& s, float mx, uint32_t n, uint32_t tbr,
                                            uint32_t c0, uint32_t c1, uint32_t lo, uint2* st, float* scale, int* act_sum) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    constexpr uint32_t kW = NI / 64;  // waves that hold elements
    if (wave < kW) {
        mx = wave_max_f32(mx);
        if (lane == 0) s.red_f[wave] = mx;
    }
    __syncthreads();
    float m = 0.0f;
    for (uint32_t w = 0; w < kW; ++w) m = fmax_nn(m, s.red_f[w]);
    const float sc = m > 0.0f ? 127.0f / m : 0.0f;
    int sum = 0;  // the codes of the staged columns' elements (each element belongs to one column)
    const uint32_t full = n / 160u * 32u;
    for (uint32_t c = c0 + tid; c < c1; c += kNT) {
        uint32_t lo_n = 0, hi_n = 0;
        const uint32_t base = c < full ? (c / 32u) * 160u + (c % 32u) : (n / 160u) * 160u + 5u * (c - full);
        const uint32_t step = c < full ? 32u : 1u;
#pragma unroll
        for (uint32_t k = 0; k < 5; ++k) {
            const uint32_t idx = base + k * step;
            int x = 0;
            if (c < tbr && idx < n && m > 0.0f) x = quant_code(s.ys[idx - lo], sc);
            sum += x;
            lo_n |= ((static_cast<uint32_t>(x) & 15u) ^ 8u) << (4 * k);
            hi_n |= (static_cast<uint32_t>(x >> 4) & 15u) << (4 * k);
        }
        st[c - c0] = make_uint2(lo_n, hi_n);
    }
    const uint32_t cw = c1 > c0 ? min(static_cast<uint32_t>(kNT / 64), (c1 - c0 + 63u) / 64u) : 0u;  // waves with columns
    if (wave < cw) {
        sum = wave_sum_i32(sum);
        if (lane == 0) s.red_i[wave] = sum;
    }
    __syncthreads();
    int t = 0;
    for (uint32_t w = 0; w < cw; ++w) t += s.red_i[w];
    *act_sum = t;
    *scale = sc;
}

// ---- decode-step GEMV ------------------------------------------------------------------------------------------------------

// ggml_v_expf (quintrit-runtime/src/ops.rs:314-377) for one lane: n = round(x log2 e) by the 1.5 2^23 shift,
// b = x - n ln 2 in two parts, j = the degree-5 polynomial of b without its constant term, k = 2^n in the exponent
// field; |n| <= 126 gives k + k j, beyond that 2^n is split as s1 s2 to reach the subnormal and overflow ranges and
// |n| > 192 gives s1 s1. Every multiply-add of the reference is a fused one here too (no contraction elsewhere).
__device__ __forceinline__ float ggml_expf(float x) {
    const float r = bits_f32(0x4b400000u);
    const float z = __builtin_fmaf(x, bits_f32(0x3fb8aa3bu), r);
    const float n = z - r;
    const float b = __builtin_fmaf(-n, bits_f32(0x35bfbe8eu), __builtin_fmaf(-n, bits_f32(0x3f317200u), x));
    const uint32_t e = f32_bits(z) << 23;
    const float k = bits_f32(e + 0x3f800000u);
    const float u = b * b;
    const float j = __builtin_fmaf(__builtin_fmaf(__builtin_fmaf(bits_f32(0x3c072010u), b, bits_f32(0x3d2b9f17u)), u,
                                                  __builtin_fmaf(bits_f32(0x3e2aaf33u), b, bits_f32(0x3efffedbu))),
                                   u, bits_f32(0x3f7ffff6u) * b);
    const float an = __builtin_fabsf(n);
    if (!(an > 126.0f)) return __builtin_fmaf(k, j, k);
    const uint32_t g = n <= 0.0f ? 0x82000000u : 0u;
    const float s1 = bits_f32(g + 0x7f000000u);
    const float s2 = bits_f32(e - g);
    if (an > 192.0f) return s1 * s1;
    return __builtin_fmaf(s2, j, s2) * s1;
}

enum GateAct : uint32_t {
    kActRelu2 = 0,  // relu2(g) * u (ops.rs:301-308, 467-473)
    kActSilu = 1,   // swiglu (ops.rs:430-464): whole blocks of 8 use ggml_v_silu, the last n % 8 values libm's expf
};

// One projection of a stage. A work item is (64-row tile, K slice): the 16 waves of a workgroup split the slice's
// chunks and add their int32 sums in LDS, and the tile's slice sums (with the row corrections on slice 0) are stored
// as part[ks][row]; the consumers add the slices and apply the epilogue (ProjOut).
// A gated pair (w2 set: gate = w, up = w2, one K slice) instead treats the two matrices' chunks of a tile as one list,
// applies the layer epilogue to both rows and stores act(gate, up) as f32 in act_out[row].
struct DJob {
    const uint8_t* w;      // device layout (vx_layout)
    const int32_t* dsum;   // per padded row: digit sum of the device row
    int32_t* part;         // [kslices][padded_rows]
    const uint8_t* w2;     // gated pair: the up projection (same geometry), else null
    const int32_t* dsum2;
    float* act_out;        // gated pair: [padded_rows]
    float ws, ws2;         // gated pair: weight scales
    uint32_t act, n8;      // gated pair: GateAct; rows below n8 take the vector exponential
    uint32_t* amax_out;    // gated pair: atomic maximum of |act_out| as float bits (a plain unnormed consumer), or null
    uint32_t rows, padded_rows, n_tiles, n_chunks, kslices, slice_chunks, item_begin;
    uint32_t w_bytes;      // bytes of w (and w2) in the device layout, below kBufferOutOfRange
    // gated pair split into chunk ranges: per tile and row one word that the workgroups whose ranges meet the tile add
    // to atomically ([tile][64], zero between launches): bits 0-23 and 24-47 the gate and up sums, each contribution
    // raised by kRangeBias, bits 48-63 the count of contributions
    unsigned long long* accum;
};
// Each contribution to a packed 24-bit field is v + kRangeBias, with |v| at most 80 x 272 per chunk of one matrix that
// the workgroup's range covers in the tile (80 weights per 16-byte chunk, digits 0..2 times staged values of magnitude
// at most 136). range_fields_fit() admits a range split only where |v| < kRangeBias and the contributions to one word,
// each in (0, 2 kRangeBias), add up below 2^24.
constexpr int kRangeBias = 1 << 21;
constexpr uint64_t kRangeChunkMax = 80u * 272u;
inline bool range_fields_fit(uint64_t n_chunks, uint64_t C, uint64_t G) {
    const uint64_t per_wg = C / G;  // every workgroup's range holds at least this many chunks
    if (per_wg == 0) return false;
    const uint64_t covered = std::min(n_chunks, (C + G - 1) / G);  // chunks of one matrix in one contribution
    const uint64_t contributions = (2u * n_chunks + per_wg - 1) / per_wg + 1u;  // workgroups that meet one tile
    return covered * kRangeChunkMax < static_cast<uint64_t>(kRangeBias) &&
           contributions * 2u * static_cast<uint64_t>(kRangeBias) <= (1ull << 24) && contributions < (1u << 16);
}

constexpr int kMaxStageJobs = 3;
constexpr int kMaxClear = 6;
// Buffer loads of the weights: the resource's fourth word for raw (unformatted, unswizzled) access, an offset past any
// matrix (such a load returns zeros without touching memory) and the non-temporal cache policy.
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr uint32_t kBufferOutOfRange = 0x80000000u;
constexpr int kLoadNt = 2;
constexpr int kDPer = 7;  // chunks of a work item per wave at most (kStChunks / 16)
// Tiles a workgroup's chunk range of a gated pair touches at most: a range of at most 16 kDPer chunks starting inside a
// tile of 2 n_chunks chunks, with 2 n_chunks >= 8 kDPer (the host's condition), ends within the third tile.
constexpr int kRangeSegs = 3;
constexpr int kRangeEarly = 1;  // chunks per wave of a range issued before the stage input is computed

struct DStageArgs {
    DJob job[kMaxStageJobs];
    uint32_t n_jobs, total_items;
    StageInput in;
    uint32_t tbr;       // tile row bytes of in.n columns
    float* as_out;      // the stage's activation scale (workgroup 0)
    uint32_t variant;   // the kernel instance (host side: the input's length and kinds)
    uint32_t loop;      // every job has one K slice: a workgroup takes items blockIdx.x and blockIdx.x + gridDim.x
    uint32_t grid;      // workgroups of the launch
    uint32_t* amax_clear;  // zeroed by the stage (the StageInput::amax a later stage of the layer accumulates), or null
    uint32_t dper;         // chunk loads per wave and item of the kernel instance (1, 4 or 7): at least any wave's count
    // A gated pair split into equal chunk ranges (0: split into items): the pair's chunks listed tile by tile, the gate
    // chunks of a tile before its up chunks, range_chunks of them in all; workgroup w takes [w C / G, (w + 1) C / G).
    uint32_t range_chunks;
    // accumulators this stage zeroes once it is done (outputs of projections whose consumers have run, which a later
    // stage adds to again), or null
    int32_t* clear[kMaxClear];
    uint32_t clear_words[kMaxClear];
};

__constant__ DigitTable g_digits = make_digit_table();

// One workgroup per work item, or (loop) a workgroup per two items of the same K slice, which computes the stage input
// once for both. Order of the loads: the stage input, the digit table, then wave w's chunks q0 + w, q0 + w + 16, ... of
// the tile (1 KiB each in the device layout) of the first item, so the input is computed while the weights are in
// flight; the second item's chunks go out one by one as the first item's are consumed. Every wave issues exactly DPER
// chunk loads per item (buffer loads; a chunk the wave does not have reads past the buffer's end, which returns zeros
// without a memory access), so each chunk is waited for on its own. The digit-nibble table and the arithmetic are those
// of the lone GEMV (vx_gemv.hip). Only the entries of the item's own chunks are staged.
template <int P4, int SA, int SB, bool MULTI, int DPER, bool RANGE, uint32_t NI>
__global__ __launch_bounds__(kNT) void dgemv_kernel(DStageArgs a) {
    static_assert(!RANGE || (MULTI && DPER == kDPer), "the chunk-range split runs on the gated-pair instance");
    __shared__ uint32_t tab[256 * 64];  // row B: 32 copies of the digit nibbles of byte B (first half)
    __shared__ uint2 st[kStChunks * 16];
    __shared__ InputLds s;
    __shared__ int red[MULTI ? kRangeSegs : 1][MULTI ? 2 : 1][kNT / 64][64];  // [item or tile][gate, up][wave][lane]

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const char* tabb = reinterpret_cast<const char*>(tab);
    const uint32_t lane_off = (lane & 31u) * 4u;

    // A work item: its job, tile and K slice, and where wave `wave`'s chunks are (byte offsets in the matrix).
    struct Item {
        DJob jb;
        uint32_t tile, ks, q0, nq, cnt;
        uint32_t off;  // the lane's 16 bytes of chunk 0 of the tile
        uint32_t cs;   // bytes between chunks q and q + 1 of the tile
    };
    // Every kernel argument that the stage input's loads depend on (the job geometry that places the K slice, the
    // input's kind, length and pointers) is read in one batch and held in registers: read where used, each would be a
    // scalar load waited for on its own before the next, a chain of memory latencies before the first input load.
    StageInput in = a.in;
    uint32_t jib[kMaxStageJobs], jks[kMaxStageJobs], jsc[kMaxStageJobs], jnc[kMaxStageJobs], jnt[kMaxStageJobs];
    bool jpair[kMaxStageJobs];
#pragma unroll
    for (int k = 0; k < kMaxStageJobs; ++k) {
        jib[k] = a.job[k].item_begin;
        jks[k] = a.job[k].kslices;
        jsc[k] = a.job[k].slice_chunks;
        jnc[k] = a.job[k].n_chunks;
        jnt[k] = a.job[k].n_tiles;
        jpair[k] = a.job[k].w2 != nullptr;
    }
    const uint32_t n_jobs = a.n_jobs, tbr = a.tbr;
    asm volatile("" : : "s"(n_jobs), "s"(tbr), "s"(jib[1]), "s"(jib[2]), "s"(jks[0]), "s"(jks[1]), "s"(jks[2]),
                 "s"(jsc[0]), "s"(jsc[1]), "s"(jsc[2]), "s"(jnc[0]), "s"(jnc[1]), "s"(jnc[2]), "s"(jnt[0]), "s"(jnt[1]),
                 "s"(jnt[2]), "s"(in.kind), "s"(in.n), "s"(in.x_in), "s"(in.amax), "s"(in.a.part), "s"(in.a.as),
                 "s"(in.a.kslices), "s"(in.a.stride), "s"(in.b.part), "s"(in.b.as), "s"(in.b.kslices), "s"(in.b.stride),
                 "s"(in.gamma), "s"(in.ctl), "s"(in.token_at));
    auto locate = [&](uint32_t item) {
        Item it;
        uint32_t j = 0;
        if (n_jobs > 1 && item >= jib[1]) j = 1;
        if (n_jobs > 2 && item >= jib[2]) j = 2;
        const uint32_t ib = j == 0 ? 0u : (j == 1 ? jib[1] : jib[2]);
        const uint32_t ks = j == 0 ? jks[0] : (j == 1 ? jks[1] : jks[2]);
        const uint32_t sc = j == 0 ? jsc[0] : (j == 1 ? jsc[1] : jsc[2]);
        const uint32_t ncj = j == 0 ? jnc[0] : (j == 1 ? jnc[1] : jnc[2]);
        const uint32_t ntj = j == 0 ? jnt[0] : (j == 1 ? jnt[1] : jnt[2]);
        const bool pr = j == 0 ? jpair[0] : (j == 1 ? jpair[1] : jpair[2]);
        it.jb = j == 0 ? a.job[0] : (j == 1 ? a.job[1] : a.job[2]);
        const uint32_t local = item - ib;
        it.tile = local / ks;
        it.ks = local - it.tile * ks;
        const uint32_t grp = it.tile / kTileGroup, tt = it.tile - grp * kTileGroup;
        const uint32_t T = min(static_cast<uint32_t>(kTileGroup), ntj - grp * kTileGroup);
        it.q0 = it.ks * sc;
        it.nq = min(sc, ncj - it.q0);
        const uint32_t nl = MULTI && pr ? 2u * it.nq : it.nq;  // gate chunks, then (pair) up chunks
        it.cnt = wave < nl ? (nl - wave + kTileGroup - 1) / kTileGroup : 0u;
        it.off = ((grp * kTileGroup * ncj + tt) * 64u + lane) * 16u;
        it.cs = T * 1024u;
        return it;
    };
    // chunk i of an item for this wave (an absent chunk, or any chunk when !valid, reads past the end)
    auto issue_one = [&](const Item& it, bool valid, int i) {
        const uint32_t c = wave + kTileGroup * static_cast<uint32_t>(i);
        const bool up = MULTI && it.jb.w2 != nullptr && c >= it.nq;
        const uint32_t q = up ? c - it.nq : c;
        const bool have = valid && static_cast<uint32_t>(i) < it.cnt;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(up ? it.jb.w2 : it.jb.w), 0, it.jb.w_bytes, kBufferRsrcWord3);
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             r, have ? it.off + (it.q0 + q) * it.cs : kBufferOutOfRange, 0, kLoadNt));
    };

    const Item ia = locate(blockIdx.x);
    // The staged slice: both items of a workgroup have the same K slice (a looping stage's jobs have one slice each).
    const uint32_t c0 = ia.q0 * 16u, c1 = min((ia.q0 + ia.nq) * 16u, tbr);
    uint32_t lo, hi;
    slice_window(in.n, c0, c1, &lo, &hi);
    InputRegs<P4, SA, SB> r;
    stage_load<P4, SA, SB, NI>(in, r, lo, hi);
    uint32_t dig[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) dig[k] = g_digits.v[(tid + k * kNT) >> 3];
    if (a.amax_clear != nullptr && blockIdx.x == 0 && tid == 0) *a.amax_clear = 0u;
    // The weight loads go out once the input and the digit table have arrived (the waits for the input would otherwise
    // also wait for the weights, which complete after them).
    input_arrived(r, dig[0] ^ dig[1]);
    // A gated pair in chunk ranges: this workgroup's chunks [rb, re) of the pair's list; chunk rb + i is chunk j0 + i
    // counted from the start of tile t_first (so in tile t_first + seg, seg < kRangeSegs).
    constexpr bool range = RANGE;
    const uint32_t nc = ia.jb.n_chunks, nc2 = 2u * nc;
    uint32_t rb = 0, re = 0, t_first = 0, j0 = 0;
    if constexpr (RANGE) {
        rb = static_cast<uint32_t>(static_cast<uint64_t>(blockIdx.x) * a.range_chunks / gridDim.x);
        re = static_cast<uint32_t>(static_cast<uint64_t>(blockIdx.x + 1u) * a.range_chunks / gridDim.x);
        t_first = rb / nc2;
        j0 = rb - t_first * nc2;
    }
    struct RChunk {
        uint32_t seg, q;  // tile segment, chunk of the row
        bool up;
    };
    auto rchunk = [&](uint32_t i) {
        const uint32_t jj = j0 + i;
        RChunk c;
        c.seg = (jj >= nc2 ? 1u : 0u) + (jj >= 2u * nc2 ? 1u : 0u);
        const uint32_t within = jj - c.seg * nc2;
        c.up = within >= nc;
        c.q = c.up ? within - nc : within;
        return c;
    };
    // chunk k of this wave in the range: its matrix and byte offset (a chunk past the range reads past the end); the
    // load itself is issued in one place for both modes, so that the waits for it stay exact
    auto issue_first = [&](int k) {
        const uint32_t i = wave + kTileGroup * static_cast<uint32_t>(k);
        const uint8_t* base;
        uint32_t off;
        if constexpr (RANGE) {
            const RChunk c = rchunk(i);
            const uint32_t t = min(t_first + c.seg, ia.jb.n_tiles - 1u);
            const uint32_t grp = t / kTileGroup, tt = t - grp * kTileGroup;
            const uint32_t T = min(static_cast<uint32_t>(kTileGroup), ia.jb.n_tiles - grp * kTileGroup);
            base = c.up ? ia.jb.w2 : ia.jb.w;
            off = rb + i < re ? ((grp * kTileGroup * nc + tt) * 64u + lane) * 16u + c.q * T * 1024u : kBufferOutOfRange;
        } else {
            const bool up = MULTI && ia.jb.w2 != nullptr && i >= ia.nq;
            const uint32_t q = up ? i - ia.nq : i;
            base = up ? ia.jb.w2 : ia.jb.w;
            off = static_cast<uint32_t>(k) < ia.cnt ? ia.off + (ia.q0 + q) * ia.cs : kBufferOutOfRange;
        }
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, ia.jb.w_bytes, kBufferRsrcWord3);
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kLoadNt));
    };
    // A range issues its first kRangeEarly chunks per wave now and each next one as an earlier one is consumed (then
    // kRangeEarly chunks ahead): the fewer weight loads there are in flight while the stage input is loaded, the sooner
    // its loads return (all seven at once held the input's waves at their loads until most of the stage's weights had
    // arrived; one, two and three measured 2.073, 2.083 and 2.089 ms per Falcon3-10B token).
    u32x4 ba[DPER];
#pragma unroll
    for (int i = 0; i < DPER; ++i)
        if (!range || i < kRangeEarly) ba[i] = issue_first(i);
    const uint32_t item_b = blockIdx.x + gridDim.x;
    const bool has_b = MULTI && a.loop && item_b < a.total_items;
    Item ib{};
    u32x4 bb[MULTI ? DPER : 1];
    if constexpr (MULTI) ib = locate(has_b ? item_b : blockIdx.x);
    // The row digit sums the epilogue adds (wave 0: the rows of the items; a range: wave sg, the rows of tile
    // t_first + sg), issued after the weights so that they do not delay them, and first used after the last chunk.
    // Every wave loads them (unconditional loads at valid rows, so that every wait stays exact); only those waves use
    // them.
    int dsa, dsa2, dsb = 0, dsb2 = 0;
    {
        uint32_t t = ia.tile;
        if constexpr (RANGE) t = min(t_first + min(wave, static_cast<uint32_t>(kRangeSegs) - 1u), ia.jb.n_tiles - 1u);
        const uint32_t row = t * kTileRows + lane;
        dsa = ia.jb.dsum[row];
        dsa2 = (ia.jb.dsum2 != nullptr ? ia.jb.dsum2 : ia.jb.dsum)[row];
        if constexpr (MULTI && !RANGE) {
            const uint32_t rowb = ib.tile * kTileRows + lane;
            dsb = ib.jb.dsum[rowb];
            dsb2 = (ib.jb.dsum2 != nullptr ? ib.jb.dsum2 : ib.jb.dsum)[rowb];
        }
    }

    float y[P4][4];
    stage_y<P4, SA, SB, NI>(in, r, s, blockIdx.x == 0, y);
    float mx = stage_window<P4, NI>(y, in.n, lo, hi, s);
    if (in.amax != nullptr) mx = __uint_as_float(r.amax);
    // The table is filled after the input's values are computed (its loads were issued after the input's, so waiting
    // for them earlier would also wait for the input) and before the quantization's first barrier.
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // 8 uint4 stores per entry
        const uint32_t i = tid + k * kNT;
        *reinterpret_cast<uint4*>(reinterpret_cast<char*>(tab) + (i >> 3) * 256u + (i & 7u) * 16u) =
            make_uint4(dig[k], dig[k], dig[k], dig[k]);
    }
    float act_scale;
    int act_sum;
    stage_quant<P4, NI>(y, s, mx, in.n, tbr, c0, (ia.q0 + ia.nq) * 16u, lo, st, &act_scale, &act_sum);
    if (blockIdx.x == 0 && tid == 0) *a.as_out = act_scale;

    // The sums of an item's chunks (from b) into red[slot] (gate, and up for a pair); with `next`, chunk i of the second
    // item goes out once chunk i of this one is consumed.
    auto accumulate = [&](const Item& it, const u32x4 (&b)[DPER], uint32_t slot, bool next) {
        const bool pair = MULTI && it.jb.w2 != nullptr;
        int acc_lo = 0, acc_hi = 0, acc2_lo = 0, acc2_hi = 0;
#pragma unroll
        for (int i = 0; i < DPER; ++i) {
            if (static_cast<uint32_t>(i) < it.cnt) {
                const uint32_t c = wave + kTileGroup * i;
                const bool up = pair && c >= it.nq;
                const uint32_t q = up ? c - it.nq : c;  // chunk of the slice
                const uint32_t dw[4] = {b[i].x, b[i].y, b[i].z, b[i].w};
                const uint2 e = st[q * 16u + (lane & 15u)];
                __builtin_amdgcn_sched_barrier(0);
                uint32_t t[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const uint32_t addr = __builtin_amdgcn_perm(dw[k >> 2], lane_off, 0x0c0c0000u | ((4u + (k & 3)) << 8));
                    t[k] = *reinterpret_cast<const uint32_t*>(tabb + addr);
                }
                if (!pair) {
                    dot4_bcast<0>(acc_lo, acc_hi, e.x, e.y, t[0], t[1], t[2], t[3]);
                    dot4_bcast<4>(acc_lo, acc_hi, e.x, e.y, t[4], t[5], t[6], t[7]);
                    dot4_bcast<8>(acc_lo, acc_hi, e.x, e.y, t[8], t[9], t[10], t[11]);
                    dot4_bcast<12>(acc_lo, acc_hi, e.x, e.y, t[12], t[13], t[14], t[15]);
                } else {
                    int l = 0, h = 0;
                    dot4_bcast<0>(l, h, e.x, e.y, t[0], t[1], t[2], t[3]);
                    dot4_bcast<4>(l, h, e.x, e.y, t[4], t[5], t[6], t[7]);
                    dot4_bcast<8>(l, h, e.x, e.y, t[8], t[9], t[10], t[11]);
                    dot4_bcast<12>(l, h, e.x, e.y, t[12], t[13], t[14], t[15]);
                    if (up) {
                        acc2_lo += l;
                        acc2_hi += h;
                    } else {
                        acc_lo += l;
                        acc_hi += h;
                    }
                }
            }
            if constexpr (MULTI) {
                if (next) bb[i] = issue_one(ib, has_b, i);
            }
        }
        red[slot][0][wave][lane] = acc_lo + 16 * acc_hi;
        if (pair) red[slot][MULTI ? 1 : 0][wave][lane] = acc2_lo + 16 * acc2_hi;
    };
    // The sums of this wave's chunks of the range (from b) into red[tile segment][gate, up].
    auto accumulate_range = [&](u32x4 (&b)[DPER]) {
        int s00 = 0, s01 = 0, s10 = 0, s11 = 0, s20 = 0, s21 = 0;
#pragma unroll
        for (int k = 0; k < DPER; ++k) {
            if (k + kRangeEarly < DPER) b[k + kRangeEarly] = issue_first(k + kRangeEarly);
            const uint32_t i = wave + kTileGroup * static_cast<uint32_t>(k);
            if (rb + i < re) {
                const RChunk c = rchunk(i);
                const uint32_t dw[4] = {b[k].x, b[k].y, b[k].z, b[k].w};
                const uint2 e = st[c.q * 16u + (lane & 15u)];
                __builtin_amdgcn_sched_barrier(0);
                uint32_t t[16];
#pragma unroll
                for (int m = 0; m < 16; ++m) {
                    const uint32_t addr = __builtin_amdgcn_perm(dw[m >> 2], lane_off, 0x0c0c0000u | ((4u + (m & 3)) << 8));
                    t[m] = *reinterpret_cast<const uint32_t*>(tabb + addr);
                }
                int l = 0, h = 0;
                dot4_bcast<0>(l, h, e.x, e.y, t[0], t[1], t[2], t[3]);
                dot4_bcast<4>(l, h, e.x, e.y, t[4], t[5], t[6], t[7]);
                dot4_bcast<8>(l, h, e.x, e.y, t[8], t[9], t[10], t[11]);
                dot4_bcast<12>(l, h, e.x, e.y, t[12], t[13], t[14], t[15]);
                const int v = l + 16 * h;
                const uint32_t slot = c.seg * 2u + (c.up ? 1u : 0u);  // the same in every lane
                if (slot == 0) s00 += v;
                else if (slot == 1) s01 += v;
                else if (slot == 2) s10 += v;
                else if (slot == 3) s11 += v;
                else if (slot == 4) s20 += v;
                else s21 += v;
            }
        }
        if constexpr (MULTI) {  // a range split is a multi-item launch: red has kRangeSegs x 2 slots
            red[0][0][wave][lane] = s00;
            red[0][1][wave][lane] = s01;
            red[1][0][wave][lane] = s10;
            red[1][1][wave][lane] = s11;
            red[2][0][wave][lane] = s20;
            red[2][1][wave][lane] = s21;
        }
    };
    // The outputs of row `row` of a gated pair from the complete sums v (gate) and v2 (up) of its row, corrections
    // included: the layer epilogue of both projections (layer.rs:246-253), then the gating of model.rs:155-170. A whole
    // wave calls it (the absmax is a wave reduction).
    auto gate_out = [&](const DJob& jb, uint32_t row, int v, int v2, bool own) {
        const bool zero = !(act_scale > 0.0f);
        const float g = zero ? 0.0f : static_cast<float>(v) * (jb.ws / act_scale);
        const float u = zero ? 0.0f : static_cast<float>(v2) * (jb.ws2 / act_scale);
        float o;
        if (jb.act == kActSilu) {
            const float ex = row < jb.n8 ? ggml_expf(0.0f - g) : glibc_expf(-g);
            const float den = 1.0f + ex;
            const float sl = g / den;
            o = sl * u;
        } else {
            const float pos = g > 0.0f ? g : 0.0f;
            const float sq = pos * pos;
            o = sq * u;
        }
        if (own && row < jb.rows) jb.act_out[row] = o;
        if (jb.amax_out != nullptr) {  // the consumer's absmax (NaN never counts, as in stage_window)
            float ao = own && row < jb.rows ? __builtin_fabsf(o) : 0.0f;
            if (!(ao > 0.0f)) ao = 0.0f;
            ao = wave_max_f32(ao);
            if (lane == 0 && ao > 0.0f) atomicMax(jb.amax_out, __float_as_uint(ao));
        }
    };
    // Wave 0 after the barrier: the slice sums of an item from red[slot] and its outputs.
    auto epilogue = [&](const Item& it, uint32_t slot, int dsum, int dsum2) {
        const bool pair = MULTI && it.jb.w2 != nullptr;
        // sum t x = 16 hi + lo + 8 sum d - sum x (the lone GEMV's row_result): the corrections once per row, in slice 0
        const DJob& jb = it.jb;
        int v = 0;
#pragma unroll
        for (int w = 0; w < kNT / 64; ++w) v += red[slot][0][w][lane];
        const uint32_t row = it.tile * kTileRows + lane;
        // act_sum holds the codes of this slice's elements only: every slice subtracts its own
        if (it.ks == 0) v += 8 * dsum;
        v -= act_sum;
        if (!pair) {
            // the K slices of a row add up in one int32 (exact and order-independent, zero before the stage)
            if (jb.kslices > 1) atomicAdd(jb.part + row, v);
            else jb.part[row] = v;
            return;
        }
        int v2 = 0;
#pragma unroll
        for (int w = 0; w < kNT / 64; ++w) v2 += red[slot][MULTI ? 1 : 0][w][lane];
        v2 += 8 * dsum2 - act_sum;
        gate_out(jb, row, v, v2, true);
    };
    if constexpr (RANGE) {
        {
            accumulate_range(ba);
            __syncthreads();
            // Wave sg takes tile t_first + sg of the range: with the whole tile here its outputs directly; otherwise
            // each row's gate and up sums go into the row's accumulator word together with a count, and the
            // contribution that completes the count (the workgroups whose ranges meet the tile) takes the totals,
            // clears the word and writes the outputs.
            const uint32_t t_last = (re - 1u) / nc2;
            if (wave <= t_last - t_first) {
                const DJob& jb = ia.jb;
                const uint32_t sg = wave, t = t_first + sg, tb = t * nc2, te = tb + nc2;
                const int rd = dsa, rd2 = dsa2;  // the digit sums of tile t's rows
                int v = 0, v2 = 0;
#pragma unroll
                for (int w = 0; w < kNT / 64; ++w) {
                    v += red[sg][0][w][lane];
                    v2 += red[sg][1][w][lane];
                }
                bool own = true;
                if (rb > tb || re < te) {
                    // workgroups whose ranges meet chunks tb and te - 1: w(g) = floor(((g + 1) G - 1) / C)
                    const uint64_t C = a.range_chunks, G = gridDim.x;
                    const uint32_t wf = static_cast<uint32_t>(((tb + 1ull) * G - 1ull) / C);
                    const uint32_t wl = static_cast<uint32_t>((static_cast<uint64_t>(te) * G - 1ull) / C);
                    const unsigned long long mine = (1ull << 48) |
                                                    (static_cast<unsigned long long>(v2 + kRangeBias) << 24) |
                                                    static_cast<unsigned long long>(v + kRangeBias);
                    unsigned long long* acc = jb.accum + static_cast<size_t>(t) * 64u + lane;
                    const unsigned long long sum = atomicAdd(acc, mine) + mine;
                    // the row's last contribution takes the totals and clears the word for the next launch
                    const uint32_t c = static_cast<uint32_t>(sum >> 48);
                    own = c == wl - wf + 1u;
                    if (own) {
                        v = static_cast<int>(static_cast<uint32_t>(sum) & 0xffffffu) - static_cast<int>(c) * kRangeBias;
                        v2 = static_cast<int>(static_cast<uint32_t>(sum >> 24) & 0xffffffu) - static_cast<int>(c) * kRangeBias;
                        __hip_atomic_store(acc, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
                gate_out(jb, t * kTileRows + lane, v + 8 * rd - act_sum, v2 + 8 * rd2 - act_sum, own);
            }
        }
    } else {
        accumulate(ia, ba, 0u, true);
        if constexpr (MULTI) {
            if (has_b) accumulate(ib, bb, 1u, false);
        }
        __syncthreads();
        if (wave == 0) {
            epilogue(ia, 0u, dsa, dsa2);
            if constexpr (MULTI) {
                if (has_b) epilogue(ib, 1u, dsb, dsb2);
            }
        }
    }
    // zero the accumulators the stage clears (their consumers have run; a later stage adds to them again)
#pragma unroll
    for (int c = 0; c < kMaxClear; ++c) {
        int32_t* z = a.clear[c];
        if (z == nullptr) continue;
        for (uint32_t i = blockIdx.x * kNT + tid; i < a.clear_words[c]; i += gridDim.x * kNT) z[i] = 0;
    }
}

// ---- attention ------------------------------------------------------------------------------------------------------------

struct AttnArgs {
    const Ctl* ctl;
    ProjOut q, k, v;       // the q, k, v projections of this layer
    const float* rope;     // [max_ctx][head_dim]: (cos, sin) of pair i at 2i, 2i + 1
    uint16_t* kc;          // this layer: [kv_head][max_ctx][head_dim] f16
    uint16_t* vc;          // this layer: [kv_head][vstride / 8][head_dim][8] f16 (V in tiles of 8 positions)
    uint32_t vstride;      // positions per row of vc: max_ctx rounded up to 8
    float* out;            // n_heads x head_dim
    uint32_t n_heads, gqa, max_ctx;
    uint32_t rope_normal;  // 1: pairs (2i, 2i + 1) (RopeMode::Normal), 0: (i, i + head_dim / 2) (NEOX)
    float scale;
    // prefill: n_tok tokens at positions ctl->pos + 1 - n_tok .. ctl->pos, their rotated f16 queries in
    // qbuf[token][n_heads * head_dim] and their k, v already in the cache; out is [token][n_heads * head_dim]
    const uint16_t* qbuf;
    uint32_t n_tok;
    // decode in two kernels: the scores [n_heads][max_ctx], then per chunk its f16 accumulators cy [n_heads][4][HD]
    // (one per word), its (max, sum) pairs cms [n_heads][slices][4][2] and a ticket per (head, slice) (0 between steps)
    float* scores;
    uint32_t* cy;
    float* cms;
    uint32_t* ticket;
};

constexpr uint32_t kAttnMaxCtx = 8192;  // KV positions held in LDS (scores, running maxima)
constexpr uint32_t kVDepth = 8;         // groups of 8 positions of V in flight per lane in the accumulator chain
// Positions per row of the transposed V cache: max_ctx rounded up to 8 (one 16-byte load is 8 positions).
inline uint32_t vstride_of(uint32_t max_ctx) { return (max_ctx + 7u) / 8u * 8u; }
// The attention kernel's shape for a head dimension: coordinates per lane, waves (4 chunks of attn_waves / 4), threads.
__host__ __device__ constexpr uint32_t attn_cpl(uint32_t hd) { return hd >= 256u ? hd / 128u : 1u; }
__host__ __device__ constexpr uint32_t attn_waves(uint32_t hd) { return hd >= 128u ? 8u : 4u; }
__host__ __device__ constexpr uint32_t attn_threads(uint32_t hd) { return 64u * attn_waves(hd); }

// f16 value of an f32 (round to nearest even, after the f32 rounding of x), kept in an f32
__device__ __forceinline__ float r16(float x) { return static_cast<float>(static_cast<_Float16>(keep_f32(x))); }
// r16 of every value of a lane's coordinates; two at a time with one packed conversion (v_cvt_pk_f16_f32, each value
// rounded to nearest even after its own f32 rounding, as r16 does).
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
template <uint32_t N>
__device__ __forceinline__ void r16_all(float (&y)[N]) {
#pragma unroll
    for (uint32_t m = 0; m + 1 < N; m += 2) {
        half2_t h;
        h.x = static_cast<_Float16>(keep_f32(y[m]));
        h.y = static_cast<_Float16>(keep_f32(y[m + 1]));
        uint32_t u = __builtin_bit_cast(uint32_t, h);
        asm volatile("" : "+v"(u));  // the pair stays one packed conversion (not folded back into two)
        y[m] = f16_f32(static_cast<uint16_t>(u));
        y[m + 1] = f16_f32(static_cast<uint16_t>(u >> 16));
    }
    if constexpr (N % 2 == 1) y[N - 1] = r16(y[N - 1]);
}

// One workgroup per query head (and token, PREFILL). First the inputs of the position: q of this head and k, v of its KV
// head, RoPE over all head_dim coordinates (ops.rs:199-221, NEOX or Normal pairing: x0' = fma(x0, c, -(x1 s)),
// x1' = fma(x0, s, x1 c)) and the f16 rounding of the cache (kv_cache.rs:24-182); the first query head of each KV head
// appends k and v to the cache, and every workgroup uses its own copy of them for the position itself (the other
// positions come from earlier steps). PREFILL: the query comes rotated from qbuf and the position's k and v from the
// cache (pf_rope_kernel wrote them), nothing is appended.
// Then the reference's attend_head (attention.rs:483-542) over the positions 0..pos. Below a padded KV length of 512 one
// online softmax covers all positions; from 512 on, 4 chunks of ceil(n_kv / 4) positions run one each and are combined
// in order. The online softmax of a chunk (attend_range, attention.rs:436-468) is rebuilt without its serial
// dependences except the FP16 accumulator itself:
//   scores        every position in parallel (four lanes each): ggml_vec_dot_f16(q, k) * scale
//   running max   a scan per chunk; the reference's max moves only on score > max, the scan combines the same way
//   factors       every position in parallel: a new maximum gives ms = expf(m_old - score), vs = 1; otherwise ms = 1,
//                 vs = expf(score - max); stored as -ms or vs (the sign marks the case)
//   accumulator   per coordinate, in position order: y = f16(y * ms), y = f16(fma(v, vs, y)), s = fma(s, ms, vs)
// The accumulator chains: each chunk has attn_waves(HD) / 4 waves, a lane attn_cpl(HD) coordinates (independent
// chains). V is cached in tiles of 8 positions, [kv_head][position / 8][coordinate][position % 8]: one 16-byte load is
// eight consecutive positions of one coordinate, and a wave's load of 64 coordinates reads 1 KiB of contiguous memory;
// kVDepth such loads per coordinate are in flight ahead of the chain.
template <int HD, bool PREFILL>
__global__ __launch_bounds__(attn_threads(HD)) void attention_kernel(AttnArgs a) {
    constexpr uint32_t kCpl = attn_cpl(HD);           // coordinates (chains) per lane
    constexpr uint32_t kWpc = attn_waves(HD) / 4u;    // waves per chunk
    constexpr uint32_t kLanes = HD / (kWpc * kCpl);   // lanes of a wave with coordinates (64, or 32 at head_dim 32)
    constexpr uint32_t kThreads = attn_threads(HD);
    constexpr uint32_t kHalf = HD / 2;        // RoPE pairs
    constexpr int kBlk = HD / 32;             // 32-value blocks of a row
    __shared__ __align__(16) float sc[kAttnMaxCtx];
    __shared__ float pm[kAttnMaxCtx];
    __shared__ __align__(16) uint16_t qs[HD];
    __shared__ __align__(16) uint16_t kp[HD];  // k and v of the position itself
    __shared__ __align__(16) uint16_t vp[HD];
    __shared__ float cm[4], cs[4];
    __shared__ uint16_t cv[4][HD];
    const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t kvh = h / a.gqa;
    const uint32_t tok = PREFILL ? blockIdx.y : 0u;
    const uint32_t pos = PREFILL ? a.ctl->pos + 1u - a.n_tok + tok : a.ctl->pos;
    const uint32_t seq = pos + 1;
    const uint16_t* kb = a.kc + static_cast<size_t>(kvh) * a.max_ctx * HD;
    uint16_t* vt = a.vc + static_cast<size_t>(kvh) * HD * a.vstride;  // this KV head's tiles: [vstride / 8][HD][8]
    auto vt_at = [&](uint32_t p, uint32_t dd) -> size_t {
        return (static_cast<size_t>(p >> 3) * HD + dd) * 8u + (p & 7u);
    };

    uint32_t n_kv = (seq + 255u) / 256u * 256u;
    if (n_kv > a.max_ctx) n_kv = a.max_ctx;
    const bool split = n_kv >= 512u;
    const uint32_t chunk = split ? (n_kv + 3u) / 4u : seq;
    const uint32_t n_chunks = split ? 4u : 1u;
    // This wave's chunk; the lane's coordinates are d0 + 64 m (m < kCpl) when it has any.
    const uint32_t c = wave / kWpc;
    const uint32_t d0 = (wave % kWpc) * 64u * kCpl + lane;
    const bool has_d = lane < kLanes;
    uint32_t st = 0, en = 0;
    if (c < n_chunks) {
        st = c * chunk;
        en = min(min(st + chunk, n_kv), seq);
    }

    if (PREFILL) {
        if (tid < HD) {
            qs[tid] = a.qbuf[(static_cast<size_t>(tok) * a.n_heads + h) * HD + tid];
            kp[tid] = kb[static_cast<size_t>(pos) * HD + tid];
            vp[tid] = vt[vt_at(pos, tid)];
        }
    } else {
        const float* cache = a.rope + static_cast<size_t>(pos) * HD;
        if (tid < HD) {  // q (tid < HD / 2) or k: the rotation of pair i
            const bool isq = tid < kHalf;
            const uint32_t i = tid & (kHalf - 1u);
            const uint32_t i0 = a.rope_normal ? 2u * i : i, i1 = a.rope_normal ? 2u * i + 1u : i + kHalf;
            const ProjOut& o = isq ? a.q : a.k;
            const uint32_t base = (isq ? h : kvh) * HD;
            bool zero;
            const float post = proj_post(o, &zero);
            const float x0 = proj_at(o, base + i0, post, zero), x1 = proj_at(o, base + i1, post, zero);
            const float cc = cache[2 * i], ss = cache[2 * i + 1];
            const float x1s = x1 * ss, x1c = x1 * cc;
            const float y0 = __builtin_fmaf(x0, cc, -x1s);
            const float y1 = __builtin_fmaf(x0, ss, x1c);
            uint16_t* dst = isq ? qs : kp;
            dst[i0] = f32_f16(y0);
            dst[i1] = f32_f16(y1);
        } else if (tid < 2u * HD) {
            const uint32_t dd = tid - HD;
            bool zero;
            const float post = proj_post(a.v, &zero);
            vp[dd] = f32_f16(proj_at(a.v, kvh * HD + dd, post, zero));
        }
    }
    __syncthreads();
    if (!PREFILL && h % a.gqa == 0 && tid < HD) {
        a.kc[(static_cast<size_t>(kvh) * a.max_ctx + pos) * HD + tid] = kp[tid];
        vt[vt_at(pos, tid)] = vp[tid];
    }

    // The chain's V: group g holds positions 8 g .. 8 g + 7 (every tile read is below vstride: groups run to the chunk's
    // end rounded up to 8). Its first kVDepth groups are requested once the scores are done, so that they arrive during
    // the scan and the exponentials without adding to the scores' registers. The value of the position itself, not yet
    // visible in the cache to every workgroup, is patched from vp when its group is used.
    const bool chain = c < n_chunks && st < en;
    const uint32_t g_first = st / 8u, g_end = chain ? (en + 7u) / 8u : g_first + 1u;
    const uint32_t dl = has_d ? d0 : 0u;  // a lane without coordinates reads coordinate 0 and never uses it
    u32x4 ring[kVDepth][kCpl];
    auto load_group = [&](uint32_t g, u32x4 (&r)[kCpl]) {
        const uint32_t gg = min(g, g_end - 1u);
#pragma unroll
        for (uint32_t m = 0; m < kCpl; ++m)
            r[m] = *reinterpret_cast<const u32x4*>(vt + (static_cast<size_t>(gg) * HD + dl + 64u * m) * 8u);
    };

    // Scores, four lanes per position (ggml_vec_dot_f16, ops.rs:960-1015): lane j of a group holds accumulator j
    // (values 32 i + 8 j .. + 7 of every 32-value block i) with q in registers as f32; (a0 + a2) + (a1 + a3) across the
    // group, then red[k] + red[k + 4] and (t0 + t1) + (t2 + t3) in lane 0. The next position's k is loaded while the
    // current one is summed.
    {
        const uint32_t j = tid & 3u, g = tid >> 2;
        constexpr uint32_t kGroups = kThreads / 4u;
        // q is read from LDS at each use (the 4-lane groups of a wave all read the same addresses: broadcasts), two
        // f16 per register; each product widens both operands exactly, as f16_f32 does. Held in registers as f32 for
        // the whole loop, it took 4 kBlk of them, which left room for one workgroup per CU instead of two.
        auto load_k = [&](uint32_t p, uint4 (&kr)[kBlk]) {
            if (p == pos) {
#pragma unroll
                for (int i = 0; i < kBlk; ++i) kr[i] = *reinterpret_cast<const uint4*>(kp + 32 * i + 8 * j);
            } else {
                const uint16_t* row = kb + static_cast<size_t>(p) * HD + 8 * j;
#pragma unroll
                for (int i = 0; i < kBlk; ++i) kr[i] = *reinterpret_cast<const uint4*>(row + 32 * i);
            }
        };
        auto score = [&](uint32_t p, const uint4 (&kr)[kBlk]) {
            uint32_t qo = 8u * j;
            asm volatile("" : "+v"(qo));  // keeps q's reads in the loop (the compiler would hoist them into registers)
            float acc[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
#pragma unroll
            for (int i = 0; i < kBlk; ++i) {
                const uint32_t kw[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
                const uint4 qv = *reinterpret_cast<const uint4*>(qs + 32 * i + qo);
                const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
                for (int l = 0; l < 8; ++l)
                    acc[l] = __builtin_fmaf(f16_f32(static_cast<uint16_t>(qw[l >> 1] >> ((l & 1) * 16))),
                                            f16_f32(static_cast<uint16_t>(kw[l >> 1] >> ((l & 1) * 16))), acc[l]);
            }
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                acc[l] = acc[l] + bits_f32(dpp32<kDppXor2>(f32_bits(acc[l])));  // lane j ^ 2 of the quad (DPP)
                acc[l] = acc[l] + bits_f32(dpp32<kDppXor1>(f32_bits(acc[l])));  // lane j ^ 1
            }
            if (j == 0) {
                const float t0 = acc[0] + acc[4], t1 = acc[1] + acc[5], t2 = acc[2] + acc[6], t3 = acc[3] + acc[7];
                sc[p] = ((t0 + t1) + (t2 + t3)) * a.scale;
            }
        };
        uint4 ka[kBlk], kn[kBlk];
        uint32_t p = g;
        if (p < seq) load_k(p, ka);
        for (; p < seq; p += 2u * kGroups) {  // unrolled by two so that the buffers keep their registers
            if (p + kGroups < seq) load_k(p + kGroups, kn);
            score(p, ka);
            if (p + kGroups >= seq) break;
            if (p + 2u * kGroups < seq) load_k(p + 2u * kGroups, ka);
            score(p + kGroups, kn);
        }
    }
#pragma unroll
    for (uint32_t k = 0; k < kVDepth; ++k) load_group(g_first + k, ring[k]);
    uint16_t vself[kCpl];
#pragma unroll
    for (uint32_t m = 0; m < kCpl; ++m) vself[m] = vp[dl + 64u * m];
    __syncthreads();

    if (wave < n_chunks) {  // the running maximum of chunk `wave`
        const uint32_t s0 = wave * chunk, s1 = min(min(s0 + chunk, n_kv), seq);
        float carry = -__builtin_inff();
        for (uint32_t base = s0; base < s1; base += 64u) {
            const uint32_t p = base + lane;
            float v = p < s1 ? sc[p] : -__builtin_inff();
#pragma unroll
            for (int sh = 1; sh < 64; sh <<= 1) {
                const float o = __shfl_up(v, sh);
                if (lane >= static_cast<uint32_t>(sh)) v = v > o ? v : o;
            }
            v = v > carry ? v : carry;
            if (p < s1) pm[p] = v;
            carry = __shfl(v, 63);
        }
    }
    __syncthreads();

    for (uint32_t p = tid; p < seq; p += kThreads) {
        const uint32_t s0 = split ? p / chunk * chunk : 0u;
        const float prev = p == s0 ? -__builtin_inff() : pm[p - 1];
        const float s = sc[p];
        sc[p] = s > prev ? -glibc_expf(prev - s) : glibc_expf(s - prev);
    }
    __syncthreads();

    // The accumulator chains of this lane's coordinates over positions st .. en - 1, eight positions per group; a group
    // with no new maximum (ms = 1 throughout) takes the shorter step.
    float y[kCpl], ssum = 0.0f;
#pragma unroll
    for (uint32_t m = 0; m < kCpl; ++m) y[m] = 0.0f;
    if (chain) {
        // the factors of the next group are read from LDS while the current group is summed, into the other of two
        // slots (slot k & 1 of group slot k: kVDepth is even, so the pattern repeats on every pass of the loop)
        static_assert(kVDepth % 2 == 0, "two factor slots alternate over the ring");
        float4 fq[2][2];
        fq[0][0] = *reinterpret_cast<const float4*>(sc + 8u * g_first);
        fq[0][1] = *reinterpret_cast<const float4*>(sc + 8u * g_first + 4u);
        for (uint32_t g0 = g_first; g0 < g_end; g0 += kVDepth) {
            static_for<kVDepth>([&](auto kc) {  // the ring's slot as a constant: no rotation of its registers
                constexpr uint32_t k = decltype(kc)::value;
                const uint32_t gg = g0 + k;
                {
                    const uint32_t pn = 8u * min(gg + 1u, g_end - 1u);
                    fq[(k + 1u) & 1u][0] = *reinterpret_cast<const float4*>(sc + pn);
                    fq[(k + 1u) & 1u][1] = *reinterpret_cast<const float4*>(sc + pn + 4u);
                }
                if (gg < g_end) {  // wave-uniform
                    // the group's V words, used in place; the slot is refilled (kVDepth groups ahead) once they are
                    // consumed, so that the refill lands in the same registers (no register rotation)
                    u32x4(&w)[kCpl] = ring[k];
                    const uint32_t p0 = 8u * gg;
                    const float4 fa = fq[k & 1u][0], fb = fq[k & 1u][1];
                    if (pos >= p0 && pos < p0 + 8u) {  // the position itself, from this workgroup's copy
                        const uint32_t e = pos - p0, sh = (e & 1u) * 16u, keep = ~(0xffffu << sh);
#pragma unroll
                        for (uint32_t m = 0; m < kCpl; ++m) {
                            const uint32_t ins = static_cast<uint32_t>(vself[m]) << sh;
                            const uint32_t q = e >> 1;
                            w[m].x = q == 0 ? ((w[m].x & keep) | ins) : w[m].x;
                            w[m].y = q == 1 ? ((w[m].y & keep) | ins) : w[m].y;
                            w[m].z = q == 2 ? ((w[m].z & keep) | ins) : w[m].z;
                            w[m].w = q == 3 ? ((w[m].w & keep) | ins) : w[m].w;
                        }
                    }
                    float f[8] = {fa.x, fa.y, fa.z, fa.w, fb.x, fb.y, fb.z, fb.w};
                    // A group that starts inside the chunk is summed whole: at its positions from en on (the chunk's
                    // last group) the factor becomes +0 (vs = 0, no new maximum) and V -0, so that a step there adds
                    // -0 and leaves y and the sum as they are.
                    const bool whole = p0 >= st;
                    if (whole && p0 + 8u > en) {
                        const uint32_t n = en - p0;
#pragma unroll
                        for (int e = 0; e < 8; ++e) f[e] = static_cast<uint32_t>(e) < n ? f[e] : 0.0f;
#pragma unroll
                        for (uint32_t m = 0; m < kCpl; ++m) {
                            uint32_t ww[4] = {w[m].x, w[m].y, w[m].z, w[m].w};
#pragma unroll
                            for (uint32_t q = 0; q < 4; ++q) {
                                const uint32_t keep = (2u * q < n ? 0xffffu : 0u) | (2u * q + 1u < n ? 0xffff0000u : 0u);
                                ww[q] = (ww[q] & keep) | (0x80008000u & ~keep);
                            }
                            w[m] = u32x4{ww[0], ww[1], ww[2], ww[3]};
                        }
                    }
                    uint32_t neg = 0;
#pragma unroll
                    for (int e = 0; e < 8; ++e) neg |= f32_bits(f[e]) >> 31;
                    neg = __builtin_amdgcn_readfirstlane(neg);
                    if (whole && neg == 0) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
#pragma unroll
                            for (uint32_t m = 0; m < kCpl; ++m) {
                                const uint32_t wv[4] = {w[m].x, w[m].y, w[m].z, w[m].w};
                                const float v = f16_f32(static_cast<uint16_t>(wv[e >> 1] >> ((e & 1) * 16)));
                                y[m] = __builtin_fmaf(v, f[e], y[m]);
                            }
                            r16_all(y);
                            ssum = ssum + f[e];
                        }
                    } else if (whole) {
                        // a group with a new maximum: the full step at every position (ms = 1 where there is none,
                        // which leaves y as it is), straight-line
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const bool nm = __builtin_signbit(f[e]);
                            const float ev = __builtin_fabsf(f[e]);
                            const float ms = nm ? ev : 1.0f, vs = nm ? 1.0f : ev;
#pragma unroll
                            for (uint32_t m = 0; m < kCpl; ++m) y[m] = y[m] * ms;
                            r16_all(y);
#pragma unroll
                            for (uint32_t m = 0; m < kCpl; ++m) {
                                const uint32_t wv[4] = {w[m].x, w[m].y, w[m].z, w[m].w};
                                const float v = f16_f32(static_cast<uint16_t>(wv[e >> 1] >> ((e & 1) * 16)));
                                y[m] = __builtin_fmaf(v, vs, y[m]);
                            }
                            r16_all(y);
                            ssum = __builtin_fmaf(ssum, ms, vs);
                        }
                    } else {  // the chunk starts inside this group (positions before it skipped)
                        const uint32_t e0 = p0 < st ? st - p0 : 0u, e1 = min(8u, en - p0);
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            if (static_cast<uint32_t>(e) >= e0 && static_cast<uint32_t>(e) < e1) {
                                const bool nm = __builtin_signbit(f[e]);
                                const float ev = __builtin_fabsf(f[e]);
                                const float ms = nm ? ev : 1.0f, vs = nm ? 1.0f : ev;
#pragma unroll
                                for (uint32_t m = 0; m < kCpl; ++m) y[m] = y[m] * ms;
                                r16_all(y);
#pragma unroll
                                for (uint32_t m = 0; m < kCpl; ++m) {
                                    const uint32_t wv[4] = {w[m].x, w[m].y, w[m].z, w[m].w};
                                    const float v = f16_f32(static_cast<uint16_t>(wv[e >> 1] >> ((e & 1) * 16)));
                                    y[m] = __builtin_fmaf(v, vs, y[m]);
                                }
                                r16_all(y);
                                ssum = __builtin_fmaf(ssum, ms, vs);
                            }
                        }
                    }
                }
                // every slot is refilled, used or not (the index stays inside the cache), so that the number of
                // loads issued after a slot's refill, and with it the wait for the slot, is the same on every path
                load_group(gg + kVDepth, ring[k]);
            });
        }
    }
    float* out = a.out + (static_cast<size_t>(tok) * a.n_heads + h) * HD;
    if (!split) {
        if (c == 0 && has_d) {
            const float s_inv = ssum == 0.0f ? 0.0f : 1.0f / ssum;
#pragma unroll
            for (uint32_t m = 0; m < kCpl; ++m) out[d0 + 64u * m] = y[m] * s_inv;
        }
        return;
    }
    if (c < 4) {
        if (has_d) {
#pragma unroll
            for (uint32_t m = 0; m < kCpl; ++m) cv[c][d0 + 64u * m] = f32_f16(y[m]);
        }
        if (wave % kWpc == 0 && lane == 0) {
            cm[c] = st < en ? pm[en - 1] : -__builtin_inff();
            cs[c] = ssum;
        }
    }
    __syncthreads();
    if (c != 0 || !has_d) return;
#pragma unroll
    for (uint32_t m = 0; m < kCpl; ++m) {
        const uint32_t d = d0 + 64u * m;
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
}

// ---- decode attention: scores, then the accumulator chains ---------------------------------------------------------------
//
// The decode step spreads attention over many workgroups: attn_score_kernel computes every score of a position range
// (and the RoPE and KV append of the position itself), attn_chain_kernel runs one chunk's online softmax for 64
// coordinates of one query head, and the last chunk of a (head, coordinates) pair to finish combines the chunks.

constexpr uint32_t kScoreTile = 64;   // positions per score workgroup: one per 4-lane group of 256 threads
constexpr uint32_t kScoreHeads = 8;   // query heads (of one KV head) per score workgroup at most
constexpr uint32_t kChainBlocks = 4;  // blocks of 32 positions of V in flight in a chain (four 8-position tiles each)
constexpr uint32_t kChunkMax = kAttnMaxCtx / 4u;  // the longest chunk (n_kv / 4 at the largest context)
constexpr uint32_t kShortCtx = 256;   // positions below which one chunk covers the context (n_kv < 512)
__host__ __device__ constexpr uint32_t attn_slices(uint32_t hd) { return hd >= 64u ? hd / 64u : 1u; }

// RoPE of pair i of the row at `base` of a projection (ops.rs:199-221, NEOX or Normal pairing): x0' = fma(x0, c, -(x1 s)),
// x1' = fma(x0, s, x1 c), stored as f16 (kv_cache.rs:24-182).
template <int HD>
__device__ __forceinline__ void rope_pair(const ProjOut& o, uint32_t base, uint32_t i, bool normal, const float* cache,
                                          uint16_t* dst) {
    const uint32_t i0 = normal ? 2u * i : i, i1 = normal ? 2u * i + 1u : i + HD / 2u;
    bool zero;
    const float post = proj_post(o, &zero);
    const float x0 = proj_at(o, base + i0, post, zero), x1 = proj_at(o, base + i1, post, zero);
    const float cc = cache[2 * i], ss = cache[2 * i + 1];
    const float x1s = x1 * ss, x1c = x1 * cc;
    dst[i0] = f32_f16(__builtin_fmaf(x0, cc, -x1s));
    dst[i1] = f32_f16(__builtin_fmaf(x0, ss, x1c));
}

// q . k of one position in ggml_vec_dot_f16's order (ops.rs:960-1015), four lanes per position: lane j holds accumulator
// j (values 32 i + 8 j .. + 7 of every 32-value block i, q from LDS and k from kr, both f16), then (a0 + a2) + (a1 + a3)
// across the group and red[k] + red[k + 4], (t0 + t1) + (t2 + t3); the result is lane 0's (the four lanes of a group
// must run together).
template <int HD>
__device__ __forceinline__ float score_dot4(const uint16_t* q, const uint4 (&kr)[HD / 32], uint32_t j) {
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) {
        const uint4 qv = *reinterpret_cast<const uint4*>(q + 32 * i + 8 * j);
        const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
        const uint32_t kw[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
        for (int l = 0; l < 8; ++l)
            acc[l] = __builtin_fmaf(f16_f32(static_cast<uint16_t>(qw[l >> 1] >> ((l & 1) * 16))),
                                    f16_f32(static_cast<uint16_t>(kw[l >> 1] >> ((l & 1) * 16))), acc[l]);
    }
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        acc[l] = acc[l] + bits_f32(dpp32<kDppXor2>(f32_bits(acc[l])));  // lane j ^ 2 of the quad (DPP)
        acc[l] = acc[l] + bits_f32(dpp32<kDppXor1>(f32_bits(acc[l])));  // lane j ^ 1
    }
    const float t0 = acc[0] + acc[4], t1 = acc[1] + acc[5], t2 = acc[2] + acc[6], t3 = acc[3] + acc[7];
    return (t0 + t1) + (t2 + t3);
}

// Scores of positions p0 .. p0 + 63 (p0 = blockIdx.y * 64, below pos + 1) for up to kScoreHeads query heads of one KV
// head (blockIdx.x: KV head, head group), so that each K row is read once for the heads that share it. The workgroup
// whose range holds the position itself rotates its k (the first head group also appends k and v to the cache); every
// workgroup rotates its heads' q. Four lanes per position as ggml_vec_dot_f16 (ops.rs:960-1015): lane j holds
// accumulator j (values 32 i + 8 j .. + 7 of every 32-value block i), then (a0 + a2) + (a1 + a3) across the group,
// red[k] + red[k + 4] and (t0 + t1) + (t2 + t3) in lane 0, times the scale.
template <int HD>
__global__ __launch_bounds__(256) void attn_score_kernel(AttnArgs a) {
    constexpr int kBlk = HD / 32;
    __shared__ __align__(16) uint16_t qh[kScoreHeads][HD];
    __shared__ __align__(16) uint16_t kp[HD];
    __shared__ __align__(16) uint16_t vp[HD];
    const uint32_t tid = threadIdx.x;
    const uint32_t hgroups = (a.gqa + kScoreHeads - 1u) / kScoreHeads;
    const uint32_t kvh = blockIdx.x / hgroups, hg = blockIdx.x - kvh * hgroups;
    const uint32_t h0 = kvh * a.gqa + hg * kScoreHeads;
    const uint32_t nh = min(kScoreHeads, a.gqa - hg * kScoreHeads);
    const uint32_t pos = a.ctl->pos, seq = pos + 1u;
    const uint32_t p0 = blockIdx.y * kScoreTile;
    if (p0 >= seq) return;
    const bool own = pos - p0 < kScoreTile;
    const bool normal = a.rope_normal != 0u;
    const float* cache = a.rope + static_cast<size_t>(pos) * HD;
    // this thread's K row goes out first (its latency overlaps the rotations' loads); the position itself comes later
    const uint32_t j = tid & 3u, p = p0 + (tid >> 2);
    uint4 kr[kBlk];
    if (p < seq && p != pos) {
        const uint16_t* row = a.kc + (static_cast<size_t>(kvh) * a.max_ctx + p) * HD + 8 * j;
#pragma unroll
        for (int i = 0; i < kBlk; ++i) kr[i] = *reinterpret_cast<const uint4*>(row + 32 * i);
    }
    for (uint32_t t = tid; t < nh * (HD / 2u); t += 256u) {
        const uint32_t hh = t / (HD / 2u), i = t - hh * (HD / 2u);
        rope_pair<HD>(a.q, (h0 + hh) * HD, i, normal, cache, qh[hh]);
    }
    if (own) {
        for (uint32_t t = tid; t < HD / 2u + HD; t += 256u) {
            if (t < HD / 2u) {
                rope_pair<HD>(a.k, kvh * HD, t, normal, cache, kp);
            } else {
                bool zero;
                const float post = proj_post(a.v, &zero);
                vp[t - HD / 2u] = f32_f16(proj_at(a.v, kvh * HD + (t - HD / 2u), post, zero));
            }
        }
    }
    __syncthreads();
    if (own && hg == 0) {
        uint16_t* vt = a.vc + static_cast<size_t>(kvh) * HD * a.vstride;
        for (uint32_t t = tid; t < HD; t += 256u) {
            a.kc[(static_cast<size_t>(kvh) * a.max_ctx + pos) * HD + t] = kp[t];
            vt[(static_cast<size_t>(pos >> 3) * HD + t) * 8u + (pos & 7u)] = vp[t];
        }
    }
    if (p >= seq) return;  // all four lanes of a position leave together; no barrier follows
    if (p == pos) {
#pragma unroll
        for (int i = 0; i < kBlk; ++i) kr[i] = *reinterpret_cast<const uint4*>(kp + 32 * i + 8 * j);
    }
    for (uint32_t hh = 0; hh < nh; ++hh) {
        const float sv = score_dot4<HD>(qh[hh], kr, j);
        if (j == 0) a.scores[static_cast<size_t>(h0 + hh) * a.max_ctx + p] = sv * a.scale;
    }
}

// The running maximum's combine (attend_range, attention.rs:436-468: the maximum moves only on score > max): `later`
// replaces `earlier` only when larger. A NaN score never moves the maximum, so it enters a scan as -inf.
__device__ __forceinline__ float max_later(float earlier, float later) { return later > earlier ? later : earlier; }

// The pieces of one chunk's online softmax (attend_range, attention.rs:436-468) over positions st .. en - 1, in blocks
// of 32 positions b_first .. b_end - 1 (fac[i] is the factor of position 32 b_first + i; bit e of bflag[i] marks position
// 32 (b_first + i) + e when it holds a new maximum).
//
// chunk_factors (all NT threads; one barrier inside, one expected after): the running maximum by a scan (runs of
// R = ceil(len / NT) positions per thread, an inclusive scan of the run maxima over the lanes and a prefix over the
// waves), then per position ms = expf(m_old - score), vs = 1 at a new maximum and ms = 1, vs = expf(score - max)
// otherwise, stored as -ms or vs (the sign marks the case). Returns the chunk's maximum (-inf when empty).
template <int NT>
__device__ __forceinline__ float chunk_factors(const float* scores, uint32_t st, uint32_t en, uint32_t b_first, float* fac,
                                               uint32_t* bflag, float* wtot, const uint64_t* etab) {
    constexpr uint32_t kW = NT / 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t len = en - st, R = (len + NT - 1u) / NT;  // R <= 8
    const uint32_t nb = (en + 31u) / 32u - b_first;
    for (uint32_t i = tid; i < nb; i += NT) bflag[i] = 0u;
    float sv[8];
    float loc = -__builtin_inff();
#pragma unroll
    for (uint32_t r = 0; r < 8; ++r) {
        const uint32_t i = tid * R + r;
        sv[r] = r < R && i < len ? scores[i] : 0.0f;
        if (r < R && i < len) loc = max_later(loc, sv[r] != sv[r] ? -__builtin_inff() : sv[r]);
    }
    float v = loc;  // inclusive scan over the lanes, earlier lanes first
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
        const float o = __shfl_up(v, sh);
        if (lane >= static_cast<uint32_t>(sh)) v = max_later(o, v);
    }
    if (lane == 63) wtot[wave] = v;
    __syncthreads();
    float before = -__builtin_inff(), cmax = -__builtin_inff();
    for (uint32_t w = 0; w < wave; ++w) before = max_later(before, wtot[w]);
    for (uint32_t w = 0; w < kW; ++w) cmax = max_later(cmax, wtot[w]);
    float prev = __shfl_up(v, 1);
    prev = max_later(before, lane == 0 ? -__builtin_inff() : prev);
    const uint32_t off = st - 32u * b_first;
    const auto tab = [&](uint32_t k) { return etab[k]; };
#pragma unroll
    for (uint32_t r = 0; r < 8; ++r) {
        const uint32_t i = tid * R + r;
        if (r < R && i < len) {
            const float sc = sv[r];
            const float f = sc > prev ? -glibc_expf_with(prev - sc, tab) : glibc_expf_with(sc - prev, tab);
            fac[off + i] = f;
            if (__builtin_signbit(f)) atomicOr(bflag + ((off + i) >> 5), 1u << ((off + i) & 31u));
            prev = max_later(prev, sc != sc ? -__builtin_inff() : sc);
        }
    }
    return cmax;
}

// The V tiles of 8 positions (16 bytes per coordinate) of a KV head for coordinate d, up to tile t_last (the last one
// with a position of the chunk: every read stays inside the cache), as a buffer: the lane's offset is fixed, a tile's
// is a scalar, so a tile costs one load and no address arithmetic.
struct VTiles {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t voff;  // the lane's coordinate: d * 16 bytes
};
template <int HD>
__device__ __forceinline__ VTiles vtiles(const uint16_t* vt, uint32_t d, uint32_t t_last) {
    VTiles v;
    v.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vt), 0, (t_last + 1u) * HD * 16u, kBufferRsrcWord3);
    v.voff = d * 16u;
    return v;
}
// The tiles of block b (4 b .. 4 b + 3, clamped at t_last).
template <int HD>
__device__ __forceinline__ void load_vblock(const VTiles& v, uint32_t b, uint32_t t_last, u32x4 (&r)[4]) {
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t t = min(4u * b + i, t_last);
        r[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(v.rsrc, v.voff, t * HD * 16u, 0));
    }
}

__device__ __forceinline__ float vhalf(const u32x4 (&w)[4], int e) {
    const u32x4 ww = w[e >> 3];
    const uint32_t word = (e & 7) < 2 ? ww.x : (e & 7) < 4 ? ww.y : (e & 7) < 6 ? ww.z : ww.w;
    return f16_f32(static_cast<uint16_t>(word >> ((e & 1) * 16)));
}

// The FP16 accumulator of one coordinate (one wave, a coordinate per lane): y = f16(y * ms), y = f16(fma(v, vs, y)) per
// position, a block per step with the V tiles kChainBlocks blocks ahead in `ring` (already requested for b_first ..). A
// block that starts inside the chunk is summed whole: its positions from en on are padding, V set to -0 here and the
// factors +0 (the caller writes them), so that a step there adds -0 and leaves y as it is. A block without a new
// maximum takes y = f16(fma(v, vs, y)) alone; one with new maxima takes the full step at every position (ms = 1 where
// there is none, which leaves y as it is), straight-line: a branch per position costs more than the longer step. A
// block that starts before the chunk (a chunk start that is not a multiple of 32) masks its leading positions.
template <int HD>
__device__ __forceinline__ float chain_y(u32x4 (&ring)[kChainBlocks][4], const VTiles& vtl, uint32_t st, uint32_t en,
                                         uint32_t b_first, uint32_t b_end, uint32_t t_last, const float* fac,
                                         const uint32_t* bflag) {
    float y = 0.0f;
    // The factors and mask of a block, read from LDS one block ahead into the other of two slots (slot k & 1 for ring
    // slot k: kChainBlocks is even, so the pattern repeats on every pass), every read unconditional: no copies.
    static_assert(kChainBlocks % 2 == 0, "two factor slots alternate over the ring");
    float4 fq[2][8];
    uint32_t fl[2];
    auto load_fac = [&](uint32_t b, float4 (&q)[8], uint32_t& m) {
        const float* fb = fac + 32u * (b - b_first);
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = *reinterpret_cast<const float4*>(fb + 4 * i);
        m = bflag[b - b_first];
    };
    load_fac(b_first, fq[0], fl[0]);
    for (uint32_t b0 = b_first; b0 < b_end; b0 += kChainBlocks) {
        static_for<kChainBlocks>([&](auto kc) {  // the ring's slot as a constant: no rotation of its registers
            constexpr uint32_t k = decltype(kc)::value;
            const uint32_t b = b0 + k;
            load_fac(min(b + 1u, b_end - 1u), fq[(k + 1u) & 1u], fl[(k + 1u) & 1u]);
            if (b < b_end) {  // wave-uniform
                // the block's V tiles, used in place; the slot is refilled (kChainBlocks blocks ahead) once they are
                // consumed, so that the refill lands in the same registers
                u32x4(&w)[4] = ring[k];
                float f[32];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    f[4 * i] = fq[k & 1u][i].x;
                    f[4 * i + 1] = fq[k & 1u][i].y;
                    f[4 * i + 2] = fq[k & 1u][i].z;
                    f[4 * i + 3] = fq[k & 1u][i].w;
                }
                const uint32_t flag = __builtin_amdgcn_readfirstlane(fl[k & 1u]);
                const uint32_t p0 = 32u * b;
                if (p0 >= st) {
                    if (p0 + 32u > en) {  // the chunk's last block: V of the positions from en on set to -0
                        const uint32_t n = en - p0;
#pragma unroll
                        for (uint32_t i = 0; i < 4; ++i) {
                            uint32_t ww[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
                            for (uint32_t q = 0; q < 4; ++q) {
                                const uint32_t e = 8u * i + 2u * q;
                                const uint32_t keep = (e < n ? 0xffffu : 0u) | (e + 1u < n ? 0xffff0000u : 0u);
                                ww[q] = (ww[q] & keep) | (0x80008000u & ~keep);
                            }
                            w[i] = u32x4{ww[0], ww[1], ww[2], ww[3]};
                        }
                    }
                    if (flag == 0u) {
#pragma unroll
                        for (int e = 0; e < 32; ++e) y = r16(__builtin_fmaf(vhalf(w, e), f[e], y));
                    } else {
#pragma unroll
                        for (int e = 0; e < 32; ++e) {
                            const bool nm = __builtin_signbit(f[e]);
                            const float ev = __builtin_fabsf(f[e]);
                            const float t = r16(y * (nm ? ev : 1.0f));
                            y = r16(__builtin_fmaf(vhalf(w, e), nm ? 1.0f : ev, t));
                        }
                    }
                } else {  // the chunk starts inside this block: positions outside [st, en) keep y
                    const uint32_t e0 = st - p0, e1 = min(32u, en - p0);
#pragma unroll
                    for (int e = 0; e < 32; ++e) {
                        const bool in = static_cast<uint32_t>(e) >= e0 && static_cast<uint32_t>(e) < e1;
                        const bool nm = __builtin_signbit(f[e]);
                        const float ev = __builtin_fabsf(f[e]);
                        const float ms = nm ? ev : 1.0f, vs = nm ? 1.0f : ev;
                        float t = r16(y * ms);
                        t = r16(__builtin_fmaf(vhalf(w, e), vs, t));
                        y = in ? t : y;
                    }
                }
            }
            // every slot is refilled, used or not (the tile index stays inside the cache), so that the number of loads
            // issued after a slot's refill, and with it the wait for the slot, is the same on every path
            load_vblock<HD>(vtl, b + kChainBlocks, t_last, ring[k]);
        });
    }
    return y;
}

// The chunk's sum s = fma(s, ms, vs) over its positions in order (one wave, the same value in every lane); the padding
// after en has factors +0, which leave s as it is (s >= +0).
__device__ __forceinline__ float chain_sum(uint32_t st, uint32_t en, uint32_t b_first, uint32_t b_end, const float* fac,
                                           const uint32_t* bflag) {
    float ssum = 0.0f;
    for (uint32_t b = b_first; b < b_end; ++b) {
        const float* fb = fac + 32u * (b - b_first);
        float f[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 q = *reinterpret_cast<const float4*>(fb + 4 * i);
            f[4 * i] = q.x;
            f[4 * i + 1] = q.y;
            f[4 * i + 2] = q.z;
            f[4 * i + 3] = q.w;
        }
        const uint32_t flag = __builtin_amdgcn_readfirstlane(bflag[b - b_first]);
        const uint32_t p0 = 32u * b;
        if (p0 >= st && flag == 0u) {
#pragma unroll
            for (int e = 0; e < 32; ++e) ssum = ssum + f[e];
        } else if (p0 >= st) {
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                const bool nm = __builtin_signbit(f[e]);
                const float ev = __builtin_fabsf(f[e]);
                ssum = __builtin_fmaf(ssum, nm ? ev : 1.0f, nm ? 1.0f : ev);
            }
        } else {
            const uint32_t e0 = st - p0, e1 = min(32u, en - p0);
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                const bool in = static_cast<uint32_t>(e) >= e0 && static_cast<uint32_t>(e) < e1;
                const bool nm = __builtin_signbit(f[e]);
                const float ev = __builtin_fabsf(f[e]);
                const float t = __builtin_fmaf(ssum, nm ? ev : 1.0f, nm ? 1.0f : ev);
                ssum = in ? t : ssum;
            }
        }
    }
    return ssum;
}

// The exponential's table in LDS (from literals, so that no load goes out ahead of the V tiles).
__device__ __forceinline__ void fill_etab(uint64_t* etab) {
    if (threadIdx.x == 0) {
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) etab[i] = expf_tab(i);
    }
}

// One chunk (blockIdx.y) of the online softmax of query head h for coordinates 64 sl .. 64 sl + 63 (blockIdx.x =
// h * slices + sl), from the scores of attn_score_kernel; below a padded KV length of 512 one chunk covers every
// position, from 512 on four chunks of ceil(n_kv / 4) (attend_head, attention.rs:483-542). All 256 threads turn the
// scores into factors, then wave 0 runs the accumulators of the slice's coordinates while wave 1 runs the sum. One
// chunk writes the output; of four, each stores its f16 accumulators and (max, sum), and the last to take the ticket
// of (h, sl) combines them in chunk order (attention.rs:526-541).
template <int HD>
__global__ __launch_bounds__(256) void attn_chain_kernel(AttnArgs a) {
    constexpr uint32_t kSlices = attn_slices(HD);
    constexpr uint32_t kLanes = HD >= 64 ? 64u : static_cast<uint32_t>(HD);
    __shared__ __align__(16) float fac[kChunkMax + 64u];
    __shared__ uint32_t bflag[kChunkMax / 32u + 2u];
    __shared__ float wtot[4];
    __shared__ float s_sum;
    __shared__ uint32_t s_last;
    __shared__ uint64_t etab[32];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t h = blockIdx.x / kSlices, sl = blockIdx.x - h * kSlices, c = blockIdx.y;
    const uint32_t pos = a.ctl->pos, seq = pos + 1u;
    uint32_t n_kv = (seq + 255u) / 256u * 256u;
    if (n_kv > a.max_ctx) n_kv = a.max_ctx;
    const bool split = n_kv >= 512u;
    const uint32_t chunk = split ? (n_kv + 3u) / 4u : seq;
    if (c >= (split ? 4u : 1u)) return;
    const uint32_t st = c * chunk, en = min(min(st + chunk, n_kv), seq);
    const bool any = st < en;
    const uint32_t kvh = h / a.gqa;
    const uint32_t d = sl * 64u + (lane < kLanes ? lane : 0u);  // a lane without a coordinate reads coordinate 0
    const uint16_t* vt = a.vc + static_cast<size_t>(kvh) * HD * a.vstride;
    const uint32_t b_first = st / 32u, b_end = any ? (en + 31u) / 32u : b_first + 1u;
    const uint32_t t_last = any ? (en - 1u) / 8u : st / 8u;
    fill_etab(etab);
    const VTiles vtl = vtiles<HD>(vt, d, t_last);
    u32x4 ring[kChainBlocks][4];
    if (wave == 0 && any) {
#pragma unroll
        for (uint32_t k = 0; k < kChainBlocks; ++k) load_vblock<HD>(vtl, b_first + k, t_last, ring[k]);
    }
    float cmax = -__builtin_inff();
    if (any) cmax = chunk_factors<256>(a.scores + static_cast<size_t>(h) * a.max_ctx + st, st, en, b_first, fac, bflag, wtot, etab);
    if (any && tid < 32u && en + tid < 32u * b_end) fac[en + tid - 32u * b_first] = 0.0f;  // the last block's padding
    __syncthreads();
    float y = 0.0f;
    if (any && wave == 0) {
        y = chain_y<HD>(ring, vtl, st, en, b_first, b_end, t_last, fac, bflag);
    } else if (wave == 1) {
        const float ssum = any ? chain_sum(st, en, b_first, b_end, fac, bflag) : 0.0f;
        if (lane == 0) s_sum = ssum;
    }
    __syncthreads();
    const float ssum = s_sum;
    float* out = a.out + static_cast<size_t>(h) * HD;
    if (!split) {
        if (wave == 0 && lane < kLanes) {
            const float s_inv = ssum == 0.0f ? 0.0f : 1.0f / ssum;
            out[sl * 64u + lane] = y * s_inv;
        }
        return;
    }
    // four chunks: this chunk's part, then the ticket of (h, sl); the fourth to arrive combines in chunk order. The
    // parts are written and read with agent-scope atomic stores and loads (coherent across the L2 caches without a
    // cache writeback), every store complete before the ticket is taken.
    uint32_t* cy = a.cy + static_cast<size_t>(h) * 4u * HD;
    float* cms = a.cms + (static_cast<size_t>(h) * kSlices + sl) * 8u;
    if (wave == 0) {
        if (lane < kLanes)
            __hip_atomic_store(cy + c * HD + sl * 64u + lane, static_cast<uint32_t>(f32_f16(y)), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) {
            __hip_atomic_store(cms + 2u * c, any ? cmax : -__builtin_inff(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(cms + 2u * c + 1u, ssum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    if (tid == 0) s_last = take_ticket(a.ticket + blockIdx.x, 3u);
    __syncthreads();
    if (s_last == 0u || wave != 0) return;
    if (lane == 0) atomicExch(a.ticket + blockIdx.x, 0u);
    if (lane >= kLanes) return;
    const uint32_t dd = sl * 64u + lane;
    float mf = -__builtin_inff(), sf = 0.0f, acc = 0.0f;
    for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t ks = k * chunk, ke = min(min(ks + chunk, n_kv), seq);
        if (ks >= ke) continue;
        const float sk = __hip_atomic_load(cms + 2u * k + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (sk == 0.0f) continue;
        const float mk = __hip_atomic_load(cms + 2u * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float mn = __builtin_fmaxf(mf, mk);
        const float so = glibc_expf(mf - mn);
        const float sn = glibc_expf(mk - mn);
        const uint32_t yk = __hip_atomic_load(cy + k * HD + dd, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float vn = f16_f32(static_cast<uint16_t>(yk)) * sn;
        acc = __builtin_fmaf(acc, so, vn);
        const float ssn = sk * sn;
        sf = __builtin_fmaf(sf, so, ssn);
        mf = mn;
    }
    out[dd] = sf != 0.0f ? acc * (1.0f / sf) : acc;
}

// The decode step's attention while the context is short (pos < kShortCtx: one chunk, no split) in one kernel per
// (head, 64 coordinates): the RoPE of q, k, v of the position (the first slice of the first head of each KV head
// appends k and v; every workgroup uses its own copy of the position itself), the scores of every position
// (1024 threads, four lanes per position, as attn_score_kernel), the factors, then the accumulators and the sum (one
// wave), and the output. The loads go out in the order they are needed: the RoPE inputs, the K rows, then the V tiles of
// the workgroup's 64 coordinates, which all threads stage into LDS during the scores, so that the chain reads V and the
// factors from LDS in a compact loop.
template <int HD>
__global__ __launch_bounds__(1024) void attn_short_kernel(AttnArgs a) {
    constexpr uint32_t kSlices = attn_slices(HD);
    constexpr uint32_t kLanes = HD >= 64 ? 64u : static_cast<uint32_t>(HD);
    constexpr int kBlk = HD / 32;
    constexpr uint32_t kTiles = kShortCtx / 8u;           // 8-position V tiles of the context at most
    constexpr uint32_t kVPer = kTiles * 64u / 1024u;      // V entries (tile, coordinate) per thread
    static_assert(kShortCtx * 4u == 1024u, "four lanes per position of the context");
    __shared__ __align__(16) uint16_t qh[HD];
    __shared__ __align__(16) uint16_t kp[HD];
    __shared__ __align__(16) uint16_t vp[HD];
    __shared__ __align__(16) float sc[kShortCtx];
    __shared__ __align__(16) float fac[kShortCtx + 64u];
    __shared__ uint32_t bflag[kShortCtx / 32u + 2u];
    __shared__ uint64_t etab[32];
    __shared__ __align__(16) u32x4 vl[kTiles][64];  // [tile][coordinate]: positions 8 t .. 8 t + 7
    __shared__ float s_sum;
    __shared__ uint32_t s_ready;  // 32-position blocks whose factors and mask are in fac and bflag
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t h = blockIdx.x / kSlices, sl = blockIdx.x - h * kSlices;
    const uint32_t pos = a.ctl->pos, seq = pos + 1u;  // seq <= kShortCtx (the host's choice of graph)
    const uint32_t kvh = h / a.gqa;
    const uint16_t* kb = a.kc + static_cast<size_t>(kvh) * a.max_ctx * HD;
    uint16_t* vt = a.vc + static_cast<size_t>(kvh) * HD * a.vstride;
    const uint32_t t_last = (seq - 1u) / 8u;
    fill_etab(etab);
    if (tid == 0) s_ready = 0u;

    // RoPE inputs: thread i < HD / 2 rotates pair i of q, HD / 2 <= i < HD pair i - HD / 2 of k; HD <= i < 2 HD takes
    // coordinate i - HD of v. The raw sums, the scale and the rotation are loaded before anything else.
    const bool normal = a.rope_normal != 0u;
    const bool is_q = tid < HD / 2u, is_k = !is_q && tid < HD, is_v = tid >= HD && tid < 2u * HD;
    const ProjOut& po = is_q ? a.q : (is_k ? a.k : a.v);
    const uint32_t pi = is_q ? tid : tid - HD / 2u;  // the pair (q, k)
    const uint32_t i0 = normal ? 2u * pi : pi, i1 = normal ? 2u * pi + 1u : pi + HD / 2u;
    float r_as = 0.0f, r_cc = 0.0f, r_ss = 0.0f;
    int32_t r_x0 = 0, r_x1 = 0;
    if (is_q || is_k) {
        const uint32_t base = (is_q ? h : kvh) * HD;
        r_as = *po.as;
        r_x0 = po.part[base + i0];
        r_x1 = po.part[base + i1];
        const float* cache = a.rope + static_cast<size_t>(pos) * HD;
        r_cc = cache[2u * pi];
        r_ss = cache[2u * pi + 1u];
    } else if (is_v) {
        r_as = *a.v.as;
        r_x0 = a.v.part[kvh * HD + (tid - HD)];
    }
    // K row of this thread's position (the position itself later, from kp)
    const uint32_t j = tid & 3u, g = tid >> 2;
    uint4 k0[kBlk];
    if (g < seq && g != pos) {
#pragma unroll
        for (int i = 0; i < kBlk; ++i) k0[i] = *reinterpret_cast<const uint4*>(kb + static_cast<size_t>(g) * HD + 8 * j + 32 * i);
    }
    // V tiles of the slice's coordinates: entry e = tid + 1024 r is (tile e / 64, coordinate e % 64)
    u32x4 vr[kVPer];
#pragma unroll
    for (uint32_t r = 0; r < kVPer; ++r) {
        const uint32_t e = tid + 1024u * r, t = e >> 6, c = e & 63u;
        if (t <= t_last && c < kLanes)
            vr[r] = *reinterpret_cast<const u32x4*>(vt + (static_cast<size_t>(t) * HD + sl * 64u + c) * 8u);
    }
    if (is_q || is_k) {
        bool zero;
        const float post = proj_post(po, r_as, &zero);
        const float x0 = proj_value(r_x0, post, zero), x1 = proj_value(r_x1, post, zero);
        const float x1s = x1 * r_ss, x1c = x1 * r_cc;
        uint16_t* dst = is_q ? qh : kp;
        dst[i0] = f32_f16(__builtin_fmaf(x0, r_cc, -x1s));
        dst[i1] = f32_f16(__builtin_fmaf(x0, r_ss, x1c));
    } else if (is_v) {
        bool zero;
        const float post = proj_post(a.v, r_as, &zero);
        vp[tid - HD] = f32_f16(proj_value(r_x0, post, zero));
    }
    __syncthreads();
    if (h % a.gqa == 0 && sl == 0 && tid < HD) {
        a.kc[(static_cast<size_t>(kvh) * a.max_ctx + pos) * HD + tid] = kp[tid];
        vt[(static_cast<size_t>(pos >> 3) * HD + tid) * 8u + (pos & 7u)] = vp[tid];
    }
    // The V tiles into LDS, the position's own value (not yet visible in the cache to every workgroup) from vp, and
    // positions from seq to the end of the last 32-position block as -0: with a factor of +0 there (vs = 0, ms = 1) a
    // step adds v * vs = -0, which leaves every accumulator value as it is (-0 + y = y, also for y = +0 or -0), so the
    // last block needs no edge handling.
    const uint32_t t_pad = (seq + 31u) / 32u * 4u;  // tiles up to the end of the last block
#pragma unroll
    for (uint32_t r = 0; r < kVPer; ++r) {
        const uint32_t e = tid + 1024u * r, t = e >> 6, c = e & 63u;
        if (t < t_pad && c < kLanes) {
            u32x4 w = t <= t_last ? vr[r] : u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
            if (t == t_last) {
                const uint32_t el = pos & 7u;
                const uint32_t self = vp[sl * 64u + c];
                uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (uint32_t i = 0; i < 8; ++i) {
                    const uint32_t sh = (i & 1u) * 16u, keep = ~(0xffffu << sh);
                    const uint32_t val = i == el ? self : 0x8000u;  // the position itself, then the padding
                    if (i >= el) ww[i >> 1] = (ww[i >> 1] & keep) | (val << sh);
                }
                w = u32x4{ww[0], ww[1], ww[2], ww[3]};
            }
            vl[t][c] = w;
        }
    }
    if (g == pos) {
#pragma unroll
        for (int i = 0; i < kBlk; ++i) k0[i] = *reinterpret_cast<const uint4*>(kp + 32 * i + 8 * j);
    }
    if (g < seq) {
        const float s0 = score_dot4<HD>(qh, k0, j);
        if (j == 0) sc[g] = s0 * a.scale;
    }
    __syncthreads();

    // The factors (attend_range, attention.rs:436-468, as chunk_factors computes them) come from wave 2, 64 positions
    // at a time: the running maximum before each position by a scan over the lanes with the previous positions' maximum
    // carried in (the combine keeps the earliest of equal values, so the scan equals the sequential fold), then ms =
    // expf(m_old - score) with vs = 1 at a new maximum and ms = 1, vs = expf(score - max) otherwise, stored as -ms or
    // vs; the positions from seq to the end of the last 32-position block get +0. After each 64 positions wave 2
    // publishes the count of complete blocks (a workgroup-scope release), and the accumulator and sum waves start on a
    // block once it is published (an acquire), so the chain does not wait for the factors of the whole context.
    //
    // The accumulator of the lane's coordinate (wave 0: y, f16) and the sum (wave 1: ssum, f32) over the positions in
    // order, a block of 32 per step (the last one padded), its V words, factors and new-maximum mask read from LDS at
    // the start of the step. A block without a new maximum takes the short step (one f16 rounding of fma(v, vs, y));
    // one with new maxima takes the full step everywhere, y = f16(y * ms), y = f16(fma(v, vs, y)), with ms = 1, where
    // the multiply and its rounding leave y as it is, at the positions without one. Both are straight-line code: a
    // branch per position costs more than the longer step.
    const uint32_t nb = (seq + 31u) / 32u;
    // Waits until block b is published. The bound (far beyond the producer's few microseconds) only keeps a wave from
    // spinning for ever should the producer not run; it is never reached when it does.
    auto wait_block = [&](uint32_t b) {
        for (uint32_t spin = 0; spin < (1u << 20); ++spin) {
            if (__hip_atomic_load(&s_ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) > b) break;
            __builtin_amdgcn_s_sleep(1);
        }
    };
    if (wave == 0) {
        const uint32_t cl = lane < kLanes ? lane : 0u;
        _Float16 yh = 0;
        for (uint32_t b = 0; b < nb; ++b) {
            wait_block(b);
            u32x4 w[4];
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) w[i] = vl[4u * b + i][cl];
            float f[32];
#pragma unroll
            for (uint32_t i = 0; i < 8; ++i) {
                const float4 q = *reinterpret_cast<const float4*>(fac + 32u * b + 4u * i);
                f[4 * i] = q.x;
                f[4 * i + 1] = q.y;
                f[4 * i + 2] = q.z;
                f[4 * i + 3] = q.w;
            }
            if (__builtin_amdgcn_readfirstlane(bflag[b]) == 0u) {
#pragma unroll
                for (int e = 0; e < 32; ++e)
                    yh = static_cast<_Float16>(keep_f32(__builtin_fmaf(vhalf(w, e), f[e], static_cast<float>(yh))));
            } else {
#pragma unroll
                for (int e = 0; e < 32; ++e) {
                    const bool nm = __builtin_signbit(f[e]);
                    const float ev = __builtin_fabsf(f[e]);
                    yh = static_cast<_Float16>(keep_f32(static_cast<float>(yh) * (nm ? ev : 1.0f)));
                    yh = static_cast<_Float16>(keep_f32(__builtin_fmaf(vhalf(w, e), nm ? 1.0f : ev, static_cast<float>(yh))));
                }
            }
        }
        __syncthreads();  // wave 1's sum
        if (lane < kLanes) {
            const float ssum = s_sum;
            const float s_inv = ssum == 0.0f ? 0.0f : 1.0f / ssum;
            a.out[static_cast<size_t>(h) * HD + sl * 64u + lane] = static_cast<float>(yh) * s_inv;
        }
    } else if (wave == 1) {
        float ssum = 0.0f;
        for (uint32_t b = 0; b < nb; ++b) {
            wait_block(b);
            float f[32];
#pragma unroll
            for (uint32_t i = 0; i < 8; ++i) {
                const float4 q = *reinterpret_cast<const float4*>(fac + 32u * b + 4u * i);
                f[4 * i] = q.x;
                f[4 * i + 1] = q.y;
                f[4 * i + 2] = q.z;
                f[4 * i + 3] = q.w;
            }
            if (__builtin_amdgcn_readfirstlane(bflag[b]) == 0u) {
#pragma unroll
                for (int e = 0; e < 32; ++e) ssum = ssum + f[e];
            } else {
#pragma unroll
                for (int e = 0; e < 32; ++e) {
                    const bool nm = __builtin_signbit(f[e]);
                    const float ev = __builtin_fabsf(f[e]);
                    ssum = __builtin_fmaf(ssum, nm ? ev : 1.0f, nm ? 1.0f : ev);
                }
            }
        }
        if (lane == 0) s_sum = ssum;
        __syncthreads();
    } else if (wave == 2) {
        const auto tab = [&](uint32_t k) { return etab[k]; };
        const uint32_t n_pad = 32u * nb;
        float carry = -__builtin_inff();  // the maximum of the positions before this group of 64
        for (uint32_t base = 0; base < n_pad; base += 64u) {
            const uint32_t p = base + lane;
            const bool in = p < seq;
            const float sv = in ? sc[p] : 0.0f;
            float v = in && sv == sv ? sv : -__builtin_inff();  // a NaN score never moves the maximum
#pragma unroll
            for (int sh = 1; sh < 64; sh <<= 1) {
                const float o = __shfl_up(v, sh);
                if (lane >= static_cast<uint32_t>(sh)) v = max_later(o, v);
            }
            float prev = __shfl_up(v, 1);
            prev = max_later(carry, lane == 0 ? -__builtin_inff() : prev);
            carry = max_later(carry, __shfl(v, 63));
            float f = 0.0f;
            if (in) f = sv > prev ? -glibc_expf_with(prev - sv, tab) : glibc_expf_with(sv - prev, tab);
            if (p < n_pad) fac[p] = f;
            const uint64_t neg = __ballot(in && __builtin_signbit(f));
            if (lane == 0) {
                bflag[base / 32u] = static_cast<uint32_t>(neg);
                if (base / 32u + 1u < nb) bflag[base / 32u + 1u] = static_cast<uint32_t>(neg >> 32);
                __hip_atomic_store(&s_ready, min(nb, base / 32u + 2u), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        __syncthreads();
    } else {
        __syncthreads();
    }
}

// ---- head and greedy argmax ----------------------------------------------------------------------------------------------

// Ordered key of a logit for the greedy argmax (sampler.rs:73-83: max_val = logits[0], then the first i with
// logits[i] > max_val): larger values first, then lower indices; -0 counts as +0, NaN never wins except at index 0,
// where it wins outright (the reference then returns 0). The maximum key over all rows names the token (0 if none).
__device__ __forceinline__ unsigned long long logit_key(float v, uint32_t r) {
    if (v != v) return r == 0 ? ~0ull : 0ull;
    uint32_t u = f32_bits(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(u) << 32) | (0xffffffffu - r);
}

struct HeadArgs {
    StageInput in;         // the final residual add (x + down of the last layer) and the output norm
    const uint16_t* w;     // the head: vocab x hidden, bf16 or f16 (the embedding when tied)
    uint32_t hidden, vocab;
    float* logits;
    Ctl* ctl;
    uint32_t* out_tokens;
    unsigned long long* key;  // argmax across workgroups: the largest logit_key (0 between steps)
    uint32_t* ticket;         // workgroups done (0 between steps)
};

// Every workgroup computes the normed vector itself, rounds it to the head's type (model.rs:347-351), then rows
// r0 + tid / 4 in blocks of kNT / 4. Lane (r, j) of four per row holds the eight lanes of accumulator j over the
// 32-value blocks, the cross-lane sums give (a0 + a2) + (a1 + a3), and inside one lane:
//   bf16 (ggml_vec_dot_bf16, ops.rs:669-713)   acc + x*y rounded separately; ((l0+l4) + (l2+l6)) + ((l1+l5) + (l3+l7))
//   f16  (ggml_vec_dot_f16, ops.rs:960-1015)   fma(x, y, acc);                ((l0+l4) + (l1+l5)) + ((l2+l6) + (l3+l7))
// hidden must be a multiple of 32. The workgroup's best key goes into *key with an atomic maximum; the last workgroup
// to finish reads the winner, resets key and ticket, and advances the loop state: the token is recorded once the
// prompt is consumed and the position moves on.
template <bool F16>
__global__ __launch_bounds__(kNT) void head_kernel(HeadArgs a) {
    __shared__ InputLds s;
    __shared__ uint4 xs[kNormMax / 8];
    __shared__ unsigned long long wbest[kNT / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    InputRegs<2, 1, 0> r;
    stage_load(a.in, r, 0u, a.in.n);
    float y[2][4];
    stage_y(a.in, r, s, false, y);
    uint16_t* xh = reinterpret_cast<uint16_t*>(xs);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t i = elem4(tid, k);
        if (i < a.hidden) {
            uint16_t hv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) hv[e] = F16 ? f32_f16(y[k][e]) : f32_bf16(y[k][e]);
            *reinterpret_cast<uint2*>(xh + i) = make_uint2(hv[0] | (static_cast<uint32_t>(hv[1]) << 16),
                                                           hv[2] | (static_cast<uint32_t>(hv[3]) << 16));
        }
    }
    __syncthreads();
    const uint32_t j = tid & 3u;
    unsigned long long best = 0;
    for (uint32_t r0 = blockIdx.x * (kNT / 4u); r0 < a.vocab; r0 += gridDim.x * (kNT / 4u)) {
        const uint32_t row_i = r0 + (tid >> 2);
        const u32x4* row = reinterpret_cast<const u32x4*>(a.w + static_cast<size_t>(min(row_i, a.vocab - 1u)) * a.hidden);
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        auto block = [&](const u32x4& w, uint32_t i) {  // the 32-value block i: lane j's accumulator j
            const uint4 x = xs[4u * i + j];
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w}, xx[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const uint16_t wb = static_cast<uint16_t>(ww[l >> 1] >> ((l & 1) * 16));
                const uint16_t xb = static_cast<uint16_t>(xx[l >> 1] >> ((l & 1) * 16));
                if (F16) {
                    acc[l] = __builtin_fmaf(f16_f32(xb), f16_f32(wb), acc[l]);
                } else {
                    const float p = bf16_f32(xb) * bf16_f32(wb);
                    acc[l] = acc[l] + p;
                }
            }
        };
        const uint32_t nblk = a.hidden / 32u, nblk8 = nblk & ~7u;
        for (uint32_t i0 = 0; i0 < nblk8; i0 += 8u) {  // eight loads in flight per lane
            u32x4 w[8];
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) w[u] = __builtin_nontemporal_load(row + 4u * (i0 + u) + j);
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) block(w[u], i0 + u);
        }
        for (uint32_t i = nblk8; i < nblk; ++i) block(__builtin_nontemporal_load(row + 4u * i + j), i);
        // (a0 + a2) + (a1 + a3): lanes j and j ^ 2, then j and j ^ 1
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            acc[l] = acc[l] + bits_f32(dpp32<kDppXor2>(f32_bits(acc[l])));  // lane j ^ 2 of the quad (DPP)
            acc[l] = acc[l] + bits_f32(dpp32<kDppXor1>(f32_bits(acc[l])));  // lane j ^ 1
        }
        if (j == 0 && row_i < a.vocab) {
            const float g0 = acc[0] + acc[4], g1 = acc[1] + acc[5], g2 = acc[2] + acc[6], g3 = acc[3] + acc[7];
            const float v = F16 ? (g0 + g1) + (g2 + g3) : (g0 + g2) + (g1 + g3);
            a.logits[row_i] = v;
            const unsigned long long k = logit_key(v, row_i);
            if (k > best) best = k;
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(best, off);
        if (o > best) best = o;
    }
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (tid != 0) return;
    for (int w = 1; w < kNT / 64; ++w)
        if (wbest[w] > best) best = wbest[w];
    atomicMax(a.key, best);
    __builtin_amdgcn_s_waitcnt(0);  // the maximum is in place (at the atomics' coherence point) before the ticket
    if (take_ticket(a.ticket, gridDim.x - 1u) == 0u) return;
    const unsigned long long k = atomicExch(a.key, 0ull);
    atomicExch(a.ticket, 0u);
    const uint32_t idx = k == 0 ? 0u : 0xffffffffu - static_cast<uint32_t>(k);
    const uint32_t pos = a.ctl->pos;
    a.ctl->token = idx;
    if (pos + 1 >= a.ctl->n_prompt) {
        const uint32_t t = pos + 1 - a.ctl->n_prompt;
        if (t < a.ctl->n_out) a.out_tokens[t] = idx;
    }
    a.ctl->pos = pos + 1;
}

// ---- prefill: the prompt's tokens in one pass per layer ---------------------------------------------------------------------
//
// The reference ingests a prompt one forward_token per position (quintrit-runtime/src/engine.rs:627-630). A prefill
// runs n tokens through each layer at once: the projections as one batched GEMM per matrix (vx_gemm.hip, exact int32,
// the same sums as n GEMVs), everything else per token with the decode step's arithmetic (stage_y, the quantizer, the
// epilogue, RoPE, the attention kernel), so that the KV cache, the logits and the greedy token equal those of n decode
// steps bit for bit. Positions: the loop state's pos is the last token's (ctl->pos + 1 - n_tok + t for token t).

// One workgroup per token: the token's stage input (embedding row, residual add or a plain vector, with the RMSNorm
// when gamma is set) and its per-token absmax int8 codes (quantize_activations_int8_with_range, ops.rs:241-267) into
// codes[t], its scale into as_out[t]. An input with x_out writes the new residual row in place.
struct PfStageArgs {
    StageInput in;          // the input of token 0; rows of x_in / x_out are x_stride floats apart, of a.part a_stride
    uint32_t x_stride, a_stride, n_tok;
    const uint32_t* prompt;  // kInEmbed: the token at each position
    int8_t* codes;          // [n_tok][codes_stride]
    uint32_t codes_stride;
    float* as_out;          // [n_tok]
};

template <int P4, int SA>
__global__ __launch_bounds__(kNT) void pf_stage_kernel(PfStageArgs a) {
    __shared__ InputLds s;
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    StageInput in = a.in;
    if (in.x_in != nullptr) in.x_in += static_cast<size_t>(t) * a.x_stride;
    if (in.x_out != nullptr) in.x_out += static_cast<size_t>(t) * a.x_stride;
    if (in.kind == kInResidual) {
        in.a.part += static_cast<size_t>(t) * a.a_stride;
        in.a.as += t;
    }
    if (in.kind == kInEmbed) in.token_at = a.prompt + (in.ctl->pos + 1u - a.n_tok + t);
    InputRegs<P4, SA, 0> r{};
    stage_load(in, r, 0u, in.n);
    float y[P4][4];
    stage_y(in, r, s, true, y);
    float mx = 0.0f;  // the largest |y|; NaN never counts (as in stage_window)
#pragma unroll
    for (int k = 0; k < P4; ++k)
        if (elem4(tid, k) < in.n) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ay = __builtin_fabsf(y[k][e]);
                if (ay > mx) mx = ay;
            }
        }
    mx = wave_max_f32(mx);
    if (lane == 0) s.red_f[wave] = mx;
    __syncthreads();
    float m = 0.0f;
    for (int w = 0; w < kNT / 64; ++w) m = fmax_nn(m, s.red_f[w]);
    const float sc = m > 0.0f ? 127.0f / m : 0.0f;
    int8_t* row = a.codes + static_cast<size_t>(t) * a.codes_stride;
#pragma unroll
    for (int k = 0; k < P4; ++k) {
        const uint32_t i = elem4(tid, k);
        if (i < in.n) {
            uint32_t w4 = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int x = m > 0.0f ? quant_code(y[k][e], sc) : 0;
                w4 |= (static_cast<uint32_t>(x) & 0xffu) << (8 * e);
            }
            *reinterpret_cast<uint32_t*>(row + i) = w4;
        }
    }
    if (tid == 0) a.as_out[t] = sc;
}

// RoPE of every token's q and k and the KV append (the first part of attention_kernel, for n tokens): q, k, v of token
// t from the GEMM outputs with the layer epilogue (layer.rs:246-253), rotated at the token's position (ops.rs:199-221),
// rounded to f16; k and v into the cache, q into qbuf.
struct PfRopeArgs {
    const Ctl* ctl;
    uint32_t n_tok;
    const int32_t *yq, *yk, *yv;  // [n_tok][ld*]
    uint32_t ldq, ldk, ldv;
    const float* as;              // [n_tok] activation scale of the q/k/v input
    float wsq, wsk, wsv;
    const float* rope;            // [max_ctx][head_dim]: (cos, sin) of pair i at 2i, 2i + 1
    uint16_t *kc, *vc;            // this layer: k [kv_head][max_ctx][head_dim], v [kv_head][vstride / 8][head_dim][8]
    uint16_t* qbuf;               // [n_tok][n_heads * head_dim]
    uint32_t n_heads, n_kv, hd, max_ctx, rope_normal, vstride;
};

__global__ __launch_bounds__(256) void pf_rope_kernel(PfRopeArgs a) {
    const uint32_t t = blockIdx.x;
    const uint32_t pos = a.ctl->pos + 1u - a.n_tok + t;
    const float as = a.as[t];
    const bool zero = !(as > 0.0f);
    const float pq = zero ? 0.0f : a.wsq / as, pk = zero ? 0.0f : a.wsk / as, pv = zero ? 0.0f : a.wsv / as;
    const uint32_t half = a.hd / 2u, nq = a.n_heads * half, nk = a.n_kv * half, nv = a.n_kv * a.hd;
    const float* cache = a.rope + static_cast<size_t>(pos) * a.hd;
    // blockIdx.y spreads the token's elements over several workgroups, so each thread waits for about one load of
    // the GEMM outputs instead of a dozen in a row
    for (uint32_t i = blockIdx.y * blockDim.x + threadIdx.x; i < nq + nk + nv; i += gridDim.y * blockDim.x) {
        if (i < nq + nk) {
            const bool isq = i < nq;
            const uint32_t j = isq ? i : i - nq, head = j / half, pr = j - head * half;
            const uint32_t i0 = a.rope_normal ? 2u * pr : pr, i1 = a.rope_normal ? 2u * pr + 1u : pr + half;
            const int32_t* y = isq ? a.yq + static_cast<size_t>(t) * a.ldq : a.yk + static_cast<size_t>(t) * a.ldk;
            const float post = isq ? pq : pk;
            const float x0 = proj_value(y[head * a.hd + i0], post, zero), x1 = proj_value(y[head * a.hd + i1], post, zero);
            const float cc = cache[2 * pr], ss = cache[2 * pr + 1];
            const float x1s = x1 * ss, x1c = x1 * cc;
            const float y0 = __builtin_fmaf(x0, cc, -x1s);
            const float y1 = __builtin_fmaf(x0, ss, x1c);
            uint16_t* dst = isq ? a.qbuf + (static_cast<size_t>(t) * a.n_heads + head) * a.hd
                                : a.kc + (static_cast<size_t>(head) * a.max_ctx + pos) * a.hd;
            dst[i0] = f32_f16(y0);
            dst[i1] = f32_f16(y1);
        } else {
            const uint32_t j = i - nq - nk, head = j / a.hd, e = j - head * a.hd;
            a.vc[static_cast<size_t>(head) * a.hd * a.vstride + (static_cast<size_t>(pos >> 3) * a.hd + e) * 8u + (pos & 7u)] =
                f32_f16(proj_value(a.yv[static_cast<size_t>(t) * a.ldv + j], pv, zero));
        }
    }
}

// The gated activation of every token (model.rs:155-170): g and u from the gate and up GEMM outputs with their layer
// epilogues, then relu2(g) * u (ops.rs:301-308) or swiglu (ops.rs:430-464: ggml's vector expf for the whole blocks
// of 8, libm's expf for the last ffn % 8 values), as the decode step's gated pair computes them.
struct PfActArgs {
    const int32_t *yg, *yu;  // [n_tok][ld]
    uint32_t ld;
    const float* as;         // [n_tok]
    float wsg, wsu;
    float* out;              // [n_tok][ffn]
    uint32_t ffn, n8, act;
};

__global__ __launch_bounds__(256) void pf_act_kernel(PfActArgs a) {
    const uint32_t t = blockIdx.y, i = blockIdx.x * 256u + threadIdx.x;
    if (i >= a.ffn) return;
    const float as = a.as[t];
    const bool zero = !(as > 0.0f);
    const float g = zero ? 0.0f : static_cast<float>(a.yg[static_cast<size_t>(t) * a.ld + i]) * (a.wsg / as);
    const float u = zero ? 0.0f : static_cast<float>(a.yu[static_cast<size_t>(t) * a.ld + i]) * (a.wsu / as);
    float o;
    if (a.act == kActSilu) {
        const float ex = i < a.n8 ? ggml_expf(0.0f - g) : glibc_expf(-g);
        const float den = 1.0f + ex;
        const float sl = g / den;
        o = sl * u;
    } else {
        const float pos = g > 0.0f ? g : 0.0f;
        const float sq = pos * pos;
        o = sq * u;
    }
    a.out[static_cast<size_t>(t) * a.ffn + i] = o;
}

// Sets the loop state from kernel arguments (no host buffer is read when the kernel runs).
__global__ void set_ctl_kernel(Ctl* ctl, uint32_t pos, uint32_t token, uint32_t n_prompt, uint32_t n_out) {
    if (threadIdx.x == 0) {
        ctl->pos = pos;
        ctl->token = token;
        ctl->n_prompt = n_prompt;
        ctl->n_out = n_out;
    }
}

int launch_pf_stage(const PfStageArgs& a, hipStream_t s) {
    const bool res = a.in.kind == kInResidual;
    if (a.in.n <= 4u * kNT) {
        if (res) hipLaunchKernelGGL((pf_stage_kernel<1, 1>), dim3(a.n_tok), dim3(kNT), 0, s, a);
        else hipLaunchKernelGGL((pf_stage_kernel<1, 0>), dim3(a.n_tok), dim3(kNT), 0, s, a);
    } else if (a.in.n <= 8u * kNT) {
        if (res) hipLaunchKernelGGL((pf_stage_kernel<2, 1>), dim3(a.n_tok), dim3(kNT), 0, s, a);
        else hipLaunchKernelGGL((pf_stage_kernel<2, 0>), dim3(a.n_tok), dim3(kNT), 0, s, a);
    } else {
        if (res || a.in.gamma != nullptr) VX_FAIL(VX_ERR_INTERNAL, "a prefill input of %u elements needs a norm", a.in.n);
        hipLaunchKernelGGL((pf_stage_kernel<kPlainMax / (4 * kNT), 0>), dim3(a.n_tok), dim3(kNT), 0, s, a);
    }
    VX_HIP(hipGetLastError());
    return VX_OK;
}

// ---- launches ----------------------------------------------------------------------------------------------------------------

// dgemv_kernel instances (DStageArgs::variant): inputs of up to 4096 and 8192 elements of every kind, and plain or
// embedding inputs of up to kPlainMax elements without a norm (the SwiGLU output of a model without sub-norms).
enum DVariant : uint32_t { kDv4K = 0, kDv8K = 1, kDvPlain = 2 };

template <int P4, int SA, int SB, bool MULTI>
static void launch_dgemv_d(const DStageArgs& a, hipStream_t s) {
    if constexpr (MULTI) {
        if (a.range_chunks != 0) {
            hipLaunchKernelGGL((dgemv_kernel<P4, SA, SB, true, kDPer, true, kNT>), dim3(a.grid), dim3(kNT), 0, s, a);
            return;
        }
    }
    if (a.dper <= 1) hipLaunchKernelGGL((dgemv_kernel<P4, SA, SB, MULTI, 1, false, kNT>), dim3(a.grid), dim3(kNT), 0, s, a);
    else if (a.dper <= 4) hipLaunchKernelGGL((dgemv_kernel<P4, SA, SB, MULTI, 4, false, kNT>), dim3(a.grid), dim3(kNT), 0, s, a);
    else hipLaunchKernelGGL((dgemv_kernel<P4, SA, SB, MULTI, kDPer, false, kNT>), dim3(a.grid), dim3(kNT), 0, s, a);
}

// MULTI: the instance that takes two items per workgroup and runs gated pairs; the others take one plain item.
int launch_dgemv(const DStageArgs& a, hipStream_t s) {
    const bool multi = a.loop || a.job[0].w2 != nullptr;
    if (a.dper == 0 || a.dper > static_cast<uint32_t>(kDPer)) VX_FAIL(VX_ERR_INTERNAL, "stage with %u chunks per wave", a.dper);
    switch (a.variant) {
        case kDv4K:
            if (multi) launch_dgemv_d<1, 1, 1, true>(a, s);
            else launch_dgemv_d<1, 1, 1, false>(a, s);
            break;
        case kDv8K:
            if (multi) launch_dgemv_d<2, 1, 1, true>(a, s);
            else launch_dgemv_d<2, 1, 1, false>(a, s);
            break;
        default:  // a wide plain input is a down projection's, split into several K slices: one item per workgroup
            if (multi) VX_FAIL(VX_ERR_INTERNAL, "a looping stage with a %u-element input", a.in.n);
            launch_dgemv_d<kPlainMax / (4 * kNT), 0, 0, false>(a, s);
            break;
    }
    VX_HIP(hipGetLastError());
    return VX_OK;
}

template <bool PREFILL>
static int launch_attention_mode(const AttnArgs& a, uint32_t head_dim, hipStream_t s) {
    const dim3 grid(a.n_heads, PREFILL ? a.n_tok : 1u);
    if (head_dim == 256) hipLaunchKernelGGL((attention_kernel<256, PREFILL>), grid, dim3(attn_threads(256)), 0, s, a);
    else if (head_dim == 128) hipLaunchKernelGGL((attention_kernel<128, PREFILL>), grid, dim3(attn_threads(128)), 0, s, a);
    else if (head_dim == 64) hipLaunchKernelGGL((attention_kernel<64, PREFILL>), grid, dim3(attn_threads(64)), 0, s, a);
    else if (head_dim == 32) hipLaunchKernelGGL((attention_kernel<32, PREFILL>), grid, dim3(attn_threads(32)), 0, s, a);
    else VX_FAIL(VX_ERR_INTERNAL, "no attention kernel for head_dim %u", head_dim);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

// The decode step's attention: the score kernel over every 64-position range of max_ctx (ranges past the position
// return at once), then the chain kernel over (head, 64 coordinates) x 4 chunks (chunks past the split return).
int launch_attention(const AttnArgs& a, uint32_t head_dim, hipStream_t s) {
    const uint32_t hgroups = (a.gqa + kScoreHeads - 1u) / kScoreHeads;
    const dim3 sgrid(a.n_heads / a.gqa * hgroups, (a.max_ctx + kScoreTile - 1u) / kScoreTile);
    const dim3 cgrid(a.n_heads * attn_slices(head_dim), 4u);
    if (a.max_ctx > kAttnMaxCtx) VX_FAIL(VX_ERR_INTERNAL, "attention context %u above %u", a.max_ctx, kAttnMaxCtx);
    if (head_dim == 256) {
        hipLaunchKernelGGL(attn_score_kernel<256>, sgrid, dim3(256), 0, s, a);
        hipLaunchKernelGGL(attn_chain_kernel<256>, cgrid, dim3(256), 0, s, a);
    } else if (head_dim == 128) {
        hipLaunchKernelGGL(attn_score_kernel<128>, sgrid, dim3(256), 0, s, a);
        hipLaunchKernelGGL(attn_chain_kernel<128>, cgrid, dim3(256), 0, s, a);
    } else if (head_dim == 64) {
        hipLaunchKernelGGL(attn_score_kernel<64>, sgrid, dim3(256), 0, s, a);
        hipLaunchKernelGGL(attn_chain_kernel<64>, cgrid, dim3(256), 0, s, a);
    } else if (head_dim == 32) {
        hipLaunchKernelGGL(attn_score_kernel<32>, sgrid, dim3(256), 0, s, a);
        hipLaunchKernelGGL(attn_chain_kernel<32>, cgrid, dim3(256), 0, s, a);
    } else {
        VX_FAIL(VX_ERR_INTERNAL, "no attention kernel for head_dim %u", head_dim);
    }
    VX_HIP(hipGetLastError());
    return VX_OK;
}

// The short-context form (every position below kShortCtx): one kernel per (head, 64 coordinates).
int launch_attention_short(const AttnArgs& a, uint32_t head_dim, hipStream_t s) {
    const dim3 grid(a.n_heads * attn_slices(head_dim));
    if (head_dim == 256) hipLaunchKernelGGL(attn_short_kernel<256>, grid, dim3(1024), 0, s, a);
    else if (head_dim == 128) hipLaunchKernelGGL(attn_short_kernel<128>, grid, dim3(1024), 0, s, a);
    else if (head_dim == 64) hipLaunchKernelGGL(attn_short_kernel<64>, grid, dim3(1024), 0, s, a);
    else if (head_dim == 32) hipLaunchKernelGGL(attn_short_kernel<32>, grid, dim3(1024), 0, s, a);
    else VX_FAIL(VX_ERR_INTERNAL, "no attention kernel for head_dim %u", head_dim);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_attention_prefill(const AttnArgs& a, uint32_t head_dim, hipStream_t s) {
    return launch_attention_mode<true>(a, head_dim, s);
}

int launch_head(const HeadArgs& a, bool f16, uint32_t grid, hipStream_t s) {
    if (f16)
        hipLaunchKernelGGL(head_kernel<true>, dim3(grid), dim3(kNT), 0, s, a);
    else
        hipLaunchKernelGGL(head_kernel<false>, dim3(grid), dim3(kNT), 0, s, a);
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
constexpr int kStages = 4;  // projection stages of a layer: q/k/v, o, gate/up, down

}  // namespace vx

struct vx_decoder {
    uint32_t magic;
    int device, num_cus;
    vx_decoder_config_t cfg;
    size_t qd, kvd;
    std::vector<vx_matrix_t*> proj;   // [layer * 7 + kind]
    std::vector<float*> norms;        // [layer * 4 + kind]; the output norm at [n_layers * 4]
    std::vector<uint8_t> norm_set;
    bool emb_set, head_set;
    bool pair;                        // gate and up run as one gated pair (the down input is d_inter)
    uint16_t* d_emb;
    uint16_t* d_head;                 // the untied head, or null
    float* d_inter;                   // gated pair output: act(gate, up), [ffn rounded up to 64]
    uint32_t* d_amax;                 // per layer: max |act(gate, up)| bits for an unnormed down input (pair, no sub-norms)
    int32_t* d_pacc;                  // pair: per tile and row one 64-bit word (gate, up, count) of the chunk-range split
    float* d_rope;
    uint16_t *d_kc, *d_vc;            // [layer][kv_head][max_ctx][head_dim]
    float *d_xa, *d_xb;               // the residual stream (written alternately by the stages that add to it)
    int32_t* d_part[vx::kProjKinds];  // K-slice sums of the q, k, v, o, gate, up, down outputs, reused by every layer
    uint32_t kslices[vx::kProjKinds];
    float* d_as;                      // activation scale of each projection stage, reused by every layer
    float *d_att, *d_logits;
    float* d_scores;                  // decode attention: scores [n_heads][max_ctx]
    uint32_t* d_cy;                   // per chunk f16 accumulators [n_heads][4][head_dim], one per word
    float* d_cms;                     // per chunk (max, sum) [n_heads][slices][4][2]
    uint32_t* d_aticket;              // chunks done per (head, slice) (0 between steps)
    unsigned long long* d_key;        // argmax key and ticket of the head kernel
    uint32_t* d_ticket;
    vx::Ctl* d_ctl;
    uint32_t* d_prompt;
    uint32_t* d_tokens;
    std::vector<vx::DStageArgs> stages;  // [layer * 4 + stage]
    // prefill: buffers for chunks of up to pf_cap tokens, and the recorded chunk graphs by (tokens, with head)
    uint32_t pf_cap;
    float* pf_x;                      // [pf_cap][hidden] residual stream
    int8_t* pf_codes;                 // [pf_cap][pf_codes_ld] int8 inputs of a GEMM
    uint32_t pf_codes_ld;
    float* pf_as;                     // [4][pf_cap] activation scales of the q/k/v, o, gate/up and down inputs
    int32_t* pf_y[vx::kProjKinds];    // [pf_cap][pf_ld[kind]] GEMM outputs
    uint32_t pf_ld[vx::kProjKinds];
    uint16_t* pf_q;                   // [pf_cap][n_heads * head_dim] rotated f16 queries
    float* pf_att;                    // [pf_cap][n_heads * head_dim] attention outputs
    float* pf_act;                    // [pf_cap][ffn] gated activations
    uint8_t* pf_staged;               // the GEMM's staged activations
    uint8_t* pf_part;                 // the GEMM's K-slice partial sums
    struct PfGraph {
        uint32_t n;
        bool head;
        hipGraph_t graph;
        hipGraphExec_t exec;
    };
    std::vector<PfGraph> pf_graphs;
    vx::Ctl* h_ctl;                   // pinned
    hipStream_t stream;
    hipGraph_t graph;                 // the decode step; graph_short: the same for positions below kShortCtx
    hipGraphExec_t exec;
    hipGraph_t graph_short;
    hipGraphExec_t exec_short;
    bool ready;
    size_t bytes;
    mutable std::mutex mu;  // serialises the calls that launch work or read the KV cache
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
    if (d->exec_short) (void)hipGraphExecDestroy(d->exec_short);
    if (d->graph_short) (void)hipGraphDestroy(d->graph_short);
    d->exec = nullptr;
    d->graph = nullptr;
    d->exec_short = nullptr;
    d->graph_short = nullptr;
    d->ready = false;
    for (auto& g : d->pf_graphs) {
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
        if (g.graph) (void)hipGraphDestroy(g.graph);
    }
    d->pf_graphs.clear();
}

static void free_prefill(vx_decoder* d) {
    void* bufs[] = {d->pf_x, d->pf_codes, d->pf_as, d->pf_q, d->pf_att, d->pf_act, d->pf_staged, d->pf_part};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    for (int32_t*& y : d->pf_y) {
        if (y) (void)hipFree(y);
        y = nullptr;
    }
    d->pf_x = nullptr;
    d->pf_codes = nullptr;
    d->pf_as = nullptr;
    d->pf_q = nullptr;
    d->pf_att = nullptr;
    d->pf_act = nullptr;
    d->pf_staged = nullptr;
    d->pf_part = nullptr;
    d->pf_cap = 0;
}

static void destroy_decoder(vx_decoder* d) {
    drop_graph(d);
    free_prefill(d);
    for (auto* m : d->proj)
        if (m) {
            m->owner = nullptr;
            (void)vx_matrix_free(m);
        }
    for (auto* p : d->norms)
        if (p) (void)hipFree(p);
    void* bufs[] = {d->d_emb, d->d_head, d->d_inter, d->d_rope,   d->d_kc,    d->d_vc,    d->d_xa,
                    d->d_xb,  d->d_att,  d->d_logits, d->d_key, d->d_ctl, d->d_prompt, d->d_tokens, d->d_amax,
                    d->d_scores, d->d_cy, d->d_cms, d->d_aticket, d->d_pacc};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    for (int32_t* b : d->d_part)
        if (b) (void)hipFree(b);
    if (d->d_as) (void)hipFree(d->d_as);
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

static bool has_sub_norms(const vx_decoder* d) { return d->cfg.no_sub_norm == 0; }

static int create_decoder(const vx_decoder_config_t* cin, vx_decoder_t** out) {
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_decoder is NULL");
    *out = nullptr;
    if (cin == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "config is NULL");
    // The first version of the struct ended at rope_theta; its switches are 0 (BitNet).
    constexpr size_t kV1Size = offsetof(vx_decoder_config_t, act);
    if (cin->struct_size != sizeof(vx_decoder_config_t) && cin->struct_size != kV1Size)
        VX_FAIL(VX_ERR_INVALID_ARGUMENT, "config.struct_size is %u, expected %zu (or %zu)", cin->struct_size,
                sizeof(vx_decoder_config_t), kV1Size);
    vx_decoder_config_t cfg{};
    std::memcpy(&cfg, cin, cin->struct_size);
    cfg.struct_size = sizeof(vx_decoder_config_t);
    const vx_decoder_config_t* c = &cfg;
    if (c->n_layers == 0 || c->n_layers > 1024) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "n_layers must be in 1..=1024");
    if (c->act > VX_ACT_SILU || c->rope_mode > VX_ROPE_NORMAL || c->no_sub_norm > 1 || c->emb_f16 > 1 || c->untied > 1)
        VX_FAIL(VX_ERR_INVALID_ARGUMENT, "act, rope_mode, no_sub_norm, emb_f16 and untied take 0 or 1");
    if (c->head_dim != 32 && c->head_dim != 64 && c->head_dim != 128 && c->head_dim != 256)
        VX_FAIL(VX_ERR_UNSUPPORTED, "head_dim %u is not supported (32, 64, 128 or 256)", c->head_dim);
    if (c->n_heads == 0 || c->n_kv_heads == 0 || c->n_heads % c->n_kv_heads)
        VX_FAIL(VX_ERR_INVALID_ARGUMENT, "n_heads (%u) must be a positive multiple of n_kv_heads (%u)", c->n_heads, c->n_kv_heads);
    if (c->max_ctx == 0 || c->max_ctx > kAttnMaxCtx) VX_FAIL(VX_ERR_UNSUPPORTED, "max_ctx must be in 1..=%u", kAttnMaxCtx);
    if (c->hidden == 0 || c->hidden % 32 || c->hidden > kNormMax)
        VX_FAIL(VX_ERR_UNSUPPORTED, "hidden must be a positive multiple of 32 up to %u", kNormMax);
    if (static_cast<size_t>(c->n_heads) * c->head_dim > kNormMax)
        VX_FAIL(VX_ERR_UNSUPPORTED, "n_heads * head_dim must be at most %u", kNormMax);
    // SiLU (and any ffn beyond kNormMax) runs gate and up as one gated pair: both matrices' chunks of a tile in one
    // workgroup (at most kStChunks), the down input then a plain vector (normed only up to kNormMax).
    const bool pair = c->act == VX_ACT_SILU || c->ffn > kNormMax;
    const size_t ffn_max = pair && c->no_sub_norm ? kPlainMax : kNormMax;
    if (c->ffn == 0 || c->ffn > ffn_max || c->ffn % 4)
        VX_FAIL(VX_ERR_UNSUPPORTED, "ffn must be a multiple of 4 in 1..=%zu for this architecture", ffn_max);
    if (pair && 2 * device_row_bytes(c->hidden) / kChunk > kStChunks)
        VX_FAIL(VX_ERR_UNSUPPORTED, "hidden %u is too wide for the gated gate/up pair (SiLU)", c->hidden);
    if (c->vocab == 0 || c->vocab > (1u << 24)) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "vocab must be in 1..=2^24");
    if (!(c->rms_eps >= 0.0f) || !(c->rope_theta > 0.0f)) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "rms_eps must be >= 0 and rope_theta > 0");
    DeviceInfo di;
    VX_TRY(device_info(&di));
    vx_decoder* d = new vx_decoder();
    d->magic = kDecoderMagic;
    d->device = di.device;
    d->num_cus = di.num_cus;
    d->cfg = *c;
    d->pair = pair;
    d->qd = static_cast<size_t>(c->n_heads) * c->head_dim;
    d->kvd = static_cast<size_t>(c->n_kv_heads) * c->head_dim;
    d->proj.assign(static_cast<size_t>(c->n_layers) * kProjKinds, nullptr);
    d->norms.assign(static_cast<size_t>(c->n_layers + 1) * kNormKinds, nullptr);
    d->norm_set.assign(d->norms.size(), 0);
    const size_t L = c->n_layers, H = c->hidden;
    // K [layer][kv_head][max_ctx][head_dim]; V in tiles of 8 positions, [layer][kv_head][vstride / 8][head_dim][8]
    const size_t kv_elems = L * d->kvd * c->max_ctx;
    const size_t v_elems = L * d->kvd * vstride_of(c->max_ctx);
    hipError_t e = dalloc(d, &d->d_emb, static_cast<size_t>(c->vocab) * H * 2);
    if (e == hipSuccess && c->untied) e = dalloc(d, &d->d_head, static_cast<size_t>(c->vocab) * H * 2);
    if (e == hipSuccess && pair) e = dalloc(d, &d->d_inter, round_up(c->ffn, kTileRows) * 4);
    if (e == hipSuccess && pair) e = dalloc(d, &d->d_amax, static_cast<size_t>(c->n_layers) * 4);
    if (e == hipSuccess && pair) e = hipMemset(d->d_amax, 0, static_cast<size_t>(c->n_layers) * 4);
    const size_t pair_tiles = round_up(c->ffn, kTileRows) / kTileRows;
    if (e == hipSuccess && pair) e = dalloc(d, &d->d_pacc, pair_tiles * (128 + 1) * 4);
    if (e == hipSuccess && pair) e = hipMemset(d->d_pacc, 0, pair_tiles * (128 + 1) * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_rope, static_cast<size_t>(c->max_ctx) * c->head_dim * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_kc, kv_elems * 2);
    if (e == hipSuccess) e = dalloc(d, &d->d_vc, v_elems * 2);
    if (e == hipSuccess) e = dalloc(d, &d->d_xa, H * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_xb, H * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_att, d->qd * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_logits, static_cast<size_t>(c->vocab) * 4);
    const size_t n_sl = static_cast<size_t>(c->n_heads) * attn_slices(c->head_dim);
    if (e == hipSuccess) e = dalloc(d, &d->d_scores, static_cast<size_t>(c->n_heads) * c->max_ctx * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_cy, d->qd * 4 * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_cms, n_sl * 8 * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_aticket, n_sl * 4);
    if (e == hipSuccess) e = hipMemset(d->d_aticket, 0, n_sl * 4);
    if (e == hipSuccess) e = dalloc(d, &d->d_as, kStages * sizeof(float));
    if (e == hipSuccess) e = dalloc(d, &d->d_key, 16);
    if (e == hipSuccess) e = hipMemset(d->d_key, 0, 16);
    if (e == hipSuccess) d->d_ticket = reinterpret_cast<uint32_t*>(d->d_key + 1);
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

static StageInput stage_input(const vx_decoder* d, uint32_t kind, size_t n, const float* x_in, float* x_out,
                              const float* gamma) {
    StageInput p{};
    p.kind = kind;
    p.n = static_cast<uint32_t>(n);
    p.x_in = x_in;
    p.x_out = x_out;
    p.gamma = gamma;
    p.eps = d->cfg.rms_eps;
    p.emb_f16 = d->cfg.emb_f16;
    return p;
}

static const int kStageKinds[kStages][kMaxStageJobs] = {{VX_PROJ_Q, VX_PROJ_K, VX_PROJ_V}, {VX_PROJ_O, -1, -1},
                                                       {VX_PROJ_GATE, VX_PROJ_UP, -1}, {VX_PROJ_DOWN, -1, -1}};
static int stage_of(int kind) {
    for (int s = 0; s < kStages; ++s)
        for (int k : kStageKinds[s])
            if (k == kind) return s;
    return 0;
}

// Projection `kind` of `layer` as its consumers read it.
static ProjOut proj_out(const vx_decoder* d, size_t layer, int kind) {
    const vx_matrix* m = d->proj[layer * kProjKinds + kind];
    ProjOut o{};
    o.part = d->d_part[kind];
    o.as = d->d_as + stage_of(kind);
    o.ws = m->weight_scale;
    o.kslices = 1;  // the producer's K slices add up in the one array
    o.stride = static_cast<uint32_t>(m->g.padded_rows);
    return o;
}

// K slices of a projection of n_chunks chunks per row: about one work item per CU for the stage's `tiles` tiles,
// at most `limit` (what its consumers read), and short enough for the staged slice: a slice of q chunks spans at most
// (ceil(q / 2) + 1) 160 input elements, which must fit the kNormMax window, and 16 waves x kDPer chunks.
static uint32_t plan_kslices(uint32_t n_chunks, uint32_t tiles, uint32_t limit, int num_cus, bool* ok) {
    constexpr uint32_t kMaxSliceChunks = 2 * (kNormMax / 160 - 1);  // 100
    static_assert(kMaxSliceChunks <= kStChunks, "a slice's entries fit in LDS");
    uint32_t ks = (static_cast<uint32_t>(num_cus) + tiles / 2) / tiles;
    ks = std::max(1u, std::min({ks, limit, n_chunks}));
    ks = std::max(ks, (n_chunks + kMaxSliceChunks - 1) / kMaxSliceChunks);
    const uint32_t sc = (n_chunks + ks - 1) / ks;
    *ok = ks <= limit && sc <= kMaxSliceChunks;
    return (n_chunks + sc - 1) / sc;
}

static uint32_t input_variant(const StageInput& in) {
    if (in.n <= 4u * kNT) return kDv4K;
    if (in.n <= 8u * kNT) return kDv8K;
    return kDvPlain;  // create_decoder admits only plain, unnormed inputs beyond kNormMax
}

// The accumulators stage s clears once it is done: a projection split into K slices adds them atomically into one
// zeroed array, so its array is cleared by a stage that runs after all of its consumers and before its producer runs
// again. q, k, v (read by the attention) and down (read by the next layer's q/k/v stage, or by the head after the last
// layer) are cleared by the o stage; o (read by the FFN stage) by the down stage; a ReLU^2 model's separate gate and up
// (read by the down stage) by the next q/k/v stage (the next step's first one after the last layer).
static void clear_after(const vx_decoder* d, int s, DStageArgs& a) {
    uint32_t n = 0;
    auto add = [&](int kind) {
        if (d->kslices[kind] <= 1 || d->d_part[kind] == nullptr) return;  // one slice: the producer stores its sums
        a.clear[n] = d->d_part[kind];
        a.clear_words[n] = static_cast<uint32_t>(d->proj[kind]->g.padded_rows);
        ++n;
    };
    if (s == 0 && !d->pair) {
        add(VX_PROJ_GATE);
        add(VX_PROJ_UP);
    } else if (s == 1) {
        add(VX_PROJ_Q);
        add(VX_PROJ_K);
        add(VX_PROJ_V);
        add(VX_PROJ_DOWN);
    } else if (s == 3) {
        add(VX_PROJ_O);
    }
}

// The stage launches of every layer. A stage's work items are (64-row tile, K slice) pairs of its projections; the K
// split gives each stage about one item per CU (a 2560-row projection has only 40 tiles). A gated pair (gate and up
// with SiLU) is one job of one slice whose items cover a tile of both matrices.
static int build_stages(vx_decoder* d) {
    const size_t L = d->cfg.n_layers, H = d->cfg.hidden, F = d->cfg.ffn;
    const bool sub = has_sub_norms(d);
    for (int s = 0; s < kStages; ++s) {
        if (s == 2 && d->pair) continue;  // one slice, no partials
        uint32_t tiles = 0;
        for (int k : kStageKinds[s])
            if (k >= 0) tiles += static_cast<uint32_t>(d->proj[k]->g.n_tiles);
        const uint32_t limit = s == 2 ? kMaxSlicesB : kMaxSlicesA;
        for (int k : kStageKinds[s]) {
            if (k < 0) continue;
            const Geometry& g = d->proj[k]->g;
            bool ok = false;
            d->kslices[k] = plan_kslices(static_cast<uint32_t>(g.n_chunks), tiles, limit, d->num_cus, &ok);
            if (!ok) VX_FAIL(VX_ERR_UNSUPPORTED, "projection %d has too many chunks per row (%zu)", k, g.n_chunks);
            if (d->d_part[k]) (void)hipFree(d->d_part[k]);
            d->d_part[k] = nullptr;
            // one int32 per row: the K slices add their sums atomically (zero before the producing stage: the stages
            // after its consumers clear it, see clear_after)
            VX_HIP(hipMalloc(&d->d_part[k], g.padded_rows * 4));
            VX_HIP(hipMemset(d->d_part[k], 0, g.padded_rows * 4));
        }
    }
    d->stages.assign(L * kStages, DStageArgs{});
    for (size_t l = 0; l < L; ++l) {
        const float* const* nw = d->norms.data() + l * kNormKinds;
        for (int s = 0; s < kStages; ++s) {
            DStageArgs& a = d->stages[l * kStages + s];
            uint32_t items = 0;
            if (s == 2 && d->pair) {
                const vx_matrix* mg = d->proj[l * kProjKinds + VX_PROJ_GATE];
                const vx_matrix* mu = d->proj[l * kProjKinds + VX_PROJ_UP];
                DJob& j = a.job[a.n_jobs++];
                j.w = mg->d_w;
                j.dsum = mg->d_dsum;
                j.w2 = mu->d_w;
                j.dsum2 = mu->d_dsum;
                j.w_bytes = static_cast<uint32_t>(mg->g.device_bytes);
                if (mg->g.device_bytes >= kBufferOutOfRange || mu->g.device_bytes != mg->g.device_bytes)
                    VX_FAIL(VX_ERR_UNSUPPORTED, "gate/up matrices of %zu and %zu bytes", mg->g.device_bytes, mu->g.device_bytes);
                j.act_out = d->d_inter;
                j.amax_out = sub ? nullptr : d->d_amax + l;
                j.ws = mg->weight_scale;
                j.ws2 = mu->weight_scale;
                j.act = d->cfg.act == VX_ACT_SILU ? kActSilu : kActRelu2;
                j.n8 = static_cast<uint32_t>(F / 8 * 8);
                j.rows = static_cast<uint32_t>(mg->g.rows);
                j.padded_rows = static_cast<uint32_t>(mg->g.padded_rows);
                j.n_tiles = static_cast<uint32_t>(mg->g.n_tiles);
                j.n_chunks = static_cast<uint32_t>(mg->g.n_chunks);
                j.kslices = 1;
                j.slice_chunks = j.n_chunks;
                items = j.n_tiles;
                // Equal chunk ranges over one workgroup per CU when every range is non-empty, fits 16 waves x kDPer
                // chunks and meets at most kRangeSegs tiles; else one or two tiles per workgroup.
                const uint64_t C = static_cast<uint64_t>(j.n_tiles) * 2u * j.n_chunks, G = static_cast<uint64_t>(d->num_cus);
                if (C >= G && (C + G - 1) / G <= static_cast<uint64_t>(kTileGroup * kDPer) &&
                    2u * j.n_chunks >= static_cast<uint32_t>(8 * kDPer) && j.n_tiles > G &&
                    range_fields_fit(j.n_chunks, C, G)) {
                    a.range_chunks = static_cast<uint32_t>(C);
                    j.accum = reinterpret_cast<unsigned long long*>(d->d_pacc);
                }
            } else {
                for (int k : kStageKinds[s]) {
                    if (k < 0) continue;
                    const vx_matrix* m = d->proj[l * kProjKinds + k];
                    DJob& j = a.job[a.n_jobs++];
                    j.w = m->d_w;
                    j.dsum = m->d_dsum;
                    j.part = d->d_part[k];
                    j.w_bytes = static_cast<uint32_t>(m->g.device_bytes);
                    if (m->g.device_bytes >= kBufferOutOfRange)
                        VX_FAIL(VX_ERR_UNSUPPORTED, "a projection of %zu bytes (at most 2 GiB)", m->g.device_bytes);
                    j.rows = static_cast<uint32_t>(m->g.rows);
                    j.padded_rows = static_cast<uint32_t>(m->g.padded_rows);
                    j.n_tiles = static_cast<uint32_t>(m->g.n_tiles);
                    j.n_chunks = static_cast<uint32_t>(m->g.n_chunks);
                    j.kslices = d->kslices[k];
                    j.slice_chunks = (j.n_chunks + j.kslices - 1) / j.kslices;
                    j.item_begin = items;
                    items += j.n_tiles * j.kslices;
                }
            }
            a.total_items = items;
            // A stage whose jobs have one K slice each and more items than CUs gives a workgroup two items.
            bool one_slice = true;
            for (uint32_t jj = 0; jj < a.n_jobs; ++jj) one_slice = one_slice && a.job[jj].kslices == 1;
            a.loop = one_slice && items > static_cast<uint32_t>(d->num_cus) && a.range_chunks == 0 ? 1u : 0u;
            a.grid = a.loop ? std::max(static_cast<uint32_t>(d->num_cus), (items + 1u) / 2u) : items;
            if (a.range_chunks != 0) a.grid = static_cast<uint32_t>(d->num_cus);
            // chunks per wave of the largest item (a pair's gate and up chunks count together): the instance loads
            // 1, 4 or kDPer
            uint32_t most = 0;
            for (uint32_t jj = 0; jj < a.n_jobs; ++jj) {
                const uint32_t nl = a.job[jj].w2 != nullptr ? 2u * a.job[jj].slice_chunks : a.job[jj].slice_chunks;
                most = std::max(most, (nl + kTileGroup - 1u) / kTileGroup);
            }
            if (most > static_cast<uint32_t>(kDPer))
                VX_FAIL(VX_ERR_INTERNAL, "stage %d with %u chunks per wave (at most %d)", s, most, kDPer);
            a.dper = most <= 1u ? 1u : (most <= 4u ? 4u : static_cast<uint32_t>(kDPer));
            if (a.range_chunks != 0) a.dper = static_cast<uint32_t>(kDPer);
            StageInput& in = a.in;
            if (s == 0 && l == 0) {  // embedding -> attention norm
                in = stage_input(d, kInEmbed, H, nullptr, d->d_xa, nw[VX_NORM_ATTN]);
                in.ctl = d->d_ctl;
                in.prompt = d->d_prompt;
                in.emb = d->d_emb;
            } else if (s == 0) {  // x + down of the previous layer -> attention norm
                in = stage_input(d, kInResidual, H, d->d_xb, d->d_xa, nw[VX_NORM_ATTN]);
                in.a = proj_out(d, l - 1, VX_PROJ_DOWN);
            } else if (s == 1) {  // attention output -> attention sub-norm (or none)
                in = stage_input(d, kInPlain, d->qd, d->d_att, nullptr, sub ? nw[VX_NORM_ATTN_SUB] : nullptr);
                // the o stage runs after the previous step's down stage and before this step's pair: it clears the
                // layer's maximum
                if (d->pair && !sub) a.amax_clear = d->d_amax + l;
            } else if (s == 2) {  // x + o -> FFN norm
                in = stage_input(d, kInResidual, H, d->d_xa, d->d_xb, nw[VX_NORM_FFN]);
                in.a = proj_out(d, l, VX_PROJ_O);
            } else if (d->pair) {  // act(gate, up) from the pair -> FFN sub-norm (or none)
                in = stage_input(d, kInPlain, F, d->d_inter, nullptr, sub ? nw[VX_NORM_FFN_SUB] : nullptr);
                if (!sub) in.amax = d->d_amax + l;
            } else {  // relu2(gate) * up -> FFN sub-norm (or none)
                in = stage_input(d, kInRelu2Mul, F, nullptr, nullptr, sub ? nw[VX_NORM_FFN_SUB] : nullptr);
                in.a = proj_out(d, l, VX_PROJ_GATE);
                in.b = proj_out(d, l, VX_PROJ_UP);
            }
            a.tbr = static_cast<uint32_t>(tile_row_bytes(in.n));
            a.as_out = d->d_as + s;
            a.variant = input_variant(in);
            clear_after(d, s, a);
            if (a.variant == kDvPlain && (in.kind != kInPlain || in.gamma != nullptr))
                VX_FAIL(VX_ERR_INTERNAL, "stage %d input of %u elements needs a norm", s, in.n);
        }
    }
    return VX_OK;
}

// Enqueues one decode step on `st` (also the sequence captured into the step graph).
static int record_step(const vx_decoder* d, hipStream_t st, bool short_ctx) {
    const vx_decoder_config_t& c = d->cfg;
    const size_t L = c.n_layers;
    const size_t layer_kv = d->kvd * c.max_ctx, layer_v = d->kvd * vstride_of(c.max_ctx);
    for (size_t l = 0; l < L; ++l) {
        VX_TRY(launch_dgemv(d->stages[l * kStages + 0], st));
        AttnArgs at{};
        at.ctl = d->d_ctl;
        at.q = proj_out(d, l, VX_PROJ_Q);
        at.k = proj_out(d, l, VX_PROJ_K);
        at.v = proj_out(d, l, VX_PROJ_V);
        at.rope = d->d_rope;
        at.kc = d->d_kc + l * layer_kv;
        at.vc = d->d_vc + l * layer_v;
        at.vstride = vstride_of(c.max_ctx);
        at.out = d->d_att;
        at.n_heads = c.n_heads;
        at.gqa = c.n_heads / c.n_kv_heads;
        at.max_ctx = c.max_ctx;
        at.rope_normal = c.rope_mode == VX_ROPE_NORMAL ? 1u : 0u;
        at.scale = 1.0f / sqrtf(static_cast<float>(c.head_dim));
        at.scores = d->d_scores;
        at.cy = d->d_cy;
        at.cms = d->d_cms;
        at.ticket = d->d_aticket;
        VX_TRY(short_ctx ? launch_attention_short(at, c.head_dim, st) : launch_attention(at, c.head_dim, st));
        for (int s = 1; s < kStages; ++s) VX_TRY(launch_dgemv(d->stages[l * kStages + s], st));
    }
    HeadArgs h{};
    h.in = stage_input(d, kInResidual, c.hidden, d->d_xb, nullptr, d->norms[L * kNormKinds]);
    h.in.a = proj_out(d, L - 1, VX_PROJ_DOWN);
    h.w = c.untied ? d->d_head : d->d_emb;
    h.hidden = c.hidden;
    h.vocab = c.vocab;
    h.logits = d->d_logits;
    h.ctl = d->d_ctl;
    h.out_tokens = d->d_tokens;
    h.key = d->d_key;
    h.ticket = d->d_ticket;
    // One workgroup per CU (its registers allow one), each computing the normed vector once and looping over blocks
    // of kNT / 4 rows.
    const uint32_t rows_per_wg = kNT / 4;
    const uint32_t grid = std::min<uint32_t>((c.vocab + rows_per_wg - 1) / rows_per_wg, static_cast<uint32_t>(d->num_cus));
    return launch_head(h, c.emb_f16 != 0, grid, st);
}

// ---- prefill ---------------------------------------------------------------------------------------------------------------

constexpr uint32_t kPrefillChunk = 512;  // tokens per prefill pass; longer prompts run in several

// The prefill buffers, sized for chunks of pf_cap tokens (allocated on the first prefill).
static int ensure_prefill(vx_decoder* d) {
    if (d->pf_cap) return VX_OK;
    const vx_decoder_config_t& c = d->cfg;
    const uint32_t cap = std::min<uint32_t>(kPrefillChunk, c.max_ctx);
    const size_t widest = std::max({static_cast<size_t>(c.hidden), d->qd, static_cast<size_t>(c.ffn)});
    d->pf_codes_ld = static_cast<uint32_t>(round_up(widest, 16));
    size_t stage_bytes = 0, part_bytes = 0;
    for (size_t cols : {static_cast<size_t>(c.hidden), d->qd, static_cast<size_t>(c.ffn)})
        stage_bytes = std::max(stage_bytes, gemm_stage_bytes(cols, cap));
    for (int k = 0; k < kProjKinds; ++k) {
        const Geometry& g = d->proj[k]->g;  // every layer's projection k has this shape
        for (uint32_t m = 1; m <= cap; ++m) part_bytes = std::max(part_bytes, gemm_part_bytes(g, m, d->num_cus));
    }
    {  // q, k and v, and gate and up, in one launch each (record_prefill)
        GemmSub qkv[3], gu[2];
        for (int k = 0; k < 3; ++k) qkv[k] = GemmSub{nullptr, &d->proj[VX_PROJ_Q + k]->g, nullptr, 0};
        for (int k = 0; k < 2; ++k) gu[k] = GemmSub{nullptr, &d->proj[VX_PROJ_GATE + k]->g, nullptr, 0};
        for (uint32_t m = 1; m <= cap; ++m) {
            if (gemm_group_small_path(qkv, 3, m, d->num_cus))
                part_bytes = std::max(part_bytes, gemm_group_part_bytes(qkv, 3, m, d->num_cus));
            if (gemm_group_small_path(gu, 2, m, d->num_cus))
                part_bytes = std::max(part_bytes, gemm_group_part_bytes(gu, 2, m, d->num_cus));
        }
    }
    hipError_t e = hipSuccess;
    auto grab = [&](auto** p, size_t bytes) {
        if (e == hipSuccess) e = dalloc(d, p, std::max<size_t>(bytes, 256));
    };
    grab(&d->pf_x, static_cast<size_t>(cap) * c.hidden * 4);
    grab(&d->pf_codes, static_cast<size_t>(cap) * d->pf_codes_ld);
    grab(&d->pf_as, 4u * cap * 4);
    for (int k = 0; k < kProjKinds; ++k) {
        d->pf_ld[k] = static_cast<uint32_t>(round_up(proj_rows(d, k), 4));
        grab(&d->pf_y[k], static_cast<size_t>(cap) * d->pf_ld[k] * 4);
    }
    grab(&d->pf_q, static_cast<size_t>(cap) * d->qd * 2);
    grab(&d->pf_att, static_cast<size_t>(cap) * d->qd * 4);
    grab(&d->pf_act, static_cast<size_t>(cap) * c.ffn * 4);
    grab(&d->pf_staged, stage_bytes);
    grab(&d->pf_part, part_bytes);
    if (e != hipSuccess) {
        free_prefill(d);
        VX_FAIL(VX_ERR_DEVICE, "prefill buffers: %s", hipGetErrorString(e));
    }
    d->pf_cap = cap;
    return VX_OK;
}

// The output of projection `kind` of `layer` for token 0 of a prefill (kslices 1; token t is t * pf_ld[kind] further).
static ProjOut pf_proj_out(const vx_decoder* d, size_t layer, int kind, const float* as) {
    ProjOut o{};
    o.part = d->pf_y[kind];
    o.as = as;
    o.ws = d->proj[layer * kProjKinds + kind]->weight_scale;
    o.kslices = 1;
    o.stride = d->pf_ld[kind];
    return o;
}

// Enqueues one prefill pass over n tokens (the last at the loop state's position) on `st`; with `head`, the final norm,
// head and greedy argmax of the last token follow and advance the loop state as a decode step does.
static int record_prefill(const vx_decoder* d, uint32_t n, bool head, hipStream_t st) {
    const vx_decoder_config_t& c = d->cfg;
    const size_t L = c.n_layers, H = c.hidden, F = c.ffn;
    const bool sub = has_sub_norms(d);
    const size_t layer_kv = d->kvd * c.max_ctx, layer_v = d->kvd * vstride_of(c.max_ctx);
    const uint32_t cap = d->pf_cap;
    float* as_qkv = d->pf_as;
    float* as_o = d->pf_as + cap;
    float* as_ffn = d->pf_as + 2 * cap;
    float* as_down = d->pf_as + 3 * cap;
    auto stage = [&](const StageInput& in, uint32_t x_stride, uint32_t a_stride, float* as_out) -> int {
        PfStageArgs a{};
        a.in = in;
        a.x_stride = x_stride;
        a.a_stride = a_stride;
        a.n_tok = n;
        a.prompt = d->d_prompt;
        a.codes = d->pf_codes;
        a.codes_stride = d->pf_codes_ld;
        a.as_out = as_out;
        return launch_pf_stage(a, st);
    };
    // GEMMs on the small path read the codes themselves; the others read them staged once per input
    auto small = [&](int kind) { return gemm_small_path(d->proj[kind]->g, n, d->num_cus); };
    auto gemm_stage = [&](size_t cols, std::initializer_list<int> kinds) -> int {
        bool need = false;
        for (int k : kinds) need = need || !small(k);
        return need ? launch_gemm_stage(d->pf_codes, n, d->pf_codes_ld, cols, d->pf_staged, st) : VX_OK;
    };
    auto gemm = [&](size_t layer, int kind) -> int {
        const vx_matrix* m = d->proj[layer * kProjKinds + kind];
        if (small(kind))
            return launch_gemm(m->d_w, m->g, d->num_cus, d->pf_codes, n, d->pf_codes_ld, d->pf_y[kind], d->pf_ld[kind],
                               d->pf_part, st);
        return launch_gemm_staged(m->d_w, m->g, d->num_cus, d->pf_staged, n, d->pf_y[kind], d->pf_ld[kind], d->pf_part, st);
    };
    for (size_t l = 0; l < L; ++l) {
        const float* const* nw = d->norms.data() + l * kNormKinds;
        // the attention input: the embedding or the residual of the previous layer, the attention norm
        StageInput in;
        if (l == 0) {
            in = stage_input(d, kInEmbed, H, nullptr, d->pf_x, nw[VX_NORM_ATTN]);
            in.ctl = d->d_ctl;
            in.emb = d->d_emb;
        } else {
            in = stage_input(d, kInResidual, H, d->pf_x, d->pf_x, nw[VX_NORM_ATTN]);
            in.a = pf_proj_out(d, l - 1, VX_PROJ_DOWN, as_down);
        }
        VX_TRY(stage(in, static_cast<uint32_t>(H), d->pf_ld[VX_PROJ_DOWN], as_qkv));
        // q, k and v in one small-path launch where each takes that path
        GemmSub qkv[3];
        for (int k = 0; k < 3; ++k) {
            const vx_matrix* m = d->proj[l * kProjKinds + VX_PROJ_Q + k];
            qkv[k] = GemmSub{m->d_w, &m->g, d->pf_y[VX_PROJ_Q + k], d->pf_ld[VX_PROJ_Q + k]};
        }
        if (gemm_group_small_path(qkv, 3, n, d->num_cus)) {
            VX_TRY(launch_gemm_group(qkv, 3, d->num_cus, d->pf_codes, n, d->pf_codes_ld, d->pf_part, st));
        } else {
            VX_TRY(gemm_stage(H, {VX_PROJ_Q, VX_PROJ_K, VX_PROJ_V}));
            for (int k : {VX_PROJ_Q, VX_PROJ_K, VX_PROJ_V}) VX_TRY(gemm(l, k));
        }
        PfRopeArgs ra{};
        ra.ctl = d->d_ctl;
        ra.n_tok = n;
        ra.yq = d->pf_y[VX_PROJ_Q];
        ra.yk = d->pf_y[VX_PROJ_K];
        ra.yv = d->pf_y[VX_PROJ_V];
        ra.ldq = d->pf_ld[VX_PROJ_Q];
        ra.ldk = d->pf_ld[VX_PROJ_K];
        ra.ldv = d->pf_ld[VX_PROJ_V];
        ra.as = as_qkv;
        ra.wsq = d->proj[l * kProjKinds + VX_PROJ_Q]->weight_scale;
        ra.wsk = d->proj[l * kProjKinds + VX_PROJ_K]->weight_scale;
        ra.wsv = d->proj[l * kProjKinds + VX_PROJ_V]->weight_scale;
        ra.rope = d->d_rope;
        ra.kc = d->d_kc + l * layer_kv;
        ra.vc = d->d_vc + l * layer_v;
        ra.vstride = vstride_of(c.max_ctx);
        ra.qbuf = d->pf_q;
        ra.n_heads = c.n_heads;
        ra.n_kv = c.n_kv_heads;
        ra.hd = c.head_dim;
        ra.max_ctx = c.max_ctx;
        ra.rope_normal = c.rope_mode == VX_ROPE_NORMAL ? 1u : 0u;
        const uint32_t n_elem = c.n_heads * c.head_dim / 2u + c.n_kv_heads * c.head_dim / 2u + c.n_kv_heads * c.head_dim;
        hipLaunchKernelGGL(pf_rope_kernel, dim3(n, (n_elem + 255u) / 256u), dim3(256), 0, st, ra);
        VX_HIP(hipGetLastError());
        AttnArgs at{};
        at.ctl = d->d_ctl;
        at.kc = d->d_kc + l * layer_kv;
        at.vc = d->d_vc + l * layer_v;
        at.vstride = vstride_of(c.max_ctx);
        at.out = d->pf_att;
        at.n_heads = c.n_heads;
        at.gqa = c.n_heads / c.n_kv_heads;
        at.max_ctx = c.max_ctx;
        at.rope_normal = ra.rope_normal;
        at.scale = 1.0f / sqrtf(static_cast<float>(c.head_dim));
        at.qbuf = d->pf_q;
        at.n_tok = n;
        VX_TRY(launch_attention_prefill(at, c.head_dim, st));
        // the o input: attention output (sub-norm or none)
        in = stage_input(d, kInPlain, d->qd, d->pf_att, nullptr, sub ? nw[VX_NORM_ATTN_SUB] : nullptr);
        VX_TRY(stage(in, static_cast<uint32_t>(d->qd), 0, as_o));
        VX_TRY(gemm_stage(d->qd, {VX_PROJ_O}));
        VX_TRY(gemm(l, VX_PROJ_O));
        // x + o, FFN norm
        in = stage_input(d, kInResidual, H, d->pf_x, d->pf_x, nw[VX_NORM_FFN]);
        in.a = pf_proj_out(d, l, VX_PROJ_O, as_o);
        VX_TRY(stage(in, static_cast<uint32_t>(H), d->pf_ld[VX_PROJ_O], as_ffn));
        VX_TRY(gemm_stage(H, {VX_PROJ_GATE, VX_PROJ_UP}));
        {
            // a staged gate/up pair as one launch when that needs no K split (twice the workgroups of one matrix)
            const vx_matrix* mg = d->proj[l * kProjKinds + VX_PROJ_GATE];
            const vx_matrix* mu = d->proj[l * kProjKinds + VX_PROJ_UP];
            GemmSub gu[2] = {GemmSub{mg->d_w, &mg->g, d->pf_y[VX_PROJ_GATE], d->pf_ld[VX_PROJ_GATE]},
                             GemmSub{mu->d_w, &mu->g, d->pf_y[VX_PROJ_UP], d->pf_ld[VX_PROJ_UP]}};
            if (gemm_group_small_path(gu, 2, n, d->num_cus)) {
                VX_TRY(launch_gemm_group(gu, 2, d->num_cus, d->pf_codes, n, d->pf_codes_ld, d->pf_part, st));
            } else if (!small(VX_PROJ_GATE) && !small(VX_PROJ_UP) && d->pf_ld[VX_PROJ_GATE] == d->pf_ld[VX_PROJ_UP] &&
                mg->g.rows == mu->g.rows && mg->g.cols == mu->g.cols && gemm_staged_pair_ok(mg->g, n, d->num_cus)) {
                VX_TRY(launch_gemm_staged_pair(mg->d_w, mu->d_w, mg->g, d->num_cus, d->pf_staged, n,
                                               d->pf_y[VX_PROJ_GATE], d->pf_y[VX_PROJ_UP], d->pf_ld[VX_PROJ_GATE], st));
            } else {
                VX_TRY(gemm(l, VX_PROJ_GATE));
                VX_TRY(gemm(l, VX_PROJ_UP));
            }
        }
        PfActArgs aa{};
        aa.yg = d->pf_y[VX_PROJ_GATE];
        aa.yu = d->pf_y[VX_PROJ_UP];
        aa.ld = d->pf_ld[VX_PROJ_GATE];
        aa.as = as_ffn;
        aa.wsg = d->proj[l * kProjKinds + VX_PROJ_GATE]->weight_scale;
        aa.wsu = d->proj[l * kProjKinds + VX_PROJ_UP]->weight_scale;
        aa.out = d->pf_act;
        aa.ffn = static_cast<uint32_t>(F);
        aa.n8 = static_cast<uint32_t>(F / 8 * 8);
        aa.act = c.act == VX_ACT_SILU ? kActSilu : kActRelu2;
        hipLaunchKernelGGL(pf_act_kernel, dim3(static_cast<uint32_t>((F + 255) / 256), n), dim3(256), 0, st, aa);
        VX_HIP(hipGetLastError());
        // the down input: the gated activation (sub-norm or none)
        in = stage_input(d, kInPlain, F, d->pf_act, nullptr, sub ? nw[VX_NORM_FFN_SUB] : nullptr);
        VX_TRY(stage(in, static_cast<uint32_t>(F), 0, as_down));
        VX_TRY(gemm_stage(F, {VX_PROJ_DOWN}));
        VX_TRY(gemm(l, VX_PROJ_DOWN));
    }
    if (!head) return VX_OK;
    HeadArgs h{};
    h.in = stage_input(d, kInResidual, c.hidden, d->pf_x + static_cast<size_t>(n - 1) * H, nullptr, d->norms[L * kNormKinds]);
    h.in.a = pf_proj_out(d, L - 1, VX_PROJ_DOWN, as_down + (n - 1));
    h.in.a.part = d->pf_y[VX_PROJ_DOWN] + static_cast<size_t>(n - 1) * d->pf_ld[VX_PROJ_DOWN];
    h.w = c.untied ? d->d_head : d->d_emb;
    h.hidden = c.hidden;
    h.vocab = c.vocab;
    h.logits = d->d_logits;
    h.ctl = d->d_ctl;
    h.out_tokens = d->d_tokens;
    h.key = d->d_key;
    h.ticket = d->d_ticket;
    const uint32_t rows_per_wg = kNT / 4;
    const uint32_t grid = std::min<uint32_t>((c.vocab + rows_per_wg - 1) / rows_per_wg, static_cast<uint32_t>(d->num_cus));
    return launch_head(h, c.emb_f16 != 0, grid, st);
}

// The graph of a prefill pass over n tokens (recorded on first use; a few are kept).
static int prefill_graph(vx_decoder* d, uint32_t n, bool head, hipGraphExec_t* out) {
    for (const auto& g : d->pf_graphs)
        if (g.n == n && g.head == head) {
            *out = g.exec;
            return VX_OK;
        }
    if (d->pf_graphs.size() >= 4) {
        auto& g = d->pf_graphs.front();
        (void)hipGraphExecDestroy(g.exec);
        (void)hipGraphDestroy(g.graph);
        d->pf_graphs.erase(d->pf_graphs.begin());
    }
    VX_HIP(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
    const int st = record_prefill(d, n, head, d->stream);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(d->stream, &graph);
    if (st != VX_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return st;
    }
    VX_HIP(e);
    hipGraphExec_t exec = nullptr;
    const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (ei != hipSuccess) {
        (void)hipGraphDestroy(graph);
        VX_HIP(ei);
    }
    d->pf_graphs.push_back({n, head, graph, exec});
    *out = exec;
    return VX_OK;
}

// Prefills positions pos0 .. pos0 + n - 1 with the tokens already in d_prompt at those positions, in chunks of pf_cap;
// the last chunk ends with the head (greedy token and logits of the last position). n_prompt and n_out are the loop
// state's (the head records the token generated after position n_prompt - 1 as out_tokens[0]).
static int run_prefill(vx_decoder* d, uint32_t pos0, uint32_t n, uint32_t n_prompt, uint32_t n_out) {
    VX_TRY(ensure_prefill(d));
    for (uint32_t done = 0; done < n;) {
        const uint32_t m = std::min(d->pf_cap, n - done);
        const bool last = done + m == n;
        hipGraphExec_t exec = nullptr;
        VX_TRY(prefill_graph(d, m, last, &exec));
        hipLaunchKernelGGL(set_ctl_kernel, dim3(1), dim3(64), 0, d->stream, d->d_ctl, pos0 + done + m - 1, 0u, n_prompt, n_out);
        VX_HIP(hipGetLastError());
        VX_HIP(hipGraphLaunch(exec, d->stream));
        done += m;
    }
    return VX_OK;
}

static bool norm_needed(const vx_decoder* d, size_t layer, int kind) {
    if (layer == d->cfg.n_layers) return kind == VX_NORM_ATTN;
    return has_sub_norms(d) || (kind != VX_NORM_ATTN_SUB && kind != VX_NORM_FFN_SUB);
}

// Builds the stage launches and captures the step graph once every weight is set.
static int prepare(vx_decoder* d) {
    if (d->ready) return VX_OK;
    const size_t L = d->cfg.n_layers;
    for (size_t i = 0; i < L * kProjKinds; ++i)
        if (!d->proj[i]) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "projection %zu of layer %zu is not set", i % kProjKinds, i / kProjKinds);
    for (size_t l = 0; l <= L; ++l)
        for (int k = 0; k < kNormKinds; ++k)
            if (norm_needed(d, l, k) && !d->norm_set[l * kNormKinds + k])
                VX_FAIL(VX_ERR_INVALID_ARGUMENT, "norm %d of layer %zu is not set", k, l);
    if (!d->emb_set) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the embedding is not set");
    if (d->cfg.untied && !d->head_set) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the head is not set");
    drop_graph(d);
    VX_TRY(build_stages(d));
    for (int form = 0; form < 2; ++form) {  // 0: any position, 1: positions below kShortCtx
        VX_HIP(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
        const int st = record_step(d, d->stream, form == 1);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(d->stream, &g);
        if (st != VX_OK) {
            if (g) (void)hipGraphDestroy(g);
            return st;
        }
        VX_HIP(e);
        (form == 0 ? d->graph : d->graph_short) = g;
        VX_HIP(hipGraphInstantiate(form == 0 ? &d->exec : &d->exec_short, g, nullptr, nullptr, 0));
    }
    d->ready = true;
    return VX_OK;
}

// The step graph for position pos (the short-context attention below kShortCtx).
static hipGraphExec_t step_exec(const vx_decoder* d, size_t pos) { return pos < kShortCtx ? d->exec_short : d->exec; }

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
        m->owner = d;
        vx_matrix_t*& slot = d->proj[static_cast<size_t>(layer) * kProjKinds + kind];
        if (slot) {
            slot->owner = nullptr;
            (void)vx_matrix_free(slot);
        }
        slot = m;
        drop_graph(d);
        return VX_OK;
    });
}

int vx_decoder_adopt_projection(vx_decoder_t* d, uint32_t layer, uint32_t kind, vx_matrix_t* m) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        std::lock_guard<std::mutex> lk(d->mu);
        if (layer >= d->cfg.n_layers) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "layer %u out of range (n_layers %u)", layer, d->cfg.n_layers);
        if (kind >= static_cast<uint32_t>(kProjKinds)) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "projection kind %u is not 0..6", kind);
        if (m == nullptr || m->magic != kMatrixMagic) VX_FAIL(VX_ERR_INVALID_HANDLE, "matrix handle is not valid");
        if (m->kind != kKindVelurex) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "a Q2_0 matrix cannot be a decoder projection");
        if (m->device != d->device) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the matrix is on device %d, the decoder on %d", m->device, d->device);
        if (m->g.rows != proj_rows(d, kind) || m->g.cols != proj_cols(d, kind))
            VX_FAIL(VX_ERR_INVALID_SHAPE, "projection %u is %zu x %zu, the matrix %zu x %zu", kind, proj_rows(d, kind),
                    proj_cols(d, kind), m->g.rows, m->g.cols);
        vx_matrix_t*& slot = d->proj[static_cast<size_t>(layer) * kProjKinds + kind];
        if (slot == m) return VX_OK;
        // one owner per matrix: a handle already held by a slot (of this or another decoder) would be freed twice
        if (m->owner != nullptr) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the matrix already belongs to a decoder");
        if (slot) {
            slot->owner = nullptr;
            (void)vx_matrix_free(slot);
        }
        m->owner = d;
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
        if (kind >= static_cast<uint32_t>(kNormKinds) || !norm_needed(d, layer, static_cast<int>(kind)))
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "norm kind %u is not valid for layer %u of this model", kind, layer);
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

// The embedding (head = false) or the untied head, vocab x hidden 16-bit values of the type the config names.
static int set_table(vx_decoder_t* d, const uint16_t* src, size_t n, bool head, bool f16) {
    VX_TRY(check_decoder(d));
    std::lock_guard<std::mutex> lk(d->mu);
    const char* what = head ? "head" : "embedding";
    if (src == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "%s is NULL", what);
    if (head && !d->cfg.untied) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the model's head is its embedding (untied = 0)");
    if (f16 != (d->cfg.emb_f16 != 0))
        VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the model's %s holds %s values", what, d->cfg.emb_f16 ? "f16" : "bf16");
    const size_t need = static_cast<size_t>(d->cfg.vocab) * d->cfg.hidden;
    if (n != need) VX_FAIL(VX_ERR_INVALID_SHAPE, "the %s has %zu values, expected vocab * hidden = %zu", what, n, need);
    VX_TRY(set_device(d->device));
    VX_HIP(hipMemcpy(head ? d->d_head : d->d_emb, src, need * 2, hipMemcpyHostToDevice));
    (head ? d->head_set : d->emb_set) = true;
    return VX_OK;
}

int vx_decoder_set_embedding_bf16(vx_decoder_t* d, const uint16_t* embedding, size_t n) {
    return guard([&]() -> int { return set_table(d, embedding, n, false, false); });
}

int vx_decoder_set_embedding_f16(vx_decoder_t* d, const uint16_t* embedding, size_t n) {
    return guard([&]() -> int { return set_table(d, embedding, n, false, true); });
}

int vx_decoder_set_head(vx_decoder_t* d, const uint16_t* head, size_t n) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        return set_table(d, head, n, true, d->cfg.emb_f16 != 0);
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
        VX_HIP(hipGraphLaunch(step_exec(d, pos), d->stream));
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
        // the prompt in prefill passes (their last head gives the first new token), then one step per further token
        VX_TRY(run_prefill(d, 0, static_cast<uint32_t>(n_prompt), static_cast<uint32_t>(n_prompt), static_cast<uint32_t>(n_new)));
        for (size_t i = n_prompt; i < steps; ++i) VX_HIP(hipGraphLaunch(step_exec(d, i), d->stream));
        VX_HIP(hipStreamSynchronize(d->stream));
        if (n_new) VX_HIP(hipMemcpy(out_tokens, d->d_tokens, n_new * 4, hipMemcpyDeviceToHost));
        return VX_OK;
    });
}

int vx_decoder_generate_stepwise(vx_decoder_t* d, const uint32_t* prompt, size_t n_prompt, size_t n_new,
                                 uint32_t* out_tokens, size_t out_capacity) {
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
        for (size_t i = 0; i < steps; ++i) VX_HIP(hipGraphLaunch(step_exec(d, i), d->stream));
        VX_HIP(hipStreamSynchronize(d->stream));
        if (n_new) VX_HIP(hipMemcpy(out_tokens, d->d_tokens, n_new * 4, hipMemcpyDeviceToHost));
        return VX_OK;
    });
}

int vx_decoder_prefill(vx_decoder_t* d, const uint32_t* tokens, size_t n, uint32_t pos0, float* logits,
                       size_t logits_capacity, uint32_t* out_next) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        std::lock_guard<std::mutex> lk(d->mu);
        if (n == 0) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "no tokens to prefill");
        if (tokens == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "tokens is NULL");
        if (pos0 > d->cfg.max_ctx || n > d->cfg.max_ctx - pos0)
            VX_FAIL(VX_ERR_CONTEXT_OVERFLOW, "positions %u .. %zu exceed the context of %u", pos0, pos0 + n - 1, d->cfg.max_ctx);
        if (logits && logits_capacity < d->cfg.vocab)
            VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "logits hold %zu values but vocab = %u", logits_capacity, d->cfg.vocab);
        for (size_t i = 0; i < n; ++i)
            if (tokens[i] >= d->cfg.vocab) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "tokens[%zu] = %u out of range (vocab %u)", i, tokens[i], d->cfg.vocab);
        VX_TRY(set_device(d->device));
        VX_TRY(prepare(d));
        VX_HIP(hipMemcpy(d->d_prompt + pos0, tokens, n * 4, hipMemcpyHostToDevice));
        // n_prompt beyond every position: the head records no generated token
        VX_TRY(run_prefill(d, pos0, static_cast<uint32_t>(n), 0xffffffffu, 0u));
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

int vx_decoder_kv_get(const vx_decoder_t* d, uint32_t layer, uint32_t pos, uint32_t kv_head, uint16_t* k, uint16_t* v,
                      size_t n) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        if (layer >= d->cfg.n_layers || pos >= d->cfg.max_ctx || kv_head >= d->cfg.n_kv_heads)
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "layer %u / pos %u / kv_head %u out of range", layer, pos, kv_head);
        if (n < d->cfg.head_dim) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "k and v hold %zu values, head_dim is %u", n, d->cfg.head_dim);
        const size_t hd = d->cfg.head_dim, vs = vstride_of(d->cfg.max_ctx);
        const size_t off = (static_cast<size_t>(layer) * d->kvd * d->cfg.max_ctx) +
                           (static_cast<size_t>(kv_head) * d->cfg.max_ctx + pos) * hd;
        const size_t voff = static_cast<size_t>(layer) * d->kvd * vs + static_cast<size_t>(kv_head) * hd * vs +
                            (static_cast<size_t>(pos / 8) * hd) * 8 + pos % 8;
        std::lock_guard<std::mutex> lk(d->mu);  // no step or prefill is half way through the cache meanwhile
        VX_TRY(set_device(d->device));
        VX_HIP(hipStreamSynchronize(d->stream));
        if (k) VX_HIP(hipMemcpy(k, d->d_kc + off, hd * 2, hipMemcpyDeviceToHost));
        // V is cached in tiles of 8 positions: the position's values are 8 elements apart
        if (v) VX_HIP(hipMemcpy2D(v, 2, d->d_vc + voff, 16, 2, hd, hipMemcpyDeviceToHost));
        return VX_OK;
    });
}

int vx_decoder_norm_fallbacks(const vx_decoder_t* d, uint64_t* out_count) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        if (out_count == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_count is NULL");
        std::lock_guard<std::mutex> lk(d->mu);
        VX_TRY(set_device(d->device));
        VX_HIP(hipStreamSynchronize(d->stream));
        unsigned int c = 0;
        VX_HIP(hipMemcpyFromSymbol(&c, HIP_SYMBOL(g_norm_fallbacks), sizeof(c), 0, hipMemcpyDeviceToHost));
        *out_count = c;
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

int vx_decoder_config(const vx_decoder_t* d, vx_decoder_config_t* out_config) {
    return guard([&]() -> int {
        VX_TRY(check_decoder(d));
        if (out_config == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_config is NULL");
        if (out_config->struct_size != sizeof(vx_decoder_config_t))
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "out_config->struct_size is %u, expected %zu", out_config->struct_size,
                    sizeof(vx_decoder_config_t));
        *out_config = d->cfg;
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
