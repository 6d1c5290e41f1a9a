// Batched ternary GEMM for gfx950 (MI355X): Y[m][i] = sum_j W[i][j] X[m][j] for M tokens, exact int32, on the matrix
// cores (v_mfma_i32_16x16x64_i8).
//
// The reference has no multi-token kernel: its prefill runs one GEMV per token (quintrit-runtime/src/engine.rs:625-631),
// so the definition is M independent GEMVs (quintrit-core/src/simd/avx512.rs:1526-1626), and the result must equal
// them bit for bit. Weights stay in the velurex device layout of the GEMV (1.60 bits per weight in HBM) and are
// decoded to int8 trits in registers right before the matrix-core instruction; activations are staged once per call
// in the order of the MFMA B operand.
//
// K order. A 16-byte chunk of a weight row holds 16 byte-columns x 5 planes = 80 trits. Four chunks (64 byte-columns,
// 320 trits) make one K step of five 64-deep MFMA blocks: block kb < 4 holds planes 0..3 of chunk kb, block 4 holds
// plane 4 of the four chunks. In block kb < 4, lane (i, s) (i = lane % 16 the row, s = lane / 16) supplies the 4 x 4
// trits of bytes 4s .. 4s+3 of its row's chunk: one 32-bit word of weights, decoded by four lookups of a 256-entry
// table (t0..t3 as int8). In block 4 the lane supplies plane 4 of the same word in each of the four chunks; d4 (the
// digit, t4 + 1) comes from two byte-wise compares done four bytes at a time (B >= 84, B >= 168), and the missing
// "- 1" is subtracted once per token as the sum of that token's plane-4 activations. The activation staging writes X
// in exactly this order, so A and B pair every weight with its activation.
#include "vx_internal.h"

#include <algorithm>

namespace vx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(4))) const uint32_t c_u32;

// t0..t3 of byte B as int8 in a dword; non-values give zero trits (pack.rs:41-58).
__device__ inline uint32_t trits03(uint32_t b) {
    const uint32_t u = b / 28u, l = b - 28u * u;
    if (b > 250u || l > 26u) return 0u;
    const uint32_t d0 = l % 3u, d1 = l / 3u % 3u, d2 = l / 9u, d3 = u % 3u;
    return ((d0 - 1u) & 0xffu) | (((d1 - 1u) & 0xffu) << 8) | (((d2 - 1u) & 0xffu) << 16) | (((d3 - 1u) & 0xffu) << 24);
}

// d4 = floor(B / 84) of each byte of w, as bytes (B >= 84 and B >= 168 tested with 7-bit adds that cannot carry).
__device__ __forceinline__ uint32_t d4_bytes(uint32_t w) {
    const uint32_t x = (w >> 1) & 0x7f7f7f7fu;
    return (((x + 0x56565656u) >> 7) & 0x01010101u) + (((x + 0x2c2c2c2cu) >> 7) & 0x01010101u);
}

// ---- activation staging --------------------------------------------------------------------------------------------

// Activation p of device byte-column c of token m (column_activation_index, pack.rs:230-237), 0 outside.
__device__ inline int act_at(const int8_t* __restrict__ x, uint32_t ldx, uint32_t m, uint32_t M, uint32_t cols,
                             uint32_t tbr, uint32_t c, uint32_t p) {
    if (m >= M || c >= tbr) return 0;
    const uint32_t full = cols / 160u * 32u;
    const uint32_t idx = c < full ? (c / 32u) * 160u + p * 32u + (c % 32u) : (cols / 160u) * 160u + 5u * (c - full) + p;
    return idx < cols ? x[static_cast<size_t>(m) * ldx + idx] : 0;
}

// One thread per 16-byte B fragment: xs[kstep][kb][tg][lane] (see the K order above).
__global__ void gemm_stage_kernel(const int8_t* __restrict__ x, uint32_t ldx, uint32_t M, uint32_t n_tg, uint32_t cols,
                                  uint32_t tbr, uint32_t n_ksteps, uint4* __restrict__ xs) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(n_ksteps) * 5u * n_tg * 64u;
    if (idx >= total) return;
    const uint32_t lane = static_cast<uint32_t>(idx & 63u);
    uint64_t r = idx >> 6;
    const uint32_t tg = static_cast<uint32_t>(r % n_tg);
    r /= n_tg;
    const uint32_t kb = static_cast<uint32_t>(r % 5u);
    const uint32_t ks = static_cast<uint32_t>(r / 5u);
    const uint32_t m = tg * 16u + (lane & 15u), s = lane >> 4;
    uint32_t w[4];
    for (uint32_t d = 0; d < 4; ++d) {
        uint32_t v = 0;
        for (uint32_t e = 0; e < 4; ++e) {
            uint32_t c, p;
            if (kb < 4) {  // dword d = byte-column 4s + d of chunk kb, bytes = planes 0..3
                c = (4u * ks + kb) * 16u + 4u * s + d;
                p = e;
            } else {       // dword d = chunk d, byte e = byte-column 4s + e, plane 4
                c = (4u * ks + d) * 16u + 4u * s + e;
                p = 4;
            }
            v |= (static_cast<uint32_t>(act_at(x, ldx, m, M, cols, tbr, c, p)) & 0xffu) << (8 * e);
        }
        w[d] = v;
    }
    xs[idx] = make_uint4(w[0], w[1], w[2], w[3]);
}

// s4[m] = sum over byte-columns of activation plane 4 (the correction for using d4 = t4 + 1). One block per token.
__global__ __launch_bounds__(256) void gemm_s4_kernel(const int8_t* __restrict__ x, uint32_t ldx, uint32_t M,
                                                       uint32_t cols, uint32_t tbr, int* __restrict__ s4) {
    __shared__ int red[4];
    const uint32_t m = blockIdx.x;
    int s = 0;
    for (uint32_t c = threadIdx.x; c < tbr; c += 256u) s += act_at(x, ldx, m, M, cols, tbr, c, 4);
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) s4[m] = red[0] + red[1] + red[2] + red[3];
}

// ---- GEMM -------------------------------------------------------------------------------------------------------------

struct GemmArgs {
    const uint8_t* w;      // device layout
    const uint4* xs;       // staged activations
    const int* s4;         // per-token plane-4 sums
    int32_t* y;            // M x ldy (kslices == 1)
    int32_t* part;         // kslices x Mp x rows_p partial sums (kslices > 1)
    uint32_t rows, n_tiles, n_chunks, n_ksteps;
    uint32_t M, n_tg, ldy;
    uint32_t kslices, ksteps_per_slice, rows_p;
};

constexpr int kGemmWaves = 4;   // one 64-row tile per wave
constexpr int kGemmTg = 4;      // 16-token groups per workgroup

__global__ __launch_bounds__(kGemmWaves * 64) void gemm_kernel(GemmArgs a) {
    __shared__ uint32_t tab[256 * 64];
    __shared__ uint4 bsm[2][5 * kGemmTg * 64];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t tile = blockIdx.x * kGemmWaves + wave;
    const uint32_t tg0 = blockIdx.y * kGemmTg;
    const uint32_t ntg = min(static_cast<uint32_t>(kGemmTg), a.n_tg - tg0);
    const uint32_t kz = blockIdx.z;
    const uint32_t ks0 = kz * a.ksteps_per_slice;
    const uint32_t ks1 = min(ks0 + a.ksteps_per_slice, a.n_ksteps);

    for (uint32_t i = tid; i < 256u * 16u; i += kGemmWaves * 64u) {
        const uint32_t e = trits03(i >> 4);
        reinterpret_cast<uint4*>(tab)[i] = make_uint4(e, e, e, e);
    }
    const char* tabb = reinterpret_cast<const char*>(tab);
    const uint32_t lane_off = lane * 4u;
    const bool active = tile < a.n_tiles;
    // Base of this wave's tile in the device layout, and the byte of lane (i, s) inside a chunk.
    const uint32_t grp = tile / kTileGroup, tt = tile - grp * kTileGroup;
    const uint32_t T = active ? min(static_cast<uint32_t>(kTileGroup), a.n_tiles - grp * kTileGroup) : 1u;
    const uint8_t* wbase = a.w + (static_cast<size_t>(grp) * kTileGroup * a.n_chunks + tt) * 1024u + (lane & 15u) * 16u + (lane >> 4) * 4u;

    v4i acc[4][kGemmTg];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int g = 0; g < kGemmTg; ++g) acc[rb][g] = v4i{0, 0, 0, 0};

    // weights of one K step: 4 row blocks x 4 chunks, one 32-bit word each (byte 125 = zero trits past the row)
    auto load_w = [&](uint32_t (&wv)[4][4], uint32_t ks) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t chunk = 4u * ks + q;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
                wv[rb][q] = chunk < a.n_chunks
                                ? __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(
                                      wbase + (static_cast<size_t>(chunk) * T) * 1024u + rb * 256u))
                                : 0x7d7d7d7du;
        }
    };
    uint32_t wv[4][4], wn[4][4];
    if (active && ks0 < ks1) load_w(wv, ks0);
    uint32_t buf = 0;
    for (uint32_t ks = ks0; ks < ks1; ++ks, buf ^= 1u) {
        if (active && ks + 1 < ks1) load_w(wn, ks + 1);  // next step's weights stream in during this step's MFMAs
        // stage the B fragments of this K step
        const uint4* src = a.xs + static_cast<size_t>(ks) * 5u * a.n_tg * 64u;
        uint4* dst = bsm[buf];
        for (uint32_t i = tid; i < 5u * ntg * 64u; i += kGemmWaves * 64u) {
            const uint32_t kb = i / (ntg * 64u), rem = i - kb * ntg * 64u;
            dst[kb * kGemmTg * 64u + rem] = src[(static_cast<size_t>(kb) * a.n_tg + tg0) * 64u + rem];
        }
        __syncthreads();
        if (active) {
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                v4i A[5];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t w = wv[rb][q];
                    int t[4];
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const uint32_t addr = __builtin_amdgcn_perm(w, lane_off, 0x0c0c0000u | ((4u + b) << 8));
                        t[b] = static_cast<int>(*reinterpret_cast<const uint32_t*>(tabb + addr));
                    }
                    A[q] = v4i{t[0], t[1], t[2], t[3]};
                }
                A[4] = v4i{static_cast<int>(d4_bytes(wv[rb][0])), static_cast<int>(d4_bytes(wv[rb][1])),
                           static_cast<int>(d4_bytes(wv[rb][2])), static_cast<int>(d4_bytes(wv[rb][3]))};
#pragma unroll
                for (int g = 0; g < kGemmTg; ++g) {
                    if (static_cast<uint32_t>(g) < ntg) {
#pragma unroll
                        for (int kb = 0; kb < 5; ++kb) {
                            const uint4 bv = bsm[buf][(kb * kGemmTg + g) * 64u + lane];
                            const v4i B = v4i{static_cast<int>(bv.x), static_cast<int>(bv.y), static_cast<int>(bv.z),
                                              static_cast<int>(bv.w)};
                            acc[rb][g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[kb], B, acc[rb][g], 0, 0, 0);
                        }
                    }
                }
            }
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int q = 0; q < 4; ++q) wv[rb][q] = wn[rb][q];
        }
    }
    if (!active) return;
    // C fragment: lane (j, s) holds rows 4s + r of the 16-row block, token j.
    const uint32_t j = lane & 15u, s = lane >> 4;
#pragma unroll
    for (int g = 0; g < kGemmTg; ++g) {
        if (static_cast<uint32_t>(g) >= ntg) continue;
        const uint32_t m = (tg0 + g) * 16u + j;
        if (m >= a.M) continue;
        const int corr = a.kslices == 1 ? a.s4[m] : 0;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t n = tile * 64u + rb * 16u + 4u * s + r;
                if (n >= a.rows) continue;
                if (a.kslices == 1) a.y[static_cast<size_t>(m) * a.ldy + n] = acc[rb][g][r] - corr;
                else a.part[(static_cast<size_t>(kz) * a.n_tg * 16u + m) * a.rows_p + n] = acc[rb][g][r];
            }
        }
    }
}

__global__ __launch_bounds__(256) void gemm_finish_kernel(GemmArgs a) {
    const uint32_t n = blockIdx.x * 256u + threadIdx.x, m = blockIdx.y;
    if (n >= a.rows) return;
    int s = -a.s4[m];
    for (uint32_t k = 0; k < a.kslices; ++k) s += a.part[(static_cast<size_t>(k) * a.n_tg * 16u + m) * a.rows_p + n];
    a.y[static_cast<size_t>(m) * a.ldy + n] = s;
}

// ---- host side ---------------------------------------------------------------------------------------------------------

struct GemmPlan {
    uint32_t n_ksteps, n_tg, kslices, ksteps_per_slice, grid_x, grid_y;
    size_t xs_bytes, s4_bytes, part_bytes;
};

static GemmPlan gemm_plan(const Geometry& g, size_t M, int num_cus) {
    GemmPlan p{};
    p.n_ksteps = static_cast<uint32_t>((g.n_chunks + 3) / 4);
    p.n_tg = static_cast<uint32_t>((M + 15) / 16);
    p.grid_x = static_cast<uint32_t>((g.n_tiles + kGemmWaves - 1) / kGemmWaves);
    p.grid_y = (p.n_tg + kGemmTg - 1) / kGemmTg;
    const uint32_t blocks = p.grid_x * p.grid_y;
    const uint32_t want = static_cast<uint32_t>(num_cus);  // one workgroup (104 KiB LDS) per CU
    uint32_t ks = std::max<uint32_t>(1u, std::min<uint32_t>(p.n_ksteps, (want + blocks - 1) / blocks));
    p.ksteps_per_slice = (p.n_ksteps + ks - 1) / ks;
    p.kslices = (p.n_ksteps + p.ksteps_per_slice - 1) / p.ksteps_per_slice;
    p.xs_bytes = round_up(static_cast<size_t>(p.n_ksteps) * 5u * p.n_tg * 1024u, 256);
    p.s4_bytes = round_up(static_cast<size_t>(p.n_tg) * 16u * 4u, 256);
    p.part_bytes = p.kslices > 1 ? static_cast<size_t>(p.kslices) * p.n_tg * 16u * g.padded_rows * 4u : 0;
    return p;
}

size_t gemm_workspace_bytes(const Geometry& g, size_t M, int num_cus) {
    const GemmPlan p = gemm_plan(g, M, num_cus);
    return p.xs_bytes + p.s4_bytes + p.part_bytes;
}

int launch_gemm(const uint8_t* w, const Geometry& g, int num_cus, const int8_t* x, size_t M, size_t ldx, int32_t* y,
                size_t ldy, uint8_t* ws, hipStream_t stream) {
    const GemmPlan p = gemm_plan(g, M, num_cus);
    uint4* xs = reinterpret_cast<uint4*>(ws);
    int* s4 = reinterpret_cast<int*>(ws + p.xs_bytes);
    int32_t* part = p.kslices > 1 ? reinterpret_cast<int32_t*>(ws + p.xs_bytes + p.s4_bytes) : nullptr;
    const uint64_t frags = static_cast<uint64_t>(p.n_ksteps) * 5u * p.n_tg * 64u;
    hipLaunchKernelGGL(gemm_stage_kernel, dim3(static_cast<uint32_t>((frags + 255) / 256)), dim3(256), 0, stream, x,
                       static_cast<uint32_t>(ldx), static_cast<uint32_t>(M), p.n_tg, static_cast<uint32_t>(g.cols),
                       static_cast<uint32_t>(g.tbr), p.n_ksteps, xs);
    VX_HIP(hipGetLastError());
    hipLaunchKernelGGL(gemm_s4_kernel, dim3(static_cast<uint32_t>(M)), dim3(256), 0, stream, x, static_cast<uint32_t>(ldx),
                       static_cast<uint32_t>(M), static_cast<uint32_t>(g.cols), static_cast<uint32_t>(g.tbr), s4);
    VX_HIP(hipGetLastError());
    GemmArgs a{};
    a.w = w;
    a.xs = xs;
    a.s4 = s4;
    a.y = y;
    a.part = part;
    a.rows = static_cast<uint32_t>(g.rows);
    a.n_tiles = static_cast<uint32_t>(g.n_tiles);
    a.n_chunks = static_cast<uint32_t>(g.n_chunks);
    a.n_ksteps = p.n_ksteps;
    a.M = static_cast<uint32_t>(M);
    a.n_tg = p.n_tg;
    a.ldy = static_cast<uint32_t>(ldy);
    a.kslices = p.kslices;
    a.ksteps_per_slice = p.ksteps_per_slice;
    a.rows_p = static_cast<uint32_t>(g.padded_rows);
    hipLaunchKernelGGL(gemm_kernel, dim3(p.grid_x, p.grid_y, p.kslices), dim3(kGemmWaves * 64), 0, stream, a);
    VX_HIP(hipGetLastError());
    if (p.kslices > 1) {
        hipLaunchKernelGGL(gemm_finish_kernel, dim3((a.rows + 255u) / 256u, static_cast<uint32_t>(M)), dim3(256), 0, stream, a);
        VX_HIP(hipGetLastError());
    }
    return VX_OK;
}

}  // namespace vx
