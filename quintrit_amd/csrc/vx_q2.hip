// Block-scaled (Q2_0) ternary GEMV for gfx950: ternary weights with one fp16 scale per 64 weights of a row, times int8
// activations with one fp32 scale per 32 values (Q8_0), with fp32 results bit-identical to the reference's definition.
//
// The reference (quintrit-core/src/block_scaled.rs:1-19, dot_row_scalar 175-202) reproduces ggml_vec_dot_q2_0_q8_0:
// every 32-value activation block s gives eight exact integer lane sums (lane j covers values 4j..4j+3); each is
// accumulated as acc[(s/2) & 1][j] = fma(w_scale[s/2] * a_scale[s], float(lane), acc[...][j]), s in increasing order;
// then l[j] = acc[0][j] + acc[1][j] and the result is ((l0+l4) + (l2+l6)) + ((l1+l5) + (l3+l7)). The weights are the
// velurex planar layout, so plane p of 160-trit block b is activation block s = 5b + p.
//
// Here one lane owns one (row, j) pair: its two accumulators are exactly the reference's acc[0][j], acc[1][j] of that
// row, fed in the same order, and the final tree is three xor-shuffles over the eight lanes of the row. The lane reads
// one 32-bit word of weights per 160-trit block (bytes 4j..4j+3); planes 0..3 of its four bytes come from four LDS table
// lookups (t0..t3 as int8) transposed with v_perm, plane 4 from byte-wise compares (d4 = t4 + 1, corrected by the lane's
// activation sum); each lane sum is one v_dot4_i32_i8.
//
// Device layout (vx_q2_matrix_create): rows form tiles of 8 and tiles form groups of 16. The 32-byte planar block b of
// row r lives at 256-byte unit (g * 16 * nb + b * T + t') with g = tile / 16, t' = tile % 16, T the tiles of the group and
// nb the blocks per row, at byte (r % 8) * 32; a wave (one tile) reads 256 consecutive bytes per block and the 16 waves
// of a workgroup 4 KiB. The fp16 scales of row r follow the weights: tile-major, then row % 8, then k (padded to a
// multiple of 10 per row, so a lane reads the ten scales of four blocks as five aligned words).
#include "vx_internal.h"

#include <algorithm>
#include <cstring>
#include <vector>

namespace vx {

// ---- layout -----------------------------------------------------------------------------------------------------------

size_t q2_blocks(size_t cols) { return (cols + kQK5 - 1) / kQK5; }
size_t q2_scale_stride(size_t cols) { return round_up(cols / 64, 10); }
size_t q2_weight_bytes(size_t rows, size_t cols) { return round_up(rows, 8) * q2_blocks(cols) * 32; }
size_t q2_device_bytes(size_t rows, size_t cols) {
    return q2_weight_bytes(rows, cols) + round_up(rows, 8) * q2_scale_stride(cols) * 2;
}

void q2_to_device_layout(const uint8_t* planar, const uint16_t* scales, size_t rows, size_t cols, uint8_t* dst) {
    const size_t nb = q2_blocks(cols), nk = cols / 64, ks = q2_scale_stride(cols);
    const size_t tiles = (rows + 7) / 8;
    std::memset(dst, 0, q2_device_bytes(rows, cols));
    for (size_t r = 0; r < round_up(rows, 8); ++r) {
        const size_t tile = r / 8, grp = tile / kTileGroup, t = tile % kTileGroup;
        const size_t T = std::min<size_t>(kTileGroup, tiles - grp * kTileGroup);
        for (size_t b = 0; b < nb; ++b) {
            uint8_t* d = dst + ((grp * kTileGroup * nb + b * T + t) * 256) + (r % 8) * 32;
            if (r < rows) std::memcpy(d, planar + r * nb * 32 + b * 32, 32);
            else std::memset(d, kZeroByte, 32);
        }
        uint16_t* sd = reinterpret_cast<uint16_t*>(dst + q2_weight_bytes(rows, cols)) + (tile * 8 + r % 8) * ks;
        for (size_t k = 0; k < nk; ++k) sd[k] = r < rows ? scales[r * nk + k] : 0;
    }
}

// ---- kernel -----------------------------------------------------------------------------------------------------------

__device__ inline uint32_t q2_trits03(uint32_t b) {
    const uint32_t u = b / 28u, l = b - 28u * u;
    if (b > 250u || l > 26u) return 0u;
    const uint32_t d0 = l % 3u, d1 = l / 3u % 3u, d2 = l / 9u, d3 = u % 3u;
    return ((d0 - 1u) & 0xffu) | (((d1 - 1u) & 0xffu) << 8) | (((d2 - 1u) & 0xffu) << 16) | (((d3 - 1u) & 0xffu) << 24);
}

__device__ __forceinline__ uint32_t q2_d4(uint32_t w) {
    const uint32_t x = (w >> 1) & 0x7f7f7f7fu;
    return (((x + 0x56565656u) >> 7) & 0x01010101u) + (((x + 0x2c2c2c2cu) >> 7) & 0x01010101u);
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));  // exact widening
}

constexpr int kQ2Waves = 16;
constexpr int kQ2Group = 4;  // 160-trit blocks per prefetch group (ten scales)

typedef __attribute__((address_space(4))) const Q2Job c_q2job;

// MANY: the jobs are a device array (a plan); otherwise the one job travels in the kernel arguments.
template <bool MANY>
__global__ __launch_bounds__(kQ2Waves * 64) __attribute__((amdgpu_waves_per_eu(8, 8))) void q2_kernel(Q2Args args) {
    __shared__ uint32_t tab[256 * 64];
    __shared__ uint32_t acts[kQ2MaxCols / 4];
    __shared__ float ascl[kQ2MaxCols / 32];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t j = lane & 7u, rl = lane >> 3;
    for (uint32_t i = tid; i < 256u * 16u; i += kQ2Waves * 64u) {
        const uint32_t e = q2_trits03(i >> 4);
        reinterpret_cast<uint4*>(tab)[i] = make_uint4(e, e, e, e);
    }
    const char* tabb = reinterpret_cast<const char*>(tab);
    const uint32_t lane_off = lane * 4u;

    uint32_t jj = 0;
    for (uint32_t item = blockIdx.x; item < args.total_items; item += gridDim.x) {
        const c_q2job* cj = (const c_q2job*)(args.jobs);
        if (MANY)
            while (jj + 1 < args.n_jobs && item >= cj[jj + 1].item_begin) ++jj;
        Q2Job jb;
        if (MANY) __builtin_memcpy(&jb, (const Q2Job*)(cj + jj), sizeof(Q2Job));
        else jb = args.one;
        const uint32_t grp = item - jb.item_begin;
        const uint32_t tiles = (jb.rows + 7u) / 8u;
        const uint32_t T = min(static_cast<uint32_t>(kTileGroup), tiles - grp * kTileGroup);
        const uint32_t ns = jb.cols / 32u, nb = (jb.cols + 159u) / 160u;
        __syncthreads();  // the previous item is done with acts / ascl
        const uint32_t* a32 = reinterpret_cast<const uint32_t*>(jb.acts);
        for (uint32_t i = tid; i < jb.cols / 4u; i += kQ2Waves * 64u) acts[i] = a32[i];
        for (uint32_t i = tid; i < ns; i += kQ2Waves * 64u) ascl[i] = jb.act_scales[i];
        __syncthreads();
        if (wave >= T) continue;
        const uint32_t tile = grp * kTileGroup + wave;
        const uint32_t row = tile * 8u + rl;
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(jb.w + (static_cast<size_t>(grp) * kTileGroup * nb + wave) * 256u) + lane;
        const size_t bstride = static_cast<size_t>(T) * 64u;  // dwords between blocks of this tile
        const uint32_t* sp = reinterpret_cast<const uint32_t*>(jb.scales + (static_cast<size_t>(tile) * 8u + rl) * jb.scale_stride);
        float acc0 = 0.0f, acc1 = 0.0f;
        for (uint32_t b0 = 0; b0 < nb; b0 += kQ2Group) {
            uint32_t w[kQ2Group], sc[5];
#pragma unroll
            for (int i = 0; i < kQ2Group; ++i) w[i] = __builtin_nontemporal_load(wp + min(b0 + i, nb - 1u) * bstride);
#pragma unroll
            for (int i = 0; i < 5; ++i) sc[i] = sp[5u * (b0 / 4u) + i];  // scales k0 .. k0 + 9, k0 = 5 b0 / 2
#pragma unroll
            for (int i = 0; i < kQ2Group; ++i) {
                const uint32_t b = b0 + i;
                if (b >= nb) break;
                const uint32_t wv = w[i];
                uint32_t x[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t addr = __builtin_amdgcn_perm(wv, lane_off, 0x0c0c0000u | ((4u + k) << 8));
                    x[k] = *reinterpret_cast<const uint32_t*>(tabb + addr);
                }
                uint32_t P[5];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const uint32_t sel = 0x0c0c0000u | ((4u + p) << 8) | static_cast<uint32_t>(p);
                    const uint32_t lo = __builtin_amdgcn_perm(x[1], x[0], sel);
                    const uint32_t hi = __builtin_amdgcn_perm(x[3], x[2], sel);
                    P[p] = lo | (hi << 16);
                }
                P[4] = q2_d4(wv);
#pragma unroll
                for (int p = 0; p < 5; ++p) {
                    const uint32_t s = 5u * b + p;
                    if (s >= ns) break;
                    const uint32_t av = acts[s * 8u + j];
                    int L = __builtin_amdgcn_sdot4(static_cast<int>(P[p]), static_cast<int>(av), 0, false);
                    if (p == 4) L -= __builtin_amdgcn_sdot4(0x01010101, static_cast<int>(av), 0, false);
                    const uint32_t kl = s / 2u - (b0 * 5u) / 2u;  // scale index inside this group's ten
                    const uint32_t hw = sc[kl >> 1] >> ((kl & 1u) * 16u);
                    const float d = half_bits_to_float(hw & 0xffffu) * ascl[s];
                    if ((s / 2u) & 1u) acc1 = __builtin_fmaf(d, static_cast<float>(L), acc1);
                    else acc0 = __builtin_fmaf(d, static_cast<float>(L), acc0);
                }
            }
        }
        float l = acc0 + acc1;
        l = l + __shfl_xor(l, 4);
        l = l + __shfl_xor(l, 2);
        l = l + __shfl_xor(l, 1);
        if (j == 0 && row < jb.rows) jb.out[row] = l;
    }
}

// Integer lane sums (rows x cols/32 x 8): the exact part of the product, for checking.
__global__ __launch_bounds__(256) void q2_lane_sums_kernel(Q2Job jb, int32_t* __restrict__ out) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint32_t ns = jb.cols / 32u, nb = (jb.cols + 159u) / 160u;
    if (idx >= static_cast<uint64_t>(jb.rows) * ns * 8u) return;
    const uint32_t jl = static_cast<uint32_t>(idx % 8u);
    const uint32_t s = static_cast<uint32_t>((idx / 8u) % ns);
    const uint32_t row = static_cast<uint32_t>(idx / (8u * ns));
    const uint32_t tiles = (jb.rows + 7u) / 8u, tile = row / 8u, grp = tile / kTileGroup, t = tile % kTileGroup;
    const uint32_t T = min(static_cast<uint32_t>(kTileGroup), tiles - grp * kTileGroup);
    const uint32_t b = s / 5u, p = s % 5u;
    const uint8_t* blk = jb.w + ((static_cast<size_t>(grp) * kTileGroup * nb + static_cast<size_t>(b) * T + t) * 256u) + (row % 8u) * 32u;
    int sum = 0;
    for (uint32_t k = 4u * jl; k < 4u * jl + 4u; ++k) {
        const uint32_t B = blk[k];
        const uint32_t u = B / 28u, l = B - 28u * u;
        int tr = 0;
        if (B <= 250u && l <= 26u) {
            const uint32_t dg[5] = {l % 3u, l / 3u % 3u, l / 9u, u % 3u, u / 3u};
            tr = static_cast<int>(dg[p]) - 1;
        }
        sum += tr * jb.acts[s * 32u + k];
    }
    out[idx] = sum;
}

int launch_q2(const Q2Args& a, int num_cus, hipStream_t stream) {
    if (a.total_items == 0) return VX_OK;
    const uint32_t grid = std::min<uint32_t>(a.total_items, 2u * static_cast<uint32_t>(num_cus));
    if (a.jobs) hipLaunchKernelGGL(q2_kernel<true>, dim3(grid), dim3(kQ2Waves * 64), 0, stream, a);
    else hipLaunchKernelGGL(q2_kernel<false>, dim3(grid), dim3(kQ2Waves * 64), 0, stream, a);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_q2_lane_sums(const Q2Job& j, int32_t* out, hipStream_t stream) {
    const uint64_t n = static_cast<uint64_t>(j.rows) * (j.cols / 32u) * 8u;
    hipLaunchKernelGGL(q2_lane_sums_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, stream, j, out);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

}  // namespace vx
