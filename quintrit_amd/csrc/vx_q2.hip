// Block-scaled (Q2_0) ternary GEMV for gfx950: ternary weights with one fp16 scale per 64 weights of a row, times int8
// activations with one fp32 scale per 32 values (Q8_0), with fp32 results bit-identical to the reference's definition.
//
// The reference (quintrit-core/src/block_scaled.rs:1-19, dot_row_scalar 175-202) reproduces ggml_vec_dot_q2_0_q8_0:
// every 32-value activation block s gives eight exact integer lane sums L[s][j] (lane j covers values 4j..4j+3); each
// is accumulated as acc[(s/2) & 1][j] = fma(w_scale[s/2] * a_scale[s], float(L[s][j]), acc[...][j]), s in increasing
// order; then l[j] = acc[0][j] + acc[1][j] and the result is ((l0+l4) + (l2+l6)) + ((l1+l5) + (l3+l7)). The weights are
// the velurex planar layout, so plane p of 160-trit block b is activation block s = 5b + p, and byte k of the block
// belongs to lane j = k / 4 of every plane.
//
// Lane sums on the matrix cores. For one 160-trit block b and 32 weight rows, the 40 lane sums (p, j) of every row are
// a product C = A' W^T on v_mfma_i32_32x32x32_i8, transposed so that the rows of C are lane sums and its columns
// weight rows: lane l of the output then holds column n = l % 32 (one weight row) and C rows 8 (r / 4) + 4 (l / 32) +
// r % 4, r = 0..15. With C row 8 p + j for planes 0..3, lane l holds the sums (p, j) of its row for every p < 4 and
// j = 4 (l / 32) + r % 4; a second product holds plane 4 in C rows j. So each lane runs the reference's fp32 chains of
// its row's four lanes j in registers, in the reference's order, with no exchange between lanes until the final sum.
//   W operand: the weights decoded exactly as the batched GEMM decodes its A operand (vx_gemm.hip): lane (n, h) holds
//     the 16 bytes 16 h .. 16 h + 15 of block b of row n; K block m < 4 takes bytes 4 m .. 4 m + 3 with their
//     trits t0..t3 (one LDS table lookup per byte), K block 4 takes t4 of all 16 bytes (byte arithmetic).
//   A' operand (one 32 x 32 int8 block per K block, built per lane with v_perm from the raw activations in LDS): for K
//     block m, row 8 p + j holds a(5b + p, 4 j + q) at the K position of (byte 4 j + q, plane p) when j = 4 h + m,
//     zero elsewhere; for K block 4, row j holds a(5b + 4, 4 j + q) at the position of byte 4 j + q.
//
// Device layout (vx_q2_matrix_create): the planar bytes of each row (ceil(cols / 160) blocks of 32 bytes, a partial
// last block padded with zero trits as the planar layout pads it) in the GEMV's tile layout (64-row tiles, 16-byte
// chunks interleaved over groups of 16 tiles, vx_layout), followed by the fp16 scales as [tile][group of 4 blocks]
// [row of the tile][10 scales]: the ten scales of 20 activation blocks, one 20-byte load per lane.
#include "vx_gemv_core.h"
#include "vx_internal.h"

#include <algorithm>
#include <cstring>
#include <functional>
#include <queue>
#include <vector>

namespace vx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 g_u4;

// ---- layout -----------------------------------------------------------------------------------------------------------

size_t q2_blocks(size_t cols) { return (cols + kQK5 - 1) / kQK5; }
size_t q2_kgroups(size_t cols) { return (q2_blocks(cols) + 3) / 4; }
size_t q2_weight_bytes(size_t rows, size_t cols) { return round_up(rows, kTileRows) * q2_blocks(cols) * kBlockBytes; }
size_t q2_device_bytes(size_t rows, size_t cols) {
    return q2_weight_bytes(rows, cols) + round_up(rows, kTileRows) * q2_kgroups(cols) * 10 * 2;
}

void q2_to_device_layout(const uint8_t* planar, const uint16_t* scales, size_t rows, size_t cols, uint8_t* dst) {
    const size_t nb = q2_blocks(cols), nk = cols / 64, ng = q2_kgroups(cols);
    const size_t padded = round_up(rows, kTileRows), n_tiles = padded / kTileRows, n_chunks = nb * 2;
    std::memset(dst, 0, q2_device_bytes(rows, cols));
    for (size_t r = 0; r < padded; ++r)
        for (size_t q = 0; q < n_chunks; ++q) {
            uint8_t* d = dst + layout_offset(r, static_cast<uint32_t>(q * kChunk), static_cast<uint32_t>(n_tiles),
                                             static_cast<uint32_t>(n_chunks));
            if (r < rows) std::memcpy(d, planar + r * nb * kBlockBytes + q * kChunk, kChunk);
            else std::memset(d, kZeroByte, kChunk);
        }
    uint16_t* sd = reinterpret_cast<uint16_t*>(dst + q2_weight_bytes(rows, cols));
    for (size_t r = 0; r < rows; ++r) {
        const size_t tile = r / kTileRows;
        for (size_t k = 0; k < nk; ++k)
            sd[((tile * ng + k / 10) * kTileRows + r % kTileRows) * 10 + k % 10] = scales[r * nk + k];
    }
}

// ---- kernel -----------------------------------------------------------------------------------------------------------

constexpr int kQ2Waves = 16;   // 8 tiles x 2 halves of 32 rows (plans)
constexpr int kQ2LoneWaves = 4;  // 2 tiles per item: a lone GEMV's waves spread over more CUs
constexpr int kQ2Pre = 4;      // blocks of weights in flight per wave (64 KiB per CU)

__constant__ TritTable g_trits = make_trit_table();

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));  // exact widening
}

typedef __attribute__((address_space(4))) const Q2Job c_q2job;
typedef __attribute__((address_space(4))) const float c_q2float;  // uniform reads through the scalar cache
typedef __attribute__((address_space(4))) const uint32_t c_q2u32;

// Work item: W / 2 consecutive tiles of a tile group (wave w: tile (W / 2) i + w / 2 for the item's index i in the
// group, rows 32 (w % 2) .. + 31 of it). The activations and their scales are staged in LDS once per item; every wave
// then streams its rows' blocks in order. A lone GEMV takes W = 4 while its items fit the CUs about once: a wave's
// pass over its rows' blocks sets the call's time, and with two waves per SIMD instead of four it runs faster (at
// 4096 columns 19.9 against 27.4 us per call, at 12288 48.5 against 72.9; W = 2 took 22.3 and 51.7).
template <bool MANY, int W>
__global__ __launch_bounds__(W * 64) void q2_kernel(Q2Args args) {
    static_assert(W >= 2 && W % 2 == 0 && (2 * kTileGroup) % W == 0, "whole items of a tile group");
    constexpr uint32_t kPer = W / 2u;                      // tiles per item
    constexpr uint32_t kItemsPerGroup = kTileGroup / kPer;
    // row B (256 bytes): 32 copies of t0..t3 of byte B, then 32 copies of t4 of B in every byte; lane l of a half-wave
    // reads copy l of each half (one address, offsets 0 and 128), so the t0..t3 dwords of four bytes land in the
    // registers of one MFMA operand
    __shared__ uint32_t tab[256 * 64];
    __shared__ uint32_t actw[kQ2MaxCols / 4 + 64];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (uint32_t i = tid; i < 256u * 16u; i += W * 64u) {
        const uint32_t b = i >> 4, e = (i & 8u) ? t4_bytes(b * 0x01010101u) : g_trits.v[b];
        *reinterpret_cast<uint4*>(reinterpret_cast<char*>(tab) + b * 256u + (i & 15u) * 16u) = make_uint4(e, e, e, e);
    }
    const char* tabb = reinterpret_cast<const char*>(tab);
    const uint32_t lane_off = (lane & 31u) * 4u;

    // This lane's A' rows: C row mr = lane % 32 (plane p = mr / 8, lane sum j = mr % 8) and K half hh = lane / 32.
    // Dword q of K block m places byte q of the activation dword at byte p (v_perm, selector byte 0x0c gives 0x00) in
    // the one K block m = j % 4 of the lanes with j / 4 == hh, and is zero elsewhere: selm[m][q] is that selector or
    // all 0x0c, so one v_perm builds each dword of every K block's operand. The plane-4 dword goes to dword u = j % 4
    // of the lanes with mr < 8 and mr / 4 == hh (on4[u]).
    const uint32_t mr = lane & 31u, hh = lane >> 5, pl = mr >> 3, jl = mr & 7u;
    uint32_t selm[4][4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const bool on = (jl >> 2) == hh && (jl & 3u) == static_cast<uint32_t>(m);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            selm[m][q] = on ? (0x0c0c0c0cu & ~(0xffu << (8u * pl))) | (static_cast<uint32_t>(q) << (8u * pl)) : 0x0c0c0c0cu;
    }
    bool on4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) on4[u] = mr < 8u && (mr >> 2) == hh && (mr & 3u) == static_cast<uint32_t>(u);

    // the items of this workgroup: its part of the plan's schedule, or every grid-th item
    const c_q2u32* sched = (const c_q2u32*)(args.sched);
    const bool scheduled = MANY && args.sched != nullptr;
    uint32_t k = blockIdx.x, k_end = args.total_items, k_step = gridDim.x;
    if (scheduled) {
        k = sched[blockIdx.x];
        k_end = sched[blockIdx.x + 1u];
        k_step = 1u;
    }
    uint32_t jj_job = 0;  // items come in increasing order, so the job index only moves forward
    for (; k < k_end; k += k_step) {
        const uint32_t item = scheduled ? sched[gridDim.x + 1u + k] : k;
        const c_q2job* cj = (const c_q2job*)(args.jobs);
        if (MANY)
            while (jj_job + 1 < args.n_jobs && item >= cj[jj_job + 1].item_begin) ++jj_job;
        Q2Job jb;
        if (MANY) __builtin_memcpy(&jb, (const Q2Job*)(cj + jj_job), sizeof(Q2Job));
        else jb = args.one;
        const uint32_t local = item - jb.item_begin;
        const uint32_t grp = local / kItemsPerGroup, tt = (local % kItemsPerGroup) * kPer + (wave >> 1), rb = wave & 1u;
        const uint32_t T = min(static_cast<uint32_t>(kTileGroup), jb.n_tiles - grp * kTileGroup);
        const uint32_t ns = jb.cols / 32u, nb = jb.nb, n_chunks = 2u * nb, ng = (nb + 3u) / 4u;
        __syncthreads();  // the previous item is done with actw
        const uint32_t* a32 = reinterpret_cast<const uint32_t*>(jb.acts);
        for (uint32_t i = tid; i < nb * 40u; i += W * 64u) actw[i] = i < jb.cols / 4u ? a32[i] : 0u;
        const c_q2float* asp = (const c_q2float*)(jb.act_scales);  // the activation scale of block s: asp[s]
        __syncthreads();
        if (tt >= T) continue;
        const uint32_t tile = grp * kTileGroup + tt;
        const uint32_t row = tile * kTileRows + rb * 32u + (lane & 31u);

        // weights: chunk 2 b + hh of this row (16 bytes), chunks of a tile T KiB apart
        const g_u4* wp = (const g_u4*)(jb.w + (static_cast<size_t>(grp) * kTileGroup * n_chunks + tt) * 1024u + rb * 512u +
                                       (lane & 31u) * 16u + static_cast<size_t>(hh) * T * 1024u);
        const size_t bstride = static_cast<size_t>(T) * 128u;  // uint4 between blocks b and b + 1
        const uint32_t* sp = reinterpret_cast<const uint32_t*>(jb.scales) +
                             (static_cast<size_t>(tile) * ng * kTileRows + rb * 32u + (lane & 31u)) * 5u;
        const size_t sstride = static_cast<size_t>(kTileRows) * 5u;  // dwords between scale groups of a tile

        // the loop body is two scale groups of 4 blocks, one per register set, with the same weight slots in both
        static_assert(kQ2Pre == 4, "four weight slots per scale group");
        u32x4 wq[kQ2Pre];
#pragma unroll
        for (int i = 0; i < kQ2Pre; ++i) wq[i] = __builtin_nontemporal_load(wp + min(static_cast<uint32_t>(i), nb - 1u) * bstride);
        // Scale groups alternate between two register sets (group g in set g & 1), each loaded one group ahead, so no
        // loaded register is ever copied (a copy would wait for its load). Every load is unconditional (indices clamp at
        // the last block and group) and blocks past the row skip only the arithmetic, so every wait is for its own load.
        uint32_t sa[5], sb[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) sa[i] = sp[i];

        float acc0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, acc1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        // block b with its weights w and the scales sc of its group
        auto block = [&](uint32_t b, const u32x4 w, const uint32_t (&sc)[5]) __attribute__((always_inline)) {
            // W operand: K blocks 0..3 (t0..t3 of bytes 4 m .. 4 m + 3) and 4 (t4 of the 16 bytes)
            // two table reads per byte: t0..t3, and t4 in every byte, of which byte k of a dword keeps byte k
            const uint32_t dw[4] = {w.x, w.y, w.z, w.w};
            v4i Bm[5];
            uint32_t t4w[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                int t[4];
                uint32_t e4[4];
                uint32_t addr[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    addr[k] = __builtin_amdgcn_perm(dw[m], lane_off, 0x0c0c0000u | ((4u + k) << 8));
                    t[k] = static_cast<int>(*reinterpret_cast<const uint32_t*>(tabb + addr[k]));
                }
                // the t4 reads apart from the t0..t3 reads (merged pairwise, each pair would land in two adjacent
                // registers and the operand would have to be copied together)
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int k = 0; k < 4; ++k) e4[k] = *reinterpret_cast<const uint32_t*>(tabb + addr[k] + 128u);
                Bm[m] = v4i{t[0], t[1], t[2], t[3]};
                t4w[m] = __builtin_amdgcn_perm(e4[3], e4[2], 0x07020c0cu) | __builtin_amdgcn_perm(e4[1], e4[0], 0x0c0c0500u);
            }
            Bm[4] = v4i{static_cast<int>(t4w[0]), static_cast<int>(t4w[1]), static_cast<int>(t4w[2]), static_cast<int>(t4w[3])};
            // A' operands from the activation dwords of this block
            const uint32_t x = actw[(5u * b + pl) * 8u + jl];
            const uint32_t x4 = actw[(5u * b + 4u) * 8u + (mr & 7u)];
            v16i c = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
            v16i c4 = c;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const v4i A = v4i{static_cast<int>(__builtin_amdgcn_perm(0u, x, selm[m][0])),
                                  static_cast<int>(__builtin_amdgcn_perm(0u, x, selm[m][1])),
                                  static_cast<int>(__builtin_amdgcn_perm(0u, x, selm[m][2])),
                                  static_cast<int>(__builtin_amdgcn_perm(0u, x, selm[m][3]))};
                c = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bm[m], c, 0, 0, 0);
            }
            {
                const int xi = static_cast<int>(x4);
                const v4i A = v4i{on4[0] ? xi : 0, on4[1] ? xi : 0, on4[2] ? xi : 0, on4[3] ? xi : 0};
                c4 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bm[4], c4, 0, 0, 0);
            }
            // the reference's chains: s = 5 b + p in order; register r = 4 p + jj of c holds L[s][4 hh + jj]
#pragma unroll
            for (int p = 0; p < 5; ++p) {
                const uint32_t s = 5u * b + static_cast<uint32_t>(p);
                if (s >= ns) break;
                const uint32_t kl = (5u * (b & 3u) + static_cast<uint32_t>(p)) / 2u;  // scale index in the group
                const uint32_t hw = sc[kl >> 1] >> ((kl & 1u) * 16u);
                const float d = half_bits_to_float(hw & 0xffffu) * asp[s];
                const bool odd = (s / 2u) & 1u;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int L = p < 4 ? c[4 * p + jj] : c4[jj];
                    if (odd) acc1[jj] = __builtin_fmaf(d, static_cast<float>(L), acc1[jj]);
                    else acc0[jj] = __builtin_fmaf(d, static_cast<float>(L), acc0[jj]);
                }
            }
        };
        for (uint32_t b0 = 0; b0 < nb; b0 += 8u) {
            const uint32_t g = b0 / 4u;
#pragma unroll
            for (int i = 0; i < 5; ++i) sb[i] = sp[min(g + 1u, ng - 1u) * sstride + i];
#pragma unroll
            for (int ib = 0; ib < 4; ++ib) {
                const uint32_t b = b0 + ib;
                const u32x4 w = wq[ib];
                wq[ib] = __builtin_nontemporal_load(wp + min(b + kQ2Pre, nb - 1u) * bstride);
                if (b < nb) block(b, w, sa);
            }
#pragma unroll
            for (int i = 0; i < 5; ++i) sa[i] = sp[min(g + 2u, ng - 1u) * sstride + i];
#pragma unroll
            for (int ib = 0; ib < 4; ++ib) {
                const uint32_t b = b0 + 4u + ib;
                const u32x4 w = wq[ib];
                wq[ib] = __builtin_nontemporal_load(wp + min(b + kQ2Pre, nb - 1u) * bstride);
                if (b < nb) block(b, w, sb);
            }
        }
        // l[j] = acc[0][j] + acc[1][j]; lanes hh = 0 hold j = 0..3, hh = 1 j = 4..7
        float l[4], o[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) l[jj] = acc0[jj] + acc1[jj];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) o[jj] = __shfl_xor(l[jj], 32);
        if (hh == 0 && row < jb.rows) {
            const float a0 = l[0] + o[0], a1 = l[1] + o[1], a2 = l[2] + o[2], a3 = l[3] + o[3];
            jb.out[row] = (a0 + a2) + (a1 + a3);
        }
    }
}

// Integer lane sums (rows x cols/32 x 8): the exact part of the product, for checking.
__global__ __launch_bounds__(256) void q2_lane_sums_kernel(Q2Job jb, int32_t* __restrict__ out) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint32_t ns = jb.cols / 32u;
    if (idx >= static_cast<uint64_t>(jb.rows) * ns * 8u) return;
    const uint32_t jl = static_cast<uint32_t>(idx % 8u);
    const uint32_t s = static_cast<uint32_t>((idx / 8u) % ns);
    const uint32_t row = static_cast<uint32_t>(idx / (8u * ns));
    const uint32_t b = s / 5u, p = s % 5u;
    int sum = 0;
    for (uint32_t k = 4u * jl; k < 4u * jl + 4u; ++k) {
        const uint32_t B = jb.w[layout_offset(row, b * 32u + k, jb.n_tiles, 2u * jb.nb)];
        sum += trit_of(B, p) * jb.acts[s * 32u + k];
    }
    out[idx] = sum;
}

// Items cost about their row's block count (the waves of an item stream their rows' blocks side by side) plus a
// fixed start (the activation staging and the first loads). Longest first, each to the least loaded workgroup (the
// lowest index among equals), then each workgroup's items in increasing order. Round robin leaves the last of a plan's
// long items (a 12288-column projection after 4096-column ones) on a few workgroups: at the Qwen3-8B-like token's 252
// projections the busiest workgroup then carries 388 blocks per row against a mean of 335, this order 337.
std::vector<uint32_t> q2_schedule(const std::vector<Q2Job>& jobs, uint32_t total_items, int num_cus) {
    const uint32_t grid = std::min<uint32_t>(total_items, static_cast<uint32_t>(std::max(num_cus, 1)));
    std::vector<std::pair<uint32_t, uint32_t>> items;  // (cost, item)
    items.reserve(total_items);
    for (const Q2Job& j : jobs)
        for (uint32_t i = 0; i < q2_items(j.rows); ++i) items.emplace_back(j.nb + 2u, j.item_begin + i);
    std::stable_sort(items.begin(), items.end(), [](const auto& x, const auto& y) { return x.first > y.first; });
    typedef std::pair<uint64_t, uint32_t> Bin;  // (load, workgroup)
    std::priority_queue<Bin, std::vector<Bin>, std::greater<Bin>> heap;
    for (uint32_t g = 0; g < grid; ++g) heap.emplace(0, g);
    std::vector<std::vector<uint32_t>> per(grid);
    for (const auto& it : items) {
        Bin b = heap.top();
        heap.pop();
        per[b.second].push_back(it.second);
        b.first += it.first;
        heap.push(b);
    }
    std::vector<uint32_t> out(grid + 1u);
    out.reserve(grid + 1u + total_items);
    for (uint32_t g = 0; g < grid; ++g) {
        std::sort(per[g].begin(), per[g].end());
        out[g + 1u] = out[g] + static_cast<uint32_t>(per[g].size());
    }
    for (uint32_t g = 0; g < grid; ++g) out.insert(out.end(), per[g].begin(), per[g].end());
    return out;
}

int launch_q2(const Q2Args& a, int num_cus, hipStream_t stream) {
    if (a.total_items == 0) return VX_OK;
    if (a.sched != nullptr && (a.jobs == nullptr || a.sched_grid == 0 || a.sched_grid > a.total_items))
        VX_FAIL(VX_ERR_INTERNAL, "a Q2_0 schedule for %u workgroups over %u items", a.sched_grid, a.total_items);
    if (a.jobs == nullptr) {
        // a lone GEMV: items of kQ2LoneWaves / 2 tiles while they fit two workgroups per CU, else the plan's form
        const uint32_t per = kQ2LoneWaves / 2u, items = (a.one.n_tiles + per - 1u) / per;
        if (items <= 2u * static_cast<uint32_t>(num_cus)) {
            Q2Args b = a;
            b.total_items = items;
            hipLaunchKernelGGL((q2_kernel<false, kQ2LoneWaves>), dim3(items), dim3(kQ2LoneWaves * 64), 0, stream, b);
        } else {
            const uint32_t grid = std::min<uint32_t>(a.total_items, static_cast<uint32_t>(num_cus));
            hipLaunchKernelGGL((q2_kernel<false, kQ2Waves>), dim3(grid), dim3(kQ2Waves * 64), 0, stream, a);
        }
        VX_HIP(hipGetLastError());
        return VX_OK;
    }
    const uint32_t grid =
        a.sched != nullptr ? a.sched_grid : std::min<uint32_t>(a.total_items, static_cast<uint32_t>(num_cus));
    hipLaunchKernelGGL((q2_kernel<true, kQ2Waves>), dim3(grid), dim3(kQ2Waves * 64), 0, stream, a);
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
