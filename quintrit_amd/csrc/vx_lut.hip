// Velurex GEMV through the reference's compact activation tables, for gfx950 (MI355X): the table decode of the
// production CPU kernel (quintrit-core/src/simd/avx512.rs:1178-1292 tables and decode, 1526-1604 the row loop) on the
// GPU, beside the digit-table kernel of vx_gemv.hip. Both give the exact int32 products; they differ in how a weight
// byte meets its five activations.
//
// Tables (compact_lut_kernel). Per device byte-column c and part (lo, hi) one 64-byte table, the layout of
// build_compact_wide_impl (avx512.rs:1216-1247): entry s < 9 is t3 a3 + t4 a4 for the 2-trit group U = s (t3 = s % 3 - 1,
// t4 = s / 3 - 1), entry 9 + L (L < 27) is t0 a0 + t1 a1 + t2 a2 for the 3-trit group L (t0 = L % 3 - 1,
// t1 = L / 3 % 3 - 1, t2 = L / 9 - 1), entries 36..63 are zero; a_p is the part of activation
// column_activation_index(cols, c, p) (pack.rs:230-237) split as x = 16 hi + lo with lo = ((x + 8) & 15) - 8 and
// hi = (x - lo) >> 4 (lut.rs:380-388). The lo tables of all columns come first, then the hi tables: 2 * tbr * 64 bytes,
// int8 entries (|entry| <= 24).
//
// Decode (gemv_lut_kernel). A byte B splits without a division into U = floor(B / 28) and L = B - 28 U
// (avx512.rs:1256-1292 decodes U from i = B >> 2 as floor(i / 7)). Here four bytes of a dword at once: i = (B >> 2) & 63
// per byte, floor(i / 7) = (37 i) >> 8 for i < 64, computed for the even and the odd bytes as two 16-bit products of one
// 24-bit multiply each and gathered with one v_perm; 28 U = ((U << 3) - U) << 2 and L + 9 = B - 28 U + 9 stay inside
// their bytes (U <= 8, L + 9 <= 35), so no carry crosses a byte. The two lookups per byte read entries U and 9 + L of
// the column's table, staged in LDS as int32 lo + 16 hi (the same exact sum the CPU kernel forms from its two int8
// parts, avx512.rs:1580-1600): a row's result is the plain int32 sum of its lookups, with no correction terms.
//
// LDS layout. A K slice of up to kLutSlice 16-byte chunks (16 byte-columns each) is staged per work item: column k of
// chunk q at byte q * kLutChunk + k * kLutCol, 36 int32 entries. kLutChunk = 2304 = 9 * 256, so every chunk starts on
// a 256-byte boundary and the address of a lookup is one v_perm of the entry offset (4 x index < 256, one byte of the
// SWAR result) with the chunk's base, plus the column's constant offset in the load instruction. A wave reads one
// column at a time (the 64 lanes are 64 rows of the same byte-column) and the entries of a column are consecutive
// dwords: the gather never conflicts on an LDS bank.
//
// Work split, K slices and outputs are those of the digit-table GEMV: (tile group, K slice) work items on
// 16-wave workgroups, the device layout's 16-byte chunks; a plan's split jobs write int32 slice sums that a finish
// kernel adds, a lone call adds them atomically and the last slice of each tile group writes the outputs.
#include "vx_internal.h"

#include <algorithm>

namespace vx {

typedef unsigned int lu32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const lu32x4 lg_u4;
typedef __attribute__((address_space(4))) const Job lc_job;
typedef __attribute__((address_space(4))) const float lc_float;

constexpr uint32_t kLutSlice = 16;                  // chunks per K slice
constexpr uint32_t kLutCol = 36 * 4;                // LDS bytes per byte-column: 36 int32 entries
constexpr uint32_t kLutChunk = 16 * kLutCol;        // 2304 = 9 * 256
constexpr uint32_t kLutBuf = kLutSlice * kLutChunk;  // one slice's tables (36 KiB; two per workgroup)
constexpr int kLutWaves = 16;
constexpr int kLutGroup = 4;                        // chunks loaded together by a wave
static_assert(kLutChunk % 256 == 0 && kLutBuf % 256 == 0, "chunk tables start on 256-byte boundaries");

// ---- tables -----------------------------------------------------------------------------------------------------------

// One thread per (column, part, 16-byte quarter of the 64-byte table).
__global__ __launch_bounds__(256) void compact_lut_kernel(const int8_t* __restrict__ acts, uint32_t cols, uint32_t tbr,
                                                          int8_t* __restrict__ lut) {
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    const uint32_t quarter = idx & 3u, part = (idx >> 2) & 1u, c = idx >> 3;
    if (c >= tbr) return;
    const uint32_t full = cols / 160u * 32u;
    int a[5];
#pragma unroll
    for (uint32_t p = 0; p < 5; ++p) {
        const uint32_t i = c < full ? (c / 32u) * 160u + p * 32u + (c % 32u) : (cols / 160u) * 160u + 5u * (c - full) + p;
        const int x = i < cols ? acts[i] : 0;
        const int lo = ((x + 8) & 15) - 8;
        a[p] = part ? (x - lo) >> 4 : lo;
    }
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (uint32_t k = 0; k < 16; ++k) {
        const uint32_t s = quarter * 16u + k;
        int v = 0;
        if (s < 9u) {
            v = (static_cast<int>(s % 3u) - 1) * a[3] + (static_cast<int>(s / 3u) - 1) * a[4];
        } else if (s < 36u) {
            const uint32_t l = s - 9u;
            v = (static_cast<int>(l % 3u) - 1) * a[0] + (static_cast<int>(l / 3u % 3u) - 1) * a[1] +
                (static_cast<int>(l / 9u) - 1) * a[2];
        }
        w[k >> 2] |= (static_cast<uint32_t>(v) & 0xffu) << (8u * (k & 3u));
    }
    *reinterpret_cast<uint4*>(lut + static_cast<size_t>(part) * tbr * 64u + static_cast<size_t>(c) * 64u + quarter * 16u) =
        make_uint4(w[0], w[1], w[2], w[3]);
}

// ---- GEMV ---------------------------------------------------------------------------------------------------------------

// weight_scale / act_scale for an fp32 job (layer.rs:246-253); a scale that is not > 0 (NaN included) gives zeros.
__device__ __forceinline__ float lut_post(const Job& jb, bool* zero) {
    *zero = false;
    if (jb.out_kind == kOutF32Post) return jb.post;
    if (jb.out_kind != kOutF32Dev) return 1.0f;
    const float as = *(const lc_float*)(jb.act_scale);
    *zero = !(as > 0.0f);
    return *zero ? 0.0f : jb.weight_scale / as;
}

__device__ __forceinline__ void lut_store(const Job& jb, uint32_t row, int acc) {
    if (row >= jb.rows) return;
    if (jb.out_kind == kOutI32) {
        __builtin_nontemporal_store(acc, static_cast<int32_t*>(jb.out) + row);
        return;
    }
    bool zero;
    const float post = lut_post(jb, &zero);
    __builtin_nontemporal_store(zero ? 0.0f : static_cast<float>(acc) * post, static_cast<float*>(jb.out) + row);
}

// The sum of the lookups of one dword of weights (byte-columns 4 D .. 4 D + 3 of the chunk whose tables start at gb).
template <int D>
__device__ __forceinline__ int lut_dword(const char* tabs, uint32_t w, uint32_t gb) {
    const uint32_t i6 = (w >> 2) & 0x3f3f3f3fu;
    const uint32_t pe = __umul24(i6 & 0x00ff00ffu, 37u);         // bytes 1, 3: floor(i / 7) of bytes 0, 2
    const uint32_t po = __umul24((i6 >> 8) & 0x00ff00ffu, 37u);  // bytes 1, 3: floor(i / 7) of bytes 1, 3
    const uint32_t u = __builtin_amdgcn_perm(po, pe, 0x07030501u);
    const uint32_t u7 = (u << 3) - u;
    const uint32_t al = ((w - (u7 << 2)) + 0x09090909u) << 2;  // 4 (9 + L) per byte
    const uint32_t au = u << 2;                                  // 4 U per byte
    int s = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t sel = 0x0c020100u | static_cast<uint32_t>(4 + b);
        const uint32_t xu = __builtin_amdgcn_perm(au, gb, sel);
        const uint32_t xl = __builtin_amdgcn_perm(al, gb, sel);
        const uint32_t col = static_cast<uint32_t>(4 * D + b) * kLutCol;
        s += *reinterpret_cast<const int*>(tabs + xu + col) + *reinterpret_cast<const int*>(tabs + xl + col);
    }
    return s;
}

template <bool MANY>
__global__ __launch_bounds__(kLutWaves * 64) __attribute__((amdgpu_waves_per_eu(8, 8))) void gemv_lut_kernel(LaunchArgs args) {
    __shared__ __align__(256) uint32_t tab_words[2 * kLutBuf / 4];
    __shared__ uint32_t last_slice;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const char* tabs = reinterpret_cast<const char*>(tab_words);
    const lc_job* cj = (const lc_job*)(args.jobs);

    uint32_t j = 0, buf = 0;
    for (uint32_t item = blockIdx.x; item < args.total_items; item += gridDim.x, buf ^= 1u) {
        if (MANY)
            while (j + 1 < args.n_jobs && item >= cj[j + 1].item_begin) ++j;
        Job jb;
        if (MANY) __builtin_memcpy(&jb, (const Job*)(cj + j), sizeof(Job));
        else jb = args.one;
        const uint32_t local = item - jb.item_begin;
        const uint32_t grp = local / jb.kslices, ks = local - grp * jb.kslices;
        const uint32_t T = min(static_cast<uint32_t>(kTileGroup), jb.n_tiles - grp * kTileGroup);
        const uint32_t q0 = ks * jb.slice_chunks;
        const uint32_t nq = min(jb.slice_chunks, jb.n_chunks - q0);
        const uint32_t nqp = (nq + kLutGroup - 1) / kLutGroup * kLutGroup;
        const bool active = wave < T;
        const lg_u4* wp = reinterpret_cast<const lg_u4*>(0);
        size_t cs = 0;
        // The first weight group goes out before the tables are staged, so its HBM latency overlaps the staging.
        lu32x4 b[kLutGroup];
        if (active) {
            wp = (const lg_u4*)(jb.w) + (static_cast<size_t>(grp) * kTileGroup * jb.n_chunks + static_cast<size_t>(q0) * T + wave) * 64u + lane;
            cs = static_cast<size_t>(T) * 64u;
#pragma unroll
            for (int i = 0; i < kLutGroup; ++i) b[i] = __builtin_nontemporal_load(wp + min(static_cast<uint32_t>(i), nq - 1u) * cs);
        }
        // Stage the slice's tables as int32 lo + 16 hi: task (chunk, column, dword of 4 entries); chunks past nq (the
        // clamped tail loads) and byte-columns past the tile row (padding bytes) get zero tables.
        {
            const uint32_t* lo_tab = reinterpret_cast<const uint32_t*>(jb.staged);
            const uint32_t* hi_tab = lo_tab + static_cast<size_t>(jb.tbr) * 16u;
            char* dst = reinterpret_cast<char*>(tab_words) + buf * kLutBuf;
            for (uint32_t e = tid; e < nqp * 144u; e += kLutWaves * 64u) {
                const uint32_t qc = e / 144u, r = e - qc * 144u, col = r / 9u, d = r - col * 9u;
                const uint32_t c = (q0 + qc) * 16u + col;
                uint32_t lo = 0, hi = 0;
                if (qc < nq && c < jb.tbr) {
                    lo = lo_tab[static_cast<size_t>(c) * 16u + d];
                    hi = hi_tab[static_cast<size_t>(c) * 16u + d];
                }
                int v[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    v[k] = __builtin_amdgcn_sbfe(static_cast<int>(lo), 8 * k, 8) + 16 * __builtin_amdgcn_sbfe(static_cast<int>(hi), 8 * k, 8);
                *reinterpret_cast<int4*>(dst + qc * kLutChunk + col * kLutCol + d * 16u) = make_int4(v[0], v[1], v[2], v[3]);
            }
        }
        const bool fold = !MANY && jb.kslices > 1 && jb.accum != nullptr;
        __syncthreads();

        if (active) {
            int acc = 0;
            for (uint32_t g = 0; g < nq; g += kLutGroup) {
                if (g) {
#pragma unroll
                    for (int i = 0; i < kLutGroup; ++i) b[i] = __builtin_nontemporal_load(wp + min(g + i, nq - 1u) * cs);
                }
#pragma unroll
                for (int i = 0; i < kLutGroup; ++i) {
                    const uint32_t gb = buf * kLutBuf + (g + i) * kLutChunk;
                    acc += lut_dword<0>(tabs, b[i].x, gb);
                    acc += lut_dword<1>(tabs, b[i].y, gb);
                    acc += lut_dword<2>(tabs, b[i].z, gb);
                    acc += lut_dword<3>(tabs, b[i].w, gb);
                }
            }
            const uint32_t row = grp * kTileGroup * kTileRows + wave * kTileRows + lane;
            if (jb.kslices == 1) lut_store(jb, row, acc);
            else if (fold) atomicAdd(jb.accum + row, acc);
            else jb.part[static_cast<size_t>(ks) * jb.padded_rows + row] = acc;
        }
        if (!fold) continue;
        // The sums are complete at the atomics' coherence point before the ticket is taken (release), and the last
        // slice reads them back with atomics after its ticket (acquire).
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) last_slice = take_ticket(jb.tickets + grp, jb.kslices - 1u);
        __syncthreads();
        if (last_slice != 0u) {
            const uint32_t row = grp * kTileGroup * kTileRows + wave * kTileRows + lane;
            if (active) lut_store(jb, row, atomicExch(jb.accum + row, 0));
            if (tid == 0) atomicExch(jb.tickets + grp, 0u);
        }
    }
}

// The K-slice sums of the split jobs of a plan, added per row, then the job's epilogue (block = 256 rows; blockIdx.y
// indexes `split`).
__global__ __launch_bounds__(256) void lut_finish_kernel(LaunchArgs args, const uint32_t* __restrict__ split) {
    Job jb;
    __builtin_memcpy(&jb, (const Job*)((const lc_job*)(args.jobs) + split[blockIdx.y]), sizeof(Job));
    const uint32_t row = blockIdx.x * 256u + threadIdx.x;
    if (row >= jb.rows) return;
    const int32_t* p = jb.part + row;
    int s = 0;
    for (uint32_t k = 0; k < jb.kslices; ++k) s += p[static_cast<size_t>(k) * jb.padded_rows];
    lut_store(jb, row, s);
}

// ---- host side --------------------------------------------------------------------------------------------------------------

size_t compact_lut_bytes(size_t cols) { return 2 * tile_row_bytes(cols) * 64; }

int launch_compact_lut(const int8_t* acts, size_t cols, int8_t* lut, hipStream_t stream) {
    const uint32_t tbr = static_cast<uint32_t>(tile_row_bytes(cols));
    const uint32_t threads = tbr * 8u;
    hipLaunchKernelGGL(compact_lut_kernel, dim3((threads + 255u) / 256u), dim3(256), 0, stream, acts,
                       static_cast<uint32_t>(cols), tbr, lut);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

void plan_lut_job(Job& j, const Geometry& g, uint32_t target_items) {
    const uint32_t nc = static_cast<uint32_t>(g.n_chunks);
    const uint32_t groups = static_cast<uint32_t>(g.n_groups);
    uint32_t ks = (nc + kLutSlice - 1) / kLutSlice;
    if (target_items) ks = std::max(ks, std::min(nc, (target_items + groups - 1) / groups));
    const uint32_t sc = (nc + ks - 1) / ks;
    j.slice_chunks = sc;
    j.kslices = (nc + sc - 1) / sc;
    j.rows = static_cast<uint32_t>(g.rows);
    j.padded_rows = static_cast<uint32_t>(g.padded_rows);
    j.n_tiles = static_cast<uint32_t>(g.n_tiles);
    j.n_chunks = nc;
    j.tbr = static_cast<uint32_t>(g.tbr);
}

int launch_gemv_lut(const LaunchArgs& a, uint32_t max_rows, const uint32_t* split, uint32_t n_split, int num_cus,
                    hipStream_t stream) {
    if (a.total_items == 0) return VX_OK;
    const uint32_t grid = std::min<uint32_t>(a.total_items, 2u * static_cast<uint32_t>(num_cus));
    if (a.jobs) hipLaunchKernelGGL(gemv_lut_kernel<true>, dim3(grid), dim3(kLutWaves * 64), 0, stream, a);
    else hipLaunchKernelGGL(gemv_lut_kernel<false>, dim3(grid), dim3(kLutWaves * 64), 0, stream, a);
    VX_HIP(hipGetLastError());
    if (n_split) {
        if (a.jobs == nullptr) VX_FAIL(VX_ERR_INTERNAL, "a lone table GEMV with split slices needs its atomic sums");
        hipLaunchKernelGGL(lut_finish_kernel, dim3((max_rows + 255u) / 256u, n_split), dim3(256), 0, stream, a, split);
        VX_HIP(hipGetLastError());
    }
    return VX_OK;
}

}  // namespace vx
