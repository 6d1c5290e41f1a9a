// Velurex ternary GEMV for gfx950 (MI355X): exact int32 products of a 1.60-bpw ternary matrix with int8 activations.
//
// Arithmetic. A velurex byte B = d0 + 3 d1 + 9 d2 + 28 d3 + 84 d4 holds five digits d = t + 1 in {0, 1, 2}
// (docs/velurex-encoding.md section 1; quintrit-core/src/pack.rs:28-58). The activations are split as x = 16 hi + lo with
// lo = x & 15 in [0, 15] and hi = x >> 4 in [-8, 7] (the 16 hi + lo split of quintrit-core/src/lut.rs:380-388, with
// lo taken unsigned so that both halves are 4-bit operands), and lo is staged as the signed nibble lo - 8. Then
//     sum_p t_p x_p = sum_p d_p (lo_p - 8) + 16 sum_p d_p hi_p + 8 sum_p d_p - sum_p x_p,
// and both digit sums are one signed dot product each of five 4-bit lanes (v_dot8c_i32_i4). The row's digit sum
// sum_p d_p is computed once per matrix and the activation sum once per staged vector. Everything is exact in int32 for
// cols <= 131072 (|sum| < 2^24, quintrit-core/src/limits.rs:7-19).
//
// Decode. The digit nibbles of every byte come from a 256-entry table in LDS (one dword per byte: d0..d4 in nibbles
// 0..4; bytes that are not velurex values map to five zero trits, like BYTE_TO_TRITS). The table is replicated 32
// times in the first half of a 256-byte LDS row per entry (copy k of entry B at byte B * 256 + 4k) and lane l reads
// copy l % 32: LDS serves a wave in two halves of 32 lanes, so the gather hits 32 distinct banks whatever the bytes
// are, and its address (B << 8) | ((l % 32) << 2) is one v_perm_b32. Per weight byte the inner loop is one v_perm, one
// ds_read_b32 and two dot products.
//
// Work split. The device layout (vx_layout) stores rows in tiles of 64 (lane = row) and interleaves 16-byte chunks of
// 16 consecutive tiles, so one workgroup of 16 waves that processes a tile group reads 16 consecutive KiB per chunk step:
// the whole GPU sweeps memory nearly in address order. A work item is (tile group, K slice); the activations of the
// slice are staged in LDS once per item and read back as wave-uniform values. Long rows are split into K slices whose
// partial sums are written to a workspace and added by a second kernel, so no workgroup ever waits for another.
//
// Output. Writes that reach HBM while the weight stream is running cost far more than their bytes (a few MB of scattered
// stores slow a 2 GB read stream by several percent), so a workgroup keeps the results of up to kSlots items in the
// free second halves of the table rows and writes them out, non-temporally, when the slots are full and at its end.
//
// Reference path: quintrit-core/src/simd/avx512.rs:1526-1626 (production CPU kernel: table decode, exact int8/int16/
// int32 sums) and quintrit-runtime/src/layer.rs:210-254 (the fp32 epilogue out = float(acc) * (ws / as)).
#include "vx_gemv_core.h"
#include "vx_internal.h"

#include <algorithm>
#include <cstring>
#include <vector>

namespace vx {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 g_u4;
// Wave-uniform data read through the constant address space, so the compiler uses scalar loads (s_load) into SGPRs.
typedef __attribute__((address_space(4))) const Job c_job;
typedef __attribute__((address_space(4))) const int c_int;
typedef __attribute__((address_space(4))) const float c_float;

// ---- activation staging -----------------------------------------------------------------------------------------------

// Up to kStageGroups workgroups (grid-stride over the entries). Entry c (device byte-column c): dword 2c = the low
// nibbles of the five activations of the column, stored as (x & 15) ^ 8 (the signed nibble (x & 15) - 8), dword 2c+1 =
// their high nibbles x >> 4 (signed); activation p of column c is column_activation_index(cols, c, p)
// (pack.rs:230-237), zero past the end of the row and in the padding columns. The 16 int32 of the header add up to the
// sum of all activations: workgroup w writes the sum of its entries to word w, workgroup 0 zeroes the words past the
// grid.
constexpr uint32_t kStageGroups = 16;
__device__ __forceinline__ void stage_body(const int8_t* __restrict__ acts, uint32_t cols, uint32_t tbr, uint32_t dbr,
                                           uint8_t* __restrict__ staged, uint32_t group, uint32_t n_groups) {
    __shared__ int wsum[16];
    const uint32_t tid = threadIdx.x;
    const uint32_t full = cols / 160u * 32u;
    uint2* ent = reinterpret_cast<uint2*>(staged + kStageHeader);
    int sum = 0;
    for (uint32_t c = group * 1024u + tid; c < dbr; c += n_groups * 1024u) {
        uint32_t lo = 0, hi = 0;
        for (uint32_t p = 0; p < 5; ++p) {
            const uint32_t idx = c < full ? (c / 32u) * 160u + p * 32u + (c % 32u) : (cols / 160u) * 160u + 5u * (c - full) + p;
            const int x = c < tbr && idx < cols ? acts[idx] : 0;
            lo |= ((static_cast<uint32_t>(x) & 15u) ^ 8u) << (4 * p);
            hi |= (static_cast<uint32_t>(x >> 4) & 15u) << (4 * p);
            sum += x;
        }
        ent[c] = make_uint2(lo, hi);
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if ((tid & 63u) == 0) wsum[tid >> 6] = sum;
    __syncthreads();
    if (tid < 16) {
        int s = wsum[tid];
        for (int off = 8; off > 0; off >>= 1) s += __shfl_xor(s, off, 16);
        int* hdr = reinterpret_cast<int*>(staged);
        if (tid == 0) hdr[group] = s;
        else if (group == 0 && tid >= n_groups) hdr[tid] = 0;
    }
}

__global__ __launch_bounds__(1024) void stage_kernel(const int8_t* __restrict__ acts, uint32_t cols, uint32_t tbr,
                                                     uint32_t dbr, uint8_t* __restrict__ staged) {
    stage_body(acts, cols, tbr, dbr, staged, blockIdx.x, gridDim.x);
}

// Many stagings in one launch (a plan's inputs): blockIdx.y is the staging, blockIdx.x its workgroup.
__global__ __launch_bounds__(1024) void stage_batch_kernel(const StageJob* __restrict__ jobs) {
    const uint32_t y = blockIdx.y;
    const uint32_t groups = jobs[y].groups;
    if (blockIdx.x >= groups) return;
    stage_body(jobs[y].acts, jobs[y].cols, jobs[y].tbr, jobs[y].dbr, jobs[y].staged, blockIdx.x, groups);
}

// ---- layout transform -----------------------------------------------------------------------------------------------------

// One byte of the device layout per thread: the inverse of layout_offset. Bytes past the tile row and padding rows hold
// kZeroByte; the partial last 160-trit block is re-encoded five trits per byte (pack.rs:240-256).
__global__ void device_layout_kernel(const uint8_t* __restrict__ planar, uint64_t rows, uint32_t cols, uint32_t prb,
                                     uint32_t tbr, uint32_t n_tiles, uint32_t n_chunks, uint64_t total,
                                     uint8_t* __restrict__ dst) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const uint64_t kib = idx >> 10;
    const uint32_t within = static_cast<uint32_t>(idx & 1023u);
    const uint64_t grp_kib = static_cast<uint64_t>(kTileGroup) * n_chunks;
    const uint32_t grp = static_cast<uint32_t>(kib / grp_kib);
    const uint32_t rem = static_cast<uint32_t>(kib - grp * grp_kib);
    const uint32_t T = min(static_cast<uint32_t>(kTileGroup), n_tiles - grp * kTileGroup);
    const uint32_t q = rem / T, t = rem - q * T;
    const uint64_t r = static_cast<uint64_t>(grp * kTileGroup + t) * kTileRows + (within >> 4);
    const uint32_t c = q * kChunk + (within & 15u);
    uint8_t v = kZeroByte;
    if (r < rows && c < tbr) {
        const uint8_t* src = planar + r * prb;
        const uint32_t full = cols / 160u * 32u;
        if (c < full) {
            v = src[c];
        } else {
            const uint32_t remc = cols % 160u;
            uint32_t acc = 0, radix = 1;
            for (uint32_t k = 0; k < 5; ++k) {
                const uint32_t qq = 5u * (c - full) + k;
                const int tr = qq < remc ? trit_of(src[full + qq % 32u], qq / 32u) : 0;
                acc += static_cast<uint32_t>(tr + 1) * radix;
                radix = (k == 2) ? 28u : radix * 3u;
            }
            v = static_cast<uint8_t>(acc);
        }
    }
    dst[idx] = v;
}

__global__ void find_invalid_kernel(const uint8_t* __restrict__ planar, uint64_t n, unsigned long long* __restrict__ first) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (!byte_valid(planar[i])) atomicMin(first, static_cast<unsigned long long>(i));
}

// One row per thread: the sum of the digits (t + 1) of the five trits of every device byte of the row, padding bytes
// included (their activations are zero, staged as low nibble -8, so the correction 8 * dsum cancels them). A lane reads
// its row's 16 bytes of a chunk at once (the 64 lanes of a wave read one contiguous KiB) and looks the byte sums up in
// an LDS table.
__global__ __launch_bounds__(256) void digit_sum_kernel(const uint8_t* __restrict__ w, uint32_t padded_rows,
                                                        uint32_t n_tiles, uint32_t n_chunks, int32_t* __restrict__ dsum) {
    __shared__ uint8_t tab[256];
    {
        const uint32_t e = digit_nibbles(static_cast<uint8_t>(threadIdx.x));
        tab[threadIdx.x] = static_cast<uint8_t>((e & 15u) + ((e >> 4) & 15u) + ((e >> 8) & 15u) + ((e >> 12) & 15u) +
                                                ((e >> 16) & 15u));
    }
    __syncthreads();
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= padded_rows) return;
    int s = 0;
    for (uint32_t q = 0; q < n_chunks; ++q) {
        const uint4 v = *reinterpret_cast<const uint4*>(w + layout_offset(r, q * kChunk, n_tiles, n_chunks));
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 16; ++k) s += tab[(d[k >> 2] >> (8 * (k & 3))) & 255u];
    }
    dsum[r] = s;
}

__global__ void fill_f32_kernel(float* __restrict__ out, uint32_t n, float v) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = v;
}

// ---- GEMV -----------------------------------------------------------------------------------------------------------

// The fp32 multiplier of a job: weight_scale / act_scale, one division per job as in layer.rs:246-253; a scale that is
// not > 0 (NaN included) makes the output zero.
__device__ __forceinline__ float job_post(const Job& jb, bool* zero) {
    *zero = false;
    if (jb.out_kind == kOutF32Post) return jb.post;
    if (jb.out_kind != kOutF32Dev) return 1.0f;
    const float as = *(const c_float*)(jb.act_scale);
    *zero = !(as > 0.0f);
    return *zero ? 0.0f : jb.weight_scale / as;
}

__device__ __forceinline__ float out_value(const Job& jb, int acc, float post, bool zero) {
    return zero ? 0.0f : static_cast<float>(acc) * post;
}

__device__ __forceinline__ void store_out(const Job& jb, uint32_t row, int acc, float post, bool zero) {
    if (row >= jb.rows) return;
    if (jb.out_kind == kOutI32) __builtin_nontemporal_store(acc, static_cast<int32_t*>(jb.out) + row);
    else __builtin_nontemporal_store(out_value(jb, acc, post, zero), static_cast<float*>(jb.out) + row);
}

// The sum of all activations: the 16 words of the staged header.
__device__ __forceinline__ int staged_sum(const Job& jb) {
    const c_int* h = (const c_int*)(jb.staged);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += h[i];
    return s;
}

// The integer result of row `row` from the two dot-product accumulators summed over all K slices: lo holds
// sum d (l - 8) with l = x & 15, hi holds sum d (x >> 4), so sum t x = 16 hi + lo + 8 sum d - sum x.
__device__ __forceinline__ int row_result(const Job& jb, uint32_t row, int lo_plus_16hi) {
    return lo_plus_16hi + 8 * jb.dsum[row] - staged_sum(jb);
}


constexpr int kWaves = 16;   // waves per workgroup = tiles per group
constexpr int kGroup = 4;    // chunks loaded together by a wave
constexpr int kSlots = 8;    // items whose results a workgroup holds in LDS (1024 rows each: 32 of the 128-byte holes)

// Where the results of a held item go: kOutI32/kOutF32* rows of `out` or one K slice of `part`, 4 bytes per row.
struct Held {
    void* dst;       // first row of the item's tile group
    uint32_t count;  // rows to write (the tile group, clipped to the matrix)
    uint32_t pad;
};

// LDS byte offset of row r (0..1023) of held slot s: the second half of table row s * 32 + r / 32.
__device__ __forceinline__ uint32_t held_offset(uint32_t s, uint32_t r) {
    return ((s * 32u + (r >> 5)) << 8) + 128u + ((r & 31u) << 2);
}

typedef __attribute__((address_space(3))) const u32x4 l_u4;

// Writes the n held items that precede ring position `end` (slots (end - n) % kSlots ... (end - 1) % kSlots). A unit of
// work is 256 rows of one item (one 16-byte load from LDS and one 16-byte store per lane); wave w takes units w, w + 16.
__device__ __forceinline__ void flush_held(const char* lds, const Held* held, uint32_t end, uint32_t n, uint32_t wave,
                                           uint32_t lane) {
    for (uint32_t u = wave; u < n * 4u; u += kWaves) {
        const uint32_t s = (end - n + u / 4u) % kSlots;
        const uint32_t r = (u % 4u) * 256u + lane * 4u;
        const Held h = held[s];
        const u32x4 v = *reinterpret_cast<l_u4*>(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)) + held_offset(s, r));
        uint32_t* d = static_cast<uint32_t*>(h.dst) + r;
        if (r + 3u < h.count && (reinterpret_cast<uintptr_t>(h.dst) & 15u) == 0) {
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(d));
        } else {
            if (r < h.count) __builtin_nontemporal_store(v.x, d);
            if (r + 1u < h.count) __builtin_nontemporal_store(v.y, d + 1);
            if (r + 2u < h.count) __builtin_nontemporal_store(v.z, d + 2);
            if (r + 3u < h.count) __builtin_nontemporal_store(v.w, d + 3);
        }
    }
}

// The staged entry of device byte-column c of a row of `cols` activations (stage_body's entry, the activations read
// directly; tbr the tile row bytes, full the byte-columns of whole 160-column blocks), and their sum added to *sum.
__device__ __forceinline__ uint2 raw_entry(const int8_t* __restrict__ acts, uint32_t cols, uint32_t tbr, uint32_t full,
                                           uint32_t c, int* sum) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (uint32_t p = 0; p < 5; ++p) {
        const uint32_t idx = c < full ? (c / 32u) * 160u + p * 32u + (c % 32u) : (cols / 160u) * 160u + 5u * (c - full) + p;
        const int x = c < tbr && idx < cols ? acts[idx] : 0;
        lo |= ((static_cast<uint32_t>(x) & 15u) ^ 8u) << (4 * p);
        hi |= (static_cast<uint32_t>(x >> 4) & 15u) << (4 * p);
        *sum += x;
    }
    return make_uint2(lo, hi);
}

// Two workgroups per CU (64 KiB table and held results + 11 KiB activations each), 8 waves per SIMD: at most 64 VGPRs.
// MANY: the jobs are a device array (a plan); otherwise the one job travels in the kernel arguments. RAW (a lone GEMV,
// args.acts): each item stages its K slice from the raw activations and subtracts the slice's activation sum from its
// sums (so the outputs need no whole-vector sum: sum t x = 16 hi + lo + 8 sum d - sum x, slice by slice).
template <bool MANY, bool RAW>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(8, 8))) void gemv_kernel(LaunchArgs args) {
    static_assert(!(MANY && RAW), "raw activations are a lone GEMV's");
    __shared__ uint32_t tab[256 * 64];  // row B: 32 copies of entry B, then 128 bytes of held results
    __shared__ uint4 acts[2][(kMaxSliceChunks + kGroup) * 8];
    __shared__ Held held[kSlots];
    __shared__ uint32_t last_slice;
    __shared__ int xsum[2][kWaves];  // RAW: the slice's activation sums per wave

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const char* tabb = reinterpret_cast<const char*>(tab);
    const uint32_t lane_off = (lane & 31u) * 4u;
    const c_job* cj = (const c_job*)(args.jobs);

    uint32_t j = 0, buf = 0;
    uint32_t done = 0, pending = 0;  // held items this workgroup has finished / of those, still in LDS
    bool built = false;              // the digit table is in LDS
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
        const uint32_t nqp = (nq + kGroup - 1) / kGroup * kGroup;
        const bool active = wave < T;
        const g_u4* wp = reinterpret_cast<const g_u4*>(0);
        size_t cs = 0;
        // The first weight group is requested before the table build, the activation staging and the barrier, so
        // its HBM latency overlaps them.
        u32x4 b[kGroup];
        if (active) {
            wp = (const g_u4*)(jb.w) + (static_cast<size_t>(grp) * kTileGroup * jb.n_chunks + static_cast<size_t>(q0) * T + wave) * 64u + lane;
            cs = static_cast<size_t>(T) * 64u;  // chunk stride of a tile, in uint4
#pragma unroll
            for (int i = 0; i < kGroup; ++i) b[i] = __builtin_nontemporal_load(wp + min(static_cast<uint32_t>(i), nq - 1u) * cs);
        }
        if (!built) {
            built = true;
            for (uint32_t i = tid; i < 256u * 8u; i += kWaves * 64u) {  // 8 uint4 stores per entry
                const uint32_t e = digit_nibbles(i >> 3);
                *reinterpret_cast<uint4*>(reinterpret_cast<char*>(tab) + (i >> 3) * 256u + (i & 7u) * 16u) = make_uint4(e, e, e, e);
            }
        }
        // Stage this slice's activations (zero past nq, so the clamped tail loads add nothing).
        uint4* ab = acts[buf];
        if constexpr (RAW) {
            uint2* ae = reinterpret_cast<uint2*>(ab);
            const uint32_t full = args.cols / 160u * 32u;
            int xs = 0;
            for (uint32_t i = tid; i < nqp * 16u; i += kWaves * 64u)
                ae[i] = i < nq * 16u ? raw_entry(args.acts, args.cols, jb.tbr, full, q0 * 16u + i, &xs) : make_uint2(0, 0);
            for (int off = 32; off > 0; off >>= 1) xs += __shfl_xor(xs, off);
            if (lane == 0) xsum[buf][wave] = xs;
        } else {
            const uint4* src = reinterpret_cast<const uint4*>(jb.staged + kStageHeader) + static_cast<size_t>(q0) * 8u;
            for (uint32_t i = tid; i < nqp * 8u; i += kWaves * 64u) ab[i] = i < nq * 8u ? src[i] : make_uint4(0, 0, 0, 0);
        }
        // A lone GEMV's split item adds its sums atomically; the last slice of the tile group writes the outputs.
        const bool fold = !MANY && jb.kslices > 1 && jb.accum != nullptr;
        const uint32_t slot = done % kSlots;
        if (tid == 0 && !fold) {
            const size_t first = static_cast<size_t>(grp) * kTileGroup * kTileRows;
            Held h;
            if (jb.kslices == 1) {
                h.dst = static_cast<uint32_t*>(jb.out) + first;
                h.count = static_cast<uint32_t>(min(static_cast<size_t>(kTileGroup * kTileRows), jb.rows - first));
            } else {
                h.dst = jb.part + static_cast<size_t>(ks) * jb.padded_rows + first;
                h.count = static_cast<uint32_t>(min(static_cast<size_t>(kTileGroup * kTileRows), jb.padded_rows - first));
            }
            h.pad = 0;
            held[slot] = h;
        }
        __syncthreads();
        // Every slot but this item's is full: write them out (their results and descriptors precede the barrier).
        if (pending == kSlots - 1) {
            flush_held(tabb, held, done, pending, wave, lane);
            pending = 0;
        }

        if (active) {
            int acc_lo = 0, acc_hi = 0;
            for (uint32_t g = 0; g < nq; g += kGroup) {
                if (g) {
#pragma unroll
                    for (int i = 0; i < kGroup; ++i) b[i] = __builtin_nontemporal_load(wp + min(g + i, nq - 1u) * cs);
                }
#pragma unroll
                for (int i = 0; i < kGroup; ++i) {
                    const uint32_t dw[4] = {b[i].x, b[i].y, b[i].z, b[i].w};
                    // this lane's activation entry: byte-column lane % 16 of the chunk (the same in all four rows)
                    const uint2 e = reinterpret_cast<const uint2*>(ab)[(g + i) * 16u + (lane & 15u)];
                    __builtin_amdgcn_sched_barrier(0);
                    uint32_t t[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k) {
                        const uint32_t addr =
                            __builtin_amdgcn_perm(dw[k >> 2], lane_off, 0x0c0c0000u | ((4u + (k & 3)) << 8));
                        t[k] = *reinterpret_cast<const uint32_t*>(tabb + addr);
                    }
                    dot4_bcast<0>(acc_lo, acc_hi, e.x, e.y, t[0], t[1], t[2], t[3]);
                    dot4_bcast<4>(acc_lo, acc_hi, e.x, e.y, t[4], t[5], t[6], t[7]);
                    dot4_bcast<8>(acc_lo, acc_hi, e.x, e.y, t[8], t[9], t[10], t[11]);
                    dot4_bcast<12>(acc_lo, acc_hi, e.x, e.y, t[12], t[13], t[14], t[15]);
                }
            }
            int v = acc_lo + 16 * acc_hi;
            if constexpr (RAW) {
#pragma unroll
                for (int w = 0; w < kWaves; ++w) v -= xsum[buf][w];
            }
            const uint32_t r = wave * kTileRows + lane;  // row within the tile group
            const uint32_t row = grp * kTileGroup * kTileRows + r;
            if (fold) atomicAdd(jb.accum + row, v);
            uint32_t word = static_cast<uint32_t>(v);
            if (jb.kslices == 1 && row < jb.rows) {
                const int acc = RAW ? v + 8 * jb.dsum[row] : row_result(jb, row, v);
                if (jb.out_kind == kOutI32) {
                    word = static_cast<uint32_t>(acc);
                } else {
                    bool zero;
                    const float post = job_post(jb, &zero);
                    word = __float_as_uint(out_value(jb, acc, post, zero));
                }
            }
            if (!fold) *reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(tab) + held_offset(slot, r)) = word;
        }
        if (!fold) {
            ++done;
            ++pending;
            continue;
        }
        // The sums are complete at the atomics' coherence point before the ticket is taken (every memory operation of
        // every wave waited for, then the barrier: take_ticket's hand-off), and the last slice reads them with atomics
        // after its ticket: no cache writeback.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) last_slice = take_ticket(jb.tickets + grp, jb.kslices - 1u);
        __syncthreads();
        if (last_slice != 0u) {
            const uint32_t row = grp * kTileGroup * kTileRows + wave * kTileRows + lane;
            if (active) {
                const int total = atomicExch(jb.accum + row, 0);
                if (row < jb.rows) {
                    bool zero;
                    const float post = job_post(jb, &zero);
                    store_out(jb, row, RAW ? total + 8 * jb.dsum[row] : row_result(jb, row, total), post, zero);
                }
            }
            if (tid == 0) atomicExch(jb.tickets + grp, 0u);
        }
    }
    __syncthreads();
    flush_held(tabb, held, done, pending, wave, lane);
    if constexpr (!MANY) {
        if (args.flag != nullptr) {
            // Every output this workgroup wrote has been performed before its ticket (the hand-off of take_ticket); the
            // last ticket's holder clears the counter and publishes the call's sequence number to the host.
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid == 0 && take_ticket(args.done, gridDim.x - 1u)) {
                atomicExch(args.done, 0u);
                __hip_atomic_store(args.flag, args.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
    }
}

// Adds the K-slice partial sums of the split jobs and applies their epilogue. Block = 64 rows x 4 waves; wave w adds
// the slices w, w + 4, ... of its 64 rows, then the 4 waves combine through LDS. blockIdx.y indexes `split` (the
// plan's split jobs) or, without a job array, the one job.
template <bool MANY>
__global__ __launch_bounds__(256) void finish_kernel(LaunchArgs args, const uint32_t* __restrict__ split) {
    __shared__ int red[4][64];
    Job jb;
    if (MANY) __builtin_memcpy(&jb, (const Job*)((const c_job*)(args.jobs) + split[blockIdx.y]), sizeof(Job));
    else jb = args.one;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t row0 = blockIdx.x * 64u;
    if (row0 >= jb.rows) return;
    const uint32_t row = row0 + lane;
    const int32_t* p = jb.part + row;
    int s = 0;
    uint32_t k = wave;
    for (; k + 12 < jb.kslices; k += 16)
        s += p[static_cast<size_t>(k) * jb.padded_rows] + p[static_cast<size_t>(k + 4) * jb.padded_rows] +
             p[static_cast<size_t>(k + 8) * jb.padded_rows] + p[static_cast<size_t>(k + 12) * jb.padded_rows];
    for (; k < jb.kslices; k += 4) s += p[static_cast<size_t>(k) * jb.padded_rows];
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0) {
        s = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
        bool zero;
        const float post = job_post(jb, &zero);
        store_out(jb, row, row_result(jb, row, s), post, zero);
    }
}

// ---- host side ---------------------------------------------------------------------------------------------------------------

void plan_job(Job& j, const Geometry& g, uint32_t target_items, uint32_t min_slice_chunks) {
    const uint32_t nc = static_cast<uint32_t>(g.n_chunks);
    const uint32_t groups = static_cast<uint32_t>(g.n_groups);
    uint32_t ks = (nc + kMaxSliceChunks - 1) / kMaxSliceChunks;
    if (target_items) {
        const uint32_t most = std::max(nc / std::max(min_slice_chunks, 1u), 1u);  // slices of min_slice_chunks at most
        ks = std::max(ks, std::min(most, (target_items + groups - 1) / groups));
    }
    const uint32_t sc = (nc + ks - 1) / ks;
    j.slice_chunks = sc;
    j.kslices = (nc + sc - 1) / sc;
    j.rows = static_cast<uint32_t>(g.rows);
    j.padded_rows = static_cast<uint32_t>(g.padded_rows);
    j.n_tiles = static_cast<uint32_t>(g.n_tiles);
    j.n_chunks = nc;
}

uint32_t stage_groups(size_t cols) {
    return static_cast<uint32_t>(std::max<size_t>(1, std::min<size_t>(kStageGroups, (device_row_bytes(cols) + 1023) / 1024)));
}

int launch_stage_batch(const StageJob* jobs, uint32_t n, uint32_t max_groups, hipStream_t stream) {
    if (n == 0) return VX_OK;
    hipLaunchKernelGGL(stage_batch_kernel, dim3(max_groups, n), dim3(1024), 0, stream, jobs);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_stage(const int8_t* acts, size_t cols, uint8_t* staged, hipStream_t stream) {
    const uint32_t groups = stage_groups(cols);
    hipLaunchKernelGGL(stage_kernel, dim3(std::max(groups, 1u)), dim3(1024), 0, stream, acts, static_cast<uint32_t>(cols),
                       static_cast<uint32_t>(tile_row_bytes(cols)), static_cast<uint32_t>(device_row_bytes(cols)), staged);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_gemv(const LaunchArgs& a, uint32_t max_rows, const uint32_t* split, uint32_t n_split, int num_cus,
                hipStream_t stream) {
    if (a.total_items == 0) return VX_OK;
    if (a.flag != nullptr && (a.jobs != nullptr || n_split != 0))
        VX_FAIL(VX_ERR_INTERNAL, "a completion flag on a launch whose outputs are not all written by gemv_kernel");
    if (a.acts != nullptr && (a.jobs != nullptr || n_split != 0 || (a.one.kslices > 1 && a.one.accum == nullptr)))
        VX_FAIL(VX_ERR_INTERNAL, "raw activations on a launch that is not a lone GEMV with atomic slice sums");
    const uint32_t grid = std::min<uint32_t>(a.total_items, 2u * static_cast<uint32_t>(num_cus));
    if (a.jobs) hipLaunchKernelGGL((gemv_kernel<true, false>), dim3(grid), dim3(kWaves * 64), 0, stream, a);
    else if (a.acts) hipLaunchKernelGGL((gemv_kernel<false, true>), dim3(grid), dim3(kWaves * 64), 0, stream, a);
    else hipLaunchKernelGGL((gemv_kernel<false, false>), dim3(grid), dim3(kWaves * 64), 0, stream, a);
    VX_HIP(hipGetLastError());
    if (n_split) {
        const dim3 fgrid((max_rows + 63u) / 64u, n_split);
        if (a.jobs) hipLaunchKernelGGL(finish_kernel<true>, fgrid, dim3(256), 0, stream, a, split);
        else hipLaunchKernelGGL(finish_kernel<false>, fgrid, dim3(256), 0, stream, a, split);
        VX_HIP(hipGetLastError());
    }
    return VX_OK;
}

int launch_device_layout(const uint8_t* planar_dev, const Geometry& g, uint8_t* dst, hipStream_t stream) {
    const uint64_t total = g.device_bytes;
    const uint64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(device_layout_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, planar_dev,
                       static_cast<uint64_t>(g.rows), static_cast<uint32_t>(g.cols),
                       static_cast<uint32_t>(planar_row_bytes(g.cols)), static_cast<uint32_t>(g.tbr),
                       static_cast<uint32_t>(g.n_tiles), static_cast<uint32_t>(g.n_chunks), total, dst);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_digit_sums(const uint8_t* w, const Geometry& g, int32_t* dsum, hipStream_t stream) {
    const uint32_t rows = static_cast<uint32_t>(g.padded_rows);
    hipLaunchKernelGGL(digit_sum_kernel, dim3((rows + 255u) / 256u), dim3(256), 0, stream, w, rows,
                       static_cast<uint32_t>(g.n_tiles), static_cast<uint32_t>(g.n_chunks), dsum);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_find_invalid(const uint8_t* planar_dev, uint64_t n, unsigned long long* first, hipStream_t stream) {
    const uint64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(find_invalid_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, planar_dev, n, first);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_fill_f32(float* out, size_t n, float v, hipStream_t stream) {
    const uint32_t nn = static_cast<uint32_t>(n);
    hipLaunchKernelGGL(fill_f32_kernel, dim3((nn + 255u) / 256u), dim3(256), 0, stream, out, nn, v);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

size_t find_invalid_byte(const uint8_t* planar, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!byte_valid(planar[i])) return i;
    return SIZE_MAX;
}

static inline uint8_t pack5(const int t[5]) {
    return static_cast<uint8_t>((t[0] + 1) + 3 * (t[1] + 1) + 9 * (t[2] + 1) + 28 * (t[3] + 1) + 84 * (t[4] + 1));
}

void planar_to_device_layout(const uint8_t* planar, const Geometry& g, uint8_t* dst) {
    const size_t prb = planar_row_bytes(g.cols);
    const size_t full = tile_full_columns(g.cols);
    const size_t rem = g.cols % kQK5;
    std::vector<uint8_t> row(g.dbr);
    for (size_t r = 0; r < g.padded_rows; ++r) {
        if (r < g.rows) {
            const uint8_t* src = planar + r * prb;
            std::memcpy(row.data(), src, full);
            for (size_t c = full; c < g.tbr; ++c) {  // packed tail (pack.rs:240-256)
                int t[5] = {0, 0, 0, 0, 0};
                for (size_t k = 0; k < 5; ++k) {
                    const size_t q = 5 * (c - full) + k;
                    if (q < rem) t[k] = trit_of(src[full + q % kBlockBytes], static_cast<uint32_t>(q / kBlockBytes));
                }
                row[c] = pack5(t);
            }
            for (size_t c = g.tbr; c < g.dbr; ++c) row[c] = kZeroByte;
        } else {
            std::memset(row.data(), kZeroByte, g.dbr);
        }
        for (size_t q = 0; q < g.n_chunks; ++q)
            std::memcpy(dst + layout_offset(r, static_cast<uint32_t>(q * kChunk), static_cast<uint32_t>(g.n_tiles),
                                            static_cast<uint32_t>(g.n_chunks)),
                        row.data() + q * kChunk, kChunk);
    }
}

}  // namespace vx
