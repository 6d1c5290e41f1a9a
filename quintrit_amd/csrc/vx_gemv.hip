// Velurex ternary GEMV for gfx950 (MI355X): exact int32 products of a 1.60-bpw ternary matrix with int8 activations.
//
// Hot loop (one wavefront = one tile of 64 rows, lane = row):
//   * every lane streams its row with 16-byte loads (global_load_dwordx4); the 64 lanes of a wave read 1 KiB of
//     contiguous HBM per load, because the device layout interleaves the 64 rows of a tile in 16-byte chunks;
//   * each weight byte B is decoded by one lookup in a byte-indexed LDS table that holds the five trits of B as two
//     dwords (t0..t3 packed int8, t4 in byte 0). The table is replicated 32 times, entry B of copy k at B*256 + k*8,
//     so lane l always reads banks 2(l%32), 2(l%32)+1: the lookup is free of bank conflicts whatever the bytes are.
//     The address (B << 8) | (l%32)*8 is one v_perm_b32;
//   * the activations of a byte-column are the same for all 64 lanes and are read with scalar loads from a staging
//     buffer (two dwords per byte-column: a0..a3 and a4), so the products are two v_dot4c_i32_i8 per byte with an
//     SGPR operand.
// Rows of a tile are summed over the byte-columns of a K slice; the waves of a workgroup split the slice and add their
// partial sums through LDS; slices of one tile meet in int32 accumulators (exact, order-free) and the workgroup that
// arrives last writes the result and clears the accumulators for the next call.
//
// Reference path: quintrit-core/src/simd/avx512.rs:1526-1626 (production CPU kernel) and quintrit-runtime/src/layer.rs:
// 210-254 (epilogue). The per-column activation tables of the CPU kernel are replaced by this byte-indexed trit table:
// on CDNA4 a dot-product unit with a wave-uniform operand is cheaper than two table lookups per byte.
#include "vx_internal.h"

#include <algorithm>
#include <cstring>
#include <vector>

namespace vx {

// ---- the trit table -------------------------------------------------------------------------------------------------

struct TritTable {
    uint32_t w[256][2];
};

// Entry B: (t0 | t1 << 8 | t2 << 16 | t3 << 24, t4) for the 243 velurex bytes (docs/velurex-encoding.md section 1,
// B = d0 + 3 d1 + 9 d2 + 28 d3 + 84 d4, t = d - 1); every other byte maps to zero trits, like BYTE_TO_TRITS
// (quintrit-core/src/pack.rs:41-58).
constexpr TritTable make_trit_table() {
    TritTable t{};
    for (int s = 0; s < 243; ++s) {
        int d[5] = {0, 0, 0, 0, 0};
        int v = s;
        for (int p = 0; p < 5; ++p) {
            d[p] = v % 3;
            v /= 3;
        }
        const int b = d[0] + 3 * d[1] + 9 * d[2] + 28 * d[3] + 84 * d[4];
        uint32_t lo = 0;
        for (int p = 0; p < 4; ++p) lo |= static_cast<uint32_t>(static_cast<uint8_t>(d[p] - 1)) << (8 * p);
        t.w[b][0] = lo;
        t.w[b][1] = static_cast<uint32_t>(static_cast<uint8_t>(d[4] - 1));
    }
    return t;
}

__constant__ TritTable kTritTable = make_trit_table();

constexpr int kCopies = 32;                       // table replicas (one per LDS bank pair of a half-wave)

// ---- activation staging -----------------------------------------------------------------------------------------------

// Entry c (device byte-column c) = (a(c,0) | a(c,1) << 8 | a(c,2) << 16 | a(c,3) << 24, a(c,4)) with a(c,p) the
// activation column_activation_index(cols, c, p) names (pack.rs:230-237), zero past the end of the row.
__global__ void act_prep_kernel(const int8_t* __restrict__ acts, uint32_t cols, uint32_t tbr, uint32_t dbr,
                                uint2* __restrict__ actp) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= dbr) return;
    uint32_t a[5] = {0, 0, 0, 0, 0};
    if (c < tbr) {
        const uint32_t full = cols / 160u * 32u;
        for (uint32_t p = 0; p < 5; ++p) {
            const uint32_t idx = c < full ? (c / 32u) * 160u + p * 32u + (c % 32u) : (cols / 160u) * 160u + 5u * (c - full) + p;
            a[p] = idx < cols ? static_cast<uint32_t>(static_cast<uint8_t>(acts[idx])) : 0u;
        }
    }
    actp[c] = make_uint2(a[0] | (a[1] << 8) | (a[2] << 16) | (a[3] << 24), a[4]);
}

// One byte of the device layout per thread (see vx_layout in include/velurex_hip.h): tiles of 64 rows, 16-byte chunks,
// the partial last 160-trit block re-encoded five trits per byte (pack.rs:240-256), padding = 125 (five zero trits).
__global__ void device_layout_kernel(const uint8_t* __restrict__ planar, uint64_t rows, uint32_t cols, uint32_t prb,
                                     uint32_t tbr, uint32_t dbr, uint64_t total, uint8_t* __restrict__ dst) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const uint64_t tile_bytes = 64ull * dbr;
    const uint64_t tile = idx / tile_bytes;
    const uint32_t in_tile = static_cast<uint32_t>(idx - tile * tile_bytes);
    const uint32_t q = in_tile >> 10, lr = (in_tile >> 4) & 63u, b = in_tile & 15u;
    const uint32_t c = q * 16u + b;
    const uint64_t r = tile * 64u + lr;
    uint8_t v = 125;
    if (r < rows && c < tbr) {
        const uint8_t* src = planar + r * prb;
        const uint32_t full = cols / 160u * 32u;
        if (c < full) {
            v = src[c];
        } else {
            const uint32_t rem = cols % 160u;
            uint32_t acc = 0, radix = 1;
            for (uint32_t k = 0; k < 5; ++k) {
                const uint32_t qq = 5u * (c - full) + k;
                int t = 0;
                if (qq < rem) {
                    const uint32_t plane = qq / 32u;
                    const uint32_t e = src[full + qq % 32u];
                    const uint32_t word = plane < 4 ? kTritTable.w[e][0] >> (8 * plane) : kTritTable.w[e][1];
                    t = static_cast<int8_t>(word & 0xffu);
                }
                acc += static_cast<uint32_t>(t + 1) * radix;
                radix = (k == 2) ? 28u : radix * 3u;
            }
            v = static_cast<uint8_t>(acc);
        }
    }
    dst[idx] = v;
}

// Lowest index of a byte that is not a velurex value (kTritTable marks them: only byte 125, five zero trits, has an
// all-zero entry among the valid ones).
__global__ void find_invalid_kernel(const uint8_t* __restrict__ planar, uint64_t n, unsigned long long* __restrict__ first) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t b = planar[i];
    const bool valid = (kTritTable.w[b][0] | kTritTable.w[b][1]) != 0u || b == 125u;
    if (!valid) atomicMin(first, static_cast<unsigned long long>(i));
}

__global__ void fill_f32_kernel(float* __restrict__ out, uint32_t n, float v) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = v;
}

// ---- GEMV -----------------------------------------------------------------------------------------------------------

// The staged activations are read-only for the whole kernel; reading them through the constant address space lets the
// compiler use scalar loads (s_load) into SGPRs instead of vector loads of a wave-uniform address.
typedef const __attribute__((address_space(4))) uint32_t const_u32;
__device__ __forceinline__ const const_u32* as_constant(const void* p) { return (const const_u32*)(p); }

struct GemvParams {
    const uint4* w;          // weights, device layout
    const uint2* actp;       // staged activations
    int32_t* acc;            // split-K accumulators (padded rows), zero between calls
    uint32_t* cnt;           // split-K arrival counters (tiles), zero between calls
    void* out;               // int32 or float, `rows` values
    float post;              // fp32 epilogue multiplier (out_f32)
    uint32_t rows;
    uint32_t n_chunks;       // 16-byte chunks per row
    uint32_t kslices;        // K slices per tile
    uint32_t slice_chunks;   // chunks per K slice
    uint32_t n_items;        // tiles * kslices
    uint32_t out_f32;
};

template <int WAVES, int PF>
__global__ __launch_bounds__(WAVES * 64) void gemv_lut_kernel(GemvParams p) {
    __shared__ uint2 tab[256 * kCopies];
    __shared__ int32_t red[WAVES][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    for (int i = tid; i < 256 * kCopies; i += WAVES * 64) {
        const int e = i / kCopies;
        tab[i] = make_uint2(kTritTable.w[e][0], kTritTable.w[e][1]);
    }
    __syncthreads();

    const uint32_t lane_off = static_cast<uint32_t>(lane & 31) * 8u;
    const char* tab_bytes = reinterpret_cast<const char*>(tab);

    for (uint32_t item = blockIdx.x; item < p.n_items; item += gridDim.x) {
        const uint32_t tile = item / p.kslices;
        const uint32_t ks = item - tile * p.kslices;
        const uint32_t c0 = ks * p.slice_chunks;
        const uint32_t c1 = min(c0 + p.slice_chunks, p.n_chunks);
        const uint32_t per = (c1 - c0 + WAVES - 1) / WAVES;
        const uint32_t qa = min(c0 + wave * per, c1);
        const uint32_t qb = min(qa + per, c1);
        const uint4* wp = p.w + static_cast<size_t>(tile) * p.n_chunks * 64u + lane;

        int acc = 0;
        uint4 buf[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i)
            if (qa + i < qb) buf[i] = wp[static_cast<size_t>(qa + i) * 64u];
        for (uint32_t q = qa; q < qb; q += PF) {
#pragma unroll
            for (int i = 0; i < PF; ++i) {
                const uint32_t qi = q + i;
                if (qi < qb) {
                    const uint4 v = buf[i];
                    if (qi + PF < qb) buf[i] = wp[static_cast<size_t>(qi + PF) * 64u];
                    const const_u32* ap = as_constant(p.actp) + static_cast<size_t>(qi) * 32u;
                    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int k = 0; k < 16; ++k) {
                        const uint32_t addr =
                            __builtin_amdgcn_perm(d[k >> 2], lane_off, 0x0c0c0000u | ((4u + (k & 3)) << 8));
                        const uint2 t = *reinterpret_cast<const uint2*>(tab_bytes + addr);
                        const uint32_t a03 = ap[2 * k], a4 = ap[2 * k + 1];
                        acc = __builtin_amdgcn_sdot4(static_cast<int>(t.x), static_cast<int>(a03), acc, false);
                        acc = __builtin_amdgcn_sdot4(static_cast<int>(t.y), static_cast<int>(a4), acc, false);
                    }
                }
            }
        }

        red[wave][lane] = acc;
        __syncthreads();
        if (wave == 0) {
            int s = 0;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) s += red[w][lane];
            const uint32_t row = tile * 64u + static_cast<uint32_t>(lane);
            bool write = true;
            if (p.kslices > 1) {
                __hip_atomic_fetch_add(p.acc + row, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __threadfence();
                uint32_t old = 0;
                if (lane == 0) old = __hip_atomic_fetch_add(p.cnt + tile, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
                old = __shfl(old, 0);
                write = (old == p.kslices - 1);
                if (write) {
                    __threadfence();
                    s = __hip_atomic_load(p.acc + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(p.acc + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (lane == 0) __hip_atomic_store(p.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            if (write && row < p.rows) {
                if (p.out_f32) static_cast<float*>(p.out)[row] = static_cast<float>(s) * p.post;
                else static_cast<int32_t*>(p.out)[row] = s;
            }
        }
        __syncthreads();
    }
}

constexpr int kWaves = 8;
constexpr int kPrefetch = 2;

// Chooses the K split and the grid: enough workgroups to fill every CU twice, slices no shorter than one chunk per wave.
static void plan(const Geometry& g, int num_cus, uint32_t* kslices, uint32_t* slice_chunks, uint32_t* grid) {
    const uint32_t tiles = static_cast<uint32_t>(g.n_tiles);
    const uint32_t chunks = static_cast<uint32_t>(g.n_chunks);
    const uint32_t want_wgs = static_cast<uint32_t>(num_cus) * 2u;
    uint32_t ks = (want_wgs + tiles - 1) / tiles;
    const uint32_t max_ks = std::max<uint32_t>(1u, chunks / (2u * kWaves));
    ks = std::max<uint32_t>(1u, std::min(ks, max_ks));
    uint32_t sc = (chunks + ks - 1) / ks;
    ks = (chunks + sc - 1) / sc;
    *kslices = ks;
    *slice_chunks = sc;
    const uint32_t items = tiles * ks;
    *grid = std::min<uint32_t>(items, want_wgs);
}

int launch_stage(const int8_t* acts, size_t cols, uint2* staged, hipStream_t stream) {
    const uint32_t dbr = static_cast<uint32_t>(device_row_bytes(cols));
    hipLaunchKernelGGL(act_prep_kernel, dim3((dbr + 255u) / 256u), dim3(256), 0, stream, acts, static_cast<uint32_t>(cols),
                       static_cast<uint32_t>(tile_row_bytes(cols)), dbr, staged);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_gemv_staged(vx_matrix* m, const uint2* staged, void* out, bool out_f32, float post, hipStream_t stream) {
    const Geometry& g = m->g;
    GemvParams p;
    p.w = reinterpret_cast<const uint4*>(m->d_w);
    p.actp = staged;
    p.acc = m->d_acc;
    p.cnt = m->d_cnt;
    p.out = out;
    p.post = post;
    p.rows = static_cast<uint32_t>(g.rows);
    p.n_chunks = static_cast<uint32_t>(g.n_chunks);
    uint32_t grid = 0;
    plan(g, m->num_cus, &p.kslices, &p.slice_chunks, &grid);
    p.n_items = static_cast<uint32_t>(g.n_tiles) * p.kslices;
    p.out_f32 = out_f32 ? 1u : 0u;
    hipLaunchKernelGGL((gemv_lut_kernel<kWaves, kPrefetch>), dim3(grid), dim3(kWaves * 64), 0, stream, p);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

int launch_gemv(vx_matrix* m, const int8_t* acts, void* out, bool out_f32, float post, hipStream_t stream) {
    VX_TRY(launch_stage(acts, m->g.cols, m->d_actp, stream));
    return launch_gemv_staged(m, m->d_actp, out, out_f32, post, stream);
}

int launch_device_layout(const uint8_t* planar_dev, const Geometry& g, uint8_t* dst, hipStream_t stream) {
    const uint64_t total = g.device_bytes;
    const uint64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(device_layout_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, planar_dev,
                       static_cast<uint64_t>(g.rows), static_cast<uint32_t>(g.cols),
                       static_cast<uint32_t>(planar_row_bytes(g.cols)), static_cast<uint32_t>(g.tbr),
                       static_cast<uint32_t>(g.dbr), total, dst);
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

// ---- host-side layout transform ------------------------------------------------------------------------------------------

// Valid velurex bytes and their trits (host copy of the table above).
static bool g_valid[256];
static int8_t g_trits[256][5];
static std::once_flag g_host_once;

static void init_host_tables() {
    std::call_once(g_host_once, [] {
        for (int b = 0; b < 256; ++b) {
            g_valid[b] = false;
            for (int p = 0; p < 5; ++p) g_trits[b][p] = 0;
        }
        for (int s = 0; s < 243; ++s) {
            int d[5], v = s;
            for (int p = 0; p < 5; ++p) {
                d[p] = v % 3;
                v /= 3;
            }
            const int b = d[0] + 3 * d[1] + 9 * d[2] + 28 * d[3] + 84 * d[4];
            g_valid[b] = true;
            for (int p = 0; p < 5; ++p) g_trits[b][p] = static_cast<int8_t>(d[p] - 1);
        }
    });
}

static inline uint8_t pack5(const int8_t t[5]) {
    return static_cast<uint8_t>((t[0] + 1) + 3 * (t[1] + 1) + 9 * (t[2] + 1) + 28 * (t[3] + 1) + 84 * (t[4] + 1));
}

// Returns the first invalid byte index or SIZE_MAX.
size_t find_invalid_byte(const uint8_t* planar, size_t n) {
    init_host_tables();
    for (size_t i = 0; i < n; ++i)
        if (!g_valid[planar[i]]) return i;
    return SIZE_MAX;
}

// Writes the device layout of a rows x cols planar matrix into `dst` (g.device_bytes bytes).
void planar_to_device_layout(const uint8_t* planar, const Geometry& g, uint8_t* dst) {
    init_host_tables();
    constexpr uint8_t kZeroByte = 125;  // five zero trits (d = 1 everywhere)
    const size_t prb = planar_row_bytes(g.cols);
    const size_t full = tile_full_columns(g.cols);
    const size_t rem = g.cols % kQK5;
    std::vector<uint8_t> row(g.dbr);
    for (size_t r = 0; r < g.padded_rows; ++r) {
        if (r < g.rows) {
            const uint8_t* src = planar + r * prb;
            std::memcpy(row.data(), src, full);
            for (size_t c = full; c < g.tbr; ++c) {  // packed tail (pack.rs:240-256)
                int8_t t[5] = {0, 0, 0, 0, 0};
                for (size_t k = 0; k < 5; ++k) {
                    const size_t q = 5 * (c - full) + k;
                    if (q < rem) t[k] = g_trits[src[full + q % kBlockBytes]][q / kBlockBytes];
                }
                row[c] = pack5(t);
            }
            for (size_t c = g.tbr; c < g.dbr; ++c) row[c] = kZeroByte;
        } else {
            std::memset(row.data(), kZeroByte, g.dbr);
        }
        uint8_t* tile = dst + (r / kTileRows) * kTileRows * g.dbr + (r % kTileRows) * kChunk;
        for (size_t q = 0; q < g.n_chunks; ++q) std::memcpy(tile + q * kTileRows * kChunk, row.data() + q * kChunk, kChunk);
    }
}

}  // namespace vx
