// Batched ternary GEMM for gfx950 (MI355X): Y[m][i] = sum_j W[i][j] X[m][j] for M tokens, exact int32, on the matrix
// cores (v_mfma_i32_32x32x32_i8).
//
// The reference has no multi-token kernel: its prefill runs one GEMV per token (quintrit-runtime/src/engine.rs:625-631),
// so the definition is M independent GEMVs (quintrit-core/src/simd/avx512.rs:1526-1626), and the result must equal
// them bit for bit. Weights stay in the velurex device layout of the GEMV (1.60 bits per weight in HBM) and are
// decoded to int8 trits in registers right before the matrix-core instruction; activations are staged once per call
// in the order of the MFMA B operand.
//
// MFMA operands (v_mfma_i32_32x32x32_i8): lane l supplies 16 int8 of row l % 32 of A (a weight row) and of column
// l % 32 of B (a token); lanes l and l + 32 hold the two halves of the 32-deep K block, and C register r of lane l is
// row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32. Any order of K works as long as A and B use the same one.
//
// K order. A K step is two 16-byte chunks of a weight row: 32 byte-columns x 5 planes = 160 trits = five 32-deep MFMA
// blocks. Lane (i, s) (i = row in the 32-row block, s = lane / 32) holds chunk 2 ks + s of its row in one 16-byte load.
// Block m < 4 takes dword m of that chunk: bytes 4m .. 4m+3, planes 0..3 (t0..t3 as int8, one LDS table lookup per
// byte). Block 4 takes plane 4 of all 16 bytes: t4 = floor(B / 84) - 1 per byte from carry-free byte arithmetic
// (t4_bytes). The activation staging writes X in exactly this order, so A and B pair every weight with its
// activation.
//
// Work split. A wave computes 64 weight rows (two 32-row blocks, one tile of the device layout) x T groups of 32
// tokens over a range of K steps; the A fragments of a K step are decoded once and used for all T token groups. A
// workgroup of W = 4 or 8 waves takes W consecutive tiles with the same tokens and K range, so the B fragments of a K
// step are staged once per workgroup in LDS (double-buffered, the next step's loaded while this one is multiplied).
// Long K is split into slices whose int32 partial sums a second kernel adds; the host picks T, W and the number of
// slices (4-wave workgroups while the grid fits the CUs in one round: at M <= 128 and for the 3072-row shapes they are
// 5-25 % faster than 8-wave ones; 23040 rows at M = 512 need the 8-wave form).
#include "vx_gemv_core.h"
#include "vx_internal.h"

#include <algorithm>
#include <mutex>

namespace vx {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4g __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4g g_u4g;

// t0..t3 of every byte as int8 in a dword (trits03_word: non-values give zero trits, pack.rs:41-58), built at compile
// time; a workgroup copies it into its LDS table with loads.
__constant__ TritTable g_gemm_trits = make_trit_table();

constexpr uint32_t kStepChunks = 2;  // 16-byte chunks per K step
constexpr uint32_t kZeroWord = 0x7d7d7d7du;  // four bytes of five zero trits

// ---- activation staging --------------------------------------------------------------------------------------------

// Staging: thread (token m, pair) writes the five B fragments of K step ks = pair / 2, half hs = pair % 2 of token m:
// xs[ks][kb][tg][lane] (tg = m / 32, lane = (m % 32) + 32 hs) for K blocks kb = 0..4, in the K order of the weight
// decode (column_activation_index, pack.rs:230-237). In a whole 160-trit block (ks < cols / 160) the step is the 160
// activations of block ks and half hs covers byte-columns 16 hs .. 16 hs + 15: K block kb < 4 takes, for byte-column
// 16 hs + 4 kb + d, its activations of planes 0..3, a(160 ks + 32 e + 16 hs + 4 kb + d), e = 0..3: dword kb of the
// four 16-byte loads at 160 ks + 32 e + 16 hs, transposed 4 x 4 bytes with v_perm; K block 4 takes plane 4 of the 16
// byte-columns, the 16 bytes at 160 ks + 128 + 16 hs as they are. The packed tail and unaligned rows take the
// per-byte gather. Workgroup (pair block, token group): lane j of each 32-thread row is token 32 tg + j and the rows are
// kStageRows consecutive pairs, so the 32 tokens of a row write one contiguous 512-byte run per K block.
constexpr uint32_t kStageRows = 8;  // pairs per staging workgroup (256 threads)

__global__ __launch_bounds__(256) void gemm_stage_kernel(const int8_t* __restrict__ x, uint32_t ldx, uint32_t n_tg,
                                                         uint32_t cols, uint32_t n_ksteps,
                                                         uint4* __restrict__ xs, uint32_t M) {
    const uint32_t tid = threadIdx.x, j = tid & 31u;
    const uint32_t pair = blockIdx.x * kStageRows + (tid >> 5), ks = pair >> 1, hs = pair & 1u;
    const uint32_t tg = blockIdx.y, m = tg * 32u + j;
    // B fragments of tokens past M (the rest of the last 32-token group) are left as they are: they only reach C
    // columns that are never stored.
    if (ks >= n_ksteps || m >= M) return;
    const int8_t* xr = x + static_cast<size_t>(m) * ldx;
    uint4 o[5];
    if (ks < cols / 160u && (reinterpret_cast<uintptr_t>(xr) & 15u) == 0) {
        const int8_t* blk = xr + ks * 160u + 16u * hs;
        uint4 X[5];
#pragma unroll
        for (int e = 0; e < 5; ++e) X[e] = *reinterpret_cast<const uint4*>(blk + 32 * e);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            auto dw = [&](const uint4& v) { return kb == 0 ? v.x : (kb == 1 ? v.y : (kb == 2 ? v.z : v.w)); };
            const uint32_t a0 = dw(X[0]), a1 = dw(X[1]), a2 = dw(X[2]), a3 = dw(X[3]);
            const uint32_t lo01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u), hi01 = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
            const uint32_t lo23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u), hi23 = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
            o[kb] = make_uint4(__builtin_amdgcn_perm(lo23, lo01, 0x05040100u), __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                               __builtin_amdgcn_perm(hi23, hi01, 0x05040100u), __builtin_amdgcn_perm(hi23, hi01, 0x07060302u));
        }
        o[4] = X[4];
    } else {
        // byte-column 16 hs + k of the step (k < 16), activation p: in a whole block 160 ks + 32 p + 16 hs + k, in the
        // packed tail 160 ks + 5 (16 hs + k) + p (column_activation_index); past the row (and in the tail's padding
        // columns, whose indices are all >= cols) zero
        const bool tail = ks >= cols / 160u;
        auto act = [&](uint32_t k, uint32_t p) -> uint32_t {
            const uint32_t idx = tail ? ks * 160u + 5u * (16u * hs + k) + p : ks * 160u + 32u * p + 16u * hs + k;
            return idx < cols ? static_cast<uint32_t>(static_cast<uint8_t>(xr[idx])) : 0u;
        };
#pragma unroll
        for (uint32_t kb = 0; kb < 5; ++kb) {
            uint32_t w[4];
#pragma unroll
            for (uint32_t d = 0; d < 4; ++d) {
                uint32_t v = 0;
#pragma unroll
                for (uint32_t e = 0; e < 4; ++e) v |= (kb < 4 ? act(4u * kb + d, e) : act(4u * d + e, 4u)) << (8 * e);
                w[d] = v;
            }
            o[kb] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
#pragma unroll
    for (uint32_t kb = 0; kb < 5; ++kb) xs[(static_cast<size_t>(ks * 5u + kb) * n_tg + tg) * 64u + j + 32u * hs] = o[kb];
}

// ---- GEMM -------------------------------------------------------------------------------------------------------------

struct GemmArgs {
    const uint8_t* w;      // device layout
    const uint4* xs;       // staged activations
    int32_t* y;            // M x ldy (kslices == 1)
    int32_t* part;         // kslices x (n_tg * 32) x rows_p partial sums (kslices > 1)
    uint32_t rows, n_tiles, n_chunks, n_ksteps;
    uint32_t M, n_tg, ldy, y_vec4;   // y_vec4: y and ldy allow 16-byte stores
    uint32_t kslices, ksteps_per_slice, rows_p;
    // a pair of matrices of one geometry in one launch (gemm_kernel's G2): the tiles of w (tiles1 of them), then those
    // of w2 with outputs y2; n_tiles counts both
    const uint8_t* w2;
    int32_t* y2;
    uint32_t tiles1;
};

// Workgroup (rg, tt, kz): W waves, wave w taking the R 32-row blocks (W rg + w) R .. + R - 1 of the matrix (block 2 t + h
// is half h of 64-row tile t), token groups T tt .. T tt + T - 1, K steps of slice kz. LDS: the trit table (32 copies
// of each entry in the first half of a 256-byte row; lane l reads copy l % 32, conflict-free because LDS serves a wave
// in two 32-lane halves) and two buffers of one K step's B fragments, which every wave reads (a B fragment serves the
// wave's R blocks, an A fragment its T token groups).
template <int T, int R, int W, bool G2>
__global__ __launch_bounds__(W * 64) void gemm_kernel(GemmArgs a) {
    __shared__ uint32_t tab[256 * 64];
    __shared__ uint4 bs[2][5 * T * 64];
    constexpr uint32_t kNT = W * 64u;
    constexpr uint32_t kB = 5u * T * 64u;                // B fragments of a K step
    constexpr uint32_t kBPer = (kB + kNT - 1) / kNT;     // per thread
    static_assert(kBPer <= 5, "at most five B fragments per thread and step");

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t blk0 = (blockIdx.x * W + wave) * R;  // the wave's first 32-row block of the launch
    // G2: the wave's matrix (its R blocks lie in one tile, so in one matrix) and its first block there
    const bool sec = G2 && blk0 >= 2u * a.tiles1;
    const uint32_t lb0 = sec ? blk0 - 2u * a.tiles1 : blk0;
    const uint32_t nt = G2 ? a.tiles1 : a.n_tiles;  // tiles of the wave's matrix
    const uint8_t* wm = sec ? a.w2 : a.w;
    int32_t* ym = sec ? a.y2 : a.y;
    const uint32_t n_blk = 2u * nt;
    const uint32_t tt = blockIdx.y, kz = blockIdx.z;
    const uint32_t ks0 = kz * a.ksteps_per_slice;
    const uint32_t ks1 = min(ks0 + a.ksteps_per_slice, a.n_ksteps);

    for (uint32_t i = tid; i < 256u * 8u; i += kNT) {
        const uint32_t e = g_gemm_trits.v[i >> 3];
        *reinterpret_cast<uint4*>(reinterpret_cast<char*>(tab) + (i >> 3) * 256u + (i & 7u) * 16u) = make_uint4(e, e, e, e);
    }
    const char* tabb = reinterpret_cast<const char*>(tab);
    const uint32_t lane_off = (lane & 31u) * 4u;

    // This lane's row (i = lane % 32) of each of the wave's blocks in the device layout: block 2 t + h is rows
    // 32 h .. 32 h + 31 of tile t (16 bytes a row per chunk, the chunks of a tile T_g KiB apart in its tile group). A
    // block past the matrix reads the last block (and stores nothing), so every load has a valid address and none sits
    // behind a branch (the compiler would then wait for all loads before the next use).
    const uint8_t* wbase[R];
    uint32_t cstride[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t blk = min(lb0 + r, n_blk - 1u), tile = blk >> 1;
        const uint32_t grp = tile / kTileGroup, t16 = tile - grp * kTileGroup;
        const uint32_t Tg = min(static_cast<uint32_t>(kTileGroup), nt - grp * kTileGroup);
        wbase[r] = wm + (static_cast<size_t>(grp) * kTileGroup * a.n_chunks + t16) * 1024u + (blk & 1u) * 512u +
                   (lane & 31u) * 16u;
        cstride[r] = Tg * 1024u;
    }
    const uint32_t half = lane >> 5;

    // Chunk 2 ks + s of the lane's rows; a chunk past the row (odd n_chunks) reads the last one and is replaced by
    // zero trits when it is decoded.
    auto load_w = [&](uint32_t ks, u32x4g (&wv)[R]) __attribute__((always_inline)) {
        const uint32_t q = min(ks * kStepChunks + half, a.n_chunks - 1u);
#pragma unroll
        for (int r = 0; r < R; ++r)
            wv[r] = __builtin_nontemporal_load((g_u4g*)(wbase[r] + static_cast<size_t>(q) * cstride[r]));
    };
    // B fragments of step ks (kBPer per thread, in named registers: an array here would be moved to scratch memory
    // once the steps rotate through three sets); slots past the token groups read a valid fragment that no stored
    // output depends on (only C columns of tokens >= M).
    auto b_index = [&](uint32_t ks, uint32_t k) -> size_t {
        const uint32_t idx = min(tid + k * kNT, kB - 1u);
        const uint32_t kb = idx / (T * 64u), rem = idx - kb * T * 64u;
        const uint32_t tg = min(tt * T + rem / 64u, a.n_tg - 1u);
        return (static_cast<size_t>(ks * 5u + kb) * a.n_tg + tg) * 64u + (rem & 63u);
    };
#define VX_LOAD_B(ks, r0, r1, r2, r3, r4)                   \
    do {                                                    \
        r0 = a.xs[b_index((ks), 0)];                        \
        if (kBPer > 1) r1 = a.xs[b_index((ks), 1)];         \
        if (kBPer > 2) r2 = a.xs[b_index((ks), 2)];         \
        if (kBPer > 3) r3 = a.xs[b_index((ks), 3)];         \
        if (kBPer > 4) r4 = a.xs[b_index((ks), 4)];         \
    } while (0)
#define VX_STORE_B(buf, r0, r1, r2, r3, r4)                                             \
    do {                                                                                \
        if (tid < kB) bs[(buf)][tid] = r0;                                              \
        if (kBPer > 1 && tid + kNT < kB) bs[(buf)][tid + kNT] = r1;                     \
        if (kBPer > 2 && tid + 2u * kNT < kB) bs[(buf)][tid + 2u * kNT] = r2;           \
        if (kBPer > 3 && tid + 3u * kNT < kB) bs[(buf)][tid + 3u * kNT] = r3;           \
        if (kBPer > 4 && tid + 4u * kNT < kB) bs[(buf)][tid + 4u * kNT] = r4;           \
    } while (0)

    v16i acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int g = 0; g < T; ++g) acc[r][g] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    // The products of step ks: weights wc, B fragments from bs[buf].
    auto multiply = [&](uint32_t ks, const u32x4g (&wc)[R], uint32_t buf) __attribute__((always_inline)) {
        const bool inside = ks * kStepChunks + half < a.n_chunks;
        v4i A[R][5];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t dw[4] = {inside ? wc[r].x : kZeroWord, inside ? wc[r].y : kZeroWord,
                                    inside ? wc[r].z : kZeroWord, inside ? wc[r].w : kZeroWord};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                int t[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t addr = __builtin_amdgcn_perm(dw[m], lane_off, 0x0c0c0000u | ((4u + b) << 8));
                    t[b] = static_cast<int>(*reinterpret_cast<const uint32_t*>(tabb + addr));
                }
                A[r][m] = v4i{t[0], t[1], t[2], t[3]};
            }
            A[r][4] = v4i{static_cast<int>(t4_bytes(dw[0])), static_cast<int>(t4_bytes(dw[1])),
                          static_cast<int>(t4_bytes(dw[2])), static_cast<int>(t4_bytes(dw[3]))};
        }
        // K block outer, token group, then block: R T independent accumulators between two MFMAs on the same one.
#pragma unroll
        for (int kb = 0; kb < 5; ++kb) {
#pragma unroll
            for (int g = 0; g < T; ++g) {
                const uint4 b = bs[buf][(kb * T + g) * 64u + lane];
                const v4i B = v4i{static_cast<int>(b.x), static_cast<int>(b.y), static_cast<int>(b.z), static_cast<int>(b.w)};
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[r][kb], B, acc[r][g], 0, 0, 0);
            }
        }
    };

    // Two K steps ahead: step ks issues the loads of step ks + 2 (B fragments first, then weights), multiplies step ks
    // (weights loaded two steps earlier, B fragments stored in LDS at the end of the previous step) and stores the B
    // fragments of step ks + 1 (loaded one step earlier). Three register sets rotate through the steps of a 3x
    // unrolled loop, so no loaded register is ever copied (a copy would wait for its load). Every load is unconditional
    // (indices clamp at the last step) and the steps past the slice's end only skip the multiply, so the compiler's
    // waits stay exact.
    u32x4g w0[R], w1[R], w2[R];
    uint4 b00, b01, b02, b03, b04, b10, b11, b12, b13, b14, b20, b21, b22, b23, b24;
    const uint32_t last = ks1 > ks0 ? ks1 - 1u : ks0;
    VX_LOAD_B(ks0, b00, b01, b02, b03, b04);
    load_w(ks0, w0);
    VX_LOAD_B(min(ks0 + 1u, last), b10, b11, b12, b13, b14);
    load_w(min(ks0 + 1u, last), w1);
    VX_STORE_B(0, b00, b01, b02, b03, b04);
    const bool active = blk0 < 2u * a.n_tiles;
#define VX_STEP(ks, WC, N0, N1, N2, N3, N4, M0, M1, M2, M3, M4, WN)      \
    do {                                                                 \
        VX_LOAD_B(min((ks) + 2u, last), M0, M1, M2, M3, M4);             \
        load_w(min((ks) + 2u, last), WN);                                \
        __syncthreads();                                                 \
        if (active && (ks) < ks1) multiply((ks), WC, ((ks) - ks0) & 1u); \
        VX_STORE_B((((ks) - ks0) & 1u) ^ 1u, N0, N1, N2, N3, N4);        \
    } while (0)
    for (uint32_t ks = ks0; ks < ks1; ks += 3u) {
        VX_STEP(ks, w0, b10, b11, b12, b13, b14, b20, b21, b22, b23, b24, w2);
        VX_STEP(ks + 1u, w1, b20, b21, b22, b23, b24, b00, b01, b02, b03, b04, w0);
        VX_STEP(ks + 2u, w2, b00, b01, b02, b03, b04, b10, b11, b12, b13, b14, w1);
    }
#undef VX_STEP
#undef VX_LOAD_B
#undef VX_STORE_B
    if (!active) return;
    // C of (block, token group g): lane l, register r -> row 8 (r / 4) + 4 (l / 32) + r % 4 of the block, token l % 32.
    const uint32_t j = lane & 31u;
#pragma unroll
    for (int g = 0; g < T; ++g) {
        const uint32_t m = (tt * T + g) * 32u + j;
        if (m >= a.M) continue;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (lb0 + r >= n_blk) continue;
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const uint32_t n = (lb0 + r) * 32u + 8u * r4 + 4u * half;
                const int v0 = acc[r][g][4 * r4], v1 = acc[r][g][4 * r4 + 1];
                const int v2 = acc[r][g][4 * r4 + 2], v3 = acc[r][g][4 * r4 + 3];
                if (a.kslices > 1) {
                    *reinterpret_cast<int4*>(a.part + (static_cast<size_t>(kz) * a.n_tg * 32u + m) * a.rows_p + n) =
                        make_int4(v0, v1, v2, v3);
                } else if (a.y_vec4 && n + 3 < a.rows) {
                    *reinterpret_cast<int4*>(ym + static_cast<size_t>(m) * a.ldy + n) = make_int4(v0, v1, v2, v3);
                } else {
                    int32_t* yr = ym + static_cast<size_t>(m) * a.ldy;
                    if (n < a.rows) yr[n] = v0;
                    if (n + 1 < a.rows) yr[n + 1] = v1;
                    if (n + 2 < a.rows) yr[n + 2] = v2;
                    if (n + 3 < a.rows) yr[n + 3] = v3;
                }
            }
        }
    }
}

__global__ __launch_bounds__(256) void gemm_finish_kernel(GemmArgs a) {
    const uint32_t n = blockIdx.x * 256u + threadIdx.x, m = blockIdx.y;
    if (n >= a.rows) return;
    const size_t stride = static_cast<size_t>(a.n_tg) * 32u * a.rows_p;
    const int32_t* p = a.part + static_cast<size_t>(m) * a.rows_p + n;
    int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    uint32_t k = 0;
    for (; k + 4 <= a.kslices; k += 4) {
        s0 += p[k * stride];
        s1 += p[(k + 1) * stride];
        s2 += p[(k + 2) * stride];
        s3 += p[(k + 3) * stride];
    }
    for (; k < a.kslices; ++k) s0 += p[k * stride];
    a.y[static_cast<size_t>(m) * a.ldy + n] = (s0 + s1) + (s2 + s3);
}

// ---- host side ---------------------------------------------------------------------------------------------------------

struct GemmPlan {
    uint32_t n_ksteps, n_tg, T, R, W, n_tt, grid_x, kslices, ksteps_per_slice;
    size_t xs_bytes, part_bytes;
};

// T (token groups per wave) from M; then the K split that minimises an estimate of the time: rounds of workgroups
// times K steps per workgroup times the time of a K step, plus the HBM traffic of the partial sums and their finish.
// A K step of a wave is 10 T MFMAs (32 cycles each, two waves per SIMD), but not less than the HBM latency (the
// weights are loaded one step ahead).
static GemmPlan gemm_plan(const Geometry& g, size_t M, int num_cus) {
    GemmPlan p{};
    p.n_ksteps = static_cast<uint32_t>((g.n_chunks + kStepChunks - 1) / kStepChunks);
    p.n_tg = static_cast<uint32_t>((M + 31) / 32);
    p.T = p.n_tg >= 4 ? 4u : (p.n_tg >= 2 ? 2u : 1u);
    p.n_tt = (p.n_tg + p.T - 1) / p.T;
    // Two 32-row blocks per wave; 4-wave workgroups while they fit the CUs in one round without a K split (more,
    // smaller workgroups spread a narrow grid over more CUs), else 8-wave workgroups (the B fragments of a step serve
    // twice the rows).
    p.R = 2;
    const uint64_t blocks = 2 * g.n_tiles;
    p.W = (blocks + 7) / 8 * p.n_tt <= static_cast<uint64_t>(std::max(num_cus, 1)) ? 4u : 8u;
    p.grid_x = static_cast<uint32_t>((blocks + p.R * p.W - 1) / (p.R * p.W));
    const uint64_t base = static_cast<uint64_t>(p.grid_x) * p.n_tt;
    const uint64_t slots = static_cast<uint64_t>(std::max(num_cus, 1)) * (p.T == 1 ? 2u : 1u);  // workgroups per CU (LDS)
    // a K step of a wave is 10 T MFMAs (32 cycles each, W / 4 waves per SIMD), but not less than the HBM latency
    const double t_step = std::max(0.29e-6 * p.T * p.W / 8.0, 1.0e-6);
    double best = 1e30;
    uint32_t best_ks = 1;
    for (uint32_t ks = 1; ks <= std::min<uint32_t>(p.n_ksteps, 64u); ++ks) {
        const uint32_t per = (p.n_ksteps + ks - 1) / ks;
        const uint32_t slices = (p.n_ksteps + per - 1) / per;
        if (slices != ks) continue;
        const double rounds = static_cast<double>((base * slices + slots - 1) / slots);
        const double part = slices > 1 ? 8.0 * slices * static_cast<double>(M) * g.padded_rows / 2.5e12 + 4.0e-6 : 0.0;
        const double t = rounds * per * t_step + part;
        if (t < best) {
            best = t;
            best_ks = slices;
        }
    }
    p.ksteps_per_slice = (p.n_ksteps + best_ks - 1) / best_ks;
    p.kslices = (p.n_ksteps + p.ksteps_per_slice - 1) / p.ksteps_per_slice;
    p.xs_bytes = round_up(static_cast<size_t>(p.n_ksteps) * 5u * p.n_tg * 1024u, 256);
    p.part_bytes = p.kslices > 1 ? static_cast<size_t>(p.kslices) * p.n_tg * 32u * g.padded_rows * 4u : 0;
    return p;
}

static size_t small_part_bytes(const Geometry& g, size_t M, int num_cus);
static bool small_path(const Geometry& g, size_t M, int num_cus);

size_t gemm_workspace_bytes(const Geometry& g, size_t M, int num_cus) {
    if (small_path(g, M, num_cus)) return std::max<size_t>(small_part_bytes(g, M, num_cus), 256);
    const GemmPlan p = gemm_plan(g, M, num_cus);
    return p.xs_bytes + p.part_bytes;
}

size_t gemm_stage_bytes(size_t cols, size_t M) {
    const GemmPlan p = gemm_plan(geometry(1, cols), M, 1);  // the staged activations depend on cols and M only
    return p.xs_bytes;
}

size_t gemm_part_bytes(const Geometry& g, size_t M, int num_cus) {
    return small_path(g, M, num_cus) ? small_part_bytes(g, M, num_cus) : gemm_plan(g, M, num_cus).part_bytes;
}

// Stages x (M rows of cols int8) into the MFMA operand order at ws (gemm_stage_bytes(cols, M) bytes): the staged
// activations of one call serve every matrix with cols columns.
int launch_gemm_stage(const int8_t* x, size_t M, size_t ldx, size_t cols, uint8_t* ws, hipStream_t stream) {
    const GemmPlan p = gemm_plan(geometry(1, cols), M, 1);
    const dim3 grid((2u * p.n_ksteps + kStageRows - 1) / kStageRows, p.n_tg);
    hipLaunchKernelGGL(gemm_stage_kernel, grid, dim3(256), 0, stream, x, static_cast<uint32_t>(ldx), p.n_tg,
                       static_cast<uint32_t>(cols), p.n_ksteps,
                       reinterpret_cast<uint4*>(ws), static_cast<uint32_t>(M));
    VX_HIP(hipGetLastError());
    return VX_OK;
}

// The product of matrix w with activations staged by launch_gemm_stage at `staged`; `part` holds
// gemm_part_bytes(g, M, num_cus) bytes of K-slice partial sums (unused when the plan has one slice).
template <bool G2>
static void launch_staged_kernel(const GemmPlan& p, const GemmArgs& a, hipStream_t stream) {
    const dim3 grid(p.grid_x, p.n_tt, p.kslices);
    const dim3 block(p.W * 64);
    if (p.W == 8) {
        if (p.T == 4) hipLaunchKernelGGL((gemm_kernel<4, 2, 8, G2>), grid, block, 0, stream, a);
        else if (p.T == 2) hipLaunchKernelGGL((gemm_kernel<2, 2, 8, G2>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((gemm_kernel<1, 2, 8, G2>), grid, block, 0, stream, a);
    } else {
        if (p.T == 4) hipLaunchKernelGGL((gemm_kernel<4, 2, 4, G2>), grid, block, 0, stream, a);
        else if (p.T == 2) hipLaunchKernelGGL((gemm_kernel<2, 2, 4, G2>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((gemm_kernel<1, 2, 4, G2>), grid, block, 0, stream, a);
    }
}

static GemmArgs staged_args(const GemmPlan& p, const uint8_t* w, const Geometry& g, const uint8_t* staged, size_t M,
                            int32_t* y, size_t ldy, uint8_t* part) {
    GemmArgs a{};
    a.w = w;
    a.xs = reinterpret_cast<const uint4*>(staged);
    a.y = y;
    a.part = p.kslices > 1 ? reinterpret_cast<int32_t*>(part) : nullptr;
    a.rows = static_cast<uint32_t>(g.rows);
    a.n_tiles = static_cast<uint32_t>(g.n_tiles);
    a.n_chunks = static_cast<uint32_t>(g.n_chunks);
    a.n_ksteps = p.n_ksteps;
    a.M = static_cast<uint32_t>(M);
    a.n_tg = p.n_tg;
    a.ldy = static_cast<uint32_t>(ldy);
    a.y_vec4 = (ldy % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0) ? 1u : 0u;
    a.kslices = p.kslices;
    a.ksteps_per_slice = p.ksteps_per_slice;
    a.rows_p = static_cast<uint32_t>(g.padded_rows);
    return a;
}

int launch_gemm_staged(const uint8_t* w, const Geometry& g, int num_cus, const uint8_t* staged, size_t M, int32_t* y,
                       size_t ldy, uint8_t* part, hipStream_t stream) {
    const GemmPlan p = gemm_plan(g, M, num_cus);
    const GemmArgs a = staged_args(p, w, g, staged, M, y, ldy, part);
    launch_staged_kernel<false>(p, a, stream);
    VX_HIP(hipGetLastError());
    if (p.kslices > 1) {
        hipLaunchKernelGGL(gemm_finish_kernel, dim3((a.rows + 255u) / 256u, static_cast<uint32_t>(M)), dim3(256), 0, stream, a);
        VX_HIP(hipGetLastError());
    }
    return VX_OK;
}

// The concatenation of two matrices of one geometry as one launch, when its plan needs no K split.
static GemmPlan pair_plan(const Geometry& g, size_t M, int num_cus) {
    return gemm_plan(geometry(2 * g.padded_rows, g.cols), M, num_cus);
}

bool gemm_staged_pair_ok(const Geometry& g, size_t M, int num_cus) { return pair_plan(g, M, num_cus).kslices == 1; }

int launch_gemm_staged_pair(const uint8_t* w, const uint8_t* w2, const Geometry& g, int num_cus, const uint8_t* staged,
                            size_t M, int32_t* y, int32_t* y2, size_t ldy, hipStream_t stream) {
    const GemmPlan p = pair_plan(g, M, num_cus);
    if (p.kslices != 1) VX_FAIL(VX_ERR_INTERNAL, "a paired GEMM with %u K slices", p.kslices);
    GemmArgs a = staged_args(p, w, g, staged, M, y, ldy, nullptr);
    a.n_tiles = static_cast<uint32_t>(2 * g.n_tiles);
    a.w2 = w2;
    a.y2 = y2;
    a.tiles1 = static_cast<uint32_t>(g.n_tiles);
    a.y_vec4 = a.y_vec4 && reinterpret_cast<uintptr_t>(y2) % 16 == 0 ? 1u : 0u;
    launch_staged_kernel<true>(p, a, stream);
    VX_HIP(hipGetLastError());
    return VX_OK;
}

// ---- one token group (M <= 32): one launch ------------------------------------------------------------------------

// Workgroup (c, kz): W waves, wave w the 64-row tile W c + w, over the K steps of slice kz (at most
// small_max_steps(T)), for T token groups of 32 (1, 2 or 4). G: the call's tiles may belong to several matrices of the
// same columns (each wave finds its own; without G the instance reads only the first). Each thread first loads the activations of its B-fragment tasks (task = step, token
// group, half, token) and the trit table's entries, then each wave loads all its weights of the slice at once (2
// chunks per K step per lane, every load unconditional: steps past the slice read its last step again), so
// the wait for the activations and the table does
// not include the weights' latency (loads return in order); the
// workgroup then builds the trit table and the slice's B fragments in LDS (the staging of gemm_stage_kernel, so no
// staging kernel runs) and each wave multiplies with no further barrier. With one slice the wave writes Y; otherwise
// it stores its slice's sums, which gemm_small_finish_kernel adds. (Gathering them in the kernel instead, each tile's
// last slice reading the others' sums with agent-scope atomic loads after a ticket, was slower: 30-160 us per call
// at M = 8-32.)
constexpr uint32_t kSmallSteps = 8;  // K steps per slice at most (40 KiB of B fragments per token group in LDS)

// K steps per slice at most for T token groups: the B fragments stay within 80 KiB of LDS (the table takes 64 KiB).
constexpr uint32_t small_max_steps(int T) { return T <= 2 ? kSmallSteps : kSmallSteps / 2; }

// One matrix of a small-path call (up to kSmallSubs matrices with the same columns share a launch): its tiles are
// tiles tile0 .. tile0 + n_tiles - 1 of the call, its rows rows row0 .. row0 + rows_p - 1 of the slice sums.
constexpr int kSmallSubs = 3;
struct SmallSub {
    const uint8_t* w;
    int32_t* y;
    uint32_t ldy, rows, rows_p, n_tiles, tile0, row0;
};

struct SmallArgs {
    SmallSub sub[kSmallSubs];
    uint32_t n_sub;
    const int8_t* x;
    int32_t* part;       // [kslices][M][rows_p] slice sums (kslices > 1)
    uint32_t ldx, rows_p, cols, n_tiles, n_chunks, n_ksteps, M, kslices;  // rows_p, n_tiles: of all the matrices
    uint32_t steps;      // K steps per slice (at most small_max_steps(T))
};

template <int T, int W, bool G>
__global__ __launch_bounds__(W * 64) void gemm_small_kernel(SmallArgs a) {
    __shared__ uint32_t tab[256 * 64];
    constexpr uint32_t S = small_max_steps(T);
    __shared__ uint4 bs[S * 5 * T * 64];
    constexpr uint32_t kTasks = S * T / W;  // B-fragment tasks per thread
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t tile = blockIdx.x * W + wave, kz = blockIdx.y;
    // the wave's matrix (wave-uniform) and its tile there (a tile past the call's tiles falls in the last matrix)
    const uint32_t j = !G ? 0u : (a.n_sub > 1u && tile >= a.sub[1].tile0 ? 1u : 0u) + (a.n_sub > 2u && tile >= a.sub[2].tile0 ? 1u : 0u);
    const SmallSub sb = j == 0u ? a.sub[0] : (j == 1u ? a.sub[1] : a.sub[2]);
    const uint32_t lt = tile - sb.tile0;
    const uint32_t ks0 = kz * a.steps, nst = min(a.steps, a.n_ksteps - ks0);
    const uint32_t half = lane >> 5;

    // The activations of this thread's tasks, loaded before the weights with every load at a valid address (no
    // branch that depends on the thread separates them from the weight loads, and nothing waits for them before the
    // weights are requested). When every row of x is 16-byte aligned: a whole 160-column block as 5 uint4 (kind 1);
    // when the slice's last step is the partial last block, its task (one per thread, a task holding W / T steps) as
    // the 80 columns of its half (kind 2). Other tasks are read by bytes after the weight loads (kind 0).
    const bool aligned = ((reinterpret_cast<uintptr_t>(a.x) | a.ldx) & 15u) == 0 && a.cols >= 160u;  // x holds a block
    const bool has_tail = a.cols % 160u != 0u && ks0 + nst == a.n_ksteps;
    uint4 X[kTasks][5];
    uint32_t kind[kTasks];
#pragma unroll
    for (uint32_t r = 0; r < kTasks; ++r) {
        const uint32_t t = tid + r * W * 64u;
        const uint32_t s = t / (64u * T), rr = t - s * 64u * T, tok = 32u * (rr >> 6) + (rr & 31u), ks = ks0 + s;
        const uint32_t hs = (rr >> 5) & 1u;
        const bool live = s < nst && tok < a.M;
        kind[r] = !live || !aligned ? 0u : (ks < a.cols / 160u ? 1u : 2u);
        if (aligned) {
            const int8_t* blk = (kind[r] == 1u ? a.x + static_cast<size_t>(tok) * a.ldx + ks * 160u : a.x) + 16u * hs;
#pragma unroll
            for (int e = 0; e < 5; ++e) X[r][e] = *reinterpret_cast<const uint4*>(blk + 32 * e);
        }
    }
    // kind 2, raw: the words at clamped addresses and the bytes of the word that straddles cols (masked where used).
    // Loaded by every workgroup (from the weights, which are 256-byte aligned, where no partial block is used) so that
    // no branch joins them before the weight loads.
    uint32_t V[20], tb[3];
    {
        const bool use = has_tail && aligned;
        const uint32_t t = tid + (nst - 1u) * T / W * W * 64u;
        const uint32_t s = t / (64u * T), rr = t - s * 64u * T, tok = 32u * (rr >> 6) + (rr & 31u), hs = (rr >> 5) & 1u;
        const int8_t* row = use ? a.x + static_cast<size_t>(tok < a.M ? tok : 0u) * a.ldx : reinterpret_cast<const int8_t*>(sb.w);
        const uint32_t base = use ? (a.n_ksteps - 1u) * 160u + 80u * hs : 0u, lastw = use ? (a.cols - 4u) & ~3u : 0u;
        const uint32_t i0 = use ? a.cols & ~3u : 0u, lastb = use ? a.cols - 1u : 0u;
#pragma unroll
        for (uint32_t d = 0; d < 20; ++d) V[d] = *reinterpret_cast<const uint32_t*>(row + min(base + 4u * d, lastw));
#pragma unroll
        for (uint32_t e = 0; e < 3; ++e) tb[e] = static_cast<uint8_t>(row[min(i0 + e, lastb)]);
    }

    // the trit table's entries (256 x 8 uint4 stores of 4 copies each)
    constexpr uint32_t kTabPer = 256u * 8u / (W * 64u);
    uint32_t te[kTabPer];
#pragma unroll
    for (uint32_t r = 0; r < kTabPer; ++r) te[r] = g_gemm_trits.v[(tid + r * W * 64u) >> 3];

    // the weights (a tile past the matrix reads the last one)
    const uint32_t ltile = min(lt, sb.n_tiles - 1u);
    const uint32_t grp = ltile / kTileGroup, t16 = ltile - grp * kTileGroup;
    const uint32_t Tg = min(static_cast<uint32_t>(kTileGroup), sb.n_tiles - grp * kTileGroup);
    const uint8_t* wbase = sb.w + (static_cast<size_t>(grp) * kTileGroup * a.n_chunks + t16) * 1024u + (lane & 31u) * 16u;
    u32x4g wv[S][2];
#pragma unroll
    for (uint32_t s = 0; s < S; ++s) {
        const uint32_t q = min((ks0 + min(s, nst - 1u)) * kStepChunks + half, a.n_chunks - 1u);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
            wv[s][rb] = __builtin_nontemporal_load((g_u4g*)(wbase + static_cast<size_t>(q) * Tg * 1024u + rb * 512u));
    }

#pragma unroll
    for (uint32_t r = 0; r < kTabPer; ++r) {
        const uint32_t i = tid + r * W * 64u;
        *reinterpret_cast<uint4*>(reinterpret_cast<char*>(tab) + (i >> 3) * 256u + (i & 7u) * 16u) =
            make_uint4(te[r], te[r], te[r], te[r]);
    }
    // B fragments of the slice; tokens past M get zeros
#pragma unroll
    for (uint32_t r = 0; r < kTasks; ++r) {
        const uint32_t t = tid + r * W * 64u;
        const uint32_t s = t / (64u * T), rr = t - s * 64u * T, g = rr >> 6, hs = (rr >> 5) & 1u, j = rr & 31u;
        const uint32_t tok = 32u * g + j, ks = ks0 + s;
        if (s >= nst) continue;
        uint4 o[5] = {};
        if (kind[r] == 1u) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                auto dw = [&](const uint4& v) { return kb == 0 ? v.x : (kb == 1 ? v.y : (kb == 2 ? v.z : v.w)); };
                const uint32_t a0 = dw(X[r][0]), a1 = dw(X[r][1]), a2 = dw(X[r][2]), a3 = dw(X[r][3]);
                const uint32_t lo01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u), hi01 = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
                const uint32_t lo23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u), hi23 = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
                o[kb] = make_uint4(__builtin_amdgcn_perm(lo23, lo01, 0x05040100u), __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                                   __builtin_amdgcn_perm(hi23, hi01, 0x05040100u), __builtin_amdgcn_perm(hi23, hi01, 0x07060302u));
            }
            o[4] = X[r][4];
        } else if (kind[r] == 2u) {
            // column ks * 160 + 80 hs + 5 k + p of the partial block is byte 5 k + p of the 80 loaded
            const uint32_t base = ks * 160u + 80u * hs, i0 = a.cols & ~3u;
            auto byte_at = [&](uint32_t i) -> uint32_t {
                const uint32_t c = base + i;
                return c < i0 ? (V[i >> 2] >> (8u * (i & 3u))) & 0xffu : (c < a.cols ? tb[c & 3u] : 0u);
            };
#pragma unroll
            for (uint32_t kb = 0; kb < 5; ++kb) {
                uint32_t w[4];
#pragma unroll
                for (uint32_t d = 0; d < 4; ++d) {
                    uint32_t v = 0;
#pragma unroll
                    for (uint32_t e = 0; e < 4; ++e)
                        v |= byte_at(kb < 4 ? 5u * (4u * kb + d) + e : 5u * (4u * d + e) + 4u) << (8 * e);
                    w[d] = v;
                }
                o[kb] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        } else if (tok < a.M) {
            const int8_t* xr = a.x + static_cast<size_t>(tok) * a.ldx;
            const bool tail = ks >= a.cols / 160u;
            auto act = [&](uint32_t k, uint32_t p) -> uint32_t {
                const uint32_t idx = tail ? ks * 160u + 5u * (16u * hs + k) + p : ks * 160u + 32u * p + 16u * hs + k;
                return idx < a.cols ? static_cast<uint32_t>(static_cast<uint8_t>(xr[idx])) : 0u;
            };
#pragma unroll
            for (uint32_t kb = 0; kb < 5; ++kb) {
                uint32_t w[4];
#pragma unroll
                for (uint32_t d = 0; d < 4; ++d) {
                    uint32_t v = 0;
#pragma unroll
                    for (uint32_t e = 0; e < 4; ++e) v |= (kb < 4 ? act(4u * kb + d, e) : act(4u * d + e, 4u)) << (8 * e);
                    w[d] = v;
                }
                o[kb] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
#pragma unroll
        for (uint32_t kb = 0; kb < 5; ++kb) bs[((s * 5u + kb) * T + g) * 64u + j + 32u * hs] = o[kb];
    }
    __syncthreads();
    if (tile >= a.n_tiles) return;

    const char* tabb = reinterpret_cast<const char*>(tab);
    const uint32_t lane_off = (lane & 31u) * 4u;
    v16i acc[2][T];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int g = 0; g < T; ++g) acc[rb][g] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (uint32_t s = 0; s < S; ++s) {
        if (s >= nst) break;
        const bool inside = (ks0 + s) * kStepChunks + half < a.n_chunks;
        v4i A[2][5];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const uint32_t dw[4] = {inside ? wv[s][rb].x : kZeroWord, inside ? wv[s][rb].y : kZeroWord,
                                    inside ? wv[s][rb].z : kZeroWord, inside ? wv[s][rb].w : kZeroWord};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                int t[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t addr = __builtin_amdgcn_perm(dw[m], lane_off, 0x0c0c0000u | ((4u + b) << 8));
                    t[b] = static_cast<int>(*reinterpret_cast<const uint32_t*>(tabb + addr));
                }
                A[rb][m] = v4i{t[0], t[1], t[2], t[3]};
            }
            A[rb][4] = v4i{static_cast<int>(t4_bytes(dw[0])), static_cast<int>(t4_bytes(dw[1])),
                           static_cast<int>(t4_bytes(dw[2])), static_cast<int>(t4_bytes(dw[3]))};
        }
#pragma unroll
        for (int kb = 0; kb < 5; ++kb) {
#pragma unroll
            for (int g = 0; g < T; ++g) {
                const uint4 b = bs[((s * 5u + kb) * T + g) * 64u + lane];
                const v4i B = v4i{static_cast<int>(b.x), static_cast<int>(b.y), static_cast<int>(b.z), static_cast<int>(b.w)};
                acc[0][g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[0][kb], B, acc[0][g], 0, 0, 0);
                acc[1][g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[1][kb], B, acc[1][g], 0, 0, 0);
            }
        }
    }
    // C of (block rb, token group g): lane l, register r -> row 8 (r / 4) + 4 (l / 32) + r % 4 of the block, token
    // 32 g + l % 32
#pragma unroll
    for (int g = 0; g < T; ++g) {
        const uint32_t m = 32u * g + (lane & 31u);
        if (m >= a.M) continue;
        if (a.kslices == 1) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t n = lt * 64u + rb * 32u + 8u * (r / 4) + 4u * half + (r % 4);
                    if (n < sb.rows) sb.y[static_cast<size_t>(m) * sb.ldy + n] = acc[rb][g][r];
                }
        } else {  // the slice's sums; gemm_small_finish_kernel adds the slices
            int32_t* pp = a.part + (static_cast<size_t>(kz) * a.M + m) * a.rows_p + sb.row0 + lt * 64u;
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    *reinterpret_cast<int4*>(pp + rb * 32u + 8u * r4 + 4u * half) =
                        make_int4(acc[rb][g][4 * r4], acc[rb][g][4 * r4 + 1], acc[rb][g][4 * r4 + 2], acc[rb][g][4 * r4 + 3]);
        }
    }
}

// Y[m][n] = sum over the slices of gemm_small_kernel's sums (block = 256 rows of the call's slice sums, one token).
template <bool G>
__global__ __launch_bounds__(256) void gemm_small_finish_kernel(SmallArgs a) {
    const uint32_t n = blockIdx.x * 256u + threadIdx.x, m = blockIdx.y;
    const uint32_t j = !G ? 0u : (a.n_sub > 1u && n >= a.sub[1].row0 ? 1u : 0u) + (a.n_sub > 2u && n >= a.sub[2].row0 ? 1u : 0u);
    const SmallSub sb = j == 0u ? a.sub[0] : (j == 1u ? a.sub[1] : a.sub[2]);  // no indexing of the arguments
    const uint32_t ln = n - sb.row0;
    if (n >= a.rows_p || ln >= sb.rows) return;
    const size_t stride = static_cast<size_t>(a.M) * a.rows_p;
    const int32_t* p = a.part + static_cast<size_t>(m) * a.rows_p + n;
    int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    uint32_t k = 0;
    for (; k + 4 <= a.kslices; k += 4) {
        s0 += p[k * stride];
        s1 += p[(k + 1) * stride];
        s2 += p[(k + 2) * stride];
        s3 += p[(k + 3) * stride];
    }
    for (; k < a.kslices; ++k) s0 += p[k * stride];
    sb.y[static_cast<size_t>(m) * sb.ldy + ln] = (s0 + s1) + (s2 + s3);
}


// The small kernel's shape: waves per workgroup (4 or 8) and K steps per slice (2 to small_max_steps). A round is one
// workgroup per CU (the trit table and the B fragments take 104-144 KiB of LDS); a round costs about 3 K steps of
// loads and staging plus its K steps, each T x W / 4 one-wave steps of matrix-core work per SIMD, and the finish
// about a quarter step per slice (measured at the configs[2] shapes). The cheapest pair; on a tie the longer slices.
struct SmallShape {
    uint32_t waves, steps, kslices;
};

static SmallShape small_shape(const Geometry& g, int num_cus, size_t M) {
    const uint64_t n_ksteps = (g.n_chunks + kStepChunks - 1) / kStepChunks;
    const uint64_t cus = static_cast<uint64_t>(std::max(num_cus, 1));
    const int Ti = M <= 32 ? 1 : (M <= 64 ? 2 : 4);
    const double T = Ti;
    const uint32_t S = small_max_steps(Ti);
    double best = 1e300;
    SmallShape sh{4, S, 1};
    for (uint32_t st = S; st >= 2; --st)
        for (uint32_t w : {4u, 8u}) {
            const uint64_t ks = (n_ksteps + st - 1) / st;
            const uint64_t rounds = ((g.n_tiles + w - 1) / w * ks + cus - 1) / cus;
            const double cost = static_cast<double>(rounds) * (3.0 + st * T * w / 4.0) + (ks > 1 ? 0.25 * ks : 0.0);
            if (cost < best - 1e-9) {
                best = cost;
                sh = SmallShape{w, st, static_cast<uint32_t>(ks)};
            }
        }
    return sh;
}

static uint32_t small_kslices(const Geometry& g, int num_cus, size_t M) { return small_shape(g, num_cus, M).kslices; }

// M <= 32 always; 33-128 tokens (two or four token groups) only for matrices of at most 128 tiles (8192 rows) and
// 32768 columns whose slice sums take at most 64 MiB: at 23040 x 3072 the staged kernel was faster (28.4 against
// 31.0 us at M = 64, 41.5 against 42.6 us at M = 128), at 3072 x 23040 and 3072 x 3072 slower (24.0 against 20.0 us at
// M = 64; 34.8 against 33.4 and 24.0 against 19.9 us at M = 128, 54 MiB of slice sums at 3072 x 23040).
constexpr size_t kSmallPartCap = size_t(64) << 20;
static bool small_path(const Geometry& g, size_t M, int num_cus) {
    if (M <= 32) return true;
    return M <= 128 && g.n_tiles <= 128 && g.cols <= 32768 && small_part_bytes(g, M, num_cus) <= kSmallPartCap;
}

bool gemm_small_path(const Geometry& g, size_t M, int num_cus) { return small_path(g, M, num_cus); }

static size_t small_part_bytes(const Geometry& g, size_t M, int num_cus) {
    const uint32_t ks = small_kslices(g, num_cus, M);
    return ks > 1 ? round_up(static_cast<size_t>(ks) * M * g.padded_rows * 4u, 256) : 0;
}

// The small path over n matrices of the same columns (tiles and slice-sum rows concatenated in order).
template <bool G>
static int launch_small(const GemmSub* subs, int n, int num_cus, const int8_t* x, size_t M, size_t ldx, uint8_t* ws,
                        hipStream_t stream) {
    SmallArgs a{};
    a.n_sub = static_cast<uint32_t>(n);
    uint32_t tiles = 0, rows_p = 0;
    for (int i = 0; i < n; ++i) {
        const Geometry& gi = *subs[i].g;
        a.sub[i] = SmallSub{subs[i].w, subs[i].y, static_cast<uint32_t>(subs[i].ldy), static_cast<uint32_t>(gi.rows),
                            static_cast<uint32_t>(gi.padded_rows), static_cast<uint32_t>(gi.n_tiles), tiles, rows_p};
        tiles += static_cast<uint32_t>(gi.n_tiles);
        rows_p += static_cast<uint32_t>(gi.padded_rows);
    }
    const Geometry g = geometry(rows_p, subs[0].g->cols);  // the call's tiles, for the planner
    a.x = x;
    a.part = reinterpret_cast<int32_t*>(ws);
    a.ldx = static_cast<uint32_t>(ldx);
    a.rows_p = rows_p;
    a.cols = static_cast<uint32_t>(g.cols);
    a.n_tiles = tiles;
    a.n_chunks = static_cast<uint32_t>(g.n_chunks);
    a.n_ksteps = static_cast<uint32_t>((g.n_chunks + kStepChunks - 1) / kStepChunks);
    a.M = static_cast<uint32_t>(M);
    const SmallShape sh = small_shape(g, num_cus, M);
    a.kslices = sh.kslices;
    a.steps = sh.steps;
    const dim3 grid((a.n_tiles + sh.waves - 1) / sh.waves, a.kslices), block(sh.waves * 64);
    if (M <= 32) {
        if (sh.waves == 8) hipLaunchKernelGGL((gemm_small_kernel<1, 8, G>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((gemm_small_kernel<1, 4, G>), grid, block, 0, stream, a);
    } else if (M <= 64) {
        if (sh.waves == 8) hipLaunchKernelGGL((gemm_small_kernel<2, 8, G>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((gemm_small_kernel<2, 4, G>), grid, block, 0, stream, a);
    } else {
        if (sh.waves == 8) hipLaunchKernelGGL((gemm_small_kernel<4, 8, G>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((gemm_small_kernel<4, 4, G>), grid, block, 0, stream, a);
    }
    VX_HIP(hipGetLastError());
    if (a.kslices > 1) {
        hipLaunchKernelGGL(gemm_small_finish_kernel<G>, dim3((a.rows_p + 255u) / 256u, a.M), dim3(256), 0, stream, a);
        VX_HIP(hipGetLastError());
    }
    return VX_OK;
}

bool gemm_group_small_path(const GemmSub* subs, int n, size_t M, int num_cus) {
    if (n < 1 || n > kSmallSubs) return false;
    for (int i = 0; i < n; ++i)
        if (subs[i].g->cols != subs[0].g->cols || !small_path(*subs[i].g, M, num_cus)) return false;
    return true;
}

size_t gemm_group_part_bytes(const GemmSub* subs, int n, size_t M, int num_cus) {
    size_t rows_p = 0;
    for (int i = 0; i < n; ++i) rows_p += subs[i].g->padded_rows;
    return small_part_bytes(geometry(rows_p, subs[0].g->cols), M, num_cus);
}

int launch_gemm_group(const GemmSub* subs, int n, int num_cus, const int8_t* x, size_t M, size_t ldx, uint8_t* ws,
                      hipStream_t stream) {
    if (!gemm_group_small_path(subs, n, M, num_cus)) VX_FAIL(VX_ERR_INTERNAL, "a grouped GEMM of %d matrices off the small path", n);
    return launch_small<true>(subs, n, num_cus, x, M, ldx, ws, stream);
}

int launch_gemm(const uint8_t* w, const Geometry& g, int num_cus, const int8_t* x, size_t M, size_t ldx, int32_t* y,
                size_t ldy, uint8_t* ws, hipStream_t stream) {
    if (small_path(g, M, num_cus)) {
        const GemmSub sub{w, &g, y, ldy};
        return launch_small<false>(&sub, 1, num_cus, x, M, ldx, ws, stream);
    }
    VX_TRY(launch_gemm_stage(x, M, ldx, g.cols, ws, stream));
    return launch_gemm_staged(w, g, num_cus, ws, M, y, ldy, ws + gemm_stage_bytes(g.cols, M), stream);
}

// ---- the no-allocation entry point's workspace -----------------------------------------------------------------------

// Workspace of vx_gemm_i32_noalloc_dev: one array per GPU, allocated with the code object when the library's kernels
// are first loaded on that GPU and held until the process ends. Host code never passes `scratch` itself (in host code
// the name is only a stand-in for the symbol); it passes the device address hipGetSymbolAddress returns for the
// current device, looked up once per device. Every call on a GPU reuses that GPU's array, so calls that overlap on one
// GPU race; the kernels write every word they later read (staged activations, plane-4 parts, K-slice partials), so
// no clearing is needed between calls.
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_ptr[kMaxScratchDevices] = {};

// The device address of `scratch` on `device`, which must be the current device.
static int scratch_address(int device, uint8_t** out) {
    if (device < 0 || device >= kMaxScratchDevices)
        VX_FAIL(VX_ERR_UNSUPPORTED, "device %d is beyond the %d devices the no-allocation GEMM serves", device,
                kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device] == nullptr) {
        void* p = nullptr;
        VX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (p == nullptr) VX_FAIL(VX_ERR_DEVICE, "hipGetSymbolAddress returned no address for the GEMM scratch");
        g_scratch_ptr[device] = static_cast<uint8_t*>(p);
    }
    *out = g_scratch_ptr[device];
    return VX_OK;
}

int gemm_scratch_prepare(int device) {
    uint8_t* p = nullptr;
    return scratch_address(device, &p);
}

int launch_gemm_noalloc(const uint8_t* w, const Geometry& g, int device, int num_cus, const int8_t* x, size_t M,
                        size_t ldx, int32_t* y, size_t ldy, hipStream_t stream) {
    const size_t need = gemm_workspace_bytes(g, M, num_cus);
    if (need > kNoAllocScratchBytes)
        VX_FAIL(VX_ERR_INVALID_SHAPE,
                "m = %zu tokens on a %zu x %zu matrix need %zu bytes of workspace, more than the %zu bytes the "
                "no-allocation GEMM holds; use vx_gemm_i32_dev with a workspace",
                M, g.rows, g.cols, need, kNoAllocScratchBytes);
    uint8_t* ws = nullptr;
    VX_TRY(scratch_address(device, &ws));
    return launch_gemm(w, g, num_cus, x, M, ldx, y, ldy, ws, stream);
}

}  // namespace vx
