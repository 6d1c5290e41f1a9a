#define _GNU_SOURCE
/*
 * cpu_avx512.c - the reference's production CPU GEMV, transcribed with AVX-512 intrinsics (CPU BASELINE ONLY).
 *
 * bench.py times this beside the GPU as the reported CPU baseline; tests/ check it against the brute-force product.
 * The product (quintrit_amd/) never calls it. The Rust original cannot be built here (no Rust toolchain), so the
 * algorithm is restated in C with the same instruction sequence:
 *   - activation tables: build_compact_wide_impl (quintrit-core/src/simd/avx512.rs:1216-1247): per tile column byte c
 *     one 64-byte table per part (x = 16 hi + lo, lo = ((x + 8) & 15) - 8): entries 0..8 hold the sums over (a3, a4)
 *     for the 9 digit pairs, entries 9..35 the sums over (a0, a1, a2) for the 27 digit triples, formed by masked
 *     adds and subtracts of the broadcast parts (avx512.rs:1180-1197 for the masks);
 *   - kernel: gemv_compact_multi::<3, 4096, T0, 0, true> -> compact_multi_block (avx512.rs:1526-1626): three 64-row
 *     blocks per pass, per column two vpermb lookups per part after the shuffle decode of the weight byte
 *     (h34 = w / 28 and r3 + 9 = w - (28 h34 - 9) from two 64-entry tables on w >> 2, avx512.rs:1255-1300), int8 sums
 *     over 3 columns, vpmaddubsw with (1, 16) into int16 over chunks of 45 columns, int32 accumulators, a 4 KiB T0
 *     prefetch of the weights;
 *   - threads: whole 64-row blocks, ceil(blocks / threads) * 64 rows per thread (avx512.rs:1150-1168).
 * Weights are in the reference's 64-row tiled layout (transform_weights_lut_64, avx512.rs:53-78): block b holds, for
 * each tile column byte c, the bytes of its 64 rows contiguously at b * 64 * tbr + c * 64.
 */
#include "cpu_avx512.h"

#include <immintrin.h>
#include <omp.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "velurex_oracle.h"

#define VXC_TARGET __attribute__((target("avx512f,avx512bw,avx512vbmi")))

int vxc_supported(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vbmi");
}

size_t vxc_table_bytes(size_t cols) { return 2 * vxo_tile_row_bytes(cols) * 64; }

void vxc_tile64(const uint8_t* planar, size_t rows, size_t cols, uint8_t* out) {
    const size_t prb = vxo_planar_row_bytes(cols), bpr = vxo_tile_row_bytes(cols);
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < bpr; ++c)
            out[(r / 64) * 64 * bpr + c * 64 + r % 64] = vxo_tile_byte(planar + r * prb, cols, c);
}

/* Lane masks (positive, negative coefficient) of activation position p in a compact table. */
static void coefficient_masks(uint64_t pos[5], uint64_t neg[5]) {
    memset(pos, 0, 5 * sizeof(uint64_t));
    memset(neg, 0, 5 * sizeof(uint64_t));
    for (int s = 0; s < 9; ++s) {
        const int c3 = s % 3 - 1, c4 = s / 3 - 1;
        if (c3 > 0) pos[3] |= 1ull << s;
        if (c3 < 0) neg[3] |= 1ull << s;
        if (c4 > 0) pos[4] |= 1ull << s;
        if (c4 < 0) neg[4] |= 1ull << s;
    }
    for (int s = 0; s < 27; ++s) {
        const int lane = 9 + s;
        const int c[3] = {s % 3 - 1, (s / 3) % 3 - 1, s / 9 - 1};
        for (int p = 0; p < 3; ++p) {
            if (c[p] > 0) pos[p] |= 1ull << lane;
            if (c[p] < 0) neg[p] |= 1ull << lane;
        }
    }
}

/* column_activation_index (pack.rs:230-237), inlined as the reference's builder has it: column c of a full 160-trit
 * block holds activations (c / 32) 160 + p 32 + c % 32; a column of the packed tail holds five consecutive ones. */
static inline size_t column_index(size_t cols, size_t full, size_t c, size_t p) {
    if (c < full) return (c >> 5) * 160 + p * 32 + (c & 31);
    return cols / 160 * 160 + 5 * (c - full) + p;
}

VXC_TARGET void vxc_build_tables(const int8_t* acts, size_t cols, int8_t* tables) {
    const size_t bpr = vxo_tile_row_bytes(cols), full = vxo_tile_full_columns(cols);
    uint64_t pos[5], neg[5];
    coefficient_masks(pos, neg);
    const __mmask64 p0 = pos[0], p1 = pos[1], p2 = pos[2], p3 = pos[3], p4 = pos[4];
    const __mmask64 n0 = neg[0], n1 = neg[1], n2 = neg[2], n3 = neg[3], n4 = neg[4];
    int8_t* lo_dst = tables;
    int8_t* hi_dst = tables + bpr * 64;
    for (size_t c = 0; c < bpr; ++c) {
        int8_t l[5], h[5];
        for (size_t p = 0; p < 5; ++p) {
            const size_t idx = column_index(cols, full, c, p);
            const int x = idx < cols ? acts[idx] : 0;
            const int lv = ((x + 8) & 15) - 8;
            l[p] = (int8_t)lv;
            h[p] = (int8_t)((x - lv) >> 4);
        }
        __m512i acc_lo = _mm512_setzero_si512(), acc_hi = _mm512_setzero_si512();
#define VXC_PART(P)                                                                              \
        do {                                                                                     \
            const __m512i bl = _mm512_set1_epi8(l[P]), bh = _mm512_set1_epi8(h[P]);             \
            acc_lo = _mm512_mask_add_epi8(acc_lo, p##P, acc_lo, bl);                             \
            acc_lo = _mm512_mask_sub_epi8(acc_lo, n##P, acc_lo, bl);                             \
            acc_hi = _mm512_mask_add_epi8(acc_hi, p##P, acc_hi, bh);                             \
            acc_hi = _mm512_mask_sub_epi8(acc_hi, n##P, acc_hi, bh);                             \
        } while (0)
        VXC_PART(0);
        VXC_PART(1);
        VXC_PART(2);
        VXC_PART(3);
        VXC_PART(4);
#undef VXC_PART
        _mm512_storeu_si512((void*)(lo_dst + c * 64), acc_lo);
        _mm512_storeu_si512((void*)(hi_dst + c * 64), acc_hi);
    }
}

/* The rows of one block from its four int32 accumulators: vpunpck{l,h}bw splits each 128-bit lane into rows 0..7 and
 * 8..15 of its 16 rows; the low and high 256 bits of the int16 sums hold lanes 0-1 and 2-3. */
VXC_TARGET static void put_rows(__m512i a0, __m512i a1, __m512i b0, __m512i b1, float* out) {
    int32_t t[16];
    const __m512i acc[4] = {a0, b0, a1, b1};
    const int first[4] = {0, 8, 32, 40};
    for (int k = 0; k < 4; ++k) {
        _mm512_storeu_si512((void*)t, acc[k]);
        for (int i = 0; i < 8; ++i) {
            out[first[k] + i] = (float)t[i];
            out[first[k] + 16 + i] = (float)t[8 + i];
        }
    }
}

#define VXC_NB_MAX 3
#define VXC_CHUNK 45
#define VXC_PF 4096

/* compact_multi_block::<NB, ...> for one compile-time NB (the reference's const generic), so that the per-block
 * registers are registers: the body is always inlined into multi_block_3 / multi_block_1 with nb a constant. */
VXC_TARGET static inline __attribute__((always_inline)) void multi_block(const int nb, const uint8_t* w, size_t stride,
                                                                          const int8_t* lo, const int8_t* hi,
                                                                          size_t bpr, float* out) {
    static const uint8_t th_b[64] = {
        0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2, 3, 3, 3, 3, 3, 3, 3, 4, 4, 4, 4,
        4, 4, 4, 5, 5, 5, 5, 5, 5, 5, 6, 6, 6, 6, 6, 6, 6, 7, 7, 7, 7, 7, 7, 7, 8, 8, 8, 8, 8, 8, 8, 9};
    uint8_t tm_b[64];
    for (int i = 0; i < 64; ++i) tm_b[i] = (uint8_t)(28 * th_b[i] - 9); /* 28 floor(i / 7) - 9 (avx512.rs:1266-1275) */
    const __m512i th = _mm512_loadu_si512((const void*)th_b), tm = _mm512_loadu_si512((const void*)tm_b);
    const __m512i combine = _mm512_set1_epi16(0x1001);
    const __m512i zero = _mm512_setzero_si512();
    __m512i a0[VXC_NB_MAX], a1[VXC_NB_MAX], b0[VXC_NB_MAX], b1[VXC_NB_MAX];
#pragma GCC unroll 4
    for (int b = 0; b < nb; ++b) a0[b] = a1[b] = b0[b] = b1[b] = zero;
    for (size_t c = 0; c < bpr;) {
        const size_t len = bpr - c < VXC_CHUNK ? bpr - c : VXC_CHUNK;
        __m512i sa[VXC_NB_MAX], sb[VXC_NB_MAX];
#pragma GCC unroll 4
        for (int b = 0; b < nb; ++b) sa[b] = sb[b] = zero;
        for (size_t ci = 0; ci < len;) {
            const size_t n = len - ci < 3 ? len - ci : 3;
#pragma GCC unroll 4
            for (int b = 0; b < nb; ++b) {
                const char* base = (const char*)(w + b * stride + (c + ci) * 64);
                _mm_prefetch(base + VXC_PF, _MM_HINT_T0);
                _mm_prefetch(base + VXC_PF + 64, _MM_HINT_T0);
                _mm_prefetch(base + VXC_PF + 128, _MM_HINT_T0);
            }
            __m512i slo[VXC_NB_MAX], shi[VXC_NB_MAX];
#pragma GCC unroll 3
            for (size_t j = 0; j < 3; ++j) {
                if (j >= n) break;
                const size_t col = c + ci + j;
                const __m512i tl = _mm512_loadu_si512((const void*)(lo + col * 64));
                const __m512i tt = _mm512_loadu_si512((const void*)(hi + col * 64));
#pragma GCC unroll 4
                for (int b = 0; b < nb; ++b) {
                    const __m512i wv = _mm512_loadu_si512((const void*)(w + b * stride + col * 64));
                    const __m512i idx = _mm512_srli_epi16(wv, 2);
                    const __m512i h34 = _mm512_permutexvar_epi8(idx, th);
                    const __m512i r3 = _mm512_sub_epi8(wv, _mm512_permutexvar_epi8(idx, tm));
                    const __m512i l = _mm512_add_epi8(_mm512_permutexvar_epi8(h34, tl), _mm512_permutexvar_epi8(r3, tl));
                    const __m512i h = _mm512_add_epi8(_mm512_permutexvar_epi8(h34, tt), _mm512_permutexvar_epi8(r3, tt));
                    if (j == 0) {
                        slo[b] = l;
                        shi[b] = h;
                    } else {
                        slo[b] = _mm512_add_epi8(slo[b], l);
                        shi[b] = _mm512_add_epi8(shi[b], h);
                    }
                }
            }
#pragma GCC unroll 4
            for (int b = 0; b < nb; ++b) {
                sa[b] = _mm512_add_epi16(sa[b], _mm512_maddubs_epi16(combine, _mm512_unpacklo_epi8(slo[b], shi[b])));
                sb[b] = _mm512_add_epi16(sb[b], _mm512_maddubs_epi16(combine, _mm512_unpackhi_epi8(slo[b], shi[b])));
            }
            ci += n;
        }
#pragma GCC unroll 4
        for (int b = 0; b < nb; ++b) {
            a0[b] = _mm512_add_epi32(a0[b], _mm512_cvtepi16_epi32(_mm512_castsi512_si256(sa[b])));
            a1[b] = _mm512_add_epi32(a1[b], _mm512_cvtepi16_epi32(_mm512_extracti64x4_epi64(sa[b], 1)));
            b0[b] = _mm512_add_epi32(b0[b], _mm512_cvtepi16_epi32(_mm512_castsi512_si256(sb[b])));
            b1[b] = _mm512_add_epi32(b1[b], _mm512_cvtepi16_epi32(_mm512_extracti64x4_epi64(sb[b], 1)));
        }
        c += len;
    }
    for (int b = 0; b < nb; ++b) put_rows(a0[b], a1[b], b0[b], b1[b], out + b * 64);
}

VXC_TARGET static void multi_block_3(const uint8_t* w, size_t stride, const int8_t* lo, const int8_t* hi, size_t bpr,
                                     float* out) {
    multi_block(3, w, stride, lo, hi, bpr, out);
}

VXC_TARGET static void multi_block_1(const uint8_t* w, size_t stride, const int8_t* lo, const int8_t* hi, size_t bpr,
                                     float* out) {
    multi_block(1, w, stride, lo, hi, bpr, out);
}

VXC_TARGET static void gemv_blocks(const uint8_t* w, const int8_t* tables, size_t nblocks, size_t bpr, float* out) {
    const size_t stride = 64 * bpr;
    const int8_t* lo = tables;
    const int8_t* hi = tables + bpr * 64;
    size_t b = 0;
    for (; b + 3 <= nblocks; b += 3) multi_block_3(w + b * stride, stride, lo, hi, bpr, out + b * 64);
    for (; b < nblocks; ++b) multi_block_1(w + b * stride, stride, lo, hi, bpr, out + b * 64);
}

void vxc_gemv_tables(const uint8_t* tiles64, const int8_t* tables, size_t rows, size_t cols, float* out, int threads) {
    const size_t bpr = vxo_tile_row_bytes(cols), nblocks = rows / 64;
    if (threads <= 1 || nblocks < (size_t)threads) {
        gemv_blocks(tiles64, tables, nblocks, bpr, out);
        return;
    }
    const size_t per = (nblocks + (size_t)threads - 1) / (size_t)threads; /* blocks per thread */
    const size_t chunks = (nblocks + per - 1) / per;
#pragma omp parallel for num_threads(threads) schedule(static, 1)
    for (size_t t = 0; t < chunks; ++t) {
        const size_t b0 = t * per, nb = nblocks - b0 < per ? nblocks - b0 : per;
        gemv_blocks(tiles64 + b0 * 64 * bpr, tables, nb, bpr, out + b0 * 64);
    }
}

void vxc_gemv(const uint8_t* tiles64, const int8_t* acts, size_t rows, size_t cols, float* out, int threads,
              int8_t* table_scratch) {
    vxc_build_tables(acts, cols, table_scratch);
    vxc_gemv_tables(tiles64, table_scratch, rows, cols, out, threads);
}

/* The engine runs the projections that share an input concurrently on one pool after one table build
 * (forward_linear_triple / forward_linear_pair, quintrit-runtime/src/layer.rs:657-716, the tables built once before
 * them, attention.rs:138-163); here the blocks of the whole group are split evenly over the threads. */
void vxc_gemv_group(const uint8_t* const* tiles64, const size_t* rows, int n, const int8_t* acts, size_t cols,
                    float* const* outs, int threads, int8_t* table_scratch) {
    vxc_build_tables(acts, cols, table_scratch);
    const size_t bpr = vxo_tile_row_bytes(cols);
    size_t total = 0;
    for (int m = 0; m < n; ++m) total += rows[m] / 64;
    if (threads < 1) threads = 1;
    const size_t per = (total + (size_t)threads - 1) / (size_t)threads;
#pragma omp parallel num_threads(threads)
    {
        const size_t g0 = (size_t)omp_get_thread_num() * per, g1 = g0 + per < total ? g0 + per : total;
        size_t base = 0; /* first global block of matrix m */
        for (int m = 0; m < n && g0 < g1; ++m) {
            const size_t nb = rows[m] / 64, lo = g0 > base ? g0 - base : 0, hi = g1 - base < nb ? g1 - base : nb;
            if (g1 > base && lo < nb && lo < hi)
                gemv_blocks(tiles64[m] + lo * 64 * bpr, table_scratch, hi - lo, bpr, outs[m] + lo * 64);
            base += nb;
        }
    }
}

/* Fills out[0..n) with pseudo-random valid packed bytes (splitmix64 per 4 bytes, each 16-bit piece mapped onto the 243
 * valid values by multiply-shift), in parallel: the CPU baseline's 1.9 GB of random weights in well under a second. */
void vxc_fill_valid(uint8_t* out, size_t n, uint64_t seed) {
    uint8_t valid[243];
    int k = 0;
    for (int b = 0; b < 256; ++b)
        if (vxo_byte_is_valid((uint8_t)b)) valid[k++] = (uint8_t)b;
#pragma omp parallel for schedule(static)
    for (size_t w = 0; w < (n + 3) / 4; ++w) {
        uint64_t z = seed + (w + 1) * 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        for (size_t j = 0; j < 4 && w * 4 + j < n; ++j) out[w * 4 + j] = valid[(((z >> (16 * j)) & 0xFFFF) * 243) >> 16];
    }
}

/* Pins OpenMP thread t of a team of n to logical CPU cpus[t] (the team the GEMV and read-stream calls with n threads
 * reuse); returns the number of threads that could not be pinned. */
int vxc_pin_threads(const int* cpus, int n) {
    int failed = 0;
#pragma omp parallel num_threads(n) reduction(+ : failed)
    {
        cpu_set_t set;
        CPU_ZERO(&set);
        CPU_SET(cpus[omp_get_thread_num()], &set);
        failed += pthread_setaffinity_np(pthread_self(), sizeof set, &set) != 0;
    }
    return failed;
}

/* Sums words [w0, w1) of buf with 64-byte loads into four independent accumulators (the loop is bound by the loads,
 * not by the adds' latency), prefetching 4 KiB ahead like the GEMV. */
VXC_TARGET static uint64_t read_range(const uint64_t* buf, size_t w0, size_t w1) {
    __m512i s0 = _mm512_setzero_si512(), s1 = s0, s2 = s0, s3 = s0;
    size_t i = w0;
    for (; i + 32 <= w1; i += 32) {
        _mm_prefetch((const char*)(buf + i) + 4096, _MM_HINT_T0);
        _mm_prefetch((const char*)(buf + i) + 4160, _MM_HINT_T0);
        _mm_prefetch((const char*)(buf + i) + 4224, _MM_HINT_T0);
        _mm_prefetch((const char*)(buf + i) + 4288, _MM_HINT_T0);
        s0 = _mm512_add_epi64(s0, _mm512_loadu_si512(buf + i));
        s1 = _mm512_add_epi64(s1, _mm512_loadu_si512(buf + i + 8));
        s2 = _mm512_add_epi64(s2, _mm512_loadu_si512(buf + i + 16));
        s3 = _mm512_add_epi64(s3, _mm512_loadu_si512(buf + i + 24));
    }
    uint64_t total = (uint64_t)_mm512_reduce_add_epi64(
        _mm512_add_epi64(_mm512_add_epi64(s0, s1), _mm512_add_epi64(s2, s3)));
    for (; i < w1; ++i) total += buf[i];
    return total;
}

/* Host read bandwidth: `threads` threads each sum one contiguous share of `words` 64-bit words; returns the sum. */
uint64_t vxc_read_stream(const uint64_t* buf, size_t words, int threads) {
    uint64_t total = 0;
#pragma omp parallel num_threads(threads) reduction(+ : total)
    {
        const size_t t = (size_t)omp_get_thread_num(), n = (size_t)omp_get_num_threads();
        const size_t per = (words + n - 1) / n, w0 = t * per < words ? t * per : words;
        total += read_range(buf, w0, w0 + per < words ? w0 + per : words);
    }
    return total;
}

/* The calling thread's core clock: eight dependent register-to-register adds per iteration retire at one per cycle,
 * so cycles = 8 x iterations, timed against CLOCK_MONOTONIC. (Adds of an immediate would not do: some cores fold
 * chains of them at register renaming.) */
double vxc_clock_hz(void) {
    const uint64_t iters = 50000000;
    uint64_t x = 0;
    const uint64_t one = 1;
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (uint64_t i = 0; i < iters; ++i)
        __asm__ volatile("add %1, %0\n\tadd %1, %0\n\tadd %1, %0\n\tadd %1, %0\n\t"
                         "add %1, %0\n\tadd %1, %0\n\tadd %1, %0\n\tadd %1, %0" : "+r"(x) : "r"(one));
    clock_gettime(CLOCK_MONOTONIC, &t1);
    const double dt = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
    return x == 8 * iters ? 8.0 * (double)iters / dt : 0.0;
}
