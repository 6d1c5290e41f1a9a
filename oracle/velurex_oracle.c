/*
 * velurex_oracle.c - CPU restatement of the reference's velurex ternary GEMV path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this code, as the checker or the timed
 * CPU baseline. The product (the HIP library under quintrit_amd/) never links or calls it.
 *
 * Written from the reference's Rust sources and its docs/velurex-encoding.md as a specification; each function cites
 * the file:line it follows. Pinning: tests/test_oracle.py checks every function against something that does not
 * restate it (brute force, round trips, closed forms, numpy, the reference's own test patterns).
 */
#include "velurex_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------------------------------- */
/* Encoding                                                                                                          */
/* ---------------------------------------------------------------------------------------------------------------- */

/* pack.rs:28-36: B = d0 + 3 d1 + 9 d2 + 28 d3 + 84 d4 with d = t + 1. */
uint8_t vxo_pack_5trits(const int8_t t[5]) {
    static const int radix[5] = {1, 3, 9, 28, 84};
    int b = 0;
    for (int p = 0; p < 5; ++p) b += (t[p] + 1) * radix[p];
    return (uint8_t)b;
}

/* pack.rs:41-58: the 243 states s (base-3 digits of s, least significant first) are packed; every byte that is not
 * the packing of some state decodes to five zeros. */
static int8_t g_byte_trits[256][5];
static uint8_t g_byte_valid[256];
static int g_tables_ready;

static void init_tables(void) {
    if (g_tables_ready) return;
    memset(g_byte_trits, 0, sizeof g_byte_trits);
    memset(g_byte_valid, 0, sizeof g_byte_valid);
    for (int s = 0; s < 243; ++s) {
        int8_t t[5];
        int v = s;
        for (int p = 0; p < 5; ++p) {
            t[p] = (int8_t)(v % 3 - 1);
            v /= 3;
        }
        uint8_t b = vxo_pack_5trits(t);
        memcpy(g_byte_trits[b], t, 5);
        g_byte_valid[b] = 1;
    }
    g_tables_ready = 1;
}

void vxo_byte_to_trits(uint8_t b, int8_t t[5]) {
    init_tables();
    memcpy(t, g_byte_trits[b], 5);
}

int vxo_byte_is_valid(uint8_t b) {
    init_tables();
    return g_byte_valid[b];
}

size_t vxo_planar_row_bytes(size_t cols) { return (cols + VXO_QK5 - 1) / VXO_QK5 * VXO_BLOCK_BYTES; }

/* pack.rs:66-131: byte j of block b packs the trits at block offsets j, 32+j, 64+j, 96+j, 128+j; the partial last
 * block is padded with zero trits. */
void vxo_pack_matrix(const int8_t* trits, size_t rows, size_t cols, uint8_t* out) {
    const size_t rb = vxo_planar_row_bytes(cols);
    for (size_t r = 0; r < rows; ++r) {
        const int8_t* src = trits + r * cols;
        uint8_t* dst = out + r * rb;
        for (size_t b = 0; b < rb / VXO_BLOCK_BYTES; ++b) {
            for (size_t j = 0; j < VXO_BLOCK_BYTES; ++j) {
                int8_t t[5];
                for (size_t p = 0; p < 5; ++p) {
                    const size_t col = b * VXO_QK5 + p * VXO_BLOCK_BYTES + j;
                    t[p] = col < cols ? src[col] : 0;
                }
                dst[b * VXO_BLOCK_BYTES + j] = vxo_pack_5trits(t);
            }
        }
    }
}

/* pack.rs:134-162 */
void vxo_unpack_matrix(const uint8_t* packed, size_t rows, size_t cols, int8_t* out) {
    const size_t rb = vxo_planar_row_bytes(cols);
    for (size_t r = 0; r < rows; ++r) {
        for (size_t b = 0; b < rb / VXO_BLOCK_BYTES; ++b) {
            for (size_t j = 0; j < VXO_BLOCK_BYTES; ++j) {
                int8_t t[5];
                vxo_byte_to_trits(packed[r * rb + b * VXO_BLOCK_BYTES + j], t);
                for (size_t p = 0; p < 5; ++p) {
                    const size_t col = b * VXO_QK5 + p * VXO_BLOCK_BYTES + j;
                    if (col < cols) out[r * cols + col] = t[p];
                }
            }
        }
    }
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* Tile geometry with the packed tail                                                                                */
/* ---------------------------------------------------------------------------------------------------------------- */

size_t vxo_tile_full_columns(size_t cols) { return cols / VXO_QK5 * VXO_BLOCK_BYTES; } /* pack.rs:207-210 */

size_t vxo_tile_row_bytes(size_t cols) { /* pack.rs:222-225 */
    const size_t tail = (cols % VXO_QK5 + 4) / 5;
    return vxo_tile_full_columns(cols) + tail + (tail & 1);
}

size_t vxo_column_activation_index(size_t cols, size_t c, size_t p) { /* pack.rs:230-237 */
    const size_t full = vxo_tile_full_columns(cols);
    if (c < full) return c / VXO_BLOCK_BYTES * VXO_QK5 + p * VXO_BLOCK_BYTES + c % VXO_BLOCK_BYTES;
    return cols / VXO_QK5 * VXO_QK5 + 5 * (c - full) + p;
}

uint8_t vxo_tile_byte(const uint8_t* planar_row, size_t cols, size_t c) { /* pack.rs:240-256 */
    const size_t full = vxo_tile_full_columns(cols);
    if (c < full) return planar_row[c];
    const size_t rem = cols % VXO_QK5;
    int8_t t[5] = {0, 0, 0, 0, 0};
    for (size_t k = 0; k < 5; ++k) {
        const size_t q = 5 * (c - full) + k;
        if (q < rem) {
            int8_t d[5];
            vxo_byte_to_trits(planar_row[full + q % VXO_BLOCK_BYTES], d);
            t[k] = d[q / VXO_BLOCK_BYTES];
        }
    }
    return vxo_pack_5trits(t);
}

void vxo_untile_row(const uint8_t* tile_row, size_t cols, uint8_t* planar_row) { /* pack.rs:279-294 */
    const size_t full = vxo_tile_full_columns(cols);
    memcpy(planar_row, tile_row, full);
    const size_t rem = cols % VXO_QK5;
    if (rem == 0) return;
    int8_t trits[VXO_QK5];
    memset(trits, 0, sizeof trits);
    for (size_t q = 0; q < rem; ++q) {
        int8_t d[5];
        vxo_byte_to_trits(tile_row[full + q / 5], d);
        trits[q] = d[q % 5];
    }
    for (size_t j = 0; j < VXO_BLOCK_BYTES; ++j) {
        const int8_t t[5] = {trits[j], trits[32 + j], trits[64 + j], trits[96 + j], trits[128 + j]};
        planar_row[full + j] = vxo_pack_5trits(t);
    }
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* Activation split, compact tables, decode                                                                          */
/* ---------------------------------------------------------------------------------------------------------------- */

/* lut.rs:380-388: lo = ((x + 8) & 15) - 8 in [-8, 7], hi = (x - lo) >> 4 in [-8, 8], x = 16 hi + lo. */
void vxo_split_hi_lo(const int8_t* acts, size_t n, int8_t* hi, int8_t* lo) {
    for (size_t i = 0; i < n; ++i) {
        const int x = acts[i];
        const int l = ((x + 8) & 15) - 8;
        lo[i] = (int8_t)l;
        hi[i] = (int8_t)((x - l) >> 4);
    }
}

size_t vxo_wide_lut_len(size_t cols) { return 2 * vxo_tile_row_bytes(cols) * 64; } /* avx512.rs:935-938 */

/* avx512.rs:1178-1247: per tile column c and part (lo, hi) one 64-byte table: lanes 0..8 hold t3 a3 + t4 a4 for
 * U = d3 + 3 d4, lanes 9..35 hold t0 a0 + t1 a1 + t2 a2 for L = d0 + 3 d1 + 9 d2 (offset 9, avx512.rs:932), the rest
 * is zero. The lo part of all columns comes first, then the hi part. */
void vxo_build_compact_wide_lut(const int8_t* acts, size_t cols, int8_t* lut) {
    const size_t bpr = vxo_tile_row_bytes(cols);
    int8_t* lo_tab = lut;
    int8_t* hi_tab = lut + bpr * 64;
    memset(lut, 0, 2 * bpr * 64);
    for (size_t c = 0; c < bpr; ++c) {
        int lo[5], hi[5];
        for (size_t p = 0; p < 5; ++p) {
            const size_t idx = vxo_column_activation_index(cols, c, p);
            const int x = idx < cols ? acts[idx] : 0;
            const int l = ((x + 8) & 15) - 8;
            lo[p] = l;
            hi[p] = (x - l) >> 4;
        }
        for (int s = 0; s < 9; ++s) {
            const int t3 = s % 3 - 1, t4 = s / 3 - 1;
            lo_tab[c * 64 + s] = (int8_t)(t3 * lo[3] + t4 * lo[4]);
            hi_tab[c * 64 + s] = (int8_t)(t3 * hi[3] + t4 * hi[4]);
        }
        for (int s = 0; s < 27; ++s) {
            const int t0 = s % 3 - 1, t1 = (s / 3) % 3 - 1, t2 = s / 9 - 1;
            lo_tab[c * 64 + 9 + s] = (int8_t)(t0 * lo[0] + t1 * lo[1] + t2 * lo[2]);
            hi_tab[c * 64 + 9 + s] = (int8_t)(t0 * hi[0] + t1 * hi[1] + t2 * hi[2]);
        }
    }
}

/* avx512.rs:1256-1292 (decode_compact with PERM = true): i = B >> 2 indexes two 64-entry tables, U = floor(i / 7)
 * and 28 floor(i / 7) - 9; the second one subtracted from B gives L + 9. Returned here without the offset. */
void vxo_decode_u_l(uint8_t b, uint8_t* u, uint8_t* l) {
    const unsigned i = (unsigned)(b >> 2) & 63u;
    const unsigned h34 = i / 7u;
    const uint8_t m28 = (uint8_t)(28u * h34 - 9u);
    *u = (uint8_t)h34;
    *l = (uint8_t)((uint8_t)(b - m28) - 9u);
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* GEMV                                                                                                              */
/* ---------------------------------------------------------------------------------------------------------------- */

/* avx512.rs:1526-1626 restated per row: every byte is decoded once, both parts of the column's table are looked up
 * at U and L + 9 and the exact sums are combined as lo + 16 hi. */
void vxo_gemv_lut_tilerows(const uint8_t* tile_rows, size_t rows, size_t cols, const int8_t* acts, int32_t* out) {
    const size_t bpr = vxo_tile_row_bytes(cols);
    int8_t* lut = (int8_t*)malloc(vxo_wide_lut_len(cols) + 1);
    vxo_build_compact_wide_lut(acts, cols, lut);
    const int8_t* lo_tab = lut;
    const int8_t* hi_tab = lut + bpr * 64;
    for (size_t r = 0; r < rows; ++r) {
        int64_t lo_sum = 0, hi_sum = 0;
        const uint8_t* row = tile_rows + r * bpr;
        for (size_t c = 0; c < bpr; ++c) {
            uint8_t u, l;
            vxo_decode_u_l(row[c], &u, &l);
            lo_sum += lo_tab[c * 64 + u] + lo_tab[c * 64 + 9 + l];
            hi_sum += hi_tab[c * 64 + u] + hi_tab[c * 64 + 9 + l];
        }
        out[r] = (int32_t)(lo_sum + 16 * hi_sum);
    }
    free(lut);
}

void vxo_tile_rows(const uint8_t* planar, size_t rows, size_t cols, uint8_t* out) {
    const size_t prb = vxo_planar_row_bytes(cols);
    const size_t bpr = vxo_tile_row_bytes(cols);
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < bpr; ++c) out[r * bpr + c] = vxo_tile_byte(planar + r * prb, cols, c);
}

void vxo_gemv_lut_planar(const uint8_t* planar, size_t rows, size_t cols, const int8_t* acts, int32_t* out) {
    const size_t prb = vxo_planar_row_bytes(cols);
    const size_t bpr = vxo_tile_row_bytes(cols);
    (void)prb;
    uint8_t* tiles = (uint8_t*)malloc(rows * bpr + 1);
    vxo_tile_rows(planar, rows, cols, tiles);
    vxo_gemv_lut_tilerows(tiles, rows, cols, acts, out);
    free(tiles);
}

void vxo_gemv_bruteforce(const int8_t* trits, size_t rows, size_t cols, const int8_t* acts, int64_t* out) {
    for (size_t r = 0; r < rows; ++r) {
        int64_t s = 0;
        for (size_t k = 0; k < cols; ++k) s += (int64_t)trits[r * cols + k] * (int64_t)acts[k];
        out[r] = s;
    }
}

/* layer.rs:246-253: one division per projection, then one multiplication per row. */
void vxo_epilogue_f32(const int32_t* acc, size_t rows, float weight_scale, float act_scale, float* out) {
    if (act_scale > 0.0f) {
        const float post = weight_scale / act_scale;
        for (size_t i = 0; i < rows; ++i) out[i] = (float)acc[i] * post;
    } else {
        for (size_t i = 0; i < rows; ++i) out[i] = 0.0f;
    }
}

void vxo_scale_f32(const int32_t* acc, size_t rows, float scale, float* out) {
    for (size_t i = 0; i < rows; ++i) out[i] = (float)acc[i] * scale;
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* Quantizers and norms                                                                                              */
/* ---------------------------------------------------------------------------------------------------------------- */

/* ops.rs:241-267: s = levels / max|x|; q = clamp(round_half_away(x s), -(levels + 1), levels). A zero or NaN maximum
 * gives zero codes and s = 0. The maximum skips NaN (a NaN never compares greater). */
float vxo_quantize_i8(const float* x, size_t n, float levels, int8_t* q) {
    float max_abs = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (a > max_abs) max_abs = a;
    }
    if (!(max_abs > 0.0f)) {
        memset(q, 0, n);
        return 0.0f;
    }
    const float s = levels / max_abs;
    const float lo = -(levels + 1.0f);
    for (size_t i = 0; i < n; ++i) {
        float v = roundf(x[i] * s);
        /* f32::clamp keeps NaN; "as i8" then maps NaN to 0. */
        if (v != v) {
            q[i] = 0;
            continue;
        }
        if (v < lo) v = lo;
        if (v > levels) v = levels;
        q[i] = (int8_t)(int)v;
    }
    return s;
}

/* IEEE 754 binary32 -> binary16, round to nearest even, written from the format definition (the conversion F16C
 * performs; the reference uses F16C when present, ops.rs:914-932). Checked against numpy in the tests. */
uint16_t vxo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf or nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    const int e = (int)(ax >> 23) - 127;
    if (e < -25) return (uint16_t)sign; /* below half of the smallest subnormal: +-0 */
    uint32_t mant = (ax & 0x7fffffu) | (e == -127 ? 0u : 0x800000u);
    int shift; /* number of low bits to drop from the 24-bit significand */
    uint32_t base;
    if (e < -14) { /* subnormal half: value = mant * 2^(e-23), unit 2^-24 */
        shift = -14 - e + 13;
        base = 0;
    } else {
        shift = 13;
        base = (uint32_t)(e + 15) << 10;
    }
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (q & 1u))) q += 1u;
    /* A carry out of the significand (q = 0x800, or 0x400 for a subnormal) moves into the exponent field by itself. */
    if (e < -14) return (uint16_t)(sign | q);
    return (uint16_t)(sign | (base + q - 0x400u));
}

/* binary16 -> binary32 (exact): a normal half moves its exponent to the f32 bias (e - 15 + 127) and its 10 significand
 * bits to the top of the 23; a subnormal half is m * 2^-24 (exact in f32); inf and NaN keep their payload. */
float vxo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    float v;
    if (e == 0) {
        v = (float)m * 0x1p-24f;
        memcpy(&bits, &v, 4);
    } else if (e == 31) {
        bits = 0x7f800000u | (m << 13);
    } else {
        bits = ((e + 112u) << 23) | (m << 13);
    }
    bits |= sign;
    memcpy(&v, &bits, 4);
    return v;
}

/* ops.rs:897-910: d = f16(amax / 127) (as f32), codes round_half_even(x * (127 / amax)) clamped to int8. */
void vxo_quantize_q8_0(const float* x, size_t n, int8_t* qs, float* d) {
    for (size_t b = 0; b < n / 32; ++b) {
        float amax = 0.0f;
        for (int k = 0; k < 32; ++k) {
            const float a = fabsf(x[b * 32 + k]);
            amax = a > amax ? a : amax; /* f32::max returns the non-NaN operand */
        }
        d[b] = vxo_f16_to_f32(vxo_f32_to_f16(amax / 127.0f));
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        for (int k = 0; k < 32; ++k) {
            const float v = nearbyintf(x[b * 32 + k] * id); /* default rounding mode: ties to even */
            int i;
            if (v != v) i = 0;
            else if (v > 2147483647.0f) i = 2147483647;
            else if (v < -2147483648.0f) i = -2147483647 - 1;
            else i = (int)v;
            if (i < -128) i = -128;
            if (i > 127) i = 127;
            qs[b * 32 + k] = (int8_t)i;
        }
    }
}

/* ops.rs:43-57 (and the AVX2 path ops.rs:60-95, same order): squares rounded to f32, summed sequentially in f64;
 * mean = f32(sum / n); inv = 1 / sqrt(mean + eps) in f32; y = (x * inv) * w. */
void vxo_rms_norm(const float* x, const float* w, size_t n, float eps, float* out) {
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const float sq = x[i] * x[i];
        sum += (double)sq;
    }
    const float mean = (float)(sum / (double)n);
    const float inv = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < n; ++i) {
        const float t = x[i] * inv;
        out[i] = t * w[i];
    }
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* Q2_0 x Q8_0                                                                                                        */
/* ---------------------------------------------------------------------------------------------------------------- */

/* block_scaled.rs:175-202 and the reduction order of block_scaled.rs:140-145. */
float vxo_q2_0_dot_row(const uint8_t* row, const float* w_scales, const int8_t* acts, const float* a_scales, size_t cols) {
    float acc[2][8];
    memset(acc, 0, sizeof acc);
    for (size_t s = 0; s < cols / 32; ++s) {
        const uint8_t* block = row + (s / 5) * VXO_BLOCK_BYTES;
        const size_t plane = s % 5;
        const int8_t* a = acts + s * 32;
        const float d = w_scales[s / 2] * a_scales[s];
        float* chain = acc[(s / 2) & 1];
        for (int j = 0; j < 8; ++j) {
            int32_t p = 0;
            for (int k = 4 * j; k < 4 * j + 4; ++k) {
                int8_t t[5];
                vxo_byte_to_trits(block[k], t);
                p += (int32_t)t[plane] * (int32_t)a[k];
            }
            chain[j] = fmaf(d, (float)p, chain[j]);
        }
    }
    float l[8];
    for (int j = 0; j < 8; ++j) l[j] = acc[0][j] + acc[1][j];
    const float r0 = l[4] + l[0], r1 = l[5] + l[1], r2 = l[6] + l[2], r3 = l[7] + l[3];
    return (r0 + r2) + (r1 + r3);
}

void vxo_q2_0_gemv(const uint8_t* packed, const float* w_scales, const int8_t* acts, const float* a_scales,
                   size_t rows, size_t cols, float* out) {
    const size_t rb = vxo_planar_row_bytes(cols);
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; ++r)
        out[r] = vxo_q2_0_dot_row(packed + r * rb, w_scales + r * (cols / 64), acts, a_scales, cols);
}

void vxo_q2_0_lane_sums(const uint8_t* packed, const int8_t* acts, size_t rows, size_t cols, int32_t* out) {
    const size_t rb = vxo_planar_row_bytes(cols);
    const size_t nb = cols / 32;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t s = 0; s < nb; ++s) {
            const uint8_t* block = packed + r * rb + (s / 5) * VXO_BLOCK_BYTES;
            for (int j = 0; j < 8; ++j) {
                int32_t p = 0;
                for (int k = 4 * j; k < 4 * j + 4; ++k) {
                    int8_t t[5];
                    vxo_byte_to_trits(block[k], t);
                    p += (int32_t)t[s % 5] * (int32_t)acts[s * 32 + k];
                }
                out[(r * nb + s) * 8 + j] = p;
            }
        }
    }
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* Generators                                                                                                        */
/* ---------------------------------------------------------------------------------------------------------------- */

/* splitmix64 (Steele, Lea, Flood 2014; public-domain constants). */
uint64_t vxo_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void vxo_gen_trits(uint64_t seed, size_t n, unsigned p_minus, unsigned p_zero, int8_t* out) {
    uint64_t st = seed;
    for (size_t i = 0; i < n; ++i) {
        const unsigned u = (unsigned)(vxo_splitmix64(&st) % 100u);
        out[i] = u < p_minus ? -1 : (u < p_minus + p_zero ? 0 : 1);
    }
}

void vxo_gen_i8(uint64_t seed, size_t n, int lo, int hi, int8_t* out) {
    uint64_t st = seed;
    const uint64_t span = (uint64_t)(hi - lo + 1);
    for (size_t i = 0; i < n; ++i) out[i] = (int8_t)(lo + (int)(vxo_splitmix64(&st) % span));
}
