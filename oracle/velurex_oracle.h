/*
 * velurex_oracle.h - CPU restatement of the reference's velurex ternary GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (quintrit_amd/, the HIP library, bench.py's GPU leg) links,
 * loads or calls this code. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker or as the timed CPU baseline.
 *
 * Every function names the reference file:line it restates (paths relative to the reference repository root,
 * rust/crates/...). Where a function is pinned by a check that does not retype its formula (brute force, closed
 * form, round trip, reference test vector), the test that pins it is named in tests/test_oracle.py (encoding, GEMV,
 * Q2_0) or tests/test_oracle_decode.py (quantizer known answers, RMSNorm).
 *
 * Conventions: trits are int8 values in {-1, 0, +1}; activations are int8 over the full range; sizes are size_t;
 * integer GEMV results are exact (int32 or int64).
 */
#ifndef VELUREX_ORACLE_H
#define VELUREX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VXO_QK5 160        /* trits per planar block (quintrit-core/src/pack.rs:19-20) */
#define VXO_BLOCK_BYTES 32 /* bytes per planar block (pack.rs:22-23) */

/* ---- encoding (quintrit-core/src/pack.rs) ------------------------------------------------------------------ */
uint8_t vxo_pack_5trits(const int8_t t[5]);                 /* pack.rs:28-36 */
void vxo_byte_to_trits(uint8_t b, int8_t t[5]);             /* pack.rs:41-58 (bytes that pack_5trits never
                                                               produces, e.g. 27 or 251..255, give zeros) */
int vxo_byte_is_valid(uint8_t b);                           /* 1 iff b is one of the 243 packed values */
size_t vxo_planar_row_bytes(size_t cols);                   /* cols.div_ceil(160) * 32 (pack.rs:105) */
void vxo_pack_matrix(const int8_t* trits, size_t rows, size_t cols, uint8_t* out);   /* pack.rs:66-131 */
void vxo_unpack_matrix(const uint8_t* packed, size_t rows, size_t cols, int8_t* out); /* pack.rs:134-162 */

/* ---- tile geometry with the packed tail (pack.rs:207-294) ----------------------------------------------------- */
size_t vxo_tile_full_columns(size_t cols);                            /* pack.rs:207-210 */
size_t vxo_tile_row_bytes(size_t cols);                               /* pack.rs:222-225 */
size_t vxo_column_activation_index(size_t cols, size_t c, size_t p);  /* pack.rs:230-237 */
uint8_t vxo_tile_byte(const uint8_t* planar_row, size_t cols, size_t c); /* pack.rs:240-256 */
void vxo_untile_row(const uint8_t* tile_row, size_t cols, uint8_t* planar_row); /* pack.rs:279-294 */

/* ---- activation split and tables (quintrit-core/src/lut.rs, simd/avx512.rs) ---------------------------------- */
void vxo_split_hi_lo(const int8_t* acts, size_t n, int8_t* hi, int8_t* lo);  /* lut.rs:380-388 */
size_t vxo_wide_lut_len(size_t cols);                                        /* avx512.rs:935-938 */
void vxo_build_compact_wide_lut(const int8_t* acts, size_t cols, int8_t* lut); /* avx512.rs:1178-1247 */
void vxo_decode_u_l(uint8_t b, uint8_t* u, uint8_t* l);                        /* avx512.rs:1256-1292 */

/* ---- GEMV ----------------------------------------------------------------------------------------------------- */
/* Restatement of the production table kernel (avx512.rs:1526-1626) on rows given as tile rows (tile_row_bytes
 * bytes each, the order pack.rs:263-276 gives a row inside a tile): out[r] = sum_c lo_c + 16 * hi_c. */
void vxo_gemv_lut_tilerows(const uint8_t* tile_rows, size_t rows, size_t cols, const int8_t* acts, int32_t* out);
/* Every row of a planar matrix re-encoded as a tile row (vxo_tile_byte for each c), rows x tile_row_bytes bytes. */
void vxo_tile_rows(const uint8_t* planar, size_t rows, size_t cols, uint8_t* out);
/* The same kernel fed from the planar layout of pack_matrix (each row re-tiled with vxo_tile_byte). */
void vxo_gemv_lut_planar(const uint8_t* planar, size_t rows, size_t cols, const int8_t* acts, int32_t* out);
/* Ground truth of every reference kernel test: sum_k trit * act in int64 (quintrit-core/tests/kernel_tests.rs:59-64,
 * quintrit-cuda/src/pack.rs:92-96). */
void vxo_gemv_bruteforce(const int8_t* trits, size_t rows, size_t cols, const int8_t* acts, int64_t* out);
/* The layers' fp32 epilogue: out = float(acc) * (ws / as), zeros when as <= 0 (quintrit-runtime/src/layer.rs:246-253). */
void vxo_epilogue_f32(const int32_t* acc, size_t rows, float weight_scale, float act_scale, float* out);
/* quintrit_gemv_f32's epilogue: out = float(acc) * scale (quintrit-c/src/tiles.rs:410-418). */
void vxo_scale_f32(const int32_t* acc, size_t rows, float scale, float* out);

/* ---- activation quantizers (quintrit-runtime/src/ops.rs) -------------------------------------------------------- */
float vxo_quantize_i8(const float* x, size_t n, float levels, int8_t* q);       /* ops.rs:241-267 */
void vxo_quantize_q8_0(const float* x, size_t n, int8_t* qs, float* d);         /* ops.rs:897-910 */
uint16_t vxo_f32_to_f16(float f);                                               /* ops.rs:935-957 (RNE) */
float vxo_f16_to_f32(uint16_t h);                                               /* ops.rs:489-530 */
void vxo_rms_norm(const float* x, const float* w, size_t n, float eps, float* out); /* ops.rs:43-57 */

/* ---- Q2_0 x Q8_0 block-scaled GEMV (quintrit-core/src/block_scaled.rs) ---------------------------------------- */
/* dot_row_scalar (block_scaled.rs:175-202). w_scales: cols/64 per row; a_scales: cols/32. Its floating-point order
 * (two chains by (s/2)&1, fma(ws*as, lane, acc), lanes of both chains added, then hsum8's pairing) is pinned by
 * hand-computed rows in which f32 absorption makes each step observable, with a negative control per step
 * (tests/test_oracle.py, test_q2_0_order_*). */
float vxo_q2_0_dot_row(const uint8_t* row, const float* w_scales, const int8_t* acts, const float* a_scales, size_t cols);
void vxo_q2_0_gemv(const uint8_t* packed, const float* w_scales, const int8_t* acts, const float* a_scales,
                   size_t rows, size_t cols, float* out);
/* The exact integer lane sums behind dot_row_scalar: out[(r * (cols/32) + s) * 8 + j] = sum over k in 4j..4j+3 of
 * trit * act of activation block s of row r (block_scaled.rs:187-196). */
void vxo_q2_0_lane_sums(const uint8_t* packed, const int8_t* acts, size_t rows, size_t cols, int32_t* out);

/* ---- seeded generators used by tests and the bench ------------------------------------------------------------- */
uint64_t vxo_splitmix64(uint64_t* state);
/* i.i.d. trits with P(-1) = p_minus/100, P(0) = p_zero/100, P(+1) = rest. */
void vxo_gen_trits(uint64_t seed, size_t n, unsigned p_minus, unsigned p_zero, int8_t* out);
/* int8 uniform in [lo, hi]. */
void vxo_gen_i8(uint64_t seed, size_t n, int lo, int hi, int8_t* out);

#ifdef __cplusplus
}
#endif
#endif
