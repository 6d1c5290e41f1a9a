/* cpu_avx512.h - the reference's production CPU GEMV in AVX-512 (CPU BASELINE ONLY; see cpu_avx512.c). */
#ifndef VXC_CPU_AVX512_H
#define VXC_CPU_AVX512_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 1 when the host has AVX-512 F, BW and VBMI (the kernel's instructions). */
int vxc_supported(void);
/* Bytes of the compact wide tables of one activation vector: 2 * tile_row_bytes(cols) * 64. */
size_t vxc_table_bytes(size_t cols);
/* Planar rows -> the 64-row tiled layout (rows a multiple of 64). */
void vxc_tile64(const uint8_t* planar, size_t rows, size_t cols, uint8_t* out);
void vxc_build_tables(const int8_t* acts, size_t cols, int8_t* tables);
/* out[r] = float(sum_k t[r][k] * acts[k]) for rows a multiple of 64, from prebuilt tables. */
void vxc_gemv_tables(const uint8_t* tiles64, const int8_t* tables, size_t rows, size_t cols, float* out, int threads);
/* Tables then kernel (one call of the reference's GEMV); table_scratch holds vxc_table_bytes(cols). */
void vxc_gemv(const uint8_t* tiles64, const int8_t* acts, size_t rows, size_t cols, float* out, int threads,
              int8_t* table_scratch);
/* A projection group of the inference engine: n matrices with the same input (q/k/v, gate/up, or one alone), the
 * tables built once, then every 64-row block of the group shared out over `threads` threads. */
void vxc_gemv_group(const uint8_t* const* tiles64, const size_t* rows, int n, const int8_t* acts, size_t cols,
                    float* const* outs, int threads, int8_t* table_scratch);
/* out[0..n) = pseudo-random valid packed bytes from `seed` (random weights for the timing). */
void vxc_fill_valid(uint8_t* out, size_t n, uint64_t seed);
/* Pins OpenMP thread t of a team of n to logical CPU cpus[t]; returns the threads that could not be pinned. */
int vxc_pin_threads(const int* cpus, int n);
uint64_t vxc_read_stream(const uint64_t* buf, size_t words, int threads);
/* The calling thread's core clock in Hz, from a timed chain of dependent adds (one per cycle). */
double vxc_clock_hz(void);

#ifdef __cplusplus
}
#endif
#endif
