/* gguf_oracle.h - CPU restatement of the reference's GGUF ternary decoders (test infrastructure only; see
 * gguf_oracle.c). Pinned by tests/test_oracle_gguf.py: encode -> decode round trips for every trit pattern and the
 * extremes (the reference's tq_decoders_roundtrip_encoder_output_for_every_trit_pattern), the ggml dequantizer layouts
 * the reference's tests restate (gguf_decoder_tests.rs:431-495), every TQ1_0 byte against base-3 arithmetic, and I2_S
 * against the bit planes written out by hand for single trits. */
#ifndef GGUF_ORACLE_H
#define GGUF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int vxo_i2s_unpack(const uint8_t* packed, size_t rows, size_t cols, int8_t* trits);   /* decoders/i2_s.rs:45-66 */
int vxo_i2s_pack(const int8_t* trits, size_t rows, size_t cols, uint8_t* packed);     /* decoders/i2_s.rs:18-42 */
void vxo_tq2_0_unpack(const uint8_t* data, size_t n_blocks, int8_t* trits);            /* decoders/tq2_0.rs:69-73 */
void vxo_tq1_0_unpack(const uint8_t* data, size_t n_blocks, int8_t* trits);            /* decoders/tq1_0.rs:63-92 */
void vxo_tq2_0_pack(const int8_t* trits, size_t n_blocks, uint16_t d_bits, uint8_t* data);
void vxo_tq1_0_pack(const int8_t* trits, size_t n_blocks, uint16_t d_bits, uint8_t* data);
size_t vxo_q2_0_unpack(const uint8_t* data, size_t rows, size_t cols, size_t block_size, int8_t* trits,
                       uint16_t* scales_f16);                                          /* decoders/q2_0.rs:34-55 */

#ifdef __cplusplus
}
#endif
#endif
