/*
 * gguf_oracle.c - CPU restatement of the reference's GGUF ternary decoders (TEST INFRASTRUCTURE ONLY).
 *
 * The trits of the GGUF tensor types the reference transcodes into velurex bytes (quintrit-format/src/decoders):
 * I2_S (BitNet planar, 2 bits per weight), TQ1_0 and TQ2_0 (llama.cpp ternary blocks of 256) and Q2_0 (llama.cpp
 * 2-bit codes with an f16 scale per block of 64 or 128). Each function names the reference file:line it follows. The
 * encoders are the inverses the reference's tests write from ggml's quantizers (tests/gguf_decoder_tests.rs:497-544,
 * decoders/i2_s.rs:18-42) and serve as checks. Only tests/ load this code; the product never calls it.
 */
#include "gguf_oracle.h"

#include <string.h>

/* I2_S code -> trit: 0 -> -1, 1 -> 0, 2 -> +1, 3 -> 0 (unpack.rs:59-62). */
static int8_t i2_trit(unsigned code) { return code == 3 ? 0 : (int8_t)((int)code - 1); }

/* decoders/i2_s.rs:45-66 with unpack.rs:64-75 (PlaneOrder::HighFirst): per row, cols / 128 blocks of 32 bytes; trit
 * j of a block is the code in byte j % 32 at bits 6 - 2 (j / 32). */
int vxo_i2s_unpack(const uint8_t* packed, size_t rows, size_t cols, int8_t* trits) {
    if (cols % 128) return -1;
    const size_t rb = cols / 4;
    for (size_t r = 0; r < rows; ++r)
        for (size_t b = 0; b < cols / 128; ++b)
            for (size_t j = 0; j < 128; ++j) {
                const uint8_t byte = packed[r * rb + b * 32 + j % 32];
                trits[r * cols + b * 128 + j] = i2_trit((byte >> (6 - 2 * (j / 32))) & 3u);
            }
    return 0;
}

/* decoders/i2_s.rs:18-42 (pack_gguf_i2_s): the inverse, codes 0, 1, 2 for -1, 0, +1. */
int vxo_i2s_pack(const int8_t* trits, size_t rows, size_t cols, uint8_t* packed) {
    if (cols % 128) return -1;
    const size_t rb = cols / 4;
    memset(packed, 0, rows * rb);
    for (size_t r = 0; r < rows; ++r)
        for (size_t b = 0; b < cols / 128; ++b)
            for (size_t j = 0; j < 128; ++j) {
                const int8_t w = trits[r * cols + b * 128 + j];
                const unsigned code = w == -1 ? 0u : (w == 1 ? 2u : 1u);
                packed[r * rb + b * 32 + j % 32] |= (uint8_t)(code << (6 - 2 * (j / 32)));
            }
    return 0;
}

/* decoders/tq2_0.rs:69-73 (ggml dequantize_row_tq2_0 order, PlaneOrder::LowFirst): a 66-byte block holds 256 trits in
 * two groups of 32 bytes; element 128 g + 32 l + m is the code at bits 2 l of byte 32 g + m (0 -> -1, 2 -> +1, 1 and
 * the unused 3 -> 0); bytes 64-65 are the f16 scale. */
void vxo_tq2_0_unpack(const uint8_t* data, size_t n_blocks, int8_t* trits) {
    for (size_t blk = 0; blk < n_blocks; ++blk) {
        const uint8_t* q = data + blk * 66;
        int8_t* out = trits + blk * 256;
        for (size_t g = 0; g < 2; ++g)
            for (size_t l = 0; l < 4; ++l)
                for (size_t m = 0; m < 32; ++m) out[128 * g + 32 * l + m] = i2_trit((q[32 * g + m] >> (2 * l)) & 3u);
    }
}

/* decoders/tq1_0.rs:63-92 (ggml dequantize_row_tq1_0): digit n of byte q is ((q * 3^n mod 256) * 3) >> 8, minus 1.
 * qs[0..32] hold elements 32 n + m (n < 5), qs[32..48] elements 160 + 16 n + m, qh[0..4] elements 240 + 4 n + j
 * (n < 4); bytes 52-53 are the f16 scale. */
static int8_t tq1_digit(uint8_t byte, unsigned n) {
    static const unsigned pow3[5] = {1, 3, 9, 27, 81};
    const unsigned q = (uint8_t)(byte * pow3[n]);
    return (int8_t)((int)((q * 3u) >> 8) - 1);
}

void vxo_tq1_0_unpack(const uint8_t* data, size_t n_blocks, int8_t* trits) {
    for (size_t blk = 0; blk < n_blocks; ++blk) {
        const uint8_t* b = data + blk * 54;
        int8_t* out = trits + blk * 256;
        for (unsigned n = 0; n < 5; ++n)
            for (size_t m = 0; m < 32; ++m) out[32 * n + m] = tq1_digit(b[m], n);
        for (unsigned n = 0; n < 5; ++n)
            for (size_t m = 0; m < 16; ++m) out[160 + 16 * n + m] = tq1_digit(b[32 + m], n);
        for (unsigned n = 0; n < 4; ++n)
            for (size_t j = 0; j < 4; ++j) out[240 + 4 * n + j] = tq1_digit(b[48 + j], n);
    }
}

/* tests/gguf_decoder_tests.rs:497-512 (ggml quantize_row_tq2_0_ref's packing): the inverse of vxo_tq2_0_unpack. */
void vxo_tq2_0_pack(const int8_t* trits, size_t n_blocks, uint16_t d_bits, uint8_t* data) {
    for (size_t blk = 0; blk < n_blocks; ++blk) {
        uint8_t* q = data + blk * 66;
        const int8_t* t = trits + blk * 256;
        for (size_t g = 0; g < 2; ++g)
            for (size_t m = 0; m < 32; ++m) {
                unsigned v = 0;
                for (unsigned l = 0; l < 4; ++l) v |= ((unsigned)(t[128 * g + m + 32 * l] + 1) & 3u) << (2 * l);
                q[32 * g + m] = (uint8_t)v;
            }
        q[64] = (uint8_t)d_bits;
        q[65] = (uint8_t)(d_bits >> 8);
    }
}

/* tests/gguf_decoder_tests.rs:514-544 (ggml quantize_row_tq1_0_ref's packing): base-3 digits most significant first,
 * stored as ceil(q * 256 / 243) so that the digit extraction above reads them back. */
void vxo_tq1_0_pack(const int8_t* trits, size_t n_blocks, uint16_t d_bits, uint8_t* data) {
    for (size_t blk = 0; blk < n_blocks; ++blk) {
        uint8_t* b = data + blk * 54;
        const int8_t* t = trits + blk * 256;
        for (size_t m = 0; m < 32; ++m) {
            unsigned q = 0;
            for (unsigned n = 0; n < 5; ++n) q = q * 3 + (unsigned)(t[m + 32 * n] + 1);
            b[m] = (uint8_t)((q * 256 + 242) / 243);
        }
        for (size_t m = 0; m < 16; ++m) {
            unsigned q = 0;
            for (unsigned n = 0; n < 5; ++n) q = q * 3 + (unsigned)(t[160 + m + 16 * n] + 1);
            b[32 + m] = (uint8_t)((q * 256 + 242) / 243);
        }
        for (size_t j = 0; j < 4; ++j) {
            unsigned q = 0;
            for (unsigned m = 0; m < 4; ++m) q = q * 3 + (unsigned)(t[240 + j + 4 * m] + 1);
            b[48 + j] = (uint8_t)((q * 3 * 256 + 242) / 243);
        }
        b[52] = (uint8_t)d_bits;
        b[53] = (uint8_t)(d_bits >> 8);
    }
}

/* decoders/q2_0.rs:34-55 (decode_block): a block of block_size weights is an f16 scale then block_size / 4 bytes; weight
 * 4 i + k is code (byte i >> 2 k) & 3 minus 1; code 3 (+2) is not ternary and fails the tensor (returns the index of
 * the first such weight + 1, else 0). scales_f16 receives the scale bits once per 64 weights. */
size_t vxo_q2_0_unpack(const uint8_t* data, size_t rows, size_t cols, size_t block_size, int8_t* trits,
                       uint16_t* scales_f16) {
    const size_t n = rows * cols, bb = 2 + block_size / 4;
    for (size_t blk = 0; blk < n / block_size; ++blk) {
        const uint8_t* b = data + blk * bb;
        const uint16_t d = (uint16_t)(b[0] | (b[1] << 8));
        for (size_t s = 0; s < block_size / 64; ++s) scales_f16[blk * (block_size / 64) + s] = d;
        for (size_t i = 0; i < block_size / 4; ++i)
            for (unsigned k = 0; k < 4; ++k) {
                const unsigned code = (b[2 + i] >> (2 * k)) & 3u;
                if (code == 3) return blk * block_size + 4 * i + k + 1;
                trits[blk * block_size + 4 * i + k] = (int8_t)((int)code - 1);
            }
    }
    return 0;
}
