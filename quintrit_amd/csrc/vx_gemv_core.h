// The velurex digit arithmetic shared by the GEMV kernels (the lone/batched GEMV of vx_gemv.hip and the decode-step
// GEMV of vx_decode.hip): the digit nibbles of a byte and the broadcast 4-bit dot products.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vx {

// ---- digits of a velurex byte ---------------------------------------------------------------------------------------

// U = floor(B / 28) is the 2-trit group (d3, d4), L = B - 28 U the 3-trit group (d0, d1, d2); B is a velurex value iff
// B <= 250 and L <= 26 (docs/velurex-encoding.md sections 2-3).
__host__ __device__ constexpr bool byte_valid(uint32_t b) {
    const uint32_t u = b / 28u, l = b - 28u * u;
    return b <= 250u && l <= 26u;
}

__host__ __device__ constexpr uint32_t digit_nibbles(uint32_t b) {
    if (!byte_valid(b)) return 0x11111u;  // five zero trits
    const uint32_t u = b / 28u, l = b - 28u * u;
    return (l % 3u) | ((l / 3u % 3u) << 4) | ((l / 9u) << 8) | ((u % 3u) << 12) | ((u / 3u) << 16);
}

// digit_nibbles of every byte, built at compile time (a kernel copies it into its LDS table with loads instead of
// computing 256 entries in every thread).
struct DigitTable {
    uint32_t v[256];
};
constexpr DigitTable make_digit_table() {
    DigitTable t{};
    for (uint32_t b = 0; b < 256; ++b) t.v[b] = digit_nibbles(b);
    return t;
}

// t0..t3 of byte b as int8 in a dword (byte p = trit p); bytes that are not velurex values give zero trits.
__host__ __device__ constexpr uint32_t trits03_word(uint32_t b) {
    if (!byte_valid(b)) return 0u;
    const uint32_t e = digit_nibbles(b);
    uint32_t w = 0;
    for (uint32_t p = 0; p < 4; ++p) w |= ((((e >> (4 * p)) & 15u) - 1u) & 0xffu) << (8 * p);
    return w;
}
struct TritTable {
    uint32_t v[256];
};
constexpr TritTable make_trit_table() {
    TritTable t{};
    for (uint32_t b = 0; b < 256; ++b) t.v[b] = trits03_word(b);
    return t;
}

// t4 of each byte of w as int8: d4 = floor(B / 84) from B >= 84 and B >= 168, tested with 7-bit adds that cannot carry
// (the halved byte B >> 1 is below 128), then t4 = d4 - 1 per byte as (d4 + 0x7f) ^ 0x80, again without carries.
// Every byte must be a velurex value.
__host__ __device__ constexpr uint32_t t4_bytes(uint32_t w) {
    const uint32_t x = (w >> 1) & 0x7f7f7f7fu;
    const uint32_t d4 = (((x + 0x56565656u) >> 7) & 0x01010101u) + (((x + 0x2c2c2c2cu) >> 7) & 0x01010101u);
    return (d4 + 0x7f7f7f7fu) ^ 0x80808080u;
}

__host__ __device__ inline int trit_of(uint32_t b, uint32_t p) {
    return static_cast<int>((digit_nibbles(b) >> (4 * p)) & 15u) - 1;
}

// Four bytes of a lane's weights against their activations: lo += dot8(L of byte K + j, t_j), hi += dot8(H, t_j) for
// j = 0..3, where t_j is the digit-nibble table entry of byte j and the activation dwords of the 16 byte-columns of a
// chunk sit in lanes 0..15 of every 16-lane row of L and H, broadcast by DPP row_newbcast. v_dot8c_i32_i4 multiplies
// signed nibbles: the digits (0..2), the high nibbles x >> 4 and the low nibbles (x & 15) - 8. L and H come from LDS
// loads; the s_nop keeps the two wait states a DPP read needs after any VALU write of its source.
template <int K>
__device__ __forceinline__ void dot4_bcast(int& lo, int& hi, uint32_t L, uint32_t H, uint32_t t0, uint32_t t1, uint32_t t2,
                                           uint32_t t3) {
    asm("s_nop 1\n\t"
        "v_dot8c_i32_i4_dpp %0, %2, %4 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot8c_i32_i4_dpp %1, %3, %4 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot8c_i32_i4_dpp %0, %2, %5 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot8c_i32_i4_dpp %1, %3, %5 row_newbcast:%9 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot8c_i32_i4_dpp %0, %2, %6 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot8c_i32_i4_dpp %1, %3, %6 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot8c_i32_i4_dpp %0, %2, %7 row_newbcast:%11 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot8c_i32_i4_dpp %1, %3, %7 row_newbcast:%11 row_mask:0xf bank_mask:0xf"
        : "+v"(lo), "+v"(hi)
        : "v"(L), "v"(H), "v"(t0), "v"(t1), "v"(t2), "v"(t3), "n"(K), "n"(K + 1), "n"(K + 2), "n"(K + 3));
}

}  // namespace vx
