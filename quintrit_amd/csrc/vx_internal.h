// Internal helpers of libvelurex_hip: the per-thread error slot, argument checks and the device layout arithmetic.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/velurex_hip.h"

namespace vx {

// ---- error slot (the reference keeps one per thread: quintrit-c/src/error.rs:64-80) ---------------------------------

struct Error {
    int code;
    std::string msg;
};

void set_error(int code, const std::string& msg);
void clear_error();

// Runs `body` (returning a status) with the error slot cleared first and C++ exceptions turned into VX_ERR_INTERNAL,
// so nothing unwinds across the C boundary (the reference's `guard`, quintrit-c/src/error.rs:64-80).
template <class F>
int guard(F&& body) {
    clear_error();
    try {
        return body();
    } catch (const std::bad_alloc&) {
        set_error(VX_ERR_DEVICE, "host out of memory");
        return VX_ERR_DEVICE;
    } catch (...) {
        set_error(VX_ERR_INTERNAL, "internal error");
        return VX_ERR_INTERNAL;
    }
}

#define VX_FAIL(code, ...)                                     \
    do {                                                       \
        char vx_buf_[512];                                     \
        std::snprintf(vx_buf_, sizeof vx_buf_, __VA_ARGS__);   \
        ::vx::set_error((code), vx_buf_);                      \
        return (code);                                         \
    } while (0)

#define VX_HIP(call)                                                                                     \
    do {                                                                                                 \
        hipError_t vx_e_ = (call);                                                                       \
        if (vx_e_ != hipSuccess) VX_FAIL(VX_ERR_DEVICE, "%s failed: %s", #call, hipGetErrorString(vx_e_)); \
    } while (0)

#define VX_TRY(expr)               \
    do {                           \
        int vx_s_ = (expr);        \
        if (vx_s_ != VX_OK) return vx_s_; \
    } while (0)

// ---- layout ---------------------------------------------------------------------------------------------------------

constexpr int kTileRows = 64;   // rows per tile = lanes of a wavefront
constexpr int kChunk = 16;      // bytes one lane loads per step (global_load_dwordx4)
constexpr size_t kQK5 = 160;    // trits per planar block (pack.rs:19)
constexpr size_t kBlockBytes = 32;

inline size_t planar_row_bytes(size_t cols) { return (cols + kQK5 - 1) / kQK5 * kBlockBytes; }
inline size_t tile_full_columns(size_t cols) { return cols / kQK5 * kBlockBytes; }
inline size_t tile_row_bytes(size_t cols) {  // pack.rs:222-225
    const size_t tail = (cols % kQK5 + 4) / 5;
    return tile_full_columns(cols) + tail + (tail & 1);
}
inline size_t device_row_bytes(size_t cols) { return (tile_row_bytes(cols) + kChunk - 1) / kChunk * kChunk; }
inline size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

struct Geometry {
    size_t rows, cols, padded_rows, n_tiles, tbr, dbr, n_chunks, device_bytes;
};

inline Geometry geometry(size_t rows, size_t cols) {
    Geometry g;
    g.rows = rows;
    g.cols = cols;
    g.padded_rows = round_up(rows, kTileRows);
    g.n_tiles = g.padded_rows / kTileRows;
    g.tbr = tile_row_bytes(cols);
    g.dbr = device_row_bytes(cols);
    g.n_chunks = g.dbr / kChunk;
    g.device_bytes = g.padded_rows * g.dbr;
    return g;
}

int check_shape(size_t rows, size_t cols);

// ---- device state -------------------------------------------------------------------------------------------------------

struct DeviceInfo {
    int device;
    int num_cus;
};
int device_info(DeviceInfo* out);  // current device; VX_ERR_UNSUPPORTED if it is not a gfx950

}  // namespace vx

// ---- the matrix handle --------------------------------------------------------------------------------------------------

struct vx_matrix {
    uint32_t magic;
    vx::Geometry g;
    float weight_scale;
    int device;
    int num_cus;
    uint8_t* d_w;       // weights, device layout (vx_layout)
    int32_t* d_acc;     // split-K accumulators, padded_rows, kept at zero between calls
    uint32_t* d_cnt;    // split-K arrival counters, n_tiles, kept at zero between calls
    uint2* d_actp;      // activation staging: one entry per device byte-column
    int8_t* d_io;       // host-API staging: cols bytes of activations + padded_rows * 4 bytes of output
    std::mutex mu;      // serialises the host-pointer API on this handle
};

constexpr uint32_t kMatrixMagic = 0x56584d31u;  // "VXM1"
