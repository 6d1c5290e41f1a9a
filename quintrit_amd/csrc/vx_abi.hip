// C ABI of libvelurex_hip (include/velurex_hip.h): argument checks, the per-thread error slot and the matrix handles.
// Error conventions follow the reference's C ABI (quintrit-c/src/error.rs:8-80, quintrit-c/src/tiles.rs:192-228).
#include "vx_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

namespace vx {

static thread_local Error t_error{VX_OK, std::string()};

void set_error(int code, const std::string& msg) {
    t_error.code = code;
    t_error.msg = msg;
}

void clear_error() {
    t_error.code = VX_OK;
    t_error.msg.clear();
}

int check_shape(size_t rows, size_t cols) {
    if (rows == 0 || rows > VX_MAX_ROWS) VX_FAIL(VX_ERR_INVALID_SHAPE, "rows must be in 1..=%zu (got %zu)", (size_t)VX_MAX_ROWS, rows);
    if (cols == 0) VX_FAIL(VX_ERR_INVALID_SHAPE, "cols must be at least 1");
    if (cols > VX_MAX_GEMV_COLS)
        VX_FAIL(VX_ERR_INVALID_SHAPE, "cols = %zu exceeds %d, the largest count for which the accumulators are exact", cols,
                VX_MAX_GEMV_COLS);
    return VX_OK;
}

int device_info(DeviceInfo* out) {
    int dev = 0;
    VX_HIP(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    VX_HIP(hipGetDeviceProperties(&prop, dev));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        VX_FAIL(VX_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950 (MI355X) only", dev, prop.gcnArchName);
    out->device = dev;
    out->num_cus = prop.multiProcessorCount;
    return VX_OK;
}

static int check_matrix(const vx_matrix_t* m) {
    if (m == nullptr) VX_FAIL(VX_ERR_INVALID_HANDLE, "matrix handle is NULL");
    if (m->magic != kMatrixMagic) VX_FAIL(VX_ERR_INVALID_HANDLE, "matrix handle is not valid (freed or foreign)");
    return VX_OK;
}

// Entry points of the GEMV/GEMM layout reject Q2_0 matrices and the other way round.
static int check_kind(const vx_matrix_t* m, uint32_t kind) {
    VX_TRY(check_matrix(m));
    if (m->kind != kind)
        VX_FAIL(VX_ERR_INVALID_HANDLE, "the matrix was created for %s", m->kind == kKindQ2 ? "the Q2_0 (block-scaled) GEMV" : "the velurex GEMV");
    return VX_OK;
}

static int set_device_of(const vx_matrix_t* m) {
    int cur = -1;
    VX_HIP(hipGetDevice(&cur));
    if (cur != m->device) VX_HIP(hipSetDevice(m->device));
    return VX_OK;
}

static void destroy(vx_matrix* m) {
    if (m->d_w) (void)hipFree(m->d_w);
    if (m->d_part) (void)hipFree(m->d_part);
    if (m->d_accum) (void)hipFree(m->d_accum);
    if (m->d_dsum) (void)hipFree(m->d_dsum);
    if (m->d_staged) (void)hipFree(m->d_staged);
    if (m->d_io) (void)hipFree(m->d_io);
    if (m->io_stream) (void)hipStreamDestroy(m->io_stream);
    if (m->h_io) (void)hipHostFree(m->h_io);
    m->magic = 0;
    delete m;
}

static int check_planar(const uint8_t* planar, size_t planar_len, size_t rows, size_t cols) {
    VX_TRY(check_shape(rows, cols));
    if (planar == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "planar is NULL");
    const size_t need = rows * planar_row_bytes(cols);
    if (planar_len < need)
        VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "planar holds %zu bytes but a %zu x %zu matrix needs %zu", planar_len, rows, cols, need);
    return VX_OK;
}

// Allocates a handle and its device buffers (weights left uninitialised).
static int alloc_matrix(size_t rows, size_t cols, float weight_scale, vx_matrix** out) {
    DeviceInfo di;
    VX_TRY(device_info(&di));
    // the no-allocation GEMM's scratch address, looked up outside any graph capture (a failure is reported by that
    // entry point's own calls, not here)
    if (gemm_scratch_prepare(di.device) != VX_OK) clear_error();
    vx_matrix* m = new vx_matrix();
    m->magic = kMatrixMagic;
    m->kind = kKindVelurex;
    m->g = geometry(rows, cols);
    m->weight_scale = weight_scale;
    m->device = di.device;
    m->num_cus = di.num_cus;
    m->d_w = nullptr;
    m->d_part = nullptr;
    m->d_accum = nullptr;
    m->d_tickets = nullptr;
    m->d_done = nullptr;
    m->d_dsum = nullptr;
    m->d_staged = nullptr;
    m->d_io = nullptr;
    m->owner = nullptr;
    Job probe{};
    plan_job(probe, m->g, static_cast<uint32_t>(di.num_cus));
    m->kslices = probe.kslices;
    m->slice_chunks = probe.slice_chunks;

    const size_t io_bytes = round_up(cols, 256) + m->g.padded_rows * 4;
    hipError_t e = hipMalloc(&m->d_w, m->g.device_bytes);
    if (e == hipSuccess && m->kslices > 1) e = hipMalloc(&m->d_part, static_cast<size_t>(m->kslices) * m->g.padded_rows * 4);
    // the atomic slice sums and tickets of the lone calls (the table GEMV splits K more finely than the digit GEMV,
    // so every matrix has them)
    const size_t accum_bytes = (m->g.padded_rows + m->g.n_groups + 1) * 4;
    if (e == hipSuccess) e = hipMalloc(&m->d_accum, accum_bytes);
    if (e == hipSuccess) e = hipMemset(m->d_accum, 0, accum_bytes);
    if (e == hipSuccess) m->d_tickets = reinterpret_cast<uint32_t*>(m->d_accum + m->g.padded_rows);
    if (e == hipSuccess) m->d_done = m->d_tickets + m->g.n_groups;
    if (e == hipSuccess) e = hipMalloc(&m->d_dsum, m->g.padded_rows * 4);
    if (e == hipSuccess) e = hipMalloc(&m->d_staged, staged_bytes(cols));
    if (e == hipSuccess) e = hipMalloc(&m->d_io, io_bytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        const size_t bytes = m->g.device_bytes;
        destroy(m);
        VX_FAIL(VX_ERR_DEVICE, "device allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
    }
    *out = m;
    return VX_OK;
}

static int create_matrix(const uint8_t* planar, size_t planar_len, size_t rows, size_t cols, float weight_scale,
                         vx_matrix_t** out) {
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_matrix is NULL");
    *out = nullptr;
    VX_TRY(check_planar(planar, planar_len, rows, cols));
    const size_t need = rows * planar_row_bytes(cols);
    const size_t bad = find_invalid_byte(planar, need);
    if (bad != SIZE_MAX)
        VX_FAIL(VX_ERR_INVALID_VALUE, "byte %zu (value %u) is not a velurex byte", bad, static_cast<unsigned>(planar[bad]));
    vx_matrix* m = nullptr;
    VX_TRY(alloc_matrix(rows, cols, weight_scale, &m));
    std::vector<uint8_t> host(m->g.device_bytes);
    planar_to_device_layout(planar, m->g, host.data());
    hipError_t e = hipMemcpy(m->d_w, host.data(), m->g.device_bytes, hipMemcpyHostToDevice);
    int st = e == hipSuccess ? launch_digit_sums(m->d_w, m->g, m->d_dsum, nullptr) : VX_OK;
    if (e == hipSuccess && st == VX_OK) e = hipDeviceSynchronize();
    if (e != hipSuccess || st != VX_OK) {
        destroy(m);
        if (st != VX_OK) return st;
        VX_FAIL(VX_ERR_DEVICE, "upload failed: %s", hipGetErrorString(e));
    }
    *out = m;
    return VX_OK;
}

static int create_matrix_dev(const uint8_t* planar_dev, size_t planar_len, size_t rows, size_t cols, float weight_scale,
                             vx_matrix_t** out) {
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_matrix is NULL");
    *out = nullptr;
    VX_TRY(check_planar(planar_dev, planar_len, rows, cols));
    const size_t need = rows * planar_row_bytes(cols);
    vx_matrix* m = nullptr;
    VX_TRY(alloc_matrix(rows, cols, weight_scale, &m));
    unsigned long long* d_first = nullptr;
    unsigned long long first = ~0ull;
    hipError_t e = hipMalloc(&d_first, sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemcpy(d_first, &first, sizeof first, hipMemcpyHostToDevice);
    int st = VX_OK;
    if (e == hipSuccess) st = launch_find_invalid(planar_dev, need, d_first, nullptr);
    if (e == hipSuccess && st == VX_OK) st = launch_device_layout(planar_dev, m->g, m->d_w, nullptr);
    if (e == hipSuccess && st == VX_OK) st = launch_digit_sums(m->d_w, m->g, m->d_dsum, nullptr);
    if (e == hipSuccess && st == VX_OK) e = hipMemcpy(&first, d_first, sizeof first, hipMemcpyDeviceToHost);
    if (d_first) (void)hipFree(d_first);
    if (st != VX_OK || e != hipSuccess) {
        destroy(m);
        if (st != VX_OK) return st;
        VX_FAIL(VX_ERR_DEVICE, "device layout transform failed: %s", hipGetErrorString(e));
    }
    if (first != ~0ull) {
        destroy(m);
        VX_FAIL(VX_ERR_INVALID_VALUE, "byte %llu is not a velurex byte", first);
    }
    *out = m;
    return VX_OK;
}

static int check_io(const vx_matrix_t* m, const void* acts, size_t acts_len, const void* out, size_t out_capacity) {
    if (acts == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "activations is NULL");
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out is NULL");
    if (acts_len < m->g.cols)
        VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "activations hold %zu values but cols = %zu", acts_len, m->g.cols);
    if (out_capacity < m->g.rows)
        VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "output holds %zu values but rows = %zu", out_capacity, m->g.rows);
    return VX_OK;
}

// A lone GEMV of matrix m on staged activations, or (raw) on int8 activations that every workgroup stages for its own
// K slice: one launch (a split matrix's K slices add their sums atomically and the last of each tile group writes the
// outputs). Calls on one matrix share its sums and tickets, so they must not overlap. With `flag`, the launch's last
// workgroup stores `seq` there once every output is written. K slices hold min_slice_chunks chunks at least (1 where the
// activations are read from host memory).
static int run_single(const vx_matrix* m, const uint8_t* staged, void* out, uint32_t out_kind, float post,
                      hipStream_t s, uint32_t* flag = nullptr, uint32_t seq = 0, const int8_t* raw = nullptr,
                      uint32_t min_slice_chunks = kLoneMinSliceChunks) {
    LaunchArgs a{};
    a.done = flag != nullptr ? m->d_done : nullptr;
    a.flag = flag;
    a.seq = seq;
    a.acts = raw;
    a.cols = static_cast<uint32_t>(m->g.cols);
    a.jobs = nullptr;
    a.n_jobs = 1;
    Job& j = a.one;
    plan_job(j, m->g, static_cast<uint32_t>(m->num_cus), min_slice_chunks);
    j.w = m->d_w;
    j.staged = staged;
    j.part = m->d_part;
    j.accum = m->d_accum;
    j.tickets = m->d_tickets;
    j.dsum = m->d_dsum;
    j.out = out;
    j.act_scale = nullptr;
    j.post = post;
    j.weight_scale = m->weight_scale;
    j.out_kind = out_kind;
    j.item_begin = 0;
    j.tbr = static_cast<uint32_t>(m->g.tbr);
    a.total_items = job_items(j);
    return launch_gemv(a, j.rows, nullptr, j.kslices > 1 && j.accum == nullptr ? 1u : 0u, m->num_cus, s);
}

// A lone GEMV of matrix m through the compact activation tables `lut` (its K slices add up in m's atomic sums, as
// run_single's do).
static int run_single_lut(const vx_matrix* m, const int8_t* lut, void* out, uint32_t out_kind, float post, hipStream_t s) {
    LaunchArgs a{};
    a.jobs = nullptr;
    a.n_jobs = 1;
    Job& j = a.one;
    plan_lut_job(j, m->g, static_cast<uint32_t>(m->num_cus));
    j.w = m->d_w;
    j.staged = reinterpret_cast<const uint8_t*>(lut);
    j.accum = m->d_accum;
    j.tickets = m->d_tickets;
    j.out = out;
    j.post = post;
    j.weight_scale = m->weight_scale;
    j.out_kind = out_kind;
    a.total_items = job_items(j);
    return launch_gemv_lut(a, j.rows, nullptr, 0, m->num_cus, s);
}

// out = float(acc) * (ws / as) with the division done once here, as the layers do; zeros when as <= 0 or NaN
// (layer.rs:246-253).
static int gemv_f32_staged(const vx_matrix* m, const uint8_t* staged, float act_scale, float* out, hipStream_t s) {
    if (act_scale > 0.0f) return run_single(m, staged, out, kOutF32Post, m->weight_scale / act_scale, s);
    return launch_fill_f32(out, m->g.rows, 0.0f, s);
}

// The raw-activation calls: one launch, each workgroup staging its own K slice.
static int gemv_f32_dev(vx_matrix* m, const int8_t* acts, float act_scale, float* out, hipStream_t s) {
    if (!(act_scale > 0.0f)) return launch_fill_f32(out, m->g.rows, 0.0f, s);
    return run_single(m, nullptr, out, kOutF32Post, m->weight_scale / act_scale, s, nullptr, 0, acts);
}

static int gemv_i32_dev(vx_matrix* m, const int8_t* acts, int32_t* out, hipStream_t s) {
    return run_single(m, nullptr, out, kOutI32, 1.0f, s, nullptr, 0, acts);
}

}  // namespace vx

using namespace vx;

extern "C" {

const char* vx_status_string(int status) {
    switch (status) {
        case VX_OK: return "ok";
        case VX_ERR_NULL_POINTER: return "null pointer";
        case VX_ERR_INVALID_ARGUMENT: return "invalid argument";
        case VX_ERR_INVALID_SHAPE: return "invalid shape";
        case VX_ERR_BUFFER_TOO_SMALL: return "buffer too small";
        case VX_ERR_INVALID_VALUE: return "invalid value";
        case VX_ERR_UNSUPPORTED: return "unsupported";
        case VX_ERR_IO: return "i/o error";
        case VX_ERR_FORMAT: return "format error";
        case VX_ERR_NOT_FOUND: return "not found";
        case VX_ERR_MODEL: return "model error";
        case VX_ERR_CONTEXT_OVERFLOW: return "context overflow";
        case VX_ERR_BUSY: return "busy";
        case VX_ERR_INTERNAL: return "internal error";
        case VX_ERR_INVALID_HANDLE: return "invalid handle";
        case VX_ERR_DEVICE: return "device error";
        default: return "unknown status";
    }
}

int vx_last_error_code(void) { return t_error.code; }
const char* vx_last_error_message(void) { return t_error.msg.c_str(); }
const char* vx_version(void) { return VX_VERSION_STRING; }
uint32_t vx_abi_version(void) { return VX_ABI_VERSION; }

int vx_device_count(int32_t* out_count) {
    return guard([&]() -> int {
        if (out_count == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_count is NULL");
        *out_count = 0;
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void)hipGetLastError();
            return VX_OK;
        }
        int32_t c = 0;
        for (int d = 0; d < n; ++d) {
            hipDeviceProp_t prop;
            if (hipGetDeviceProperties(&prop, d) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ++c;
        }
        *out_count = c;
        return VX_OK;
    });
}

int vx_layout(size_t rows, size_t cols, vx_layout_t* out_layout) {
    return guard([&]() -> int {
        if (out_layout == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_layout is NULL");
        if (out_layout->struct_size != sizeof(vx_layout_t))
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "struct_size is %u, expected %zu", out_layout->struct_size, sizeof(vx_layout_t));
        VX_TRY(check_shape(rows, cols));
        const Geometry g = geometry(rows, cols);
        out_layout->tile_rows = kTileRows;
        out_layout->tile_group = kTileGroup;
        out_layout->rows = rows;
        out_layout->cols = cols;
        out_layout->padded_rows = g.padded_rows;
        out_layout->planar_row_bytes = planar_row_bytes(cols);
        out_layout->tile_row_bytes = g.tbr;
        out_layout->device_row_bytes = g.dbr;
        out_layout->device_bytes = g.device_bytes;
        return VX_OK;
    });
}

int vx_matrix_create(const uint8_t* planar, size_t planar_len, size_t rows, size_t cols, float weight_scale,
                     vx_matrix_t** out_matrix) {
    return guard([&]() -> int { return create_matrix(planar, planar_len, rows, cols, weight_scale, out_matrix); });
}

int vx_matrix_create_dev(const uint8_t* planar_dev, size_t planar_len, size_t rows, size_t cols, float weight_scale,
                         vx_matrix_t** out_matrix) {
    return guard([&]() -> int { return create_matrix_dev(planar_dev, planar_len, rows, cols, weight_scale, out_matrix); });
}

int vx_device_layout_pack(const uint8_t* planar, size_t planar_len, size_t rows, size_t cols, uint8_t* out,
                          size_t out_capacity) {
    return guard([&]() -> int {
        VX_TRY(check_planar(planar, planar_len, rows, cols));
        if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out is NULL");
        const Geometry g = geometry(rows, cols);
        if (out_capacity < g.device_bytes)
            VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "out holds %zu bytes but the device layout needs %zu", out_capacity, g.device_bytes);
        const size_t bad = find_invalid_byte(planar, rows * planar_row_bytes(cols));
        if (bad != SIZE_MAX)
            VX_FAIL(VX_ERR_INVALID_VALUE, "byte %zu (value %u) is not a velurex byte", bad, static_cast<unsigned>(planar[bad]));
        planar_to_device_layout(planar, g, out);
        return VX_OK;
    });
}

int vx_staged_bytes(size_t cols, size_t* out_bytes) {
    return guard([&]() -> int {
        if (out_bytes == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_bytes is NULL");
        VX_TRY(check_shape(1, cols));
        *out_bytes = staged_bytes(cols);
        return VX_OK;
    });
}

int vx_stage_acts_dev(const int8_t* acts, size_t acts_len, size_t cols, void* staged, size_t staged_capacity,
                      void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_shape(1, cols));
        if (acts == nullptr || staged == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "activations or staged is NULL");
        if (acts_len < cols) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "activations hold %zu values but cols = %zu", acts_len, cols);
        const size_t need = staged_bytes(cols);
        if (staged_capacity < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "staged holds %zu bytes, %zu needed", staged_capacity, need);
        return launch_stage(acts, cols, static_cast<uint8_t*>(staged), static_cast<hipStream_t>(stream));
    });
}

static int check_staged(const vx_matrix_t* m, const void* staged, size_t staged_len, const void* out, size_t out_capacity) {
    if (staged == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "staged is NULL");
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out is NULL");
    const size_t need = staged_bytes(m->g.cols);
    if (staged_len < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "staged holds %zu bytes, %zu needed", staged_len, need);
    if (out_capacity < m->g.rows)
        VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "output holds %zu values but rows = %zu", out_capacity, m->g.rows);
    return VX_OK;
}

int vx_gemv_staged_i32_dev(const vx_matrix_t* matrix, const void* staged, size_t staged_len, int32_t* out,
                           size_t out_capacity, void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindVelurex));
        VX_TRY(check_staged(matrix, staged, staged_len, out, out_capacity));
        VX_TRY(set_device_of(matrix));
        return run_single(matrix, static_cast<const uint8_t*>(staged), out, kOutI32, 1.0f, static_cast<hipStream_t>(stream));
    });
}

int vx_gemv_staged_f32_dev(const vx_matrix_t* matrix, const void* staged, size_t staged_len, float act_scale, float* out,
                           size_t out_capacity, void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindVelurex));
        VX_TRY(check_staged(matrix, staged, staged_len, out, out_capacity));
        VX_TRY(set_device_of(matrix));
        return gemv_f32_staged(matrix, static_cast<const uint8_t*>(staged), act_scale, out, static_cast<hipStream_t>(stream));
    });
}

int vx_compact_lut_bytes(size_t cols, size_t* out_bytes) {
    return guard([&]() -> int {
        if (out_bytes == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_bytes is NULL");
        VX_TRY(check_shape(1, cols));
        *out_bytes = compact_lut_bytes(cols);
        return VX_OK;
    });
}

int vx_compact_lut_dev(const int8_t* acts, size_t acts_len, size_t cols, int8_t* lut, size_t lut_capacity, void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_shape(1, cols));
        if (acts == nullptr || lut == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "activations or lut is NULL");
        if (acts_len < cols) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "activations hold %zu values but cols = %zu", acts_len, cols);
        const size_t need = compact_lut_bytes(cols);
        if (lut_capacity < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "lut holds %zu bytes, %zu needed", lut_capacity, need);
        if ((reinterpret_cast<uintptr_t>(lut) & 15u) != 0) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "lut must be 16-byte aligned");
        return launch_compact_lut(acts, cols, lut, static_cast<hipStream_t>(stream));
    });
}

static int check_lut(const vx_matrix_t* m, const int8_t* lut, size_t lut_len, const void* out, size_t out_capacity) {
    if (lut == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "lut is NULL");
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out is NULL");
    const size_t need = compact_lut_bytes(m->g.cols);
    if (lut_len < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "lut holds %zu bytes, %zu needed", lut_len, need);
    if ((reinterpret_cast<uintptr_t>(lut) & 15u) != 0) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "lut must be 16-byte aligned");
    if (out_capacity < m->g.rows)
        VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "output holds %zu values but rows = %zu", out_capacity, m->g.rows);
    return VX_OK;
}

int vx_gemv_lut_i32_dev(const vx_matrix_t* matrix, const int8_t* lut, size_t lut_len, int32_t* out, size_t out_capacity,
                        void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindVelurex));
        VX_TRY(check_lut(matrix, lut, lut_len, out, out_capacity));
        VX_TRY(set_device_of(matrix));
        return run_single_lut(matrix, lut, out, kOutI32, 1.0f, static_cast<hipStream_t>(stream));
    });
}

int vx_gemv_lut_f32_dev(const vx_matrix_t* matrix, const int8_t* lut, size_t lut_len, float act_scale, float* out,
                        size_t out_capacity, void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindVelurex));
        VX_TRY(check_lut(matrix, lut, lut_len, out, out_capacity));
        VX_TRY(set_device_of(matrix));
        const hipStream_t s = static_cast<hipStream_t>(stream);
        if (!(act_scale > 0.0f)) return launch_fill_f32(out, matrix->g.rows, 0.0f, s);
        return run_single_lut(matrix, lut, out, kOutF32Post, matrix->weight_scale / act_scale, s);
    });
}

int vx_matrix_free(vx_matrix_t* matrix) {
    return guard([&]() -> int {
        if (matrix == nullptr) return VX_OK;
        VX_TRY(check_matrix(matrix));
        if (matrix->owner != nullptr)
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the matrix belongs to a decoder (adopted); it is freed with the decoder");
        VX_TRY(set_device_of(matrix));
        VX_HIP(hipDeviceSynchronize());
        destroy(matrix);
        return VX_OK;
    });
}

int vx_matrix_shape(const vx_matrix_t* matrix, size_t* out_rows, size_t* out_cols) {
    return guard([&]() -> int {
        VX_TRY(check_matrix(matrix));
        if (out_rows == nullptr || out_cols == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "output pointer is NULL");
        *out_rows = matrix->g.rows;
        *out_cols = matrix->g.cols;
        return VX_OK;
    });
}

int vx_matrix_memory_bytes(const vx_matrix_t* matrix, size_t* out_bytes) {
    return guard([&]() -> int {
        VX_TRY(check_matrix(matrix));
        if (out_bytes == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_bytes is NULL");
        *out_bytes = matrix->g.device_bytes;
        return VX_OK;
    });
}

int vx_matrix_weight_scale(const vx_matrix_t* matrix, float* out_scale) {
    return guard([&]() -> int {
        VX_TRY(check_matrix(matrix));
        if (out_scale == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_scale is NULL");
        *out_scale = matrix->weight_scale;
        return VX_OK;
    });
}

int vx_matrix_device_weights(const vx_matrix_t* matrix, const void** out_ptr) {
    return guard([&]() -> int {
        VX_TRY(check_matrix(matrix));
        if (out_ptr == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_ptr is NULL");
        *out_ptr = matrix->d_w;
        return VX_OK;
    });
}

int vx_gemv_i32_dev(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, int32_t* out, size_t out_capacity,
                    void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindVelurex));
        VX_TRY(check_io(matrix, acts, acts_len, out, out_capacity));
        VX_TRY(set_device_of(matrix));
        return gemv_i32_dev(const_cast<vx_matrix*>(matrix), acts, out, static_cast<hipStream_t>(stream));
    });
}

int vx_gemv_f32_dev(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, float act_scale, float* out,
                    size_t out_capacity, void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindVelurex));
        VX_TRY(check_io(matrix, acts, acts_len, out, out_capacity));
        VX_TRY(set_device_of(matrix));
        return gemv_f32_dev(const_cast<vx_matrix*>(matrix), acts, act_scale, out, static_cast<hipStream_t>(stream));
    });
}

int vx_layer_forward(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, float act_scale, float* out,
                     size_t out_capacity) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindVelurex));
        VX_TRY(check_io(matrix, acts, acts_len, out, out_capacity));
        vx_matrix* m = const_cast<vx_matrix*>(matrix);
        std::lock_guard<std::mutex> lock(m->mu);
        // A scale that is not > 0 makes every output zero (layer.rs:246-253), as the device path's fill does.
        if (!(act_scale > 0.0f)) {
            std::memset(out, 0, m->g.rows * sizeof(float));
            return VX_OK;
        }
        VX_TRY(set_device_of(m));
        // The activations go into a pinned host buffer that the GEMV's workgroups read over the bus (each its own K
        // slice), and the GEMV writes its outputs into the same buffer: one launch, no copy engine (two synchronous
        // copies through pageable memory cost 15-25 us per call at the Falcon3-10B shapes). The GEMV's last workgroup
        // then stores the call's number into the buffer's flag word, on which this thread waits instead of a stream
        // synchronisation (whose completion path costs about 5 us more per call).
        const size_t out_off = round_up(m->g.cols, 256);
        const size_t flag_off = out_off + round_up(m->g.padded_rows * 4, 256);
        if (m->h_io == nullptr) {
            void* h = nullptr;
            VX_HIP(hipHostMalloc(&h, flag_off + 256, hipHostMallocDefault));
            void* hd = nullptr;
            hipError_t e = hipHostGetDevicePointer(&hd, h, 0);
            hipStream_t st = nullptr;
            if (e == hipSuccess) e = hipStreamCreate(&st);
            if (e != hipSuccess) {
                (void)hipHostFree(h);
                VX_FAIL(VX_ERR_DEVICE, "pinned staging for vx_layer_forward failed: %s", hipGetErrorString(e));
            }
            m->h_io = static_cast<int8_t*>(h);
            m->h_io_dev = static_cast<int8_t*>(hd);
            m->io_stream = st;
            m->io_seq = 0;
            __atomic_store_n(reinterpret_cast<uint32_t*>(m->h_io + flag_off), 0u, __ATOMIC_RELEASE);
        }
        uint32_t* flag = reinterpret_cast<uint32_t*>(m->h_io + flag_off);
        const uint32_t seq = m->io_seq + 1u == 0u ? 1u : m->io_seq + 1u;  // never 0, the buffer's initial value
        m->io_seq = seq;
        std::memcpy(m->h_io, acts, m->g.cols);
        VX_TRY(run_single(m, nullptr, m->h_io_dev + out_off, kOutF32Post, m->weight_scale / act_scale, m->io_stream,
                          reinterpret_cast<uint32_t*>(m->h_io_dev + flag_off), seq, m->h_io_dev, 1u));
        // Wait for the flag; every 65536 reads (tens of microseconds, longer than a call), ask the stream whether it
        // has ended (an error, or an end without the flag, is reported instead of waiting on).
        for (uint32_t i = 1;; ++i) {
            if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) == seq) break;
            if ((i & 0xffffu) == 0u) {
                const hipError_t q = hipStreamQuery(m->io_stream);
                if (q == hipErrorNotReady) continue;
                if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) == seq) break;
                if (q != hipSuccess) VX_FAIL(VX_ERR_DEVICE, "vx_layer_forward's GEMV failed: %s", hipGetErrorString(q));
                VX_FAIL(VX_ERR_INTERNAL, "vx_layer_forward's GEMV ended without storing its completion flag");
            }
        }
        std::memcpy(out, m->h_io + out_off, m->g.rows * sizeof(float));
        return VX_OK;
    });
}

static int planar_oneshot(const uint8_t* weights, size_t weights_len, size_t rows, size_t cols, const int8_t* acts,
                          size_t acts_len, void* out, size_t out_capacity, bool f32, float scale) {
    if (acts == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "activations is NULL");
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out is NULL");
    VX_TRY(check_shape(rows, cols));
    if (out_capacity < rows) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "output holds %zu values but rows = %zu", out_capacity, rows);
    if (acts_len < cols) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "activations hold %zu values but cols = %zu", acts_len, cols);
    vx_matrix_t* m = nullptr;
    VX_TRY(create_matrix(weights, weights_len, rows, cols, 1.0f, &m));
    int8_t* d_acts = m->d_io;
    void* d_out = m->d_io + round_up(cols, 256);
    int st = VX_OK;
    hipError_t e = hipMemcpy(d_acts, acts, cols, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        st = launch_stage(d_acts, cols, m->d_staged, nullptr);
        if (st == VX_OK) st = run_single(m, m->d_staged, d_out, f32 ? kOutF32Post : kOutI32, scale, nullptr);
        if (st == VX_OK) e = hipMemcpy(out, d_out, rows * 4, hipMemcpyDeviceToHost);
    }
    (void)hipDeviceSynchronize();
    destroy(m);
    if (st != VX_OK) return st;
    if (e != hipSuccess) VX_FAIL(VX_ERR_DEVICE, "copy failed: %s", hipGetErrorString(e));
    return VX_OK;
}

int vx_gemv_planar_i32(const uint8_t* weights, size_t weights_len, size_t rows, size_t cols, const int8_t* acts,
                       size_t acts_len, int32_t* out, size_t out_capacity) {
    return guard([&]() -> int {
        return planar_oneshot(weights, weights_len, rows, cols, acts, acts_len, out, out_capacity, false, 1.0f);
    });
}

int vx_gemv_planar_f32(const uint8_t* weights, size_t weights_len, size_t rows, size_t cols, const int8_t* acts,
                       size_t acts_len, float scale, float* out, size_t out_capacity) {
    return guard([&]() -> int {
        return planar_oneshot(weights, weights_len, rows, cols, acts, acts_len, out, out_capacity, true, scale);
    });
}

}  // extern "C"

// ---- batched GEMV plans -------------------------------------------------------------------------------------------------

namespace vx {

static int check_plan(const vx_plan_t* p) {
    if (p == nullptr) VX_FAIL(VX_ERR_INVALID_HANDLE, "plan handle is NULL");
    if (p->magic != kPlanMagic) VX_FAIL(VX_ERR_INVALID_HANDLE, "plan handle is not valid (freed or foreign)");
    return VX_OK;
}

static void destroy_plan(vx_plan* p) {
    if (p->d_jobs) (void)hipFree(p->d_jobs);
    if (p->d_part) (void)hipFree(p->d_part);
    if (p->d_split) (void)hipFree(p->d_split);
    if (p->d_q2jobs) (void)hipFree(p->d_q2jobs);
    if (p->d_stage) (void)hipFree(p->d_stage);
    p->magic = 0;
    delete p;
}

static int create_plan(const vx_gemv_job_t* jobs, size_t n_jobs, bool lut, vx_plan_t** out) {
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_plan is NULL");
    *out = nullptr;
    if (jobs == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "jobs is NULL");
    if (n_jobs == 0 || n_jobs > 65535) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "n_jobs must be in 1..=65535 (got %zu)", n_jobs);
    DeviceInfo di;
    VX_TRY(device_info(&di));
    std::vector<Job> hj(n_jobs);
    size_t part_ints = 0;
    uint32_t items = 0;
    std::vector<uint32_t> split;
    std::vector<StageJob> stages;  // distinct (acts, staged) pairs of jobs that bring raw activations
    constexpr size_t kJobSizeNoActs = offsetof(vx_gemv_job_t, acts);
    for (size_t i = 0; i < n_jobs; ++i) {
        const vx_gemv_job_t& u = jobs[i];
        if (u.struct_size != sizeof(vx_gemv_job_t) && u.struct_size != kJobSizeNoActs)
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "jobs[%zu].struct_size is %u, expected %zu (or %zu without acts)", i,
                    u.struct_size, sizeof(vx_gemv_job_t), kJobSizeNoActs);
        const int8_t* raw = u.struct_size == sizeof(vx_gemv_job_t) ? u.acts : nullptr;
        VX_TRY(check_kind(u.matrix, kKindVelurex));
        const vx_matrix* m = u.matrix;
        if (m->device != di.device)
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "jobs[%zu].matrix lives on device %d, the current device is %d", i, m->device, di.device);
        if (u.staged == nullptr || u.out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "jobs[%zu]: staged or out is NULL", i);
        const size_t need = lut ? compact_lut_bytes(m->g.cols) : staged_bytes(m->g.cols);
        if (u.staged_len < need)
            VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "jobs[%zu]: staged holds %zu bytes, %zu needed", i, u.staged_len, need);
        if (lut && (reinterpret_cast<uintptr_t>(u.staged) & 15u) != 0)
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "jobs[%zu]: the compact tables must be 16-byte aligned", i);
        if (u.out_capacity < m->g.rows)
            VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "jobs[%zu]: out holds %zu values but rows = %zu", i, u.out_capacity, m->g.rows);
        if (u.out_f32 != 0 && u.out_f32 != 1) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "jobs[%zu].out_f32 must be 0 or 1", i);
        if (u.out_f32 == 1 && u.act_scale_dev == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "jobs[%zu].act_scale_dev is NULL", i);
        {
            // a staging of this job's input: new, the same as an earlier job's, or a conflict
            uint8_t* dst = static_cast<uint8_t*>(const_cast<void*>(u.staged));
            bool seen = false;
            for (const StageJob& sj : stages) {
                if (sj.staged != dst) continue;
                if (sj.acts != raw || sj.cols != m->g.cols)
                    VX_FAIL(VX_ERR_INVALID_ARGUMENT, "jobs[%zu]: its staged buffer is staged by an earlier job from "
                            "other activations", i);
                seen = true;
            }
            if (raw != nullptr && lut)
                VX_FAIL(VX_ERR_UNSUPPORTED, "jobs[%zu]: raw activations are staged by velurex plans only", i);
            if (raw != nullptr && !seen)
                stages.push_back(StageJob{raw, dst, static_cast<uint32_t>(m->g.cols), static_cast<uint32_t>(m->g.tbr),
                                          static_cast<uint32_t>(m->g.dbr), stage_groups(m->g.cols)});
            if (raw == nullptr && !seen)  // a job that reads a staged input the caller keeps: remembered as such
                stages.push_back(StageJob{nullptr, dst, static_cast<uint32_t>(m->g.cols), 0, 0, 0});
        }
        Job& j = hj[i];
        j = Job{};
        if (lut) plan_lut_job(j, m->g, 0);
        else plan_job(j, m->g, 0);
        j.w = m->d_w;
        j.dsum = lut ? nullptr : m->d_dsum;
        j.staged = static_cast<const uint8_t*>(u.staged);
        j.out = u.out;
        j.act_scale = u.act_scale_dev;
        j.weight_scale = m->weight_scale;
        j.out_kind = u.out_f32 ? kOutF32Dev : kOutI32;
        j.item_begin = items;
        const uint64_t next = static_cast<uint64_t>(items) + job_items(j);
        if (next > 0x7fffffffu) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "the plan has too many work items");
        items = static_cast<uint32_t>(next);
        if (j.kslices > 1) {
            j.part = reinterpret_cast<int32_t*>(part_ints);  // offset, rebased below
            part_ints += static_cast<size_t>(j.kslices) * j.padded_rows;
            split.push_back(static_cast<uint32_t>(i));
        }
    }
    vx_plan* p = new vx_plan();
    p->magic = kPlanMagic;
    p->device = di.device;
    p->num_cus = di.num_cus;
    p->d_jobs = nullptr;
    p->d_part = nullptr;
    p->d_split = nullptr;
    p->d_q2jobs = nullptr;
    p->d_q2sched = nullptr;
    p->n_jobs = static_cast<uint32_t>(n_jobs);
    p->total_items = items;
    p->max_rows = 0;
    p->n_split = static_cast<uint32_t>(split.size());
    p->lut = lut ? 1u : 0u;
    p->d_stage = nullptr;
    p->n_stage = 0;
    p->stage_max_groups = 0;
    for (uint32_t i : split) p->max_rows = std::max(p->max_rows, hj[i].rows);
    std::vector<StageJob> st;
    for (const StageJob& sj : stages)
        if (sj.acts != nullptr) {
            st.push_back(sj);
            p->stage_max_groups = std::max(p->stage_max_groups, sj.groups);
        }
    p->n_stage = static_cast<uint32_t>(st.size());
    hipError_t e = hipMalloc(&p->d_jobs, n_jobs * sizeof(Job));
    if (e == hipSuccess && !st.empty()) e = hipMalloc(&p->d_stage, st.size() * sizeof(StageJob));
    if (e == hipSuccess && !st.empty())
        e = hipMemcpy(p->d_stage, st.data(), st.size() * sizeof(StageJob), hipMemcpyHostToDevice);
    if (e == hipSuccess && part_ints) e = hipMalloc(&p->d_part, part_ints * sizeof(int32_t));
    if (e == hipSuccess && !split.empty()) e = hipMalloc(&p->d_split, split.size() * sizeof(uint32_t));
    if (e == hipSuccess && !split.empty())
        e = hipMemcpy(p->d_split, split.data(), split.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        for (auto& j : hj)
            if (j.kslices > 1) j.part = p->d_part + reinterpret_cast<size_t>(j.part);
        e = hipMemcpy(p->d_jobs, hj.data(), n_jobs * sizeof(Job), hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        destroy_plan(p);
        VX_FAIL(VX_ERR_DEVICE, "plan allocation failed: %s", hipGetErrorString(e));
    }
    *out = p;
    return VX_OK;
}

}  // namespace vx

extern "C" {

int vx_plan_create(const vx_gemv_job_t* jobs, size_t n_jobs, vx_plan_t** out_plan) {
    return guard([&]() -> int { return create_plan(jobs, n_jobs, false, out_plan); });
}

int vx_lut_plan_create(const vx_gemv_job_t* jobs, size_t n_jobs, vx_plan_t** out_plan) {
    return guard([&]() -> int { return create_plan(jobs, n_jobs, true, out_plan); });
}

int vx_plan_run(const vx_plan_t* plan, void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_plan(plan));
        int cur = -1;
        VX_HIP(hipGetDevice(&cur));
        if (cur != plan->device) VX_HIP(hipSetDevice(plan->device));
        if (plan->d_q2jobs) {
            Q2Args q{};
            q.jobs = plan->d_q2jobs;
            q.n_jobs = plan->n_jobs;
            q.total_items = plan->total_items;
            q.sched = plan->d_q2sched;
            q.sched_grid = plan->q2_grid;
            return launch_q2(q, plan->num_cus, static_cast<hipStream_t>(stream));
        }
        LaunchArgs a{};
        a.jobs = plan->d_jobs;
        a.n_jobs = plan->n_jobs;
        a.total_items = plan->total_items;
        VX_TRY(launch_stage_batch(plan->d_stage, plan->n_stage, plan->stage_max_groups, static_cast<hipStream_t>(stream)));
        if (plan->lut)
            return launch_gemv_lut(a, plan->max_rows, plan->d_split, plan->n_split, plan->num_cus,
                                   static_cast<hipStream_t>(stream));
        return launch_gemv(a, plan->max_rows, plan->d_split, plan->n_split, plan->num_cus, static_cast<hipStream_t>(stream));
    });
}

int vx_plan_work_items(const vx_plan_t* plan, uint32_t* out_items) {
    return guard([&]() -> int {
        VX_TRY(check_plan(plan));
        if (out_items == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_items is NULL");
        *out_items = plan->total_items;
        return VX_OK;
    });
}

int vx_plan_free(vx_plan_t* plan) {
    return guard([&]() -> int {
        if (plan == nullptr) return VX_OK;
        VX_TRY(check_plan(plan));
        VX_HIP(hipSetDevice(plan->device));
        VX_HIP(hipDeviceSynchronize());
        destroy_plan(plan);
        return VX_OK;
    });
}

}  // extern "C"

// ---- batched GEMM -------------------------------------------------------------------------------------------------------

extern "C" {

int vx_gemm_workspace_bytes(const vx_matrix_t* matrix, size_t m, size_t* out_bytes) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindVelurex));
        if (out_bytes == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_bytes is NULL");
        if (m == 0 || m > VX_MAX_GEMM_TOKENS) VX_FAIL(VX_ERR_INVALID_SHAPE, "m must be in 1..=%d (got %zu)", VX_MAX_GEMM_TOKENS, m);
        *out_bytes = gemm_workspace_bytes(matrix->g, m, matrix->num_cus);
        return VX_OK;
    });
}

static int check_gemm(const vx_matrix_t* matrix, const int8_t* x, size_t m, size_t ldx, const int32_t* y, size_t ldy) {
    VX_TRY(check_kind(matrix, kKindVelurex));
    if (x == nullptr || y == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "x or y is NULL");
    if (m == 0 || m > VX_MAX_GEMM_TOKENS) VX_FAIL(VX_ERR_INVALID_SHAPE, "m must be in 1..=%d (got %zu)", VX_MAX_GEMM_TOKENS, m);
    if (ldx < matrix->g.cols) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "ldx = %zu is less than cols = %zu", ldx, matrix->g.cols);
    if (ldy < matrix->g.rows) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "ldy = %zu is less than rows = %zu", ldy, matrix->g.rows);
    return VX_OK;
}

int vx_gemm_i32_dev(const vx_matrix_t* matrix, const int8_t* x, size_t m, size_t ldx, int32_t* y, size_t ldy,
                    void* workspace, size_t workspace_len, void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_gemm(matrix, x, m, ldx, y, ldy));
        if (workspace == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "workspace is NULL");
        const size_t need = gemm_workspace_bytes(matrix->g, m, matrix->num_cus);
        if (workspace_len < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "workspace holds %zu bytes, %zu needed", workspace_len, need);
        if (reinterpret_cast<uintptr_t>(workspace) % 256u) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
        VX_TRY(set_device_of(matrix));
        return launch_gemm(matrix->d_w, matrix->g, matrix->num_cus, x, m, ldx, y, ldy, static_cast<uint8_t*>(workspace),
                           static_cast<hipStream_t>(stream));
    });
}

int vx_gemm_i32_noalloc_dev(const vx_matrix_t* matrix, const int8_t* x, size_t m, size_t ldx, int32_t* y, size_t ldy,
                            void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_gemm(matrix, x, m, ldx, y, ldy));
        VX_TRY(set_device_of(matrix));
        return launch_gemm_noalloc(matrix->d_w, matrix->g, matrix->device, matrix->num_cus, x, m, ldx, y, ldy,
                                   static_cast<hipStream_t>(stream));
    });
}

}  // extern "C"

// ---- Q2_0 (block-scaled) ------------------------------------------------------------------------------------------------

namespace vx {

static int check_q2_shape(size_t rows, size_t cols) {
    VX_TRY(check_shape(rows, cols));
    if (cols % 64 != 0) VX_FAIL(VX_ERR_INVALID_SHAPE, "cols = %zu is not a multiple of 64 (one scale per 64 weights)", cols);
    if (cols > kQ2MaxCols) VX_FAIL(VX_ERR_INVALID_SHAPE, "cols = %zu exceeds %zu for the Q2_0 GEMV", cols, kQ2MaxCols);
    return VX_OK;
}

static Q2Job q2_job(const vx_matrix* m, const int8_t* acts, const float* act_scales, float* out) {
    Q2Job j{};
    j.w = m->d_w;
    j.scales = reinterpret_cast<const uint16_t*>(m->d_w + q2_weight_bytes(m->g.rows, m->g.cols));
    j.acts = acts;
    j.act_scales = act_scales;
    j.out = out;
    j.rows = static_cast<uint32_t>(m->g.rows);
    j.cols = static_cast<uint32_t>(m->g.cols);
    j.n_tiles = static_cast<uint32_t>(m->g.n_tiles);
    j.nb = static_cast<uint32_t>(q2_blocks(m->g.cols));
    j.item_begin = 0;
    return j;
}

static int check_q2_io(const vx_matrix* m, const int8_t* acts, size_t acts_len, const float* act_scales, size_t n_scales,
                       const void* out, size_t out_capacity) {
    if (acts == nullptr || act_scales == nullptr || out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "acts, act_scales or out is NULL");
    if (acts_len < m->g.cols) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "acts hold %zu values but cols = %zu", acts_len, m->g.cols);
    if (reinterpret_cast<uintptr_t>(acts) % 4u) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "acts must be 4-byte aligned");
    if (n_scales < m->g.cols / 32) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "act_scales hold %zu values, %zu needed", n_scales, m->g.cols / 32);
    if (out_capacity < m->g.rows) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "out holds %zu values but rows = %zu", out_capacity, m->g.rows);
    return VX_OK;
}

}  // namespace vx

extern "C" {

int vx_q2_matrix_create(const uint8_t* planar, size_t planar_len, const uint16_t* scales_f16, size_t n_scales,
                        size_t rows, size_t cols, vx_matrix_t** out_matrix) {
    return guard([&]() -> int {
        if (out_matrix == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_matrix is NULL");
        *out_matrix = nullptr;
        VX_TRY(check_q2_shape(rows, cols));
        if (planar == nullptr || scales_f16 == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "planar or scales_f16 is NULL");
        const size_t need = rows * planar_row_bytes(cols);
        if (planar_len < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "planar holds %zu bytes, %zu needed", planar_len, need);
        if (n_scales < rows * (cols / 64)) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "scales hold %zu values, %zu needed", n_scales, rows * (cols / 64));
        const size_t bad = find_invalid_byte(planar, need);
        if (bad != SIZE_MAX)
            VX_FAIL(VX_ERR_INVALID_VALUE, "byte %zu (value %u) is not a velurex byte", bad, static_cast<unsigned>(planar[bad]));
        DeviceInfo di;
        VX_TRY(device_info(&di));
        vx_matrix* m = new vx_matrix();
        m->magic = kMatrixMagic;
        m->kind = kKindQ2;
        m->g = geometry(rows, cols);
        m->weight_scale = 1.0f;
        m->device = di.device;
        m->num_cus = di.num_cus;
        m->kslices = 1;
        m->slice_chunks = 0;
        m->d_w = nullptr;
        m->d_part = nullptr;
        m->d_dsum = nullptr;
        m->d_staged = nullptr;
        m->d_io = nullptr;
        m->owner = nullptr;
        const size_t bytes = q2_device_bytes(rows, cols);
        std::vector<uint8_t> host(bytes);
        q2_to_device_layout(planar, scales_f16, rows, cols, host.data());
        hipError_t e = hipMalloc(&m->d_w, bytes);
        if (e == hipSuccess) e = hipMemcpy(m->d_w, host.data(), bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            destroy(m);
            VX_FAIL(VX_ERR_DEVICE, "device allocation or upload of %zu bytes failed: %s", bytes, hipGetErrorString(e));
        }
        m->g.device_bytes = bytes;
        *out_matrix = m;
        return VX_OK;
    });
}

int vx_q2_gemv_f32_dev(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, const float* act_scales,
                       size_t n_act_scales, float* out, size_t out_capacity, void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindQ2));
        VX_TRY(check_q2_io(matrix, acts, acts_len, act_scales, n_act_scales, out, out_capacity));
        VX_TRY(set_device_of(matrix));
        Q2Args a{};
        a.jobs = nullptr;
        a.n_jobs = 1;
        a.one = q2_job(matrix, acts, act_scales, out);
        a.total_items = q2_items(a.one.rows);
        return launch_q2(a, matrix->num_cus, static_cast<hipStream_t>(stream));
    });
}

int vx_q2_lane_sums_dev(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, int32_t* out,
                        size_t out_capacity, void* stream) {
    return guard([&]() -> int {
        VX_TRY(check_kind(matrix, kKindQ2));
        if (acts == nullptr || out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "acts or out is NULL");
        if (acts_len < matrix->g.cols) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "acts hold %zu values but cols = %zu", acts_len, matrix->g.cols);
        const size_t need = matrix->g.rows * (matrix->g.cols / 32) * 8;
        if (out_capacity < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "out holds %zu values, %zu needed", out_capacity, need);
        VX_TRY(set_device_of(matrix));
        return launch_q2_lane_sums(q2_job(matrix, acts, nullptr, nullptr), out, static_cast<hipStream_t>(stream));
    });
}

int vx_q2_plan_create(const vx_q2_job_t* jobs, size_t n_jobs, vx_plan_t** out_plan) {
    return guard([&]() -> int {
        if (out_plan == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_plan is NULL");
        *out_plan = nullptr;
        if (jobs == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "jobs is NULL");
        if (n_jobs == 0 || n_jobs > 65535) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "n_jobs must be in 1..=65535 (got %zu)", n_jobs);
        DeviceInfo di;
        VX_TRY(device_info(&di));
        std::vector<Q2Job> hj(n_jobs);
        uint32_t items = 0;
        for (size_t i = 0; i < n_jobs; ++i) {
            const vx_q2_job_t& u = jobs[i];
            if (u.struct_size != sizeof(vx_q2_job_t))
                VX_FAIL(VX_ERR_INVALID_ARGUMENT, "jobs[%zu].struct_size is %u, expected %zu", i, u.struct_size, sizeof(vx_q2_job_t));
            VX_TRY(check_kind(u.matrix, kKindQ2));
            if (u.matrix->device != di.device) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "jobs[%zu].matrix lives on another device", i);
            VX_TRY(check_q2_io(u.matrix, u.acts, u.acts_len, u.act_scales, u.n_act_scales, u.out, u.out_capacity));
            hj[i] = q2_job(u.matrix, u.acts, u.act_scales, u.out);
            hj[i].item_begin = items;
            items += q2_items(hj[i].rows);
        }
        vx_plan* p = new vx_plan();
        p->magic = kPlanMagic;
        p->device = di.device;
        p->num_cus = di.num_cus;
        p->d_jobs = nullptr;
        p->d_part = nullptr;
        p->d_split = nullptr;
        p->d_q2jobs = nullptr;
        p->d_q2sched = nullptr;
        p->d_stage = nullptr;
        p->n_stage = 0;
        p->n_jobs = static_cast<uint32_t>(n_jobs);
        p->total_items = items;
        p->max_rows = 0;
        p->n_split = 0;
        // the job table, then the schedule (4-byte words after the 8-byte aligned table)
        const std::vector<uint32_t> sched = q2_schedule(hj, items, di.num_cus);
        const size_t job_bytes = n_jobs * sizeof(Q2Job);
        hipError_t e = hipMalloc(&p->d_q2jobs, job_bytes + sched.size() * sizeof(uint32_t));
        if (e == hipSuccess) e = hipMemcpy(p->d_q2jobs, hj.data(), job_bytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) {
            uint32_t* ds = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(p->d_q2jobs) + job_bytes);
            e = hipMemcpy(ds, sched.data(), sched.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
            p->d_q2sched = ds;
            p->q2_grid = static_cast<uint32_t>(sched.size() - 1u - items);
        }
        if (e != hipSuccess) {
            destroy_plan(p);
            VX_FAIL(VX_ERR_DEVICE, "plan allocation failed: %s", hipGetErrorString(e));
        }
        *out_plan = p;
        return VX_OK;
    });
}

}  // extern "C"
