// Internal helpers of libvelurex_hip: the per-thread error slot, argument checks, the device layout arithmetic and the
// GEMV job descriptors shared by the host planner and the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

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

constexpr int kTileRows = 64;    // rows per tile = lanes of a wavefront
constexpr int kChunk = 16;       // bytes one lane loads per step (global_load_dwordx4)
constexpr int kTileGroup = 16;   // tiles whose chunks are interleaved (= waves of a GEMV workgroup)
constexpr size_t kQK5 = 160;     // trits per planar block (pack.rs:19)
constexpr size_t kBlockBytes = 32;
constexpr size_t kStageHeader = 64;  // staged activations: int32 sum of the activations, then the chunk entries
constexpr uint8_t kZeroByte = 125;   // five zero trits (every digit d = t + 1 is 1)

inline size_t planar_row_bytes(size_t cols) { return (cols + kQK5 - 1) / kQK5 * kBlockBytes; }
inline size_t tile_full_columns(size_t cols) { return cols / kQK5 * kBlockBytes; }
inline size_t tile_row_bytes(size_t cols) {  // pack.rs:222-225
    const size_t tail = (cols % kQK5 + 4) / 5;
    return tile_full_columns(cols) + tail + (tail & 1);
}
inline size_t device_row_bytes(size_t cols) { return (tile_row_bytes(cols) + kChunk - 1) / kChunk * kChunk; }
inline size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }
inline size_t staged_bytes(size_t cols) { return kStageHeader + device_row_bytes(cols) * 8; }

struct Geometry {
    size_t rows, cols, padded_rows, n_tiles, n_groups, tbr, dbr, n_chunks, device_bytes;
};

inline Geometry geometry(size_t rows, size_t cols) {
    Geometry g;
    g.rows = rows;
    g.cols = cols;
    g.padded_rows = round_up(rows, kTileRows);
    g.n_tiles = g.padded_rows / kTileRows;
    g.n_groups = (g.n_tiles + kTileGroup - 1) / kTileGroup;
    g.tbr = tile_row_bytes(cols);
    g.dbr = device_row_bytes(cols);
    g.n_chunks = g.dbr / kChunk;
    g.device_bytes = g.padded_rows * g.dbr;
    return g;
}

// Byte offset of (row r, device byte-column c) in the device layout (vx_layout in include/velurex_hip.h).
__host__ __device__ inline uint64_t layout_offset(uint64_t r, uint32_t c, uint32_t n_tiles, uint32_t n_chunks) {
    const uint32_t tile = static_cast<uint32_t>(r / kTileRows);
    const uint32_t grp = tile / kTileGroup, t = tile - grp * kTileGroup;
    const uint32_t T = (n_tiles - grp * kTileGroup) < static_cast<uint32_t>(kTileGroup) ? n_tiles - grp * kTileGroup
                                                                                         : static_cast<uint32_t>(kTileGroup);
    const uint32_t q = c / kChunk;
    const uint64_t kib = static_cast<uint64_t>(grp) * kTileGroup * n_chunks + static_cast<uint64_t>(q) * T + t;
    return kib * 1024u + (r % kTileRows) * kChunk + c % kChunk;
}

int check_shape(size_t rows, size_t cols);

// One ticket of a cross-workgroup hand-off, taken by one thread after a barrier that follows the workgroup's writes of
// the handed-over data. Returns 1 for ticket `last` (the last of the workgroups that take one), else 0.
//
// The handed-over data is written and read only with device-scope atomic read-modify-writes or agent-scope atomic
// stores and loads, which are performed at the memory side, coherently for every XCD. Each writing wave waits for all
// of its memory operations (s_waitcnt 0) before the barrier, so every write is performed before the ticket is issued;
// the last holder's workgroup issues its reads only after the ticket's value has returned (and a barrier). Compiler
// signal fences keep the compiler from moving memory operations across the ticket in either direction (the barrier's
// workgroup fences already do). Agent-scope release / acquire fences would state the same ordering in the memory
// model's terms, but on gfx950 they write back and invalidate the whole L2 of the XCD (buffer_wbl2 sc1, buffer_inv
// sc1): measured at +10 % on a chain of 160 dependent lone GEMVs and +7 % on a Falcon3-10B decode step at context 7000.
__device__ inline uint32_t take_ticket(uint32_t* ticket, uint32_t last) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const uint32_t t = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return t == last ? 1u : 0u;
}

// ---- GEMV jobs --------------------------------------------------------------------------------------------------------

enum OutKind : uint32_t {
    kOutI32 = 0,       // int32 accumulators
    kOutF32Post = 1,   // float(acc) * post, post = weight_scale / act_scale computed on the host
    kOutF32Dev = 2,    // float(acc) * (weight_scale / *act_scale_dev), zeros when the scale is not > 0
};

// One GEMV of a launch: rows x cols weights in the device layout times one staged activation vector.
struct Job {
    const uint8_t* w;           // device layout
    const uint8_t* staged;      // staged activations (kStageHeader + n_chunks * 128 bytes)
    int32_t* part;              // K-slice partial sums [kslices][padded_rows] (kslices > 1)
    const int32_t* dsum;        // per row: sum of the five digits (t + 1) of every device byte of the row
    void* out;                  // rows values
    const float* act_scale;     // kOutF32Dev
    float post;                 // kOutF32Post
    float weight_scale;         // kOutF32Dev
    uint32_t out_kind;
    uint32_t rows, padded_rows, n_tiles, n_chunks;
    uint32_t kslices, slice_chunks;  // K split: slices of slice_chunks chunks (the last may be shorter)
    uint32_t item_begin;             // first work item of this job in the launch
    uint32_t tbr;                    // tile row bytes: the byte-columns of a compact-table job's tables
    // A lone GEMV's K-slice sums by atomic addition: accum[padded_rows] and tickets[tile groups], both zero between
    // calls; the last slice of a tile group to arrive takes (and clears) the sums and writes the outputs, so no finish
    // kernel runs. Null in a plan.
    int32_t* accum;
    uint32_t* tickets;
};

struct LaunchArgs {
    const Job* jobs;       // device array of n_jobs jobs, or nullptr: use `one`
    uint32_t n_jobs;
    uint32_t total_items;  // work items: (tile group, K slice) pairs summed over the jobs
    Job one;
    // A lone GEMV whose caller waits on host memory (or null): the workgroup that takes the last ticket of `done`
    // (device memory, zero between launches) after every workgroup's outputs are stored resets it and stores `seq`
    // into `flag` (pinned host memory) with a system-scope release.
    uint32_t* done;
    uint32_t* flag;
    uint32_t seq;
    // A lone GEMV on raw int8 activations (or null: the job's staged vector): every workgroup stages its own K slice
    // from acts[cols] (one.tbr the tile row bytes) and subtracts that slice's activation sum, so no staging kernel runs.
    const int8_t* acts;
    uint32_t cols;
};

constexpr uint32_t kMaxSliceChunks = 40;  // chunks per K slice staged in LDS (5 KiB of activations)

// Host planner: fills kslices/slice_chunks of a job. `target_items` spreads a lone GEMV over the GPU, with at least
// `min_slice_chunks` chunks per slice where the row has them; 0 keeps slices as long as kMaxSliceChunks allows (the
// batched launches, which have work enough).
void plan_job(Job& j, const Geometry& g, uint32_t target_items, uint32_t min_slice_chunks = 1);
// The chunks per K slice a lone GEMV on activations in device memory keeps at least: below that the slices' atomic
// sums and tickets cost more than their parallelism gains at the shapes of one to three tile groups (2560 x 2560: 7.16
// -> 6.57 us per call, 3072 x 3072: 7.95 -> 7.03 us, 1024 x 3072: 7.2 -> 6.7-7.0 us; 4 chunks were slower again), and
// the wide shapes keep their split. Activations read from host memory keep one chunk per slice (vx_layer_forward at
// 3072 x 3072: 19 us with one, 22-37 us with two or three).
constexpr uint32_t kLoneMinSliceChunks = 3;
inline uint32_t job_items(const Job& j) {
    return (j.n_tiles + kTileGroup - 1) / kTileGroup * j.kslices;
}

int launch_stage(const int8_t* acts, size_t cols, uint8_t* staged, hipStream_t stream);
// One staging of a batch (vx_plan_run of a plan whose jobs bring raw activations).
struct StageJob {
    const int8_t* acts;
    uint8_t* staged;
    uint32_t cols, tbr, dbr, groups;
};
uint32_t stage_groups(size_t cols);
int launch_stage_batch(const StageJob* jobs, uint32_t n, uint32_t max_groups, hipStream_t stream);
// Launches the GEMV kernel and, when n_split > 0, the finish kernel over the split jobs (`split`: device array of their
// indices in a.jobs; unused without a job array).
int launch_gemv(const LaunchArgs& a, uint32_t max_rows, const uint32_t* split, uint32_t n_split, int num_cus,
                hipStream_t stream);
int launch_device_layout(const uint8_t* planar_dev, const Geometry& g, uint8_t* dst, hipStream_t stream);
// dsum[r] = digit sum of the device row r (every byte of the device layout, padding included).
int launch_digit_sums(const uint8_t* w, const Geometry& g, int32_t* dsum, hipStream_t stream);
int launch_find_invalid(const uint8_t* planar_dev, uint64_t n, unsigned long long* first, hipStream_t stream);
int launch_fill_f32(float* out, size_t n, float v, hipStream_t stream);
size_t gemm_workspace_bytes(const Geometry& g, size_t M, int num_cus);
// Up to 32 tokens, and up to 128 on matrices of at most 8192 rows and 32768 columns with at most 64 MiB of slice sums
// (gemm_small_path), a call runs without a staging kernel (gemm_small_kernel builds the B fragments in LDS from x; a
// finish kernel adds the K slices when there are several) and needs gemm_part_bytes of workspace; otherwise it runs
// as staging + GEMM + finish.
bool gemm_small_path(const Geometry& g, size_t M, int num_cus);
// One matrix of a grouped small-path GEMM: its weights, geometry and output.
struct GemmSub {
    const uint8_t* w;
    const Geometry* g;
    int32_t* y;
    size_t ldy;
};
// Up to 3 matrices with the same columns in one small-path launch (their tiles concatenated), when each of them would
// take the small path at M tokens; gemm_group_part_bytes of workspace.
bool gemm_group_small_path(const GemmSub* subs, int n, size_t M, int num_cus);
size_t gemm_group_part_bytes(const GemmSub* subs, int n, size_t M, int num_cus);
int launch_gemm_group(const GemmSub* subs, int n, int num_cus, const int8_t* x, size_t M, size_t ldx, uint8_t* ws,
                      hipStream_t stream);
int launch_gemm(const uint8_t* w, const Geometry& g, int num_cus, const int8_t* x, size_t M, size_t ldx, int32_t* y,
                size_t ldy, uint8_t* ws, hipStream_t stream);
// The two halves of launch_gemm: staging of the activations (shared by every matrix with the same cols) and the
// product; gemm_workspace_bytes = gemm_stage_bytes + gemm_part_bytes outside the small path.
size_t gemm_stage_bytes(size_t cols, size_t M);
size_t gemm_part_bytes(const Geometry& g, size_t M, int num_cus);
int launch_gemm_stage(const int8_t* x, size_t M, size_t ldx, size_t cols, uint8_t* ws, hipStream_t stream);
// Two matrices of one geometry (a gated pair) as one staged launch over the same staged activations, when that launch
// needs no K split (gemm_staged_pair_ok).
bool gemm_staged_pair_ok(const Geometry& g, size_t M, int num_cus);
int launch_gemm_staged_pair(const uint8_t* w, const uint8_t* w2, const Geometry& g, int num_cus, const uint8_t* staged,
                            size_t M, int32_t* y, int32_t* y2, size_t ldy, hipStream_t stream);
int launch_gemm_staged(const uint8_t* w, const Geometry& g, int num_cus, const uint8_t* staged, size_t M, int32_t* y,
                       size_t ldy, uint8_t* part, hipStream_t stream);
// The same GEMM with its workspace in the library's per-device scratch array (kNoAllocScratchBytes): no allocation.
constexpr size_t kNoAllocScratchBytes = VX_GEMM_NOALLOC_SCRATCH_BYTES;
// Looks up (once per device; `device` must be current) the device address of the no-allocation GEMM's scratch, so
// that vx_gemm_i32_noalloc_dev finds it ready and makes no runtime call of its own under graph capture.
int gemm_scratch_prepare(int device);
int launch_gemm_noalloc(const uint8_t* w, const Geometry& g, int device, int num_cus, const int8_t* x, size_t M,
                        size_t ldx, int32_t* y, size_t ldy, hipStream_t stream);
// The GEMV through the compact activation tables (vx_lut.hip): a job's `staged` is the table of its cols
// (compact_lut_bytes), dsum is unused; plan_lut_job sets the K split for the tables' LDS slices.
size_t compact_lut_bytes(size_t cols);
int launch_compact_lut(const int8_t* acts, size_t cols, int8_t* lut, hipStream_t stream);
void plan_lut_job(Job& j, const Geometry& g, uint32_t target_items);
int launch_gemv_lut(const LaunchArgs& a, uint32_t max_rows, const uint32_t* split, uint32_t n_split, int num_cus,
                    hipStream_t stream);
size_t find_invalid_byte(const uint8_t* planar, size_t n);
void planar_to_device_layout(const uint8_t* planar, const Geometry& g, uint8_t* dst);

// ---- Q2_0 (block-scaled) jobs ---------------------------------------------------------------------------------------

struct Q2Job {
    const uint8_t* w;            // Q2 device layout (vx_q2.hip): planar blocks in the GEMV tile layout
    const uint16_t* scales;      // fp16 weight scales, [tile][group of 4 blocks][row of the tile][10]
    const int8_t* acts;          // cols int8 codes (4-byte aligned)
    const float* act_scales;     // cols / 32 fp32 scales
    float* out;                  // rows values
    uint32_t rows, cols, n_tiles, nb, item_begin;  // nb: 160-trit blocks per row
};

struct Q2Args {
    const Q2Job* jobs;  // device array, or nullptr: use `one`
    uint32_t n_jobs;
    uint32_t total_items;  // runs of 8 tiles (64 rows each) summed over the jobs
    Q2Job one;
    // The plan's schedule, or nullptr (workgroup i takes items i, i + grid, ...): workgroup i takes the items
    // sched[grid + 1 + k] for k in sched[i] .. sched[i + 1] - 1, in increasing order; the launch has sched_grid
    // workgroups, the count the schedule was made for.
    const uint32_t* sched;
    uint32_t sched_grid;
};

size_t q2_blocks(size_t cols);
size_t q2_kgroups(size_t cols);
size_t q2_weight_bytes(size_t rows, size_t cols);
size_t q2_device_bytes(size_t rows, size_t cols);
void q2_to_device_layout(const uint8_t* planar, const uint16_t* scales, size_t rows, size_t cols, uint8_t* dst);
inline uint32_t q2_items(uint32_t rows) { return ((rows + kTileRows - 1) / kTileRows + 7) / 8; }
int launch_q2(const Q2Args& a, int num_cus, hipStream_t stream);
// The plan's balanced assignment of its items to min(total_items, num_cus) workgroups (the layout of Q2Args::sched).
std::vector<uint32_t> q2_schedule(const std::vector<Q2Job>& jobs, uint32_t total_items, int num_cus);
int launch_q2_lane_sums(const Q2Job& j, int32_t* out, hipStream_t stream);

// ---- device state -------------------------------------------------------------------------------------------------------

struct DeviceInfo {
    int device;
    int num_cus;
};
int device_info(DeviceInfo* out);  // current device; VX_ERR_UNSUPPORTED if it is not a gfx950

}  // namespace vx

// ---- handles ------------------------------------------------------------------------------------------------------------

struct vx_matrix {
    uint32_t magic;
    uint32_t kind;      // kKindVelurex (GEMV/GEMM layout) or kKindQ2 (block-scaled layout)
    vx::Geometry g;
    float weight_scale;
    int device;
    int num_cus;
    uint32_t kslices, slice_chunks;  // K split of a lone GEMV on this matrix
    uint8_t* d_w;       // weights, device layout (vx_layout)
    int32_t* d_part;    // K-slice partial sums of a lone GEMV
    int32_t* d_accum;   // a lone GEMV's atomic K-slice sums (padded_rows), tickets (one per tile group) and
    uint32_t* d_tickets;  // completion counter (d_done), zero between calls
    uint32_t* d_done;
    int32_t* d_dsum;    // per padded row: digit sum of the device row (the signed low-nibble correction)
    uint8_t* d_staged;  // activation staging of the calls that take raw int8 activations
    int8_t* d_io;       // one-shot host API: cols bytes of activations + padded_rows * 4 bytes of output
    int8_t* h_io;       // vx_layer_forward: pinned host buffer of the same shape, which the kernels read and write
    int8_t* h_io_dev;   //   directly (its device address); made at the first call
    hipStream_t io_stream;  // vx_layer_forward's stream on this matrix (default priority), made at the first call
    uint32_t io_seq;        // vx_layer_forward's last call number, which its GEMV stores into the buffer's flag word
    const void* owner;  // the decoder that adopted the matrix (it frees it), or null: the caller's
    std::mutex mu;      // serialises the host-pointer API on this handle
};

constexpr uint32_t kMatrixMagic = 0x56584d32u;  // "VXM2"
constexpr uint32_t kKindVelurex = 0;
constexpr uint32_t kKindQ2 = 1;
constexpr size_t kQ2MaxCols = 12288;  // activations of one Q2_0 row staged in LDS (two workgroups per CU)

struct vx_plan {
    uint32_t magic;
    int device;
    int num_cus;
    vx::Job* d_jobs;
    int32_t* d_part;
    uint32_t* d_split;  // indices of the jobs split into K slices
    vx::Q2Job* d_q2jobs;  // Q2_0 plans: their job table (d_jobs unused), then the schedule (d_q2sched)
    const uint32_t* d_q2sched;
    uint32_t q2_grid;     // the workgroups the schedule was made for
    uint32_t n_jobs, total_items, max_rows, n_split;
    uint32_t lut;  // the jobs read compact activation tables (vx_lut_plan_create)
    vx::StageJob* d_stage;  // the distinct stagings of jobs that bring raw activations, run first (one launch)
    uint32_t n_stage, stage_max_groups;
};

constexpr uint32_t kPlanMagic = 0x56585031u;  // "VXP1"
