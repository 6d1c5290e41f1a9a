/*
 * velurex_hip.h - C ABI of the MI355X (gfx950) velurex ternary GEMV library (libvelurex_hip.so).
 *
 * Ternary weights {-1, 0, +1} are stored five to a byte (velurex encoding, 1.60 bits per weight) and multiplied with
 * int8 activations by hand-written CDNA4 HIP kernels. The integer products are exact (int32); the fp32 epilogue is the
 * one of the reference's projection layers.
 *
 * This header replaces, for one GPU, the kernel-level entry points of the reference's C ABI
 * (rust/crates/quintrit-c/include/quintrit.h:73-218) and the Rust trait the runtime calls
 * (rust/crates/quintrit-runtime/src/layer.rs:72-87, TernaryGemvLayer). Each declaration below names the reference
 * interface it stands in for.
 *
 * Conventions (the reference's, quintrit.h:11-22):
 *   - Every function that can fail returns an int status: VX_OK (0) or a VX_ERR_* code. The codes have the values of
 *     QUINTRIT_OK / QUINTRIT_ERR_* (quintrit.h:73-88), so a binding can forward them unchanged. On failure
 *     vx_last_error_message() describes the failure (per thread).
 *   - Every pointer argument is validated, every buffer comes with an explicit length, sizes are size_t. A NULL pointer,
 *     an undersized buffer or a bad shape yields an error code, never a crash.
 *   - Versioned structs start with a uint32_t struct_size the caller sets to sizeof(the struct).
 *   - No C++ exception crosses the boundary.
 *
 * Device pointers and streams: functions with the suffix _dev take device pointers and a HIP stream (hipStream_t,
 * passed as void*; NULL is the null stream); they enqueue work and return without waiting. Every other function takes
 * host pointers and returns when the result is in host memory.
 *
 * Thread safety: functions are thread-safe on distinct matrix handles. A matrix handle owns a small device workspace
 * (K-slice partial sums and activation staging); calls on one handle must be ordered: either one stream per handle,
 * or events between streams. The host-pointer functions serialise calls on one handle internally.
 */
#ifndef VELUREX_HIP_H
#define VELUREX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VX_VERSION_STRING "0.2.0"
#define VX_ABI_VERSION 2

/* ---- status codes: same values as quintrit.h:73-88 ----------------------------------------------------------------- */
#define VX_OK                      0
#define VX_ERR_NULL_POINTER        1
#define VX_ERR_INVALID_ARGUMENT    2
#define VX_ERR_INVALID_SHAPE       3
#define VX_ERR_BUFFER_TOO_SMALL    4
#define VX_ERR_INVALID_VALUE       5  /* a packed byte that is not one of the 243 velurex values */
#define VX_ERR_UNSUPPORTED         6  /* no gfx950 device, or the library was built without it */
#define VX_ERR_IO                  7
#define VX_ERR_FORMAT              8
#define VX_ERR_NOT_FOUND           9
#define VX_ERR_MODEL              10
#define VX_ERR_CONTEXT_OVERFLOW   11
#define VX_ERR_BUSY               12
#define VX_ERR_INTERNAL           13
#define VX_ERR_INVALID_HANDLE     14
#define VX_ERR_DEVICE             15  /* a HIP call failed (driver error, out of device memory) */

/* Largest column count: keeps |sum| < 2^24 so float(acc) is exact (quintrit-core/src/limits.rs:7-19). */
#define VX_MAX_GEMV_COLS 131072
/* Largest row count accepted. */
#define VX_MAX_ROWS ((size_t)1 << 31)

/* Replaces quintrit_status_string (quintrit.h:91). Static string, never NULL. */
const char* vx_status_string(int status);
/* Replaces quintrit_last_error_code (quintrit.h:94). */
int vx_last_error_code(void);
/* Replaces quintrit_last_error_message (quintrit.h:100). Valid until the next vx_* call on the same thread. */
const char* vx_last_error_message(void);
/* Replaces quintrit_version / quintrit_abi_version (quintrit.h:107-110). */
const char* vx_version(void);
uint32_t vx_abi_version(void);

/* Number of usable gfx950 devices (0 when there is none; the call itself succeeds). Counterpart of the reference's GPU
 * queries (quintrit-c/src/cuda.rs). */
int vx_device_count(int32_t* out_count);

/* ---- layout ------------------------------------------------------------------------------------------------------------ */

/*
 * Device layout of a rows x cols matrix. The interchange format is the planar layout of the reference
 * (quintrit-core/src/pack.rs:10-16: a row is ceil(cols/160) blocks of 32 bytes; byte j of block b packs columns
 * b*160 + p*32 + j, p = 0..4). On upload each row is re-encoded with the packed tail of pack.rs:212-276 (the partial
 * last block stored five trits per byte, tile_row_bytes(cols) bytes) and padded with byte 125 (five zero trits) to
 * device_row_bytes, a multiple of 16. Rows form tiles of 64 (tile_rows) and tiles form groups of 16 (tile_group); the
 * 16-byte chunk q of tile t lives at KiB (g * 16 * n_chunks + q * T + t') of the buffer, with g = t / 16, t' = t % 16,
 * T = the number of tiles in group g (16, or fewer in the last group) and n_chunks = device_row_bytes / 16; inside the
 * chunk, row r % 64 holds bytes 16 (r % 64) .. +15. A GPU wave (64 lanes = 64 rows) thus reads 1 KiB per load, and the 16
 * waves of a workgroup that work on one tile group read 16 consecutive KiB. Counterpart of quintrit_tiled_layout_t
 * (quintrit.h:181-196).
 */
typedef struct vx_layout {
    uint32_t struct_size;       /* set to sizeof(vx_layout_t) */
    uint32_t tile_rows;         /* 64 */
    uint32_t tile_group;        /* 16 */
    uint32_t reserved;
    uint64_t rows;
    uint64_t cols;
    uint64_t padded_rows;       /* rows rounded up to a multiple of 64 */
    uint64_t planar_row_bytes;  /* ceil(cols/160) * 32: bytes of one row of the interchange (planar) format */
    uint64_t tile_row_bytes;    /* bytes of one row with the packed tail (pack.rs:222-225) */
    uint64_t device_row_bytes;  /* tile_row_bytes rounded up to 16 */
    uint64_t device_bytes;      /* padded_rows * device_row_bytes */
} vx_layout_t;

/* Replaces quintrit_tiled_layout (quintrit.h:199). rows and cols must be in [1, 2^31] and cols <= VX_MAX_GEMV_COLS. */
int vx_layout(size_t rows, size_t cols, vx_layout_t* out_layout);

/*
 * Host-side conversion of a planar matrix into the device layout (out_capacity >= device_bytes of vx_layout). Checks
 * every byte like vx_matrix_create. Counterpart of quintrit_pack_matrix's tiling step (quintrit.h:222-224) for the
 * device layout; vx_matrix_create performs the same conversion.
 */
int vx_device_layout_pack(const uint8_t* planar, size_t planar_len, size_t rows, size_t cols, uint8_t* out,
                          size_t out_capacity);

/* ---- matrix handles (weights resident in HBM) ------------------------------------------------------------------------ */

typedef struct vx_matrix vx_matrix_t;

/*
 * Uploads a planar velurex matrix (planar_len >= rows * planar_row_bytes) to the current HIP device and returns an owned
 * handle. Every byte is checked: a byte outside the 243 velurex values gives VX_ERR_INVALID_VALUE. weight_scale is the
 * per-tensor scale alpha of TernaryGemvLayer::weight_scale (layer.rs:86). Stands in for the construction of a
 * QuintritLutAVX512Layer (layer.rs:192-203) plus the upload the GPU path does (quintrit-runtime/src/gpu.rs:183-260).
 */
int vx_matrix_create(const uint8_t* planar, size_t planar_len, size_t rows, size_t cols, float weight_scale,
                     vx_matrix_t** out_matrix);
/*
 * As vx_matrix_create, with the planar bytes already in device memory (planar_dev on the current device). The layout
 * transform and the byte check run on the GPU; the call returns when the handle is ready. The planar buffer is not
 * kept. Counterpart of the upload of planar weights in the reference's GPU path (quintrit-runtime/src/gpu.rs:120-138).
 */
int vx_matrix_create_dev(const uint8_t* planar_dev, size_t planar_len, size_t rows, size_t cols, float weight_scale,
                         vx_matrix_t** out_matrix);
/* Frees a handle (NULL is a no-op). */
int vx_matrix_free(vx_matrix_t* matrix);
/* TernaryGemvLayer::shape (layer.rs:83). */
int vx_matrix_shape(const vx_matrix_t* matrix, size_t* out_rows, size_t* out_cols);
/* TernaryGemvLayer::memory_bytes (layer.rs:80): bytes of the weights in device memory. */
int vx_matrix_memory_bytes(const vx_matrix_t* matrix, size_t* out_bytes);
/* TernaryGemvLayer::weight_scale (layer.rs:86). */
int vx_matrix_weight_scale(const vx_matrix_t* matrix, float* out_scale);
/* Device address of the weights in the layout of vx_layout (for callers that fuse their own kernels). */
int vx_matrix_device_weights(const vx_matrix_t* matrix, const void** out_ptr);

/* ---- GEMV ------------------------------------------------------------------------------------------------------------ */

/*
 * Integer GEMV on device memory: out[i] = sum_j W[i][j] * acts[j] for i < rows, exact for the whole int8 range.
 * acts_len >= cols, out_capacity >= rows. Enqueued on `stream`. Device counterpart of quintrit_gemv_i32
 * (quintrit.h:208-210). The device calls on one matrix (this, vx_gemv_f32_dev and the staged forms) share its staging
 * buffer and K-slice sums: calls on one matrix on different streams must be ordered by the caller (vx_layer_forward
 * takes the matrix's lock itself).
 */
int vx_gemv_i32_dev(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, int32_t* out, size_t out_capacity,
                    void* stream);

/*
 * Dequantised GEMV on device memory with the layers' epilogue (layer.rs:246-253): post = weight_scale / act_scale
 * (one fp32 division), out[i] = float(acc[i]) * post; act_scale <= 0 (or NaN) gives zeros.
 */
int vx_gemv_f32_dev(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, float act_scale, float* out,
                    size_t out_capacity, void* stream);

/*
 * Staged activations: the GEMV kernels read the activations of each device byte-column c (the five activations
 * column_activation_index(cols, c, p), p = 0..4, of quintrit-core/src/pack.rs:230-237) as two dwords of 4-bit fields:
 * the low nibbles stored as (x & 15) ^ 8, i.e. the signed value (x & 15) - 8, and the high nibbles x >> 4 (signed), so
 * that x = 16 hi + lo (lut.rs:380-388 splits the same way); activations past the end of the row and in padding columns
 * are zero. A 64-byte header of 16 int32 adds up to the sum of all activations (one part per staging workgroup).
 * vx_staged_bytes(cols) = 64 + 8 * device_row_bytes.
 * One staged vector serves every matrix with the same cols (Q, K and V share one input, gate and up another). The
 * reference stages its GPU inputs the same way, one permuted entry per byte-column (quintrit-cuda/src/pack.rs:75-85).
 */
int vx_staged_bytes(size_t cols, size_t* out_bytes);
int vx_stage_acts_dev(const int8_t* acts, size_t acts_len, size_t cols, void* staged, size_t staged_capacity,
                      void* stream);
/* GEMVs on staged activations (staged by vx_stage_acts_dev for the matrix's cols); same results as the _dev calls. */
int vx_gemv_staged_i32_dev(const vx_matrix_t* matrix, const void* staged, size_t staged_len, int32_t* out,
                           size_t out_capacity, void* stream);
int vx_gemv_staged_f32_dev(const vx_matrix_t* matrix, const void* staged, size_t staged_len, float act_scale, float* out,
                           size_t out_capacity, void* stream);

/*
 * Compact activation tables on device memory: the GPU form of build_activation_lut_wide_avx512_into /
 * build_compact_wide_impl (quintrit-core/src/simd/avx512.rs:1178-1247), byte for byte. Per device byte-column c and
 * part (lo, then hi) one 64-byte table of int8 sums: entry s < 9 is t3 a3 + t4 a4 for the 2-trit group U = s, entry
 * 9 + L is t0 a0 + t1 a1 + t2 a2 for the 3-trit group L < 27, the rest is zero, where a_p is the lo or hi part
 * (lut.rs:380-388: lo = ((x + 8) & 15) - 8, hi = (x - lo) >> 4) of activation column_activation_index(cols, c, p). The
 * lo tables of all tile_row_bytes(cols) columns come first, then the hi tables: vx_compact_lut_bytes(cols) =
 * 2 * 64 * tile_row_bytes(cols). `lut` must be 16-byte aligned. One table set serves every matrix with the same cols.
 */
int vx_compact_lut_bytes(size_t cols, size_t* out_bytes);
int vx_compact_lut_dev(const int8_t* acts, size_t acts_len, size_t cols, int8_t* lut, size_t lut_capacity, void* stream);
/*
 * GEMVs through the compact tables: each weight byte is split without a division into U = floor(B / 28) and
 * L = B - 28 U and looked up at U and 9 + L (decode_compact, avx512.rs:1256-1292; the row loop of compact_multi_block,
 * avx512.rs:1526-1604). Same results as vx_gemv_staged_i32_dev / vx_gemv_staged_f32_dev on the same activations; the
 * digit-table kernel of those calls is the faster decode on this GPU and the one the plans and the decoder use.
 */
int vx_gemv_lut_i32_dev(const vx_matrix_t* matrix, const int8_t* lut, size_t lut_len, int32_t* out, size_t out_capacity,
                        void* stream);
int vx_gemv_lut_f32_dev(const vx_matrix_t* matrix, const int8_t* lut, size_t lut_len, float act_scale, float* out,
                        size_t out_capacity, void* stream);

/*
 * TernaryGemvLayer::forward (layer.rs:74) on host memory: acts (acts_len >= cols) and out (out_capacity >= rows) are
 * host buffers; the call returns when out holds y = alpha * beta * (W x) with the epilogue of vx_gemv_f32_dev. The
 * matrix keeps a pinned host buffer and a stream for these calls (made at the first call); calls on one matrix are
 * serialised by its lock, and device calls on the same matrix still in flight on other streams must be waited for
 * by the caller first.
 */
int vx_layer_forward(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, float act_scale, float* out,
                     size_t out_capacity);

/*
 * One-shot host GEMVs with the argument order of quintrit_gemv_i32 / quintrit_gemv_f32 (quintrit.h:208-218), for the
 * planar layout: the weights are uploaded, multiplied and freed in the call. quintrit_gemv_f32's out = scale * acc.
 */
int vx_gemv_planar_i32(const uint8_t* weights, size_t weights_len, size_t rows, size_t cols, const int8_t* acts,
                       size_t acts_len, int32_t* out, size_t out_capacity);
int vx_gemv_planar_f32(const uint8_t* weights, size_t weights_len, size_t rows, size_t cols, const int8_t* acts,
                       size_t acts_len, float scale, float* out, size_t out_capacity);

/* ---- batched GEMV plans --------------------------------------------------------------------------------------------- */

/*
 * One GEMV of a plan. out_f32 = 0: out receives the int32 accumulators. out_f32 = 1: out receives
 * float(acc) * (weight_scale / *act_scale_dev), the division done once per job in fp32, and zeros when the scale is not
 * > 0 (the epilogue of layer.rs:246-253); the scale is read from device memory when the plan runs, so a producer kernel
 * on the same stream can write it.
 */
typedef struct vx_gemv_job {
    uint32_t struct_size;        /* sizeof(vx_gemv_job_t) */
    int32_t out_f32;
    const vx_matrix_t* matrix;
    const void* staged;          /* device; staged by vx_stage_acts_dev for the matrix's cols */
    size_t staged_len;
    const float* act_scale_dev;  /* device; read when out_f32 = 1 */
    void* out;                   /* device; rows values */
    size_t out_capacity;
    /* device, optional (NULL, or a struct_size that ends before this field): cols int8 activations that each run
     * stages into `staged` first, every distinct (acts, staged) pair once, all of them in one launch before the
     * GEMVs (velurex plans only; jobs that share `staged` must then share `acts`) */
    const int8_t* acts;
} vx_gemv_job_t;

typedef struct vx_plan vx_plan_t;

/*
 * Builds a plan of n_jobs GEMVs (1..65535) that run as one persistent launch (plus one launch that adds the K-slice
 * partial sums of long rows). The pointers of the jobs are fixed in the plan; their contents may change between runs.
 * The plan owns its job table and partial-sum workspace, so a run allocates nothing and can be captured in a HIP graph.
 * The reference runs the projections of a layer concurrently on its thread pool (quintrit-runtime/src/layer.rs:657-716,
 * forward_linear_pair/triple) and the projections of a token as one CUDA graph (quintrit-runtime/src/gpu.rs:389-493);
 * a plan is the single-launch form of both.
 */
int vx_plan_create(const vx_gemv_job_t* jobs, size_t n_jobs, vx_plan_t** out_plan);
/*
 * The same plan through the compact tables (vx_gemv_lut_i32_dev): each job's `staged` is the table set of its
 * matrix's cols (vx_compact_lut_dev, staged_len >= vx_compact_lut_bytes(cols), 16-byte aligned). Run, count and free
 * it with the calls below.
 */
int vx_lut_plan_create(const vx_gemv_job_t* jobs, size_t n_jobs, vx_plan_t** out_plan);
/* Enqueues the plan on `stream`. Runs of one plan must not overlap (they share the partial-sum workspace). */
int vx_plan_run(const vx_plan_t* plan, void* stream);
/* Number of work items (tile group x K slice) of the plan. */
int vx_plan_work_items(const vx_plan_t* plan, uint32_t* out_items);
/* Frees a plan (NULL is a no-op); waits for the device first. */
int vx_plan_free(vx_plan_t* plan);

/* ---- batched (multi-token) GEMM ---------------------------------------------------------------------------------- */

/* Largest token count of one GEMM call. */
#define VX_MAX_GEMM_TOKENS 65536

/*
 * Y[t][i] = sum_j W[i][j] * X[t][j] for t < m tokens, exact int32: the same numbers as m calls of vx_gemv_i32_dev, on
 * the matrix cores (v_mfma_i32_32x32x32_i8). x: m rows of ldx >= cols int8 (device); y: m rows of ldy >= rows int32
 * (device); workspace: device memory of vx_gemm_workspace_bytes(matrix, m) bytes, 256-byte aligned, owned by the
 * caller (the call allocates nothing, so it can be captured in a HIP graph; concurrent calls need distinct
 * workspaces). The reference has no multi-token kernel: its prefill calls the GEMV once per token
 * (quintrit-runtime/src/engine.rs:625-631), which defines the result.
 */
int vx_gemm_workspace_bytes(const vx_matrix_t* matrix, size_t m, size_t* out_bytes);
int vx_gemm_i32_dev(const vx_matrix_t* matrix, const int8_t* x, size_t m, size_t ldx, int32_t* y, size_t ldy,
                    void* workspace, size_t workspace_len, void* stream);

/*
 * vx_gemm_i32_dev without the workspace argument: the call allocates nothing (no hipMalloc, no library allocation).
 * It has no counterpart in the reference; it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). The workspace is a library-owned array of
 * VX_GEMM_NOALLOC_SCRATCH_BYTES per GPU, held from the first call on that GPU until the process ends; a call whose
 * workspace (vx_gemm_workspace_bytes) would exceed it returns VX_ERR_INVALID_SHAPE. Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (two streams, two threads) race and must be ordered by the caller.
 * Results are those of vx_gemm_i32_dev, bit for bit.
 */
#define VX_GEMM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int vx_gemm_i32_noalloc_dev(const vx_matrix_t* matrix, const int8_t* x, size_t m, size_t ldx, int32_t* y, size_t ldy,
                            void* stream);

/* ---- block-scaled (Q2_0) GEMV -------------------------------------------------------------------------------------- */

/*
 * Q2_0 weights against Q8_0 activations (quintrit-core/src/block_scaled.rs; llama.cpp's ggml_vec_dot_q2_0_q8_0):
 * ternary weights in the planar velurex layout plus one scale per 64 weights of a row (here fp16, stored beside the
 * trits on the device; the reference keeps them as f32: each fp16 is widened exactly), int8 activations with one fp32
 * scale per 32 values. out[r] is bit-identical to the reference's dot_row_scalar (block_scaled.rs:175-202): the eight
 * lane sums of every 32-value block s are accumulated as fma(w_scale[s/2] * a_scale[s], lane, acc[(s/2) & 1][lane])
 * in increasing s, then reduced ((l0+l4) + (l2+l6)) + ((l1+l5) + (l3+l7)).
 * cols must be a multiple of 64 and at most 12288.
 */
int vx_q2_matrix_create(const uint8_t* planar, size_t planar_len, const uint16_t* scales_f16, size_t n_scales,
                        size_t rows, size_t cols, vx_matrix_t** out_matrix);
/* acts: cols int8 (device, 4-byte aligned); act_scales: cols/32 fp32 (device); out: rows fp32 (device). */
int vx_q2_gemv_f32_dev(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, const float* act_scales,
                       size_t n_act_scales, float* out, size_t out_capacity, void* stream);
/* The exact integer part: out[(r * (cols/32) + s) * 8 + j] = sum_{k<4} t[r][32s + 4j + k] * acts[32s + 4j + k]. */
int vx_q2_lane_sums_dev(const vx_matrix_t* matrix, const int8_t* acts, size_t acts_len, int32_t* out,
                        size_t out_capacity, void* stream);

typedef struct vx_q2_job {
    uint32_t struct_size;        /* sizeof(vx_q2_job_t) */
    uint32_t reserved;
    const vx_matrix_t* matrix;   /* created by vx_q2_matrix_create */
    const int8_t* acts;          /* device */
    size_t acts_len;
    const float* act_scales;     /* device */
    size_t n_act_scales;
    float* out;                  /* device */
    size_t out_capacity;
} vx_q2_job_t;
/* A plan of Q2_0 GEMVs, run with vx_plan_run and freed with vx_plan_free like the velurex plans. */
int vx_q2_plan_create(const vx_q2_job_t* jobs, size_t n_jobs, vx_plan_t** out_plan);

/* ---- decode token loop ------------------------------------------------------------------------------------------------
 * A ternary decoder of the BitNet-b1.58 / Falcon3 families on one GPU, step for step the reference's CPU token loop
 * (QuintritModel::forward_token_with_scratchpad, quintrit-runtime/src/model.rs:282-377, with
 * AttentionBlock::forward_with_scratchpad, attention.rs:115-260, and the BitnetCpp numerics: RMSNorm with an f64 sum,
 * per-token absmax int8, velurex projections with the fp32 epilogue, RoPE (NEOX or Normal), an F16 KV cache,
 * FP16-accumulator attention with the 4-chunk split, optional sub-norms, ReLU^2 or SwiGLU (ggml's vector expf), a
 * bf16 or f16 head, tied or not, greedy argmax), so that logits and tokens are bit-identical to it. One step is one HIP
 * graph of 1 + 5 per layer kernels: per layer the q/k/v, o, gate/up and down projection stages (each computing its
 * own input: embedding or residual add or gating, RMSNorm, int8 quantization) and attention (RoPE, KV append), then
 * the final norm, head and argmax in one kernel, with the position and the token kept on the device (the reference's
 * CUDA decode graph does the same, quintrit-runtime/src/gpu.rs:459-493).
 * Supported: head_dim 32, 64, 128 or 256, max_ctx <= 8192, hidden a multiple of 32 up to 8192 (4480 with SiLU),
 * n_heads * head_dim <= 8192, ffn a multiple of 4 up to 8192 (24576 with SiLU and no sub-norms). */
typedef struct vx_decoder vx_decoder_t;

typedef struct vx_decoder_config {
    uint32_t struct_size; /* sizeof(vx_decoder_config_t); a size that ends at rope_theta leaves the switches 0 */
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx;
    float rms_eps, rope_theta;
    /* Architecture switches (ModelConfig, config.rs:155-227); all 0 is ModelConfig::bitnet_2b_default with a bf16
     * tied head, the Falcon3 defaults are VX_ACT_SILU, VX_ROPE_NORMAL, no_sub_norm 1, emb_f16 1, untied 1. */
    uint32_t act;         /* VX_ACT_RELU2: relu2(gate) * up; VX_ACT_SILU: swiglu(gate, up) (model.rs:155-170) */
    uint32_t rope_mode;   /* VX_ROPE_NEOX or VX_ROPE_NORMAL (ops.rs:199-221) */
    uint32_t no_sub_norm; /* 1: no attention / FFN sub-norms (has_sub_norm = false) */
    uint32_t emb_f16;     /* 0: bf16 embedding and head (ggml_vec_dot_bf16); 1: f16 (ggml_vec_dot_f16, model.rs:347-373) */
    uint32_t untied;      /* 1: a head of its own (lm_head_f16, vx_decoder_set_head); 0: the embedding is the head */
} vx_decoder_config_t;

enum { VX_ACT_RELU2 = 0, VX_ACT_SILU = 1 };
enum { VX_ROPE_NEOX = 0, VX_ROPE_NORMAL = 1 };

/* Projection kinds (vx_decoder_set_projection) and norm kinds (vx_decoder_set_norm). */
enum {
    VX_PROJ_Q = 0, VX_PROJ_K = 1, VX_PROJ_V = 2, VX_PROJ_O = 3, VX_PROJ_GATE = 4, VX_PROJ_UP = 5, VX_PROJ_DOWN = 6
};
enum { VX_NORM_ATTN = 0, VX_NORM_ATTN_SUB = 1, VX_NORM_FFN = 2, VX_NORM_FFN_SUB = 3 };

/* ModelConfig (quintrit-runtime/src/config.rs:155-227) of the model; allocates the KV cache and work buffers. */
int vx_decoder_create(const vx_decoder_config_t* config, vx_decoder_t** out_decoder);
/* A planar velurex matrix (host memory) with its per-tensor scale: Q/K/V rows n_heads*head_dim or n_kv_heads*head_dim,
 * cols hidden; O hidden x n_heads*head_dim; gate/up ffn x hidden; down hidden x ffn (the reference's BitLinear). */
int vx_decoder_set_projection(vx_decoder_t* decoder, uint32_t layer, uint32_t kind, const uint8_t* planar,
                              size_t planar_len, float weight_scale);
/* The same from a matrix handle (vx_matrix_create(_dev), vx_gguf_upload_matrix, vx_matrix_create_ggml_dev) of the
 * projection's shape on the decoder's device; its weight scale is the projection's. On success the decoder owns the
 * matrix (it is freed with the decoder or when replaced) and the caller must not use or free it; on failure the caller
 * keeps it. The upload of the reference's GPU loader (quintrit-runtime/src/gpu.rs:201-225) without a host copy. */
int vx_decoder_adopt_projection(vx_decoder_t* decoder, uint32_t layer, uint32_t kind, vx_matrix_t* matrix);
/* RMSNorm weights (host f32). layer == n_layers with kind VX_NORM_ATTN sets the output norm; the sub-norm kinds are
 * rejected when no_sub_norm is set. */
int vx_decoder_set_norm(vx_decoder_t* decoder, uint32_t layer, uint32_t kind, const float* weights, size_t n);
/* The embedding (also the head when tied), vocab x hidden (host): bf16 when emb_f16 is 0, else f16. */
int vx_decoder_set_embedding_bf16(vx_decoder_t* decoder, const uint16_t* embedding, size_t n);
int vx_decoder_set_embedding_f16(vx_decoder_t* decoder, const uint16_t* embedding, size_t n);
/* The untied head (untied = 1), vocab x hidden in the embedding's type (host). */
int vx_decoder_set_head(vx_decoder_t* decoder, const uint16_t* head, size_t n);
/* One token at position pos (forward_token): KV entries 0..pos-1 must come from earlier steps. logits (host, may be
 * NULL) receives vocab values; out_next (may be NULL) the greedy token. */
int vx_decoder_step(vx_decoder_t* decoder, uint32_t token, uint32_t pos, float* logits, size_t logits_capacity,
                    uint32_t* out_next);
/* Greedy generation from position 0 (engine.rs:590-686 with the greedy sampler): the prompt is ingested by prefill
 * passes (vx_decoder_prefill), then one decode step per further token; n_new tokens into out_tokens (host).
 * n_prompt >= 1 and n_prompt + n_new - 1 <= max_ctx. The tokens are those of feeding the prompt one token at a time. */
int vx_decoder_generate(vx_decoder_t* decoder, const uint32_t* prompt, size_t n_prompt, size_t n_new,
                        uint32_t* out_tokens, size_t out_capacity);
/* The same with the prompt fed one decode step per token, as the reference's loop does (engine.rs:627-630). */
int vx_decoder_generate_stepwise(vx_decoder_t* decoder, const uint32_t* prompt, size_t n_prompt, size_t n_new,
                                 uint32_t* out_tokens, size_t out_capacity);
/* Prompt ingestion (engine.rs:625-631 runs forward_token for each prompt position): the n tokens at positions
 * pos0 .. pos0 + n - 1 (positions below pos0 must already be in the KV cache) pass each layer together, their
 * projections as batched GEMMs on the matrix cores (vx_gemm_i32_dev), in chunks of up to 512 tokens. The KV cache, the
 * logits of the last position (logits, may be NULL) and its greedy token (out_next, may be NULL) are bit-identical to n
 * calls of vx_decoder_step; the next step continues at pos0 + n. VX_ERR_CONTEXT_OVERFLOW beyond max_ctx. */
int vx_decoder_prefill(vx_decoder_t* decoder, const uint32_t* tokens, size_t n, uint32_t pos0, float* logits,
                       size_t logits_capacity, uint32_t* out_next);
/* The cached f16 key and value of (layer, pos, kv_head): head_dim values each into k and v (host, either may be NULL;
 * n >= head_dim). KVCache::get_key / get_val (quintrit-runtime/src/kv_cache.rs:142-155). */
int vx_decoder_kv_get(const vx_decoder_t* decoder, uint32_t layer, uint32_t pos, uint32_t kv_head, uint16_t* k,
                      uint16_t* v, size_t n);
/* Device bytes held by the decoder (weights, KV cache, work buffers). */
int vx_decoder_memory_bytes(const vx_decoder_t* decoder, size_t* out_bytes);
/* Diagnostic, no counterpart in the reference: how many times an RMSNorm on the decoder's GPU has taken the
 * reference's sequential f64 order (rms_norm, quintrit-runtime/src/ops.rs:43-57) because its tree-summed mean lay
 * within the error bound of an f32 rounding boundary. One count per workgroup that computed such a norm, summed over
 * every decoder of the process on that GPU since the library was loaded. */
int vx_decoder_norm_fallbacks(const vx_decoder_t* decoder, uint64_t* out_count);
/* The decoder's configuration (the shape part of quintrit_model_info, quintrit.h:323-340); out_config->struct_size must be
 * sizeof(vx_decoder_config_t). */
int vx_decoder_config(const vx_decoder_t* decoder, vx_decoder_config_t* out_config);
int vx_decoder_free(vx_decoder_t* decoder);

/* ---- GGUF files ------------------------------------------------------------------------------------------------------
 * The format level of the reference's C API (quintrit-c/include/quintrit.h:221-308, over quintrit-format/src/gguf.rs):
 * an open, memory-mapped GGUF v2/v3 file, checked like the reference's reader (every count and length bounded by the
 * file, offsets aligned and inside the data section, payloads not overlapping; violations give VX_ERR_FORMAT). Names
 * and payload pointers stay valid until vx_gguf_close. Ternary tensors (I2_S, TQ1_0, TQ2_0) convert to the planar
 * velurex layout on the host, or upload in their GGUF size and convert in HBM into a GEMV matrix. */
typedef struct vx_gguf vx_gguf_t;

#define VX_MAX_DIMS 8
#define VX_GGML_F32    0
#define VX_GGML_F16    1
#define VX_GGML_Q8_0   8
#define VX_GGML_BF16   30
#define VX_GGML_TQ1_0  34
#define VX_GGML_TQ2_0  35
#define VX_GGML_I2_S   36
#define VX_GGML_Q2_0   42

typedef struct vx_gguf_info {
    uint32_t struct_size;     /* sizeof(vx_gguf_info_t) */
    uint32_t version;         /* 2 or 3 */
    uint64_t tensor_count;
    uint64_t metadata_count;
    uint64_t data_offset;     /* absolute file offset of the tensor data section */
} vx_gguf_info_t;

typedef struct vx_tensor_info {
    uint32_t    struct_size;  /* sizeof(vx_tensor_info_t) */
    int32_t     ggml_type;    /* VX_GGML_* */
    uint32_t    n_dims;
    int32_t     is_ternary;   /* 1 for I2_S, TQ1_0 and TQ2_0, which convert to velurex weights */
    uint64_t    shape[VX_MAX_DIMS]; /* as stored: shape[0] is the innermost dimension (a matrix is [cols, rows]) */
    uint64_t    num_elements;
    uint64_t    offset;       /* offset inside the data section */
    uint64_t    data_bytes;   /* payload bytes; 0 for types whose layout is not known here */
    const char* name;         /* valid until vx_gguf_close */
    const char* type_name;    /* "F32", "F16", "Q8_0", "BF16", "TQ1_0", "TQ2_0", "I2_S", "Q2_0" or "UNKNOWN" */
    uint32_t    block_size;   /* Q2_0: weights per block (64 or 128, read from the layout, gguf.rs:460-508); else 0 */
} vx_tensor_info_t;

/* quintrit_gguf_open / _close / _info (quintrit.h:260-269). A file that cannot be opened gives VX_ERR_IO. */
int vx_gguf_open(const char* path, vx_gguf_t** out_gguf);
int vx_gguf_close(vx_gguf_t* gguf);
int vx_gguf_info(const vx_gguf_t* gguf, vx_gguf_info_t* out_info);
/* Tensor `index` in [0, tensor_count), in file order; or by name (VX_ERR_NOT_FOUND). (quintrit.h:271-275) */
int vx_gguf_tensor_at(const vx_gguf_t* gguf, size_t index, vx_tensor_info_t* out_info);
int vx_gguf_tensor_find(const vx_gguf_t* gguf, const char* name, vx_tensor_info_t* out_info);
/* Metadata (quintrit.h:277-285): a string (*out_len without the NUL; BUFFER_TOO_SMALL if capacity <= *out_len), an
 * unsigned or non-negative integer, a float (f32 widened or f64), and every entry as one JSON object
 * {"key": {"type": t, ["array_type": a,] "value": v}} with exact floats (f32 widened to double, 17 digits). */
int vx_gguf_metadata_string(const vx_gguf_t* gguf, const char* key, char* buffer, size_t capacity, size_t* out_len);
int vx_gguf_metadata_u64(const vx_gguf_t* gguf, const char* key, uint64_t* out_value);
int vx_gguf_metadata_f64(const vx_gguf_t* gguf, const char* key, double* out_value);
int vx_gguf_metadata_json(const vx_gguf_t* gguf, char* buffer, size_t capacity, size_t* out_len);
/* The raw payload inside the mapping (quintrit.h:287-289); VX_ERR_UNSUPPORTED for a type of unknown layout. */
int vx_gguf_tensor_data(const vx_gguf_t* gguf, const char* name, const uint8_t** out_data, size_t* out_len);
/* The per-tensor weight scale (gguf.rs:342-360, transcoder.rs:224-236): the f32 after an I2_S payload, the common
 * block scale of TQ1_0 / TQ2_0 (VX_ERR_FORMAT if the blocks differ), 1 for other types. */
int vx_gguf_tensor_scale(const vx_gguf_t* gguf, const char* name, float* out_scale);
/* A ternary 2-D tensor in the planar velurex layout in the caller's buffer (transcoder.rs:154-205); out_rows, out_cols
 * and out_scale may be NULL. The counterpart of quintrit_gguf_convert_tensor for the GPU's layout. */
int vx_gguf_convert_planar(const vx_gguf_t* gguf, const char* name, uint8_t* out, size_t out_capacity, size_t* out_rows,
                           size_t* out_cols, float* out_scale);
/* The same for a raw payload in host memory: rows x cols weights of ggml_type (I2_S: cols a multiple of 128; TQ1_0 and
 * TQ2_0: rows * cols a multiple of 256). */
int vx_ggml_to_planar(int32_t ggml_type, const uint8_t* data, size_t len, size_t rows, size_t cols, uint8_t* out,
                      size_t out_capacity);
/* A GEMV matrix from a ternary tensor: its payload crosses to the device in its GGUF size and is converted there, with
 * the tensor's weight scale (transcoder.rs:211-249 for the GPU). */
int vx_gguf_upload_matrix(const vx_gguf_t* gguf, const char* name, vx_matrix_t** out_matrix);
/* The same from a raw payload already in device memory. */
int vx_matrix_create_ggml_dev(int32_t ggml_type, const uint8_t* data_dev, size_t len, size_t rows, size_t cols,
                              float weight_scale, vx_matrix_t** out_matrix);

/* A Q2_0 tensor (block size 64 or 128, as detected) as the block-scaled layer's inputs (BlockScaledLayer::from_q2_0,
 * quintrit-runtime/src/layer.rs:453-470, over decode_q2_0_packed, quintrit-format/src/decoders/q2_0.rs:58-155): planar
 * velurex bytes (rows * ceil(cols/160) * 32) and one f16 scale per 64 weights of a row (rows * cols / 64; a 128-weight
 * block's scale appears twice). A code 3 gives VX_ERR_FORMAT naming the first such weight. out_rows / out_cols may be
 * NULL; they are set before a VX_ERR_BUFFER_TOO_SMALL. */
int vx_gguf_convert_q2_0(const vx_gguf_t* gguf, const char* name, uint8_t* planar, size_t planar_capacity,
                         uint16_t* scales_f16, size_t scales_capacity, size_t* out_rows, size_t* out_cols);
/* The same tensor as a Q2_0 GEMV matrix (vx_q2_matrix_create's limits apply: cols a multiple of 64, at most 12288). */
int vx_gguf_upload_q2_matrix(const vx_gguf_t* gguf, const char* name, vx_matrix_t** out_matrix);

/* quintrit_gpu_options_t (quintrit.h:515-520). */
typedef struct vx_gpu_options {
    uint32_t struct_size;    /* sizeof(vx_gpu_options_t) */
    uint32_t device_index;   /* GPU to use, below hipGetDeviceCount */
    uint32_t context_length; /* largest context in tokens; 0 = min(4096, the model's maximum); at most 7936 */
    uint32_t flags;          /* 0 */
} vx_gpu_options_t;

/* Replaces quintrit_model_open_gpu (quintrit.h:527; GpuModel::load, quintrit-runtime/src/gpu.rs:149-260): a GGUF model
 * as a decoder on the GPU. The configuration comes from the metadata as ModelConfig::from_gguf reads it (config.rs:257-440;
 * BitNet: ReLU^2, sub-norms, NEOX RoPE; Falcon3 / LLaMA: SiLU, Normal RoPE); the ternary projections (I2_S, TQ1_0,
 * TQ2_0) are uploaded in their GGUF size and converted in HBM (as vx_gguf_upload_matrix); the embedding is the F16 token_embd.weight,
 * the head output.weight (F16) or the embedding. The context is rounded down to a multiple of 256 as gpu.rs:141-146
 * does. Files the reference rejects give VX_ERR_MODEL (missing or misshapen tensors, no tokenizer, absurd dimensions);
 * models it runs elsewhere than this decoder give VX_ERR_UNSUPPORTED (no I2_S tensor, Q2_0, Qwen3 / hybrid / MoE,
 * partial or scaled RoPE, head_dim other than 32 / 64 / 128 / 256). options may be NULL (device 0, default context). On failure
 * *out_decoder is NULL. The handle is used and freed like one from vx_decoder_create. */
int vx_decoder_open_gguf(const char* path, const vx_gpu_options_t* options, vx_decoder_t** out_decoder);

/* glibc's expf (the reference's f32::exp) evaluated on the device, as used by the attention softmax: n values. */
int vx_expf_dev(const float* x, size_t n, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
