// velurex_hip.hpp - header-only C++17 host interface over the C ABI of libvelurex_hip (velurex_hip.h).
//
// It mirrors, in C++, the two host interfaces of the reference that this library stands in for:
//   - the TernaryGemvLayer trait (rust/crates/quintrit-runtime/src/layer.rs:72-87) as the abstract class
//     velurex_hip::TernaryGemvLayer, with VelurexHipLayer as its GPU implementation (weights resident in HBM); the
//     kernel kinds of TernaryKernelType (layer.rs:13-68) with the one this library adds, VelurexHip;
//   - the kernel level of the reference's C++ wrapper (rust/crates/quintrit-c/include/quintrit.hpp:146-191):
//     version(), check_abi(), layout(), gemv_i32() and gemv_f32() on the planar bytes of quintrit_core::pack;
//   - its GPU model (quintrit::Model::open_gpu, quintrit.hpp:394-430) at the level of token ids: velurex_hip::Decoder,
//     the greedy token loop of the reference's engine (quintrit-runtime/src/engine.rs:590-686) on one GPU.
// Conventions of quintrit.hpp (lines 1-57):
//   - Every failing C call throws velurex_hip::Error, which carries the status code (code(): one of VX_ERR_*, whose
//     values are QUINTRIT_ERR_*) and the library's message (vx_last_error_message, else vx_status_string).
//   - The owning classes are RAII and move-only; their destructors free the handle and never throw.
//   - The helpers allocate their outputs (std::vector).
// forward() requires activations.len() == cols and out.len() == rows, as the trait's implementations assert
// (layer.rs:124,156,211,259); the Rust trait panics on a mismatch, this header throws Error with VX_ERR_INVALID_ARGUMENT.
// Thread safety is the C ABI's: host-pointer calls on one matrix are serialised by the library, so one layer may be
// shared between threads (the trait's Send + Sync).
#ifndef VELUREX_HIP_HPP
#define VELUREX_HIP_HPP

#include "velurex_hip.h"

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace velurex_hip {

/// Thrown when a call of the C ABI fails (quintrit::Error, quintrit.hpp:33-41).
class Error : public std::runtime_error {
public:
    Error(int code, const std::string& message) : std::runtime_error(message), code_(code) {}
    /// One of the VX_ERR_* status codes.
    int code() const noexcept { return code_; }

private:
    int code_;
};

namespace detail {

[[noreturn]] inline void throw_last(int status) {
    const char* msg = vx_last_error_message();
    std::string text = (msg != nullptr && msg[0] != '\0') ? msg : vx_status_string(status);
    throw Error(status, text);
}

/// Throws velurex_hip::Error unless `status` is VX_OK.
inline void check(int status) {
    if (status != VX_OK) throw_last(status);
}

}  // namespace detail

// -------------------------------------------------------------------------------------------------------------------
// Library
// -------------------------------------------------------------------------------------------------------------------

inline std::string version() { return vx_version(); }

/// Throws unless the loaded library has the ABI this header was written for (quintrit.hpp:97-101).
inline void check_abi() {
    if (vx_abi_version() != VX_ABI_VERSION)
        throw Error(VX_ERR_INVALID_ARGUMENT, "libvelurex_hip ABI version differs from the header");
}

/// Usable gfx950 devices (0 without one).
inline int device_count() {
    std::int32_t n = 0;
    detail::check(vx_device_count(&n));
    return static_cast<int>(n);
}

// -------------------------------------------------------------------------------------------------------------------
// Kernel level
// -------------------------------------------------------------------------------------------------------------------

/// The device layout of a rows x cols matrix (quintrit::tiled_layout, quintrit.hpp:146-151).
inline vx_layout_t layout(std::size_t rows, std::size_t cols) {
    vx_layout_t l{};
    l.struct_size = sizeof(l);
    detail::check(vx_layout(rows, cols, &l));
    return l;
}

/// out[i] = sum_j W[i][j] * activations[j], exact, with W the planar bytes of a rows x cols matrix
/// (quintrit::gemv_i32, quintrit.hpp:173-181; the GPU has no thread count).
inline std::vector<std::int32_t> gemv_i32(const std::vector<std::uint8_t>& planar, std::size_t rows, std::size_t cols,
                                          const std::vector<std::int8_t>& activations) {
    std::vector<std::int32_t> out(rows);
    detail::check(vx_gemv_planar_i32(planar.data(), planar.size(), rows, cols, activations.data(), activations.size(),
                                     out.data(), out.size()));
    return out;
}

/// out[i] = scale * sum_j W[i][j] * activations[j] (quintrit::gemv_f32, quintrit.hpp:183-191).
inline std::vector<float> gemv_f32(const std::vector<std::uint8_t>& planar, std::size_t rows, std::size_t cols,
                                   const std::vector<std::int8_t>& activations, float scale = 1.0f) {
    std::vector<float> out(rows);
    detail::check(vx_gemv_planar_f32(planar.data(), planar.size(), rows, cols, activations.data(), activations.size(),
                                     scale, out.data(), out.size()));
    return out;
}

// -------------------------------------------------------------------------------------------------------------------
// Layers
// -------------------------------------------------------------------------------------------------------------------

/// TernaryKernelType (layer.rs:13-32) with the kernel of this library.
enum class TernaryKernelType { QuintritLut, QuintritLutAVX512, QuintritBlockScaled, VelurexHip };

/// TernaryKernelType::as_str (layer.rs:35-45).
inline const char* kernel_name(TernaryKernelType k) {
    switch (k) {
        case TernaryKernelType::QuintritLut: return "QuintritLut";
        case TernaryKernelType::QuintritLutAVX512: return "QuintritLutAVX512";
        case TernaryKernelType::QuintritBlockScaled: return "QuintritBlockScaled";
        case TernaryKernelType::VelurexHip: return "VelurexHip";
    }
    return "unknown";
}

/// TernaryKernelType::activation_quant_levels (layer.rs:51-58): every kernel here is exact over the full int8 range.
inline float activation_quant_levels(TernaryKernelType) { return 127.0f; }

/// TernaryKernelType::bpw (layer.rs:60-67).
inline float bpw(TernaryKernelType k) { return k == TernaryKernelType::QuintritBlockScaled ? 2.1f : 1.6f; }

/// The TernaryGemvLayer trait (layer.rs:72-87): y = alpha * beta * (W x) for int8 activations x.
class TernaryGemvLayer {
public:
    virtual ~TernaryGemvLayer() = default;
    /// out[0 .. rows) = weight_scale() / act_scale * (W activations), or zeros when act_scale is not > 0 (layer.rs:74,
    /// 143-150); n_activations must be cols and n_out rows.
    virtual void forward(const std::int8_t* activations, std::size_t n_activations, float act_scale, float* out,
                         std::size_t n_out) const = 0;
    void forward(const std::vector<std::int8_t>& activations, float act_scale, std::vector<float>& out) const {
        forward(activations.data(), activations.size(), act_scale, out.data(), out.size());
    }
    /// The kernel architecture of the layer (layer.rs:77).
    virtual TernaryKernelType kernel_type() const = 0;
    /// Bytes of the packed weights (layer.rs:80).
    virtual std::size_t memory_bytes() const = 0;
    /// (rows, cols) = (N, K) (layer.rs:83).
    virtual std::pair<std::size_t, std::size_t> shape() const = 0;
    /// The weight scale alpha (layer.rs:86).
    virtual float weight_scale() const = 0;
};

/// A velurex matrix resident in HBM of the current HIP device (vx_matrix_create), as a TernaryGemvLayer. forward() runs
/// on host buffers (vx_layer_forward); the _dev forms take device buffers and a HIP stream (stream-ordered).
class VelurexHipLayer final : public TernaryGemvLayer {
public:
    /// planar: rows * ceil(cols / 160) * 32 bytes of quintrit_core::pack's planar layout (at least that many).
    VelurexHipLayer(const std::uint8_t* planar, std::size_t planar_len, std::size_t rows, std::size_t cols,
                    float weight_scale)
        : rows_(rows), cols_(cols), weight_scale_(weight_scale) {
        detail::check(vx_matrix_create(planar, planar_len, rows, cols, weight_scale, &m_));
    }
    VelurexHipLayer(const std::vector<std::uint8_t>& planar, std::size_t rows, std::size_t cols, float weight_scale)
        : VelurexHipLayer(planar.data(), planar.size(), rows, cols, weight_scale) {}
    ~VelurexHipLayer() override {
        if (m_ != nullptr) (void)vx_matrix_free(m_);
    }
    VelurexHipLayer(const VelurexHipLayer&) = delete;
    VelurexHipLayer& operator=(const VelurexHipLayer&) = delete;
    VelurexHipLayer(VelurexHipLayer&& o) noexcept
        : m_(std::exchange(o.m_, nullptr)), rows_(o.rows_), cols_(o.cols_), weight_scale_(o.weight_scale_) {}
    VelurexHipLayer& operator=(VelurexHipLayer&& o) noexcept {
        if (this != &o) {
            if (m_ != nullptr) (void)vx_matrix_free(m_);
            m_ = std::exchange(o.m_, nullptr);
            rows_ = o.rows_;
            cols_ = o.cols_;
            weight_scale_ = o.weight_scale_;
        }
        return *this;
    }

    using TernaryGemvLayer::forward;
    void forward(const std::int8_t* activations, std::size_t n_activations, float act_scale, float* out,
                 std::size_t n_out) const override {
        if (n_activations != cols_)
            throw Error(VX_ERR_INVALID_ARGUMENT, "forward: " + std::to_string(n_activations) +
                                                     " activations for a matrix of " + std::to_string(cols_) + " columns");
        if (n_out != rows_)
            throw Error(VX_ERR_INVALID_ARGUMENT, "forward: an output of " + std::to_string(n_out) +
                                                     " values for a matrix of " + std::to_string(rows_) + " rows");
        detail::check(vx_layer_forward(handle(), activations, n_activations, act_scale, out, n_out));
    }
    TernaryKernelType kernel_type() const override { return TernaryKernelType::VelurexHip; }
    std::size_t memory_bytes() const override {
        std::size_t n = 0;
        detail::check(vx_matrix_memory_bytes(handle(), &n));
        return n;
    }
    std::pair<std::size_t, std::size_t> shape() const override { return {rows_, cols_}; }
    float weight_scale() const override { return weight_scale_; }

    /// out[0 .. rows) = W acts, exact int32; acts (cols int8) and out in device memory, enqueued on `stream`.
    void gemv_i32_dev(const std::int8_t* acts, std::int32_t* out, void* stream = nullptr) const {
        detail::check(vx_gemv_i32_dev(handle(), acts, cols_, out, rows_, stream));
    }
    /// out[0 .. rows) = float(W acts) * (weight_scale / act_scale) in device memory, enqueued on `stream`.
    void gemv_f32_dev(const std::int8_t* acts, float act_scale, float* out, void* stream = nullptr) const {
        detail::check(vx_gemv_f32_dev(handle(), acts, cols_, act_scale, out, rows_, stream));
    }
    /// The C handle (owned by this object).
    vx_matrix_t* handle() const {
        if (m_ == nullptr) throw Error(VX_ERR_INVALID_HANDLE, "the layer was moved from");
        return m_;
    }
    /// Gives up the handle (the caller then owns it); the layer is left empty.
    vx_matrix_t* release() noexcept { return std::exchange(m_, nullptr); }

private:
    vx_matrix_t* m_ = nullptr;
    std::size_t rows_, cols_;
    float weight_scale_;
};

// -------------------------------------------------------------------------------------------------------------------
// Many projections in one launch, and many tokens per call
// -------------------------------------------------------------------------------------------------------------------

/// One GEMV of a plan on device buffers (vx_gemv_job_t): `acts` (cols int8) staged into `staged` by each run, outputs
/// int32 or, with `act_scale_dev`, float(acc) * (weight_scale / *act_scale_dev) read when the plan runs.
struct PlanJob {
    const VelurexHipLayer* layer;
    const std::int8_t* acts;     // device, cols values
    void* staged;                // device, staged_bytes(cols) bytes (jobs with the same acts may share it)
    void* out;                   // device, rows values
    const float* act_scale_dev;  // device, or null for int32 outputs
};

/// Bytes of one staged activation vector of `cols` columns (vx_staged_bytes).
inline std::size_t staged_bytes(std::size_t cols) {
    std::size_t n = 0;
    detail::check(vx_staged_bytes(cols, &n));
    return n;
}

/// Many GEMVs as one launch per run (vx_plan_*): the single-launch form of the reference's concurrent projections of a
/// layer and of its per-token CUDA graph (layer.rs:657-716, gpu.rs:389-493). Move-only; a run allocates nothing.
class Plan {
public:
    explicit Plan(const std::vector<PlanJob>& jobs) {
        std::vector<vx_gemv_job_t> raw(jobs.size());
        for (std::size_t i = 0; i < jobs.size(); ++i) {
            const auto shape = jobs[i].layer->shape();
            vx_gemv_job_t& j = raw[i];
            j = vx_gemv_job_t{};
            j.struct_size = sizeof(j);
            j.out_f32 = jobs[i].act_scale_dev != nullptr ? 1 : 0;
            j.matrix = jobs[i].layer->handle();
            j.staged = jobs[i].staged;
            j.staged_len = staged_bytes(shape.second);
            j.act_scale_dev = jobs[i].act_scale_dev;
            j.out = jobs[i].out;
            j.out_capacity = shape.first;
            j.acts = jobs[i].acts;
        }
        detail::check(vx_plan_create(raw.data(), raw.size(), &p_));
    }
    ~Plan() {
        if (p_ != nullptr) (void)vx_plan_free(p_);
    }
    Plan(const Plan&) = delete;
    Plan& operator=(const Plan&) = delete;
    Plan(Plan&& o) noexcept : p_(std::exchange(o.p_, nullptr)) {}
    Plan& operator=(Plan&& o) noexcept {
        if (this != &o) {
            if (p_ != nullptr) (void)vx_plan_free(p_);
            p_ = std::exchange(o.p_, nullptr);
        }
        return *this;
    }
    /// Enqueues the plan's GEMVs on `stream` (runs of one plan must not overlap).
    void run(void* stream = nullptr) const { detail::check(vx_plan_run(handle(), stream)); }
    /// Work items (tile group x K slice) of the launch.
    std::uint32_t work_items() const {
        std::uint32_t n = 0;
        detail::check(vx_plan_work_items(handle(), &n));
        return n;
    }
    vx_plan_t* handle() const {
        if (p_ == nullptr) throw Error(VX_ERR_INVALID_HANDLE, "the plan was moved from");
        return p_;
    }

private:
    vx_plan_t* p_ = nullptr;
};

/// Y = X W^T for m tokens on the matrix cores, exact int32 (vx_gemm_i32_dev): x m x ldx int8 and y m x ldy int32 in
/// device memory, `workspace` of gemm_workspace_bytes(layer, m) bytes (256-byte aligned) owned by the caller.
inline std::size_t gemm_workspace_bytes(const VelurexHipLayer& layer, std::size_t m) {
    std::size_t n = 0;
    detail::check(vx_gemm_workspace_bytes(layer.handle(), m, &n));
    return n;
}
inline void gemm_i32_dev(const VelurexHipLayer& layer, const std::int8_t* x, std::size_t m, std::size_t ldx,
                         std::int32_t* y, std::size_t ldy, void* workspace, std::size_t workspace_len,
                         void* stream = nullptr) {
    detail::check(vx_gemm_i32_dev(layer.handle(), x, m, ldx, y, ldy, workspace, workspace_len, stream));
}

// -------------------------------------------------------------------------------------------------------------------
// Decoder (the token loop on the GPU)
// -------------------------------------------------------------------------------------------------------------------

/// A ternary decoder resident on one GPU (vx_decoder_*): the counterpart of quintrit::Model opened on a GPU
/// (quintrit.hpp:394-430, Model::open_gpu) at the level of token ids, with the reference's greedy token loop
/// (quintrit-runtime/src/engine.rs:590-686). Move-only; the destructor frees the decoder and never throws.
class Decoder {
public:
    /// A decoder of the given shape and architecture (ModelConfig, config.rs:155-227) whose weights are set next.
    explicit Decoder(vx_decoder_config_t config) {
        config.struct_size = sizeof(config);
        detail::check(vx_decoder_create(&config, &d_));
    }
    /// A GGUF model on GPU `device` (quintrit::Model::open_gpu); `context` bounds the context (0 = default).
    static Decoder open_gguf(const std::string& path, std::uint32_t device = 0, std::uint32_t context = 0) {
        vx_gpu_options_t o{};
        o.struct_size = sizeof(o);
        o.device_index = device;
        o.context_length = context;
        vx_decoder_t* d = nullptr;
        detail::check(vx_decoder_open_gguf(path.c_str(), &o, &d));
        return Decoder(d);
    }
    ~Decoder() {
        if (d_ != nullptr) (void)vx_decoder_free(d_);
    }
    Decoder(const Decoder&) = delete;
    Decoder& operator=(const Decoder&) = delete;
    Decoder(Decoder&& o) noexcept : d_(std::exchange(o.d_, nullptr)) {}
    Decoder& operator=(Decoder&& o) noexcept {
        if (this != &o) {
            if (d_ != nullptr) (void)vx_decoder_free(d_);
            d_ = std::exchange(o.d_, nullptr);
        }
        return *this;
    }

    /// The configuration (quintrit::Model::info's shape part).
    vx_decoder_config_t config() const {
        vx_decoder_config_t c{};
        c.struct_size = sizeof(c);
        detail::check(vx_decoder_config(handle(), &c));
        return c;
    }
    /// The weights: a projection from planar bytes, or a matrix handed over (on success the decoder owns it).
    void set_projection(std::uint32_t layer, std::uint32_t kind, const std::vector<std::uint8_t>& planar, float weight_scale) {
        detail::check(vx_decoder_set_projection(handle(), layer, kind, planar.data(), planar.size(), weight_scale));
    }
    void adopt_projection(std::uint32_t layer, std::uint32_t kind, VelurexHipLayer&& matrix) {
        detail::check(vx_decoder_adopt_projection(handle(), layer, kind, matrix.handle()));
        (void)matrix.release();
    }
    void set_norm(std::uint32_t layer, std::uint32_t kind, const std::vector<float>& weights) {
        detail::check(vx_decoder_set_norm(handle(), layer, kind, weights.data(), weights.size()));
    }
    void set_embedding_bf16(const std::vector<std::uint16_t>& e) {
        detail::check(vx_decoder_set_embedding_bf16(handle(), e.data(), e.size()));
    }
    void set_embedding_f16(const std::vector<std::uint16_t>& e) {
        detail::check(vx_decoder_set_embedding_f16(handle(), e.data(), e.size()));
    }
    void set_head(const std::vector<std::uint16_t>& h) { detail::check(vx_decoder_set_head(handle(), h.data(), h.size())); }

    /// One token at position `pos` (forward_token); returns the greedy next token, and the logits when asked.
    std::uint32_t step(std::uint32_t token, std::uint32_t pos, std::vector<float>* logits = nullptr) {
        std::uint32_t next = 0;
        if (logits != nullptr) logits->resize(config().vocab);
        detail::check(vx_decoder_step(handle(), token, pos, logits ? logits->data() : nullptr, logits ? logits->size() : 0,
                                      &next));
        return next;
    }
    /// The tokens pos0 .. pos0 + n - 1 in batched passes; the last position's greedy token (and logits when asked).
    std::uint32_t prefill(const std::vector<std::uint32_t>& tokens, std::uint32_t pos0, std::vector<float>* logits = nullptr) {
        std::uint32_t next = 0;
        if (logits != nullptr) logits->resize(config().vocab);
        detail::check(vx_decoder_prefill(handle(), tokens.data(), tokens.size(), pos0, logits ? logits->data() : nullptr,
                                         logits ? logits->size() : 0, &next));
        return next;
    }
    /// Greedy generation from position 0 (engine.rs:590-686): n_new tokens; `stepwise` feeds the prompt one decode
    /// step per token, as the reference's loop does, instead of prefill passes (the tokens are the same).
    std::vector<std::uint32_t> generate(const std::vector<std::uint32_t>& prompt, std::size_t n_new, bool stepwise = false) {
        std::vector<std::uint32_t> out(n_new);
        detail::check(stepwise ? vx_decoder_generate_stepwise(handle(), prompt.data(), prompt.size(), n_new, out.data(), out.size())
                               : vx_decoder_generate(handle(), prompt.data(), prompt.size(), n_new, out.data(), out.size()));
        return out;
    }
    /// The cached f16 key and value of (layer, pos, kv_head) (KVCache::get_key / get_val, kv_cache.rs:142-155).
    std::pair<std::vector<std::uint16_t>, std::vector<std::uint16_t>> kv(std::uint32_t layer, std::uint32_t pos,
                                                                        std::uint32_t kv_head) const {
        const std::size_t hd = config().head_dim;
        std::vector<std::uint16_t> k(hd), v(hd);
        detail::check(vx_decoder_kv_get(handle(), layer, pos, kv_head, k.data(), v.data(), hd));
        return {std::move(k), std::move(v)};
    }
    /// Device bytes held (weights, KV cache, work buffers).
    std::size_t memory_bytes() const {
        std::size_t n = 0;
        detail::check(vx_decoder_memory_bytes(handle(), &n));
        return n;
    }
    vx_decoder_t* handle() const {
        if (d_ == nullptr) throw Error(VX_ERR_INVALID_HANDLE, "the decoder was moved from");
        return d_;
    }

private:
    explicit Decoder(vx_decoder_t* d) : d_(d) {}
    vx_decoder_t* d_ = nullptr;
};

}  // namespace velurex_hip

#endif  // VELUREX_HIP_HPP
