// C++ test of velurex_hip.hpp (the TernaryGemvLayer interface and the kernel-level GEMV over the C ABI), in the manner
// of the reference's C++ wrapper test (rust/crates/quintrit-c/tests/cpp/test_kernel.cpp): GEMVs against a brute-force
// product at the shapes of that test and of quintrit-c/tests/ffi_kernel.rs:36-49,195-265, errors as exceptions with
// their status codes, and the move-only owning classes; a plan of GEMVs and the batched GEMM on device buffers; the
// decoder through the wrapper (prefill against steps, greedy generation with and without prefill passes, its errors).
// Exit code 0 means success.
//
//   test_layer          everything (needs a gfx950 device)
//   test_layer --cpu    only what needs no device: the ABI, the layout, argument errors, the type traits
#include "velurex_hip.hpp"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <iostream>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

namespace {

int failures = 0;

#define CHECK(cond)                                                                       \
    do {                                                                                  \
        if (!(cond)) {                                                                    \
            std::cerr << __FILE__ << ":" << __LINE__ << ": CHECK failed: " #cond << "\n"; \
            ++failures;                                                                   \
        }                                                                                 \
    } while (0)

#define CHECK_THROWS_CODE(expr, expected_code)                                              \
    do {                                                                                    \
        bool threw_ = false;                                                                \
        try {                                                                               \
            expr;                                                                           \
        } catch (const velurex_hip::Error& e) {                                             \
            threw_ = true;                                                                  \
            if (e.code() != (expected_code)) {                                              \
                std::cerr << __FILE__ << ":" << __LINE__ << ": code " << e.code()            \
                          << " instead of " << (expected_code) << ": " << e.what() << "\n"; \
                ++failures;                                                                 \
            }                                                                               \
            if (std::string(e.what()).empty()) {                                            \
                std::cerr << __FILE__ << ":" << __LINE__ << ": empty message\n";            \
                ++failures;                                                                 \
            }                                                                               \
        }                                                                                   \
        if (!threw_) {                                                                      \
            std::cerr << __FILE__ << ":" << __LINE__ << ": no exception from " #expr "\n";  \
            ++failures;                                                                     \
        }                                                                                   \
    } while (0)

std::uint64_t state = 0x13198A2E03707344ULL;
std::uint32_t next() {
    state ^= state >> 12;
    state ^= state << 25;
    state ^= state >> 27;
    return static_cast<std::uint32_t>((state * 0x2545F4914F6CDD1DULL) >> 32);
}

// The planar layout of a row-major trit matrix: ceil(cols / 160) blocks of 32 bytes per row, byte j of block b holding
// the trits of columns 160 b + 32 p + j (p = 0..4) as the digits d = t + 1 of d0 + 3 d1 + 9 d2 + 28 d3 + 84 d4, zero
// trits past the row (quintrit-core/src/pack.rs:10-58).
std::vector<std::uint8_t> pack_planar(const std::vector<std::int8_t>& trits, std::size_t rows, std::size_t cols) {
    static const int kWeight[5] = {1, 3, 9, 28, 84};
    const std::size_t nb = (cols + 159) / 160;
    std::vector<std::uint8_t> out(rows * nb * 32);
    for (std::size_t r = 0; r < rows; ++r)
        for (std::size_t b = 0; b < nb; ++b)
            for (std::size_t j = 0; j < 32; ++j) {
                int v = 0;
                for (int p = 0; p < 5; ++p) {
                    const std::size_t c = b * 160 + 32 * p + j;
                    v += (c < cols ? trits[r * cols + c] + 1 : 1) * kWeight[p];
                }
                out[(r * nb + b) * 32 + j] = static_cast<std::uint8_t>(v);
            }
    return out;
}

std::vector<std::int64_t> brute_force(const std::vector<std::int8_t>& trits, std::size_t rows, std::size_t cols,
                                      const std::vector<std::int8_t>& acts) {
    std::vector<std::int64_t> y(rows, 0);
    for (std::size_t r = 0; r < rows; ++r)
        for (std::size_t c = 0; c < cols; ++c) y[r] += static_cast<std::int64_t>(trits[r * cols + c]) * acts[c];
    return y;
}

std::uint32_t bits(float f) {
    std::uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

// The layer epilogue of layer.rs:143-150: out = float(acc) * (weight_scale / act_scale), zeros when act_scale <= 0.
float epilogue(std::int64_t acc, float weight_scale, float act_scale) {
    if (!(act_scale > 0.0f)) return 0.0f;
    const float post = weight_scale / act_scale;
    return static_cast<float>(acc) * post;
}

// One shape through the kernel-level helpers and through the layer (by its interface), against brute force.
void gemv_case(std::size_t rows, std::size_t cols, int trit_fill, int act_fill) {
    std::vector<std::int8_t> trits(rows * cols);
    for (auto& t : trits) t = static_cast<std::int8_t>(trit_fill == 2 ? static_cast<int>(next() % 3) - 1 : trit_fill);
    std::vector<std::int8_t> acts(cols);
    for (auto& a : acts) a = static_cast<std::int8_t>(act_fill == 0 ? static_cast<int>(next() & 0xFF) : act_fill);
    if (act_fill == 0) acts[0] = -128;
    const std::vector<std::uint8_t> planar = pack_planar(trits, rows, cols);
    const std::vector<std::int64_t> want = brute_force(trits, rows, cols, acts);

    const std::vector<std::int32_t> got = velurex_hip::gemv_i32(planar, rows, cols, acts);
    const std::vector<float> gotf = velurex_hip::gemv_f32(planar, rows, cols, acts, 2.0f);
    CHECK(got.size() == rows && gotf.size() == rows);
    bool ok = true;
    for (std::size_t r = 0; r < rows; ++r) {
        ok = ok && got[r] == want[r];
        ok = ok && bits(gotf[r]) == bits(static_cast<float>(want[r]) * 2.0f);
    }
    CHECK(ok);

    const velurex_hip::VelurexHipLayer layer(planar, rows, cols, 0.5f);
    const velurex_hip::TernaryGemvLayer& base = layer;
    CHECK(base.shape() == std::make_pair(rows, cols));
    CHECK(base.weight_scale() == 0.5f);
    CHECK(base.memory_bytes() == velurex_hip::layout(rows, cols).device_bytes);
    CHECK(base.kernel_type() == velurex_hip::TernaryKernelType::VelurexHip);
    std::vector<float> y(rows);
    for (float as : {1.0f, 0.37f, 0.0f, -1.0f}) {
        base.forward(acts, as, y);
        bool same = true;
        for (std::size_t r = 0; r < rows; ++r) same = same && bits(y[r]) == bits(epilogue(want[r], 0.5f, as));
        CHECK(same);
    }
}

// The device-memory forms of a layer: int32 and fp32 outputs on a stream.
void device_case(std::size_t rows, std::size_t cols) {
    std::vector<std::int8_t> trits(rows * cols);
    for (auto& t : trits) t = static_cast<std::int8_t>(static_cast<int>(next() % 3) - 1);
    std::vector<std::int8_t> acts(cols);
    for (auto& a : acts) a = static_cast<std::int8_t>(next() & 0xFF);
    const std::vector<std::int64_t> want = brute_force(trits, rows, cols, acts);
    const velurex_hip::VelurexHipLayer layer(pack_planar(trits, rows, cols), rows, cols, 0.02f);
    std::int8_t* da = nullptr;
    void* dy = nullptr;
    CHECK(hipMalloc(reinterpret_cast<void**>(&da), cols) == hipSuccess);
    CHECK(hipMalloc(&dy, rows * 4) == hipSuccess);
    if (da == nullptr || dy == nullptr) return;
    CHECK(hipMemcpy(da, acts.data(), cols, hipMemcpyHostToDevice) == hipSuccess);
    std::vector<std::int32_t> yi(rows);
    std::vector<float> yf(rows);
    layer.gemv_i32_dev(da, static_cast<std::int32_t*>(dy));
    CHECK(hipMemcpy(yi.data(), dy, rows * 4, hipMemcpyDeviceToHost) == hipSuccess);
    layer.gemv_f32_dev(da, 0.25f, static_cast<float*>(dy));
    CHECK(hipMemcpy(yf.data(), dy, rows * 4, hipMemcpyDeviceToHost) == hipSuccess);
    bool ok = true;
    for (std::size_t r = 0; r < rows; ++r) {
        ok = ok && yi[r] == want[r];
        ok = ok && bits(yf[r]) == bits(epilogue(want[r], 0.02f, 0.25f));
    }
    CHECK(ok);
    (void)hipFree(da);
    (void)hipFree(dy);
}

// A plan of three GEMVs (two share an input, one has its own; int32 and fp32 outputs) run twice with new inputs, and a
// batched GEMM, all on device buffers, against brute force.
void plan_and_gemm_case() {
    struct M { std::size_t rows, cols; std::vector<std::int8_t> t; };
    std::vector<M> mats = {{1024, 3072, {}}, {3072, 3072, {}}, {512, 6000, {}}};
    std::vector<velurex_hip::VelurexHipLayer> layers;
    for (auto& m : mats) {
        m.t.resize(m.rows * m.cols);
        for (auto& v : m.t) v = static_cast<std::int8_t>(static_cast<int>(next() % 3) - 1);
        layers.emplace_back(pack_planar(m.t, m.rows, m.cols), m.rows, m.cols, 0.02f);
    }
    std::int8_t *a0 = nullptr, *a1 = nullptr;
    void *s0 = nullptr, *s1 = nullptr, *y0 = nullptr, *y1 = nullptr, *y2 = nullptr;
    float* as = nullptr;
    bool ok = hipMalloc(reinterpret_cast<void**>(&a0), 3072) == hipSuccess && hipMalloc(reinterpret_cast<void**>(&a1), 6000) == hipSuccess &&
              hipMalloc(&s0, velurex_hip::staged_bytes(3072)) == hipSuccess && hipMalloc(&s1, velurex_hip::staged_bytes(6000)) == hipSuccess &&
              hipMalloc(&y0, 1024 * 4) == hipSuccess && hipMalloc(&y1, 3072 * 4) == hipSuccess && hipMalloc(&y2, 512 * 4) == hipSuccess &&
              hipMalloc(reinterpret_cast<void**>(&as), 4) == hipSuccess;
    CHECK(ok);
    if (!ok) return;
    const velurex_hip::Plan plan({{&layers[0], a0, s0, y0, nullptr}, {&layers[1], a0, s0, y1, as}, {&layers[2], a1, s1, y2, nullptr}});
    CHECK(plan.work_items() > 0);
    for (int run = 0; run < 2; ++run) {
        std::vector<std::int8_t> x0(3072), x1(6000);
        for (auto& v : x0) v = static_cast<std::int8_t>(next() & 0xFF);
        for (auto& v : x1) v = static_cast<std::int8_t>(next() & 0xFF);
        const float scale = run == 0 ? 0.5f : 1.75f;
        CHECK(hipMemcpy(a0, x0.data(), 3072, hipMemcpyHostToDevice) == hipSuccess);
        CHECK(hipMemcpy(a1, x1.data(), 6000, hipMemcpyHostToDevice) == hipSuccess);
        CHECK(hipMemcpy(as, &scale, 4, hipMemcpyHostToDevice) == hipSuccess);
        plan.run();
        CHECK(hipDeviceSynchronize() == hipSuccess);
        std::vector<std::int32_t> g0(1024), g2(512);
        std::vector<float> g1(3072);
        CHECK(hipMemcpy(g0.data(), y0, 1024 * 4, hipMemcpyDeviceToHost) == hipSuccess);
        CHECK(hipMemcpy(g1.data(), y1, 3072 * 4, hipMemcpyDeviceToHost) == hipSuccess);
        CHECK(hipMemcpy(g2.data(), y2, 512 * 4, hipMemcpyDeviceToHost) == hipSuccess);
        const auto w0 = brute_force(mats[0].t, 1024, 3072, x0), w1 = brute_force(mats[1].t, 3072, 3072, x0);
        const auto w2 = brute_force(mats[2].t, 512, 6000, x1);
        bool same = true;
        for (std::size_t r = 0; r < 1024; ++r) same = same && g0[r] == w0[r];
        for (std::size_t r = 0; r < 3072; ++r) same = same && bits(g1[r]) == bits(epilogue(w1[r], 0.02f, scale));
        for (std::size_t r = 0; r < 512; ++r) same = same && g2[r] == w2[r];
        CHECK(same);
    }
    // 40 tokens through the GEMM on the 3072 x 3072 matrix
    const std::size_t m = 40, cols = 3072, rows = 3072;
    std::vector<std::int8_t> x(m * cols);
    for (auto& v : x) v = static_cast<std::int8_t>(next() & 0xFF);
    std::int8_t* dx = nullptr;
    void *dy = nullptr, *ws = nullptr;
    const std::size_t wsb = velurex_hip::gemm_workspace_bytes(layers[1], m);
    ok = hipMalloc(reinterpret_cast<void**>(&dx), m * cols) == hipSuccess && hipMalloc(&dy, m * rows * 4) == hipSuccess &&
         hipMalloc(&ws, wsb) == hipSuccess;
    CHECK(ok);
    if (ok) {
        CHECK(hipMemcpy(dx, x.data(), m * cols, hipMemcpyHostToDevice) == hipSuccess);
        velurex_hip::gemm_i32_dev(layers[1], dx, m, cols, static_cast<std::int32_t*>(dy), rows, ws, wsb);
        CHECK(hipDeviceSynchronize() == hipSuccess);
        std::vector<std::int32_t> y(m * rows);
        CHECK(hipMemcpy(y.data(), dy, m * rows * 4, hipMemcpyDeviceToHost) == hipSuccess);
        bool same = true;
        for (std::size_t t = 0; t < m; ++t) {
            const std::vector<std::int8_t> xt(x.begin() + t * cols, x.begin() + (t + 1) * cols);
            const auto w = brute_force(mats[1].t, rows, cols, xt);
            for (std::size_t r = 0; r < rows; ++r) same = same && y[t * rows + r] == w[r];
        }
        CHECK(same);
        CHECK_THROWS_CODE(velurex_hip::gemm_i32_dev(layers[1], dx, m, cols, static_cast<std::int32_t*>(dy), rows, ws, wsb - 1),
                          VX_ERR_BUFFER_TOO_SMALL);
    }
    for (void* p : {static_cast<void*>(a0), static_cast<void*>(a1), s0, s1, y0, y1, y2, static_cast<void*>(as),
                    static_cast<void*>(dx), dy, ws})
        (void)hipFree(p);
}

// One layer shared by four threads (the trait is Send + Sync), each with its own activations.
void threads_case() {
    const std::size_t rows = 1024, cols = 3072;
    std::vector<std::int8_t> trits(rows * cols);
    for (auto& t : trits) t = static_cast<std::int8_t>(static_cast<int>(next() % 3) - 1);
    const velurex_hip::VelurexHipLayer layer(pack_planar(trits, rows, cols), rows, cols, 1.0f);
    std::vector<std::vector<std::int8_t>> acts(4, std::vector<std::int8_t>(cols));
    std::vector<std::vector<std::int64_t>> want;
    for (auto& a : acts) {
        for (auto& v : a) v = static_cast<std::int8_t>(next() & 0xFF);
        want.push_back(brute_force(trits, rows, cols, a));
    }
    std::vector<int> bad(4, 0);
    std::vector<std::thread> pool;
    for (int t = 0; t < 4; ++t)
        pool.emplace_back([&, t]() {
            std::vector<float> y(rows);
            for (int i = 0; i < 25; ++i) {
                layer.forward(acts[t], 1.0f, y);
                for (std::size_t r = 0; r < rows; ++r)
                    if (bits(y[r]) != bits(static_cast<float>(want[t][r]))) ++bad[t];
            }
        });
    for (auto& th : pool) th.join();
    CHECK(bad[0] == 0 && bad[1] == 0 && bad[2] == 0 && bad[3] == 0);
}

// A random decoder of a small BitNet-like (ReLU^2, sub-norms, NEOX RoPE, tied bf16 embedding) or Falcon3-like (SiLU,
// Normal RoPE, no sub-norms, f16 embedding, untied head) shape: the same weights for every decoder built with one seed.
velurex_hip::Decoder small_decoder(bool falcon, std::uint64_t seed) {
    state = seed;
    vx_decoder_config_t c{};
    c.n_layers = 2;
    c.hidden = 256;
    c.n_heads = 4;
    c.n_kv_heads = 2;
    c.head_dim = 64;
    c.ffn = 512;
    c.vocab = 1000;
    c.max_ctx = 640;
    c.rms_eps = 1e-5f;
    c.rope_theta = 10000.0f;
    if (falcon) {
        c.act = VX_ACT_SILU;
        c.rope_mode = VX_ROPE_NORMAL;
        c.no_sub_norm = 1;
        c.emb_f16 = 1;
        c.untied = 1;
    }
    velurex_hip::Decoder d(c);
    auto planar = [&](std::size_t rows, std::size_t cols) {
        std::vector<std::int8_t> t(rows * cols);
        for (auto& v : t) v = static_cast<std::int8_t>(static_cast<int>(next() % 3) - 1);
        return pack_planar(t, rows, cols);
    };
    const std::size_t q = c.n_heads * c.head_dim, kv = c.n_kv_heads * c.head_dim;
    const std::size_t shapes[7][2] = {{q, c.hidden}, {kv, c.hidden}, {kv, c.hidden}, {c.hidden, q},
                                      {c.ffn, c.hidden}, {c.ffn, c.hidden}, {c.hidden, c.ffn}};
    for (std::uint32_t l = 0; l < c.n_layers; ++l) {
        for (std::uint32_t k = 0; k < 7; ++k) {
            const float ws = 0.5f + static_cast<float>(next() % 1000) / 1000.0f;
            if (k == VX_PROJ_O && l == 1) {  // one projection handed over as a matrix
                d.adopt_projection(l, k, velurex_hip::VelurexHipLayer(planar(shapes[k][0], shapes[k][1]), shapes[k][0],
                                                                      shapes[k][1], ws));
            } else {
                d.set_projection(l, k, planar(shapes[k][0], shapes[k][1]), ws);
            }
        }
        for (std::uint32_t k : {VX_NORM_ATTN, VX_NORM_ATTN_SUB, VX_NORM_FFN, VX_NORM_FFN_SUB}) {
            if (falcon && (k == VX_NORM_ATTN_SUB || k == VX_NORM_FFN_SUB)) continue;
            const std::size_t n = k == VX_NORM_ATTN_SUB ? q : (k == VX_NORM_FFN_SUB ? c.ffn : c.hidden);
            std::vector<float> w(n);
            for (auto& v : w) v = 0.8f + static_cast<float>(next() % 400) / 1000.0f;
            d.set_norm(l, k, w);
        }
    }
    std::vector<float> out_norm(c.hidden);
    for (auto& v : out_norm) v = 0.8f + static_cast<float>(next() % 400) / 1000.0f;
    d.set_norm(c.n_layers, VX_NORM_ATTN, out_norm);
    // 16-bit values of magnitude 2^-5 .. 2^-1 with random signs and mantissas: bf16 (exponent 122..126) or f16 (10..14)
    auto table = [&](bool f16) {
        std::vector<std::uint16_t> e(static_cast<std::size_t>(c.vocab) * c.hidden);
        for (auto& v : e) {
            const std::uint32_t r = next();
            v = f16 ? static_cast<std::uint16_t>(((r >> 31) << 15) | ((10u + r % 5u) << 10) | ((r >> 8) & 0x3ffu))
                    : static_cast<std::uint16_t>(((r >> 31) << 15) | ((122u + r % 5u) << 7) | ((r >> 8) & 0x7fu));
        }
        return e;
    };
    if (falcon) {
        d.set_embedding_f16(table(true));
        d.set_head(table(true));
    } else {
        d.set_embedding_bf16(table(false));
    }
    return d;
}

// The decoder through the wrapper: prefill passes and decode steps give the same logits, KV cache and tokens.
void decoder_case(bool falcon) {
    std::vector<std::uint32_t> prompt(40);
    velurex_hip::Decoder a = small_decoder(falcon, 0x5EED0001ULL);
    velurex_hip::Decoder b = small_decoder(falcon, 0x5EED0001ULL);
    for (auto& t : prompt) t = next() % 1000;
    const vx_decoder_config_t c = a.config();
    CHECK(c.hidden == 256 && c.vocab == 1000 && c.act == (falcon ? VX_ACT_SILU : VX_ACT_RELU2));
    CHECK(a.memory_bytes() > 0);
    // the prompt by one prefill on a, by steps on b
    std::vector<float> la, lb;
    const std::uint32_t na = a.prefill(prompt, 0, &la);
    std::uint32_t nb = 0;
    for (std::uint32_t p = 0; p < prompt.size(); ++p) nb = b.step(prompt[p], p, p + 1 == prompt.size() ? &lb : nullptr);
    CHECK(na == nb);
    bool same = la.size() == lb.size();
    for (std::size_t i = 0; same && i < la.size(); ++i) same = bits(la[i]) == bits(lb[i]);
    CHECK(same);
    for (std::uint32_t p : {0u, 17u, 39u})
        for (std::uint32_t l = 0; l < c.n_layers; ++l) CHECK(a.kv(l, p, 1) == b.kv(l, p, 1));
    // the next step continues both at position 40
    std::vector<float> sa, sb;
    CHECK(a.step(na, 40, &sa) == b.step(nb, 40, &sb));
    same = true;
    for (std::size_t i = 0; i < sa.size(); ++i) same = same && bits(sa[i]) == bits(sb[i]);
    CHECK(same);
    // greedy generation with prefill passes and fed step by step
    CHECK(a.generate(prompt, 24) == b.generate(prompt, 24, true));
    // beyond the context
    CHECK_THROWS_CODE(a.prefill(std::vector<std::uint32_t>(8, 1u), 636), VX_ERR_CONTEXT_OVERFLOW);
    // a projection of the wrong size, a sub-norm the architecture does not have
    CHECK_THROWS_CODE(a.set_projection(0, VX_PROJ_Q, std::vector<std::uint8_t>(100, 125), 1.0f), VX_ERR_BUFFER_TOO_SMALL);
    if (falcon) CHECK_THROWS_CODE(a.set_norm(0, VX_NORM_ATTN_SUB, std::vector<float>(256, 1.0f)), VX_ERR_INVALID_ARGUMENT);
    velurex_hip::Decoder moved(std::move(a));
    CHECK(moved.config().vocab == 1000);
    CHECK_THROWS_CODE(a.config(), VX_ERR_INVALID_HANDLE);
}

void cpu_checks() {
    velurex_hip::check_abi();
    CHECK(velurex_hip::version() == VX_VERSION_STRING);
    CHECK(std::string(velurex_hip::kernel_name(velurex_hip::TernaryKernelType::VelurexHip)) == "VelurexHip");
    CHECK(velurex_hip::bpw(velurex_hip::TernaryKernelType::VelurexHip) == 1.6f);
    CHECK(velurex_hip::activation_quant_levels(velurex_hip::TernaryKernelType::VelurexHip) == 127.0f);

    // pack.rs:222-225: 6 whole blocks (192 bytes) and a tail of 40 columns in 8 bytes, rounded to 16 on the device
    const vx_layout_t l = velurex_hip::layout(70, 1000);
    CHECK(l.padded_rows == 128 && l.planar_row_bytes == 224 && l.tile_row_bytes == 200 && l.device_row_bytes == 208);
    CHECK(l.device_bytes == 128u * 208u && l.tile_rows == 64 && l.tile_group == 16);

    // Errors become velurex_hip::Error with the status code and the message of the library.
    CHECK_THROWS_CODE(velurex_hip::layout(0, 4), VX_ERR_INVALID_SHAPE);
    CHECK_THROWS_CODE(velurex_hip::layout(4, VX_MAX_GEMV_COLS + 1), VX_ERR_INVALID_SHAPE);
    CHECK_THROWS_CODE(velurex_hip::VelurexHipLayer(nullptr, 32, 1, 160, 1.0f), VX_ERR_NULL_POINTER);
    CHECK_THROWS_CODE(velurex_hip::VelurexHipLayer(std::vector<std::uint8_t>(31, 125), 1, 160, 1.0f),
                      VX_ERR_BUFFER_TOO_SMALL);
    CHECK_THROWS_CODE(velurex_hip::gemv_i32(std::vector<std::uint8_t>(32, 125), 1, 160, std::vector<std::int8_t>(159)),
                      VX_ERR_BUFFER_TOO_SMALL);

    // The owning class is move-only and implements the interface.
    static_assert(std::is_move_constructible<velurex_hip::VelurexHipLayer>::value, "VelurexHipLayer must be movable");
    static_assert(!std::is_copy_constructible<velurex_hip::VelurexHipLayer>::value, "VelurexHipLayer must not be copyable");
    static_assert(std::is_base_of<velurex_hip::TernaryGemvLayer, velurex_hip::VelurexHipLayer>::value, "a layer");
    static_assert(std::has_virtual_destructor<velurex_hip::TernaryGemvLayer>::value, "owned through the interface");
    static_assert(std::is_move_constructible<velurex_hip::Decoder>::value, "Decoder must be movable");
    static_assert(!std::is_copy_constructible<velurex_hip::Decoder>::value, "Decoder must not be copyable");
    static_assert(!std::is_copy_constructible<velurex_hip::Plan>::value, "Plan must not be copyable");
    CHECK(velurex_hip::staged_bytes(3072) > 0);
    CHECK_THROWS_CODE(velurex_hip::Decoder::open_gguf("this-file-does-not-exist.gguf"), VX_ERR_IO);
}

void gpu_checks() {
    std::cout << "devices: " << velurex_hip::device_count() << "\n";
    // the reference C++ test's shapes (test_kernel.cpp), then ffi_kernel.rs's (a 512-row matrix, an odd column count
    // past 4096, a packed tail)
    const std::size_t shapes[][2] = {{1, 1},   {5, 7},      {33, 161},  {64, 320}, {70, 1000},
                                     {96, 3072}, {512, 3072}, {96, 6000}, {70, 777}, {100, 777}};
    for (const auto& s : shapes) gemv_case(s[0], s[1], 2, 0);
    // extreme fills (ffi_kernel.rs:195-265): every trit +1 or -1 against every activation 127 or -128
    for (int t : {1, -1})
        for (int a : {127, -128}) gemv_case(64, 1000, t, a);
    device_case(3072, 3072);
    device_case(70, 777);
    threads_case();
    plan_and_gemm_case();
    decoder_case(false);
    decoder_case(true);

    // Errors of a valid handle: a byte outside the 243 velurex values, slices of the wrong length, a moved-from layer.
    std::vector<std::uint8_t> bad(32, 125);
    bad[7] = 251;
    CHECK_THROWS_CODE(velurex_hip::VelurexHipLayer(bad, 1, 160, 1.0f), VX_ERR_INVALID_VALUE);
    velurex_hip::VelurexHipLayer layer(std::vector<std::uint8_t>(2 * 32, 125), 2, 160, 1.0f);
    std::vector<float> y(2);
    CHECK_THROWS_CODE(layer.forward(std::vector<std::int8_t>(159), 1.0f, y), VX_ERR_INVALID_ARGUMENT);
    std::vector<float> y3(3);
    CHECK_THROWS_CODE(layer.forward(std::vector<std::int8_t>(160), 1.0f, y3), VX_ERR_INVALID_ARGUMENT);
    layer.forward(std::vector<std::int8_t>(160, 5), 1.0f, y);  // zero trits: a zero result
    CHECK(y[0] == 0.0f && y[1] == 0.0f);
    velurex_hip::VelurexHipLayer moved(std::move(layer));
    CHECK(moved.shape() == std::make_pair(std::size_t{2}, std::size_t{160}));
    CHECK_THROWS_CODE(layer.forward(std::vector<std::int8_t>(160), 1.0f, y), VX_ERR_INVALID_HANDLE);
}

}  // namespace

int main(int argc, char** argv) {
    const bool cpu_only = argc > 1 && std::string(argv[1]) == "--cpu";
    try {
        cpu_checks();
        if (!cpu_only) gpu_checks();
    } catch (const velurex_hip::Error& e) {
        std::cerr << "unexpected velurex_hip::Error " << e.code() << ": " << e.what() << "\n";
        return 1;
    }
    if (failures != 0) {
        std::cerr << failures << " check(s) failed\n";
        return 1;
    }
    std::cout << (cpu_only ? "C++ test (no device) passed\n" : "C++ test passed\n");
    return 0;
}
