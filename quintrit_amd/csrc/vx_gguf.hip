// GGUF files and their ternary tensors: the reader of quintrit-format/src/gguf.rs behind the C API of
// quintrit-c/include/quintrit.h:221-308 (vx_gguf_* here), and the transcoding of I2_S / TQ1_0 / TQ2_0 / Q2_0 payloads
// into velurex weights (quintrit-format/src/transcoder.rs:154-205, decoders/*.rs).
//
// The reader trusts nothing it reads (gguf.rs:7-23): every count and length is bounded by the bytes that remain before
// anything is allocated, offsets and sizes are checked, and an inconsistent file gives VX_ERR_FORMAT. The file is
// memory-mapped read-only; names and payload pointers stay valid until vx_gguf_close.
//
// Transcoding: on the host, rows of trits are decoded and packed into the planar velurex layout on several threads
// (the layout vx_matrix_create takes). On the GPU (vx_gguf_upload_matrix, vx_matrix_create_ggml_dev), the raw payload
// goes to HBM as it is and one kernel writes each planar byte from the five source trits it covers, so a model's
// weights cross PCIe once, in their GGUF size, and are converted at HBM speed instead of on the CPU.
#include "vx_internal.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace vx {

// ---- trits of the GGUF ternary types (host and device) ------------------------------------------------------------------

constexpr uint32_t kQkTq = 256;
constexpr uint32_t kTq1Bytes = 54, kTq2Bytes = 66;

__host__ __device__ inline int8_t code_trit(uint32_t code) {  // 0 -> -1, 1 -> 0, 2 -> +1, 3 -> 0 (unpack.rs:59-62)
    return code == 3 ? 0 : static_cast<int8_t>(static_cast<int>(code) - 1);
}

// Internal type codes of Q2_0 payloads by block size (64 or 128 weights per f16 scale) for the trit gatherer.
constexpr uint32_t kQ2Block64 = 0x10000u | VX_GGML_Q2_0, kQ2Block128 = 0x20000u | VX_GGML_Q2_0;

// TQ1_0 digit n of byte q: ((q 3^n mod 256) 3) >> 8, minus 1 (decoders/tq1_0.rs:63-67).
__host__ __device__ inline int8_t tq1_digit(uint32_t byte, uint32_t n) {
    const uint32_t p3 = n == 0 ? 1u : n == 1 ? 3u : n == 2 ? 9u : n == 3 ? 27u : 81u;
    const uint32_t q = (byte * p3) & 255u;
    return static_cast<int8_t>(static_cast<int>((q * 3u) >> 8) - 1);
}

// Trit of weight (row r, column c) of a payload; for the TQ types the flattened index e = r cols + c runs over blocks
// of 256 (rows need not be whole blocks, as in transcoder.rs:166-170).
__host__ __device__ inline int8_t ggml_trit(uint32_t type, const uint8_t* src, uint64_t r, uint64_t c, uint64_t cols) {
    if (type == VX_GGML_I2_S) {  // decoders/i2_s.rs:45-66: byte j % 32 of the 128-trit block, bits 6 - 2 (j / 32)
        const uint64_t j = c & 127u;
        const uint8_t b = src[r * (cols / 4) + (c >> 7) * 32 + (j & 31u)];
        return code_trit((b >> (6 - 2 * (j >> 5))) & 3u);
    }
    const uint64_t e = r * cols + c;
    if (type == kQ2Block64 || type == kQ2Block128) {
        // decoders/q2_0.rs:32-57: an f16 scale, then the block's 2-bit codes four to a byte, low bits first (the codes
        // were checked: no 3 reaches here)
        const uint32_t bs = type == kQ2Block64 ? 64u : 128u;
        const uint8_t* blk = src + (e / bs) * (2 + bs / 4);
        const uint32_t o = static_cast<uint32_t>(e % bs);
        return code_trit((blk[2 + o / 4] >> (2 * (o & 3u))) & 3u);
    }
    const uint32_t i = static_cast<uint32_t>(e & (kQkTq - 1));
    if (type == VX_GGML_TQ2_0) {  // decoders/tq2_0.rs:69-73: element 128 g + 32 l + m at bits 2 l of byte 32 g + m
        const uint8_t* blk = src + (e / kQkTq) * kTq2Bytes;
        const uint32_t g = i >> 7, l = (i >> 5) & 3u, m = i & 31u;
        return code_trit((blk[32 * g + m] >> (2 * l)) & 3u);
    }
    // TQ1_0 (decoders/tq1_0.rs:69-89): qs[m] holds 32 n + m, qs[32 + m] 160 + 16 n + m, qh[j] 240 + 4 n + j
    const uint8_t* blk = src + (e / kQkTq) * kTq1Bytes;
    if (i < 160) return tq1_digit(blk[i & 31u], i >> 5);
    if (i < 240) return tq1_digit(blk[32 + ((i - 160) & 15u)], (i - 160) >> 4);
    return tq1_digit(blk[48 + ((i - 240) & 3u)], (i - 240) >> 2);
}

// Planar byte j of 160-trit block b of row r (pack.rs:66-131): digits d = t + 1 of columns b 160 + p 32 + j weighted
// 1, 3, 9, 28, 84; columns past the row are zero trits.
__host__ __device__ inline uint8_t planar_byte(uint32_t type, const uint8_t* src, uint64_t r, uint64_t b, uint32_t j,
                                               uint64_t cols) {
    const uint32_t w[5] = {1, 3, 9, 28, 84};
    uint32_t v = 0;
    for (uint32_t p = 0; p < 5; ++p) {
        const uint64_t c = b * kQK5 + p * 32 + j;
        const int t = c < cols ? ggml_trit(type, src, r, c, cols) : 0;
        v += static_cast<uint32_t>(t + 1) * w[p];
    }
    return static_cast<uint8_t>(v);
}

__global__ void ggml_to_planar_kernel(uint32_t type, const uint8_t* __restrict__ src, uint64_t rows, uint64_t cols,
                                      uint8_t* __restrict__ planar) {
    const uint64_t rb = (cols + kQK5 - 1) / kQK5 * kBlockBytes;
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows * rb) return;
    const uint64_t r = i / rb, k = i - r * rb;
    planar[i] = planar_byte(type, src, r, k / kBlockBytes, static_cast<uint32_t>(k % kBlockBytes), cols);
}

// Payload bytes of a rows x cols tensor of a ternary type, or 0 if the shape does not fit the type.
static size_t ggml_payload_bytes(uint32_t type, size_t rows, size_t cols) {
    const size_t n = rows * cols;
    switch (type) {
        case VX_GGML_I2_S: return cols % 128 == 0 ? n / 4 : 0;
        case VX_GGML_TQ1_0: return n % kQkTq == 0 ? n / kQkTq * kTq1Bytes : 0;
        case VX_GGML_TQ2_0: return n % kQkTq == 0 ? n / kQkTq * kTq2Bytes : 0;
        default: return 0;
    }
}

static int check_ternary(uint32_t type, size_t len, size_t rows, size_t cols) {
    if (type != VX_GGML_I2_S && type != VX_GGML_TQ1_0 && type != VX_GGML_TQ2_0)
        VX_FAIL(VX_ERR_UNSUPPORTED, "GGML type %u is not a ternary type (I2_S = 36, TQ1_0 = 34, TQ2_0 = 35)", type);
    VX_TRY(check_shape(rows, cols));
    const size_t need = ggml_payload_bytes(type, rows, cols);
    if (need == 0)
        VX_FAIL(VX_ERR_INVALID_SHAPE, "%zu x %zu weights do not fit GGML type %u (I2_S: cols a multiple of 128; TQ: "
                "a multiple of 256 weights)", rows, cols, type);
    if (len < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "the payload holds %zu bytes, %zu needed", len, need);
    return VX_OK;
}

// Host transcoding: rows split over threads, each byte computed from the payload directly.
static void host_to_planar(uint32_t type, const uint8_t* src, size_t rows, size_t cols, uint8_t* out) {
    const size_t rb = planar_row_bytes(cols);
    const size_t total = rows * cols;
    unsigned nt = std::max(1u, std::min(std::thread::hardware_concurrency(), 64u));
    if (total < (size_t{1} << 20)) nt = 1;
    auto work = [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r)
            for (size_t k = 0; k < rb; ++k) out[r * rb + k] = planar_byte(type, src, r, k / kBlockBytes, static_cast<uint32_t>(k % kBlockBytes), cols);
    };
    if (nt == 1) {
        work(0, rows);
        return;
    }
    std::vector<std::thread> th;
    const size_t per = (rows + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const size_t r0 = t * per, r1 = std::min(rows, r0 + per);
        if (r0 < r1) th.emplace_back(work, r0, r1);
    }
    for (auto& x : th) x.join();
}

// ---- the GGUF reader -----------------------------------------------------------------------------------------------

constexpr size_t kMaxNameLen = size_t{1} << 16;
constexpr uint32_t kMaxArrayDepth = 4;
constexpr uint32_t kMaxDims = VX_MAX_DIMS;
constexpr uint64_t kMaxElements = uint64_t{1} << 40;
constexpr size_t kMinMetaEntry = 13;    // key length (8), value type (4), a one-byte value
constexpr size_t kMinTensorEntry = 32;  // name length (8), n_dims (4), one dimension (8), type (4), offset (8)

struct Meta {
    uint32_t type = 0;
    uint64_t u = 0;   // unsigned and bool
    int64_t i = 0;    // signed
    double f = 0.0;   // floats (f32 widened)
    std::string s;
    uint32_t arr_type = 0;
    std::vector<Meta> arr;
};

struct TensorRec {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[kMaxDims] = {};
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t n_elem = 1;
    uint64_t byte_len = 0;  // 0: the layout of the type is not known here
    uint32_t block_size = 0;
};

struct ParseError {
    std::string msg;
};

class Reader {
  public:
    Reader(const uint8_t* b, size_t n) : buf_(b), len_(n) {}
    size_t pos() const { return pos_; }
    size_t remaining() const { return len_ - pos_; }
    const uint8_t* take(size_t n, const char* what) {
        if (n > remaining())
            throw ParseError{std::string("truncated GGUF file: ") + what + " needs " + std::to_string(n) + " bytes at offset " +
                             std::to_string(pos_) + " but only " + std::to_string(remaining()) + " remain"};
        const uint8_t* p = buf_ + pos_;
        pos_ += n;
        return p;
    }
    template <class T>
    T num(const char* what) {
        T v;
        std::memcpy(&v, take(sizeof(T), what), sizeof(T));
        return v;
    }
    size_t count(const char* what, size_t min_entry) {
        const uint64_t n = num<uint64_t>(what);
        if (n > remaining() / min_entry)
            throw ParseError{std::string(what) + " " + std::to_string(n) + " does not fit into the " + std::to_string(remaining()) +
                             " remaining bytes of the file"};
        return static_cast<size_t>(n);
    }
    std::string str(const char* what, size_t max_len) {
        const uint64_t n = num<uint64_t>(what);
        if (n > max_len || n > remaining())
            throw ParseError{std::string(what) + " of " + std::to_string(n) + " bytes is longer than the limit of " +
                             std::to_string(max_len) + " bytes or the rest of the file"};
        const uint8_t* p = take(static_cast<size_t>(n), what);
        if (!utf8_valid(p, static_cast<size_t>(n))) throw ParseError{std::string(what) + " is not valid UTF-8"};
        return std::string(reinterpret_cast<const char*>(p), static_cast<size_t>(n));
    }
    // Well-formed UTF-8: no stray continuation bytes, no truncated, overlong or surrogate sequences, nothing past
    // U+10FFFF (Rust's String::from_utf8, gguf.rs:562).
    static bool utf8_valid(const uint8_t* p, size_t n) {
        size_t i = 0;
        while (i < n) {
            const uint8_t c = p[i];
            if (c < 0x80) {
                ++i;
                continue;
            }
            size_t k;
            uint32_t cp;
            if ((c & 0xE0) == 0xC0) {
                k = 1;
                cp = c & 0x1F;
            } else if ((c & 0xF0) == 0xE0) {
                k = 2;
                cp = c & 0x0F;
            } else if ((c & 0xF8) == 0xF0) {
                k = 3;
                cp = c & 0x07;
            } else {
                return false;
            }
            if (k >= n - i) return false;
            for (size_t j = 1; j <= k; ++j) {
                if ((p[i + j] & 0xC0) != 0x80) return false;
                cp = (cp << 6) | (p[i + j] & 0x3F);
            }
            if ((k == 1 && cp < 0x80) || (k == 2 && cp < 0x800) || (k == 3 && (cp < 0x10000 || cp > 0x10FFFF)) ||
                (cp >= 0xD800 && cp <= 0xDFFF))
                return false;
            i += k + 1;
        }
        return true;
    }

  private:
    const uint8_t* buf_;
    size_t len_;
    size_t pos_ = 0;
};

static Meta read_value(Reader& r, uint32_t vtype, uint32_t depth) {  // gguf.rs:567-605
    Meta m;
    m.type = vtype;
    const char* W = "metadata value";
    switch (vtype) {
        case 0: m.u = r.num<uint8_t>(W); break;
        case 1: m.i = r.num<int8_t>(W); break;
        case 2: m.u = r.num<uint16_t>(W); break;
        case 3: m.i = r.num<int16_t>(W); break;
        case 4: m.u = r.num<uint32_t>(W); break;
        case 5: m.i = r.num<int32_t>(W); break;
        case 6: m.f = r.num<float>(W); break;
        case 7: m.u = r.num<uint8_t>(W) != 0; break;
        case 8: m.s = r.str("metadata string", SIZE_MAX); break;
        case 9: {
            if (depth >= kMaxArrayDepth)
                throw ParseError{"metadata arrays are nested deeper than " + std::to_string(kMaxArrayDepth) + " levels"};
            m.arr_type = r.num<uint32_t>("array element type");
            size_t min_item;
            switch (m.arr_type) {
                case 0: case 1: case 7: min_item = 1; break;
                case 2: case 3: min_item = 2; break;
                case 4: case 5: case 6: min_item = 4; break;
                case 8: case 10: case 11: case 12: min_item = 8; break;
                case 9: min_item = 12; break;
                default: throw ParseError{"unsupported metadata array element type " + std::to_string(m.arr_type)};
            }
            const size_t n = r.count("metadata array length", min_item);
            m.arr.reserve(n);
            for (size_t k = 0; k < n; ++k) m.arr.push_back(read_value(r, m.arr_type, depth + 1));
            break;
        }
        case 10: m.u = r.num<uint64_t>(W); break;
        case 11: m.i = r.num<int64_t>(W); break;
        case 12: m.f = r.num<double>(W); break;
        default: throw ParseError{"unsupported GGUF metadata type code " + std::to_string(vtype)};
    }
    return m;
}

// The value as an unsigned integer (unsigned types, or signed ones that are not negative; gguf.rs:88-98).
static bool meta_u64(const Meta& m, uint64_t* out) {
    switch (m.type) {
        case 0: case 2: case 4: case 10: *out = m.u; return true;
        case 5: case 11:
            if (m.i < 0) return false;
            *out = static_cast<uint64_t>(m.i);
            return true;
        default: return false;
    }
}

static uint64_t tensor_bytes(const TensorRec& t) {  // gguf.rs:159-176
    const uint64_t n = t.n_elem;
    switch (t.type) {
        case VX_GGML_F32: return n * 4;
        case VX_GGML_F16: case VX_GGML_BF16: return n * 2;
        case VX_GGML_Q8_0: return n % 32 == 0 ? n / 32 * 34 : 0;
        case VX_GGML_I2_S: return (n + 3) / 4;
        case VX_GGML_TQ1_0: return n % 256 == 0 ? n / 256 * kTq1Bytes : 0;
        case VX_GGML_TQ2_0: return n % 256 == 0 ? n / 256 * kTq2Bytes : 0;
        case VX_GGML_Q2_0: return t.block_size && n % t.block_size == 0 ? n / t.block_size * (2 + t.block_size / 4) : 0;
        default: return 0;
    }
}

// Q2_0's block size is not stored (gguf.rs:460-508): the payload ends less than one alignment before the next tensor,
// which singles out 64 or 128 for tensors of realistic size; undecided tensors take the others' size, or 64.
static void detect_q2_block(std::vector<TensorRec>& ts, uint64_t data_len, uint64_t alignment) {
    std::vector<uint64_t> starts;
    for (const auto& t : ts) starts.push_back(t.offset);
    std::sort(starts.begin(), starts.end());
    starts.erase(std::unique(starts.begin(), starts.end()), starts.end());
    int decided = 0;
    std::vector<std::pair<size_t, int>> cand;
    for (size_t k = 0; k < ts.size(); ++k) {
        const TensorRec& t = ts[k];
        if (t.type != VX_GGML_Q2_0) continue;
        const uint64_t n = t.n_elem;
        const auto it = std::upper_bound(starts.begin(), starts.end(), t.offset);  // the next tensor's start
        const uint64_t next = it == starts.end() ? data_len : *it;
        const uint64_t room = next > t.offset ? next - t.offset : 0;
        auto fits = [&](uint64_t bs) {
            if (n % bs) return false;
            const uint64_t len = n / bs * (2 + bs / 4);
            return len <= room && (next == data_len || room - len < std::max<uint64_t>(alignment, 1));
        };
        const bool f64 = fits(64), f128 = fits(128);
        if (!f64 && !f128)
            throw ParseError{"Q2_0 tensor '" + t.name + "' (" + std::to_string(n) + " elements, " + std::to_string(room) +
                             " bytes) matches neither 64- nor 128-weight blocks"};
        cand.emplace_back(k, f64 && f128 ? 0 : (f64 ? 64 : 128));
    }
    for (auto& c : cand)
        if (c.second) {
            if (decided && decided != c.second)
                throw ParseError{"Q2_0 tensors with different block sizes ('" + ts[c.first].name + "' uses " +
                                 std::to_string(c.second) + ")"};
            decided = c.second;
        }
    for (auto& c : cand) ts[c.first].block_size = decided ? decided : 64;
}

}  // namespace vx

struct vx_gguf {
    uint32_t magic;
    void* map;
    size_t len;
    uint32_t version;
    size_t data_start;
    std::vector<std::pair<std::string, vx::Meta>> meta;  // file order
    std::unordered_map<std::string, size_t> meta_idx;
    std::vector<vx::TensorRec> tensors;                  // ordered by position in the file
    std::unordered_map<std::string, size_t> tensor_idx;
    const uint8_t* base() const { return static_cast<const uint8_t*>(map); }
};

namespace vx {

constexpr uint32_t kGgufMagic = 0x56584746u;  // "VXGF"

static void parse(vx_gguf* g) {  // gguf.rs:189-313
    Reader r(g->base(), g->len);
    const uint8_t* magic = r.take(4, "magic bytes");
    if (std::memcmp(magic, "GGUF", 4) != 0) throw ParseError{"invalid GGUF magic header bytes"};
    g->version = r.num<uint32_t>("version");
    if (g->version < 2 || g->version > 3)
        throw ParseError{"unsupported GGUF version " + std::to_string(g->version) + " (supported: 2 and 3)"};
    const size_t n_tensors = r.count("tensor count", kMinTensorEntry);
    const size_t n_meta = r.count("metadata count", kMinMetaEntry);
    g->meta.reserve(n_meta);
    for (size_t k = 0; k < n_meta; ++k) {
        std::string key = r.str("metadata key", kMaxNameLen);
        const uint32_t vt = r.num<uint32_t>("metadata value type");
        Meta v = read_value(r, vt, 0);
        if (!g->meta_idx.emplace(key, g->meta.size()).second) throw ParseError{"duplicate metadata key '" + key + "'"};
        g->meta.emplace_back(std::move(key), std::move(v));
    }
    std::vector<TensorRec> ts;
    ts.reserve(n_tensors);
    for (size_t k = 0; k < n_tensors; ++k) {
        TensorRec t;
        t.name = r.str("tensor name", kMaxNameLen);
        t.n_dims = r.num<uint32_t>("tensor dimension count");
        if (t.n_dims < 1 || t.n_dims > kMaxDims)
            throw ParseError{"tensor '" + t.name + "' has " + std::to_string(t.n_dims) + " dimensions (supported: 1 to 8)"};
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            const uint64_t v = r.num<uint64_t>("tensor dimension");
            if (v != 0 && t.n_elem > kMaxElements / v)
                throw ParseError{"tensor '" + t.name + "' has more than 2^40 elements"};
            t.dims[d] = v;
            t.n_elem *= v;
        }
        t.type = r.num<uint32_t>("tensor type");
        t.offset = r.num<uint64_t>("tensor offset");
        ts.push_back(std::move(t));
    }
    uint64_t alignment = 32;
    auto it = g->meta_idx.find("general.alignment");
    if (it != g->meta_idx.end()) {
        if (!meta_u64(g->meta[it->second].second, &alignment) || alignment == 0 || (alignment & (alignment - 1)))
            throw ParseError{"general.alignment must be an unsigned integer that is a power of two"};
    }
    const uint64_t pos = r.pos();
    const uint64_t data_start = (pos + alignment - 1) / alignment * alignment;
    if (data_start < pos || data_start > g->len)
        throw ParseError{"the tensor data section would start beyond the end of the file (" + std::to_string(g->len) + " bytes)"};
    const uint64_t data_len = g->len - data_start;
    if (std::any_of(ts.begin(), ts.end(), [](const TensorRec& t) { return t.type == VX_GGML_Q2_0; }))
        detect_q2_block(ts, data_len, alignment);
    std::vector<std::pair<std::pair<uint64_t, uint64_t>, std::string>> ranges;
    std::unordered_set<std::string> names;
    for (auto& t : ts) {
        if (!names.insert(t.name).second) throw ParseError{"duplicate tensor name '" + t.name + "'"};
        if (t.offset > data_len) throw ParseError{"tensor '" + t.name + "' starts beyond the end of the file"};
        if (t.offset % alignment)
            throw ParseError{"tensor '" + t.name + "' has offset " + std::to_string(t.offset) +
                             ", which is not a multiple of the alignment " + std::to_string(alignment)};
        t.byte_len = tensor_bytes(t);
        if (t.byte_len) {
            if (t.byte_len > data_len - t.offset)
                throw ParseError{"tensor '" + t.name + "' (" + std::to_string(t.byte_len) + " bytes) extends beyond the end of the file"};
            ranges.push_back({{t.offset, t.offset + t.byte_len}, t.name});
        }
    }
    std::sort(ranges.begin(), ranges.end());
    for (size_t k = 1; k < ranges.size(); ++k)
        if (ranges[k - 1].first.second > ranges[k].first.first)
            throw ParseError{"the data of tensors '" + ranges[k - 1].second + "' and '" + ranges[k].second + "' overlaps"};
    std::stable_sort(ts.begin(), ts.end(), [](const TensorRec& a, const TensorRec& b) { return a.offset < b.offset; });
    g->data_start = static_cast<size_t>(data_start);
    g->tensors = std::move(ts);
    for (size_t k = 0; k < g->tensors.size(); ++k) g->tensor_idx.emplace(g->tensors[k].name, k);
}

static void close_file(vx_gguf* g) {
    if (g->map) munmap(g->map, g->len);
    g->magic = 0;
    delete g;
}

static int check_gguf(const vx_gguf_t* g) {
    if (g == nullptr) VX_FAIL(VX_ERR_INVALID_HANDLE, "GGUF handle is NULL");
    if (g->magic != kGgufMagic) VX_FAIL(VX_ERR_INVALID_HANDLE, "GGUF handle is not valid (closed or foreign)");
    return VX_OK;
}

static const char* type_name(uint32_t t) {
    switch (t) {
        case VX_GGML_F32: return "F32";
        case VX_GGML_F16: return "F16";
        case VX_GGML_Q8_0: return "Q8_0";
        case VX_GGML_BF16: return "BF16";
        case VX_GGML_TQ1_0: return "TQ1_0";
        case VX_GGML_TQ2_0: return "TQ2_0";
        case VX_GGML_I2_S: return "I2_S";
        case VX_GGML_Q2_0: return "Q2_0";
        default: return "UNKNOWN";
    }
}

static int fill_info(const vx_gguf* g, size_t k, vx_tensor_info_t* out) {
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_info is NULL");
    if (out->struct_size != sizeof(vx_tensor_info_t))
        VX_FAIL(VX_ERR_INVALID_ARGUMENT, "out_info.struct_size is %u, expected %zu", out->struct_size, sizeof(vx_tensor_info_t));
    const TensorRec& t = g->tensors[k];
    out->ggml_type = static_cast<int32_t>(t.type);
    out->n_dims = t.n_dims;
    out->is_ternary = t.type == VX_GGML_I2_S || t.type == VX_GGML_TQ1_0 || t.type == VX_GGML_TQ2_0;
    for (uint32_t d = 0; d < kMaxDims; ++d) out->shape[d] = d < t.n_dims ? t.dims[d] : 0;
    out->num_elements = t.n_elem;
    out->offset = t.offset;
    out->data_bytes = t.byte_len;
    out->name = t.name.c_str();
    out->type_name = type_name(t.type);
    out->block_size = t.block_size;
    return VX_OK;
}

static int find(const vx_gguf* g, const char* name, size_t* k) {
    if (name == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "name is NULL");
    auto it = g->tensor_idx.find(name);
    if (it == g->tensor_idx.end()) VX_FAIL(VX_ERR_NOT_FOUND, "no tensor '%s' in the file", name);
    *k = it->second;
    return VX_OK;
}

static const uint8_t* payload(const vx_gguf* g, const TensorRec& t) { return g->base() + g->data_start + t.offset; }

// A 2-D tensor as a matrix: shape [cols, rows] (quintrit.h:250).
static int matrix_shape(const TensorRec& t, size_t* rows, size_t* cols) {
    if (t.n_dims != 2) VX_FAIL(VX_ERR_INVALID_SHAPE, "tensor '%s' has %u dimensions, a matrix has 2", t.name.c_str(), t.n_dims);
    *cols = static_cast<size_t>(t.dims[0]);
    *rows = static_cast<size_t>(t.dims[1]);
    return VX_OK;
}

static float half_f32(uint16_t h) {  // decoders/mod.rs:89-111, an exact widening
    _Float16 v;
    std::memcpy(&v, &h, 2);
    return static_cast<float>(v);
}

// The per-tensor weight scale (gguf.rs:342-360, transcoder.rs:224-236): the f32 after an I2_S payload, the common
// block scale of TQ1_0 / TQ2_0 (differing block scales cannot be represented: VX_ERR_FORMAT), 1 otherwise.
static int tensor_scale(const vx_gguf* g, const TensorRec& t, float* out) {
    *out = 1.0f;
    if (t.type == VX_GGML_I2_S) {
        const uint64_t at = g->data_start + t.offset + t.byte_len;
        if (at + 4 <= g->len) std::memcpy(out, g->base() + at, 4);
        return VX_OK;
    }
    if (t.type != VX_GGML_TQ1_0 && t.type != VX_GGML_TQ2_0) return VX_OK;
    const size_t bb = t.type == VX_GGML_TQ1_0 ? kTq1Bytes : kTq2Bytes, so = bb - 2;
    if (t.byte_len == 0) return VX_OK;
    const uint8_t* p = payload(g, t);
    uint16_t first;
    std::memcpy(&first, p + so, 2);
    for (uint64_t off = bb; off < t.byte_len; off += bb) {
        uint16_t d;
        std::memcpy(&d, p + off + so, 2);
        if (d != first)
            VX_FAIL(VX_ERR_FORMAT, "tensor '%s' has differing per-block scales, which a per-tensor weight scale cannot represent",
                    t.name.c_str());
    }
    *out = half_f32(first);
    return VX_OK;
}

static void json_str(std::string& o, const std::string& s) {
    o += '"';
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') {
            o += '\\';
            o += static_cast<char>(c);
        } else if (c < 0x20) {
            char b[8];
            std::snprintf(b, sizeof b, "\\u%04x", c);
            o += b;
        } else {
            o += static_cast<char>(c);
        }
    }
    o += '"';
}

static void json_value(std::string& o, const Meta& m) {
    char b[40];
    switch (m.type) {
        case 0: case 2: case 4: case 10: std::snprintf(b, sizeof b, "%llu", static_cast<unsigned long long>(m.u)); o += b; break;
        case 1: case 3: case 5: case 11: std::snprintf(b, sizeof b, "%lld", static_cast<long long>(m.i)); o += b; break;
        case 6: case 12:
            if (m.f != m.f) o += "NaN";
            else if (m.f == __builtin_inf()) o += "Infinity";
            else if (m.f == -__builtin_inf()) o += "-Infinity";
            else {
                std::snprintf(b, sizeof b, "%.17g", m.f);  // an f32 is widened exactly; 17 digits round-trip a double
                o += b;
            }
            break;
        case 7: o += m.u ? "true" : "false"; break;
        case 8: json_str(o, m.s); break;
        default:
            o += '[';
            for (size_t k = 0; k < m.arr.size(); ++k) {
                if (k) o += ',';
                json_value(o, m.arr[k]);
            }
            o += ']';
    }
}

static int upload_ggml(uint32_t type, const uint8_t* data, bool data_on_device, size_t len, size_t rows, size_t cols,
                       float weight_scale, vx_matrix_t** out) {
    if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_matrix is NULL");
    *out = nullptr;
    if (data == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "data is NULL");
    VX_TRY(check_ternary(type, len, rows, cols));
    const size_t need = ggml_payload_bytes(type, rows, cols);
    const size_t planar_len = rows * planar_row_bytes(cols);
    uint8_t* d_src = nullptr;
    uint8_t* d_planar = nullptr;
    hipError_t e = hipSuccess;
    if (!data_on_device) {
        e = hipMalloc(&d_src, need);
        if (e == hipSuccess) e = hipMemcpy(d_src, data, need, hipMemcpyHostToDevice);
    }
    if (e == hipSuccess) e = hipMalloc(&d_planar, planar_len);
    if (e == hipSuccess) {
        const uint64_t n = planar_len;
        hipLaunchKernelGGL(ggml_to_planar_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, nullptr,
                           type, data_on_device ? data : d_src, static_cast<uint64_t>(rows), static_cast<uint64_t>(cols),
                           d_planar);
        e = hipGetLastError();
    }
    int st = VX_OK;
    if (e == hipSuccess) st = vx_matrix_create_dev(d_planar, planar_len, rows, cols, weight_scale, out);
    if (d_src) (void)hipFree(d_src);
    if (d_planar) (void)hipFree(d_planar);
    if (e != hipSuccess) VX_FAIL(VX_ERR_DEVICE, "GGUF upload failed: %s", hipGetErrorString(e));
    return st;
}



// decode_q2_0_packed (decoders/q2_0.rs:17-30,58-155) on the host: the planar velurex bytes of a Q2_0 tensor and one f16
// scale per 64 weights of a row (a 128-weight block's scale twice). A code 3 is an error naming the first such weight.
static int q2_0_convert(const vx_gguf* g, const TensorRec& t, std::vector<uint8_t>* planar, std::vector<uint16_t>* scales,
                        size_t* rows_out, size_t* cols_out) {
    size_t rows, cols;
    VX_TRY(matrix_shape(t, &rows, &cols));
    if (t.type != VX_GGML_Q2_0) VX_FAIL(VX_ERR_UNSUPPORTED, "tensor '%s' (type %u) is not Q2_0", t.name.c_str(), t.type);
    const uint32_t bs = t.block_size;
    if (bs != 64 && bs != 128) VX_FAIL(VX_ERR_FORMAT, "tensor '%s': Q2_0 block size %u is not supported (64 or 128)", t.name.c_str(), bs);
    VX_TRY(check_shape(rows, cols));
    if (cols % bs) VX_FAIL(VX_ERR_INVALID_SHAPE, "a Q2_0 row of %zu weights is not a multiple of the block size %u", cols, bs);
    const size_t bb = 2 + bs / 4, nblk = rows * cols / bs;
    if (t.byte_len != nblk * bb) VX_FAIL(VX_ERR_FORMAT, "tensor '%s': the payload is not %zu blocks of %zu bytes", t.name.c_str(), nblk, bb);
    const uint8_t* src = payload(g, t);
    for (size_t b = 0; b < nblk; ++b) {
        const uint8_t* q = src + b * bb + 2;
        for (uint32_t j = 0; j < bs / 4; ++j)
            if (q[j] & (q[j] >> 1) & 0x55u) {
                uint32_t k = 0;
                while (((q[j] >> (2 * k)) & 3u) != 3u) ++k;
                VX_FAIL(VX_ERR_FORMAT, "Q2_0 weight %zu uses code 3 (+2), which is not ternary", b * bs + 4 * j + k);
            }
    }
    planar->resize(rows * planar_row_bytes(cols));
    host_to_planar(bs == 64 ? kQ2Block64 : kQ2Block128, src, rows, cols, planar->data());
    scales->resize(rows * cols / 64);
    for (size_t b = 0; b < nblk; ++b) {
        uint16_t d;
        std::memcpy(&d, src + b * bb, 2);
        for (uint32_t s = 0; s < bs / 64; ++s) (*scales)[b * (bs / 64) + s] = d;
    }
    *rows_out = rows;
    *cols_out = cols;
    return VX_OK;
}

// ---- model loading (quintrit_model_open_gpu) ----------------------------------------------------------------------

static const Meta* meta_get(const vx_gguf* g, const std::string& key) {
    auto it = g->meta_idx.find(key);
    return it == g->meta_idx.end() ? nullptr : &g->meta[it->second].second;
}

// GgufMetadataValue::as_usize (gguf.rs:90-104), and config.rs:502-507 scalar_or_max: an array gives its largest entry.
static bool meta_usize(const Meta* m, bool or_max, uint64_t* out) {
    if (m == nullptr) return false;
    if (or_max && m->type == 9) {
        bool any = false;
        uint64_t best = 0, v;
        for (const Meta& e : m->arr)
            if (meta_u64(e, &v)) best = any ? std::max(best, v) : v, any = true;
        *out = best;
        return any;
    }
    return meta_u64(*m, out);
}

// GgufMetadataValue::as_f32 (gguf.rs:106-112): f32, or f64 narrowed.
static bool meta_f32(const Meta* m, float* out) {
    if (m == nullptr || (m->type != 6 && m->type != 12)) return false;
    *out = static_cast<float>(m->f);
    return true;
}

// The tensor names of a layer (quintrit-runtime/src/engine.rs:455-480), in the order of the projection / norm kinds.
static const char* const kProjNames[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
static const char* const kNormNames[4] = {"attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm"};

static const TensorRec* tensor_get(const vx_gguf* g, const std::string& name) {
    auto it = g->tensor_idx.find(name);
    return it == g->tensor_idx.end() ? nullptr : &g->tensors[it->second];
}

// ModelConfig::from_gguf (quintrit-runtime/src/config.rs:257-440) with validate_gguf_model's table checks
// (validate.rs:199-240) and GpuModel::check_supported / context_for (gpu.rs:141-179), narrowed to what this decoder
// runs. A file the reference rejects is VX_ERR_MODEL; a model it runs but not on this decoder is VX_ERR_UNSUPPORTED.
static int gguf_decoder_config(const vx_gguf* g, uint32_t context_limit, vx_decoder_config_t* c) {
    const Meta* am = meta_get(g, "general.architecture");
    const std::string arch = am != nullptr && am->type == 8 ? am->s : "bitnet-b1.58";
    auto key = [&](const char* k) { return meta_get(g, arch + "." + k); };
    if (arch == "qwen3" || arch == "qwen35" || arch == "nemotron_h_moe")
        VX_FAIL(VX_ERR_UNSUPPORTED, "architecture '%s' (query/key norms, hybrid or mixture-of-experts layers) is not "
                "supported by this decoder", arch.c_str());
    const bool bitnet = arch == "bitnet" || arch == "bitnet-b1.58";
    uint64_t vocab = 0, hidden = 2560, ffn = 6912, layers = 30, heads = 20, kv_heads = 5, ctx = 4096, v;
    const TensorRec* emb = tensor_get(g, "token_embd.weight");
    const Meta* tokens = meta_get(g, "tokenizer.ggml.tokens");
    if (meta_usize(key("vocab_size"), false, &v)) vocab = v;
    else if (emb != nullptr && emb->n_dims > 1) vocab = emb->dims[1];
    else if (tokens != nullptr && tokens->type == 9) vocab = tokens->arr.size();
    else vocab = 128256;
    if (meta_usize(key("embedding_length"), false, &v)) hidden = v;
    if (meta_usize(key("feed_forward_length"), true, &v)) ffn = v;
    if (meta_usize(key("block_count"), false, &v)) layers = v;
    if (meta_usize(key("attention.head_count"), true, &v)) heads = v;
    if (meta_usize(key("attention.head_count_kv"), true, &v)) kv_heads = v;
    if (meta_usize(key("context_length"), false, &v)) ctx = v;
    float eps = 1e-5f, theta = 500000.0f;
    meta_f32(key("attention.layer_norm_rms_epsilon"), &eps);
    meta_f32(key("rope.freq_base"), &theta);
    const uint64_t dims[] = {vocab, hidden, ffn, layers, heads, kv_heads, ctx};
    for (uint64_t d : dims)
        if (d == 0 || d > (uint64_t{1} << 24)) VX_FAIL(VX_ERR_MODEL, "a model dimension of '%s' is 0 or absurd (%llu)", arch.c_str(),
                                                       static_cast<unsigned long long>(d));
    uint64_t head_dim = hidden / heads;
    if (meta_usize(key("attention.key_length"), false, &v)) head_dim = v;
    if (head_dim == 0 || head_dim % 2 || head_dim > 4096)
        VX_FAIL(VX_ERR_MODEL, "metadata '%s.attention.key_length' = %llu must be even and in 2..=4096", arch.c_str(),
                static_cast<unsigned long long>(head_dim));
    uint64_t n_rot = head_dim;
    if (meta_usize(key("rope.dimension_count"), false, &v)) n_rot = v;
    if (n_rot == 0 || n_rot % 2 || n_rot > head_dim)
        VX_FAIL(VX_ERR_MODEL, "metadata '%s.rope.dimension_count' = %llu must be even and at most the head dimension",
                arch.c_str(), static_cast<unsigned long long>(n_rot));
    if (n_rot != head_dim) VX_FAIL(VX_ERR_UNSUPPORTED, "partial RoPE (%llu of %llu dimensions) is not supported",
                                   static_cast<unsigned long long>(n_rot), static_cast<unsigned long long>(head_dim));
    const Meta* sc = key("rope.scaling.type");
    const std::string scaling = sc != nullptr && sc->type == 8 ? sc->s : "none";
    float factor = 0.0f;
    meta_f32(key("rope.scaling.factor"), &factor);
    if (scaling != "none" && scaling != "linear" && scaling != "yarn")
        VX_FAIL(VX_ERR_MODEL, "RoPE scaling type '%s' is not supported", scaling.c_str());
    if (scaling != "none" && !(scaling == "linear" && (factor == 0.0f || factor == 1.0f)))
        VX_FAIL(VX_ERR_UNSUPPORTED, "RoPE scaling '%s' (factor %g) is not supported by this decoder", scaling.c_str(), factor);
    // validate.rs:207-240: a tokenizer, and the F16 tables and F32 output norm of the declared sizes.
    if (tokens == nullptr || tokens->type != 9 || tokens->arr.empty() || tokens->arr.size() > vocab)
        VX_FAIL(VX_ERR_MODEL, "metadata 'tokenizer.ggml.tokens' is missing, empty or longer than the vocabulary (%llu)",
                static_cast<unsigned long long>(vocab));
    bool any_i2s = false;
    for (const TensorRec& t : g->tensors) {
        if (t.type == VX_GGML_Q2_0)
            VX_FAIL(VX_ERR_UNSUPPORTED, "block-scaled (Q2_0) models run on the CPU only; the GPU decoder supports I2_S models");
        any_i2s |= t.type == VX_GGML_I2_S;
    }
    if (!any_i2s)
        VX_FAIL(VX_ERR_UNSUPPORTED, "the GPU decoder reproduces the bitnet.cpp attention numerics only (I2_S models)");
    for (const char* name : {"token_embd.weight", "output.weight"}) {
        const TensorRec* t = tensor_get(g, name);
        if (t == nullptr) {
            if (std::strcmp(name, "output.weight") == 0) continue;
            VX_FAIL(VX_ERR_MODEL, "tensor '%s' is missing", name);
        }
        if (t->type == VX_GGML_Q2_0 || t->type == VX_GGML_Q8_0)
            VX_FAIL(VX_ERR_UNSUPPORTED, "%s is not F16; the GPU decoder needs an F16 embedding and head", name);
        if (t->type != VX_GGML_F16) VX_FAIL(VX_ERR_MODEL, "tensor '%s' has type %u, expected F16", name, t->type);
        if (t->n_elem != vocab * hidden)
            VX_FAIL(VX_ERR_MODEL, "tensor '%s' has %llu elements, expected %llu", name, static_cast<unsigned long long>(t->n_elem),
                    static_cast<unsigned long long>(vocab * hidden));
    }
    const TensorRec* on = tensor_get(g, "output_norm.weight");
    if (on == nullptr || on->type != VX_GGML_F32 || on->n_elem != hidden)
        VX_FAIL(VX_ERR_MODEL, "tensor 'output_norm.weight' is missing or not %llu F32 values", static_cast<unsigned long long>(hidden));
    if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)  // gpu.rs:163-165
        VX_FAIL(VX_ERR_UNSUPPORTED, "head dimension %llu is not supported (32, 64, 128 or 256)",
                static_cast<unsigned long long>(head_dim));
    // validate.rs:241-290: every layer's projections (ternary, of the configured shapes) and F32 norms.
    const uint64_t qd = heads * head_dim, kvd = kv_heads * head_dim;
    const uint64_t shape[7][2] = {{qd, hidden}, {kvd, hidden}, {kvd, hidden}, {hidden, qd},
                                 {ffn, hidden}, {ffn, hidden}, {hidden, ffn}};
    char name[96];
    for (uint64_t l = 0; l < layers; ++l) {
        for (uint32_t k = 0; k < 7; ++k) {
            std::snprintf(name, sizeof name, "blk.%llu.%s.weight", static_cast<unsigned long long>(l), kProjNames[k]);
            const TensorRec* t = tensor_get(g, name);
            if (t == nullptr) VX_FAIL(VX_ERR_MODEL, "tensor '%s' is missing", name);
            if (t->n_dims != 2 || t->dims[0] != shape[k][1] || t->dims[1] != shape[k][0])
                VX_FAIL(VX_ERR_MODEL, "tensor '%s' has the wrong shape, expected [%llu, %llu]", name,
                        static_cast<unsigned long long>(shape[k][1]), static_cast<unsigned long long>(shape[k][0]));
            if (t->type != VX_GGML_I2_S && t->type != VX_GGML_TQ1_0 && t->type != VX_GGML_TQ2_0)
                VX_FAIL(VX_ERR_MODEL, "tensor '%s' (type %u) is not a ternary tensor", name, t->type);
            VX_TRY(check_ternary(t->type, static_cast<size_t>(t->byte_len), shape[k][0], shape[k][1]));
            float scale;
            VX_TRY(tensor_scale(g, *t, &scale));
        }
        for (uint32_t k = 0; k < 4; ++k) {
            if ((k == VX_NORM_ATTN_SUB || k == VX_NORM_FFN_SUB) && !bitnet) continue;
            std::snprintf(name, sizeof name, "blk.%llu.%s.weight", static_cast<unsigned long long>(l), kNormNames[k]);
            const TensorRec* t = tensor_get(g, name);
            // The attention sub-norm acts on the n_heads * head_dim attention output, the FFN sub-norm on the ffn-wide
            // gated vector (attention.rs:230-240, model.rs:155-190).
            // A sub-norm may hold more values than are used (validate.rs:253-256: at least q_dim / ffn).
            const bool sub = k == VX_NORM_ATTN_SUB || k == VX_NORM_FFN_SUB;
            const uint64_t n = k == VX_NORM_ATTN_SUB ? qd : k == VX_NORM_FFN_SUB ? ffn : hidden;
            if (t == nullptr || t->type != VX_GGML_F32 || t->n_elem < n || (!sub && t->n_elem != n))
                VX_FAIL(VX_ERR_MODEL, "tensor '%s' is missing or not %s%llu F32 values", name, sub ? "at least " : "",
                        static_cast<unsigned long long>(n));
        }
    }
    // gpu.rs:141-146: the model's maximum, at most the caller's limit (default 4096, gpu.rs:30) and 7936
    // (quintrit-cuda/src/layer.rs:66-67), rounded down to a multiple of 256.
    uint64_t want = std::min<uint64_t>(ctx, context_limit ? context_limit : 4096);
    want = std::min<uint64_t>(want, 7936);
    if (want >= 256) want = want / 256 * 256;
    *c = vx_decoder_config_t{};
    c->struct_size = sizeof(vx_decoder_config_t);
    c->n_layers = static_cast<uint32_t>(layers);
    c->hidden = static_cast<uint32_t>(hidden);
    c->n_heads = static_cast<uint32_t>(heads);
    c->n_kv_heads = static_cast<uint32_t>(kv_heads);
    c->head_dim = static_cast<uint32_t>(head_dim);
    c->ffn = static_cast<uint32_t>(ffn);
    c->vocab = static_cast<uint32_t>(vocab);
    c->max_ctx = static_cast<uint32_t>(want);
    c->rms_eps = eps;
    c->rope_theta = theta;
    c->act = bitnet ? VX_ACT_RELU2 : VX_ACT_SILU;  // config.rs:419-422
    // config.rs:464-467 (rope_from_gguf): NEOX for BitNet and Qwen2, Normal for Falcon3 / LLaMA.
    c->rope_mode = bitnet || arch == "qwen2" ? VX_ROPE_NEOX : VX_ROPE_NORMAL;
    c->no_sub_norm = bitnet ? 0 : 1;  // has_sub_norm (config.rs:424)
    c->emb_f16 = 1;
    c->untied = tensor_get(g, "output.weight") != nullptr ? 1 : 0;  // tie_word_embeddings (config.rs:425)
    return VX_OK;
}

// GpuModel::load (gpu.rs:183-260): every projection converted to velurex in HBM (the reference converts on the host,
// gpu.rs:120-138; the bytes are the same), the F32 norms and the F16 tables handed to the decoder.
// The tensors were checked by gguf_decoder_config.
static int gguf_load_decoder(const vx_gguf* g, vx_decoder_t* d, const vx_decoder_config_t& c) {
    char name[96];
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        for (uint32_t k = 0; k < 7; ++k) {
            // The payload goes to the GPU in its GGUF size and is converted there (vx_gguf_upload_matrix).
            std::snprintf(name, sizeof name, "blk.%u.%s.weight", l, kProjNames[k]);
            vx_matrix_t* m = nullptr;
            VX_TRY(vx_gguf_upload_matrix(g, name, &m));
            const int st = vx_decoder_adopt_projection(d, l, k, m);
            if (st != VX_OK) {
                const std::string msg = vx_last_error_message();
                vx_matrix_free(m);
                set_error(st, msg);
                return st;
            }
        }
        for (uint32_t k = 0; k < 4; ++k) {
            if ((k == VX_NORM_ATTN_SUB || k == VX_NORM_FFN_SUB) && c.no_sub_norm) continue;
            std::snprintf(name, sizeof name, "blk.%u.%s.weight", l, kNormNames[k]);
            const TensorRec* t = tensor_get(g, name);
            const size_t n = k == VX_NORM_ATTN_SUB ? size_t{c.n_heads} * c.head_dim : k == VX_NORM_FFN_SUB ? c.ffn : c.hidden;
            VX_TRY(vx_decoder_set_norm(d, l, k, reinterpret_cast<const float*>(payload(g, *t)), n));
        }
    }
    const TensorRec* on = tensor_get(g, "output_norm.weight");
    VX_TRY(vx_decoder_set_norm(d, c.n_layers, VX_NORM_ATTN, reinterpret_cast<const float*>(payload(g, *on)), c.hidden));
    const size_t table = size_t{c.vocab} * c.hidden;
    const TensorRec* emb = tensor_get(g, "token_embd.weight");
    VX_TRY(vx_decoder_set_embedding_f16(d, reinterpret_cast<const uint16_t*>(payload(g, *emb)), table));
    if (c.untied)
        VX_TRY(vx_decoder_set_head(d, reinterpret_cast<const uint16_t*>(payload(g, *tensor_get(g, "output.weight"))), table));
    return VX_OK;
}
}  // namespace vx

extern "C" {

using namespace vx;

int vx_gguf_open(const char* path, vx_gguf_t** out_gguf) {
    return guard([&]() -> int {
        if (out_gguf == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_gguf is NULL");
        *out_gguf = nullptr;
        if (path == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "path is NULL");
        const int fd = open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) VX_FAIL(VX_ERR_IO, "cannot open '%s': %s", path, std::strerror(errno));
        struct stat sb;
        if (fstat(fd, &sb) != 0) {
            const int er = errno;
            close(fd);
            VX_FAIL(VX_ERR_IO, "cannot stat '%s': %s", path, std::strerror(er));
        }
        vx_gguf* g = new vx_gguf();
        g->magic = kGgufMagic;
        g->len = static_cast<size_t>(sb.st_size);
        g->map = nullptr;
        if (g->len > 0) {
            void* p = mmap(nullptr, g->len, PROT_READ, MAP_PRIVATE, fd, 0);
            if (p == MAP_FAILED) {
                const int er = errno;
                close(fd);
                delete g;
                VX_FAIL(VX_ERR_IO, "cannot map '%s': %s", path, std::strerror(er));
            }
            g->map = p;
        }
        close(fd);
        try {
            parse(g);
        } catch (const ParseError& pe) {
            close_file(g);
            VX_FAIL(VX_ERR_FORMAT, "%s", pe.msg.c_str());
        }
        *out_gguf = g;
        return VX_OK;
    });
}

int vx_gguf_close(vx_gguf_t* g) {
    return guard([&]() -> int {
        if (g == nullptr) return VX_OK;
        VX_TRY(check_gguf(g));
        close_file(g);
        return VX_OK;
    });
}

int vx_gguf_info(const vx_gguf_t* g, vx_gguf_info_t* out) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_info is NULL");
        if (out->struct_size != sizeof(vx_gguf_info_t))
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "out_info.struct_size is %u, expected %zu", out->struct_size, sizeof(vx_gguf_info_t));
        out->version = g->version;
        out->tensor_count = g->tensors.size();
        out->metadata_count = g->meta.size();
        out->data_offset = g->data_start;
        return VX_OK;
    });
}

int vx_gguf_tensor_at(const vx_gguf_t* g, size_t index, vx_tensor_info_t* out) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        if (index >= g->tensors.size())
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "tensor index %zu out of range (%zu tensors)", index, g->tensors.size());
        return fill_info(g, index, out);
    });
}

int vx_gguf_tensor_find(const vx_gguf_t* g, const char* name, vx_tensor_info_t* out) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        size_t k;
        VX_TRY(find(g, name, &k));
        return fill_info(g, k, out);
    });
}

int vx_gguf_metadata_string(const vx_gguf_t* g, const char* key, char* buffer, size_t capacity, size_t* out_len) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        if (key == nullptr || out_len == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "key or out_len is NULL");
        auto it = g->meta_idx.find(key);
        if (it == g->meta_idx.end()) VX_FAIL(VX_ERR_NOT_FOUND, "no metadata key '%s'", key);
        const Meta& m = g->meta[it->second].second;
        if (m.type != 8) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "metadata '%s' is not a string", key);
        *out_len = m.s.size();
        if (capacity <= m.s.size())
            VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "metadata '%s' needs %zu bytes with its NUL", key, m.s.size() + 1);
        if (buffer == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "buffer is NULL");
        std::memcpy(buffer, m.s.data(), m.s.size());
        buffer[m.s.size()] = '\0';
        return VX_OK;
    });
}

int vx_gguf_metadata_u64(const vx_gguf_t* g, const char* key, uint64_t* out_value) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        if (key == nullptr || out_value == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "key or out_value is NULL");
        auto it = g->meta_idx.find(key);
        if (it == g->meta_idx.end()) VX_FAIL(VX_ERR_NOT_FOUND, "no metadata key '%s'", key);
        if (!meta_u64(g->meta[it->second].second, out_value))
            VX_FAIL(VX_ERR_INVALID_ARGUMENT, "metadata '%s' is not an unsigned integer", key);
        return VX_OK;
    });
}

int vx_gguf_metadata_f64(const vx_gguf_t* g, const char* key, double* out_value) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        if (key == nullptr || out_value == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "key or out_value is NULL");
        auto it = g->meta_idx.find(key);
        if (it == g->meta_idx.end()) VX_FAIL(VX_ERR_NOT_FOUND, "no metadata key '%s'", key);
        const Meta& m = g->meta[it->second].second;
        if (m.type != 6 && m.type != 12) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "metadata '%s' is not a float", key);
        *out_value = m.f;
        return VX_OK;
    });
}

int vx_gguf_metadata_json(const vx_gguf_t* g, char* buffer, size_t capacity, size_t* out_len) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        if (out_len == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_len is NULL");
        std::string o = "{";
        for (size_t k = 0; k < g->meta.size(); ++k) {
            if (k) o += ',';
            json_str(o, g->meta[k].first);
            char b[64];
            std::snprintf(b, sizeof b, ":{\"type\":%u,", g->meta[k].second.type);
            o += b;
            if (g->meta[k].second.type == 9) {
                std::snprintf(b, sizeof b, "\"array_type\":%u,", g->meta[k].second.arr_type);
                o += b;
            }
            o += "\"value\":";
            json_value(o, g->meta[k].second);
            o += '}';
        }
        o += '}';
        *out_len = o.size();
        if (capacity <= o.size()) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "the metadata needs %zu bytes with its NUL", o.size() + 1);
        if (buffer == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "buffer is NULL");
        std::memcpy(buffer, o.data(), o.size() + 1);
        return VX_OK;
    });
}

int vx_gguf_tensor_data(const vx_gguf_t* g, const char* name, const uint8_t** out_data, size_t* out_len) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        if (out_data == nullptr || out_len == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_data or out_len is NULL");
        size_t k;
        VX_TRY(find(g, name, &k));
        const TensorRec& t = g->tensors[k];
        if (t.byte_len == 0)
            VX_FAIL(VX_ERR_UNSUPPORTED, "tensor '%s' has type %u, whose layout is not known here", name, t.type);
        *out_data = payload(g, t);
        *out_len = static_cast<size_t>(t.byte_len);
        return VX_OK;
    });
}

int vx_gguf_tensor_scale(const vx_gguf_t* g, const char* name, float* out_scale) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        if (out_scale == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_scale is NULL");
        size_t k;
        VX_TRY(find(g, name, &k));
        return tensor_scale(g, g->tensors[k], out_scale);
    });
}

int vx_ggml_to_planar(int32_t ggml_type, const uint8_t* data, size_t len, size_t rows, size_t cols, uint8_t* out,
                      size_t out_capacity) {
    return guard([&]() -> int {
        if (data == nullptr || out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "data or out is NULL");
        VX_TRY(check_ternary(static_cast<uint32_t>(ggml_type), len, rows, cols));
        const size_t need = rows * planar_row_bytes(cols);
        if (out_capacity < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "out holds %zu bytes, the planar layout needs %zu", out_capacity, need);
        host_to_planar(static_cast<uint32_t>(ggml_type), data, rows, cols, out);
        return VX_OK;
    });
}

int vx_gguf_convert_planar(const vx_gguf_t* g, const char* name, uint8_t* out, size_t out_capacity, size_t* out_rows,
                           size_t* out_cols, float* out_scale) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        size_t k, rows, cols;
        VX_TRY(find(g, name, &k));
        const TensorRec& t = g->tensors[k];
        VX_TRY(matrix_shape(t, &rows, &cols));
        VX_TRY(check_ternary(t.type, static_cast<size_t>(t.byte_len), rows, cols));
        float scale;
        VX_TRY(tensor_scale(g, t, &scale));
        if (out_rows) *out_rows = rows;
        if (out_cols) *out_cols = cols;
        if (out_scale) *out_scale = scale;
        const size_t need = rows * planar_row_bytes(cols);
        if (out_capacity < need) VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "out holds %zu bytes, the planar layout needs %zu", out_capacity, need);
        if (out == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out is NULL");
        host_to_planar(t.type, payload(g, t), rows, cols, out);
        return VX_OK;
    });
}

int vx_matrix_create_ggml_dev(int32_t ggml_type, const uint8_t* data_dev, size_t len, size_t rows, size_t cols,
                              float weight_scale, vx_matrix_t** out_matrix) {
    return guard([&]() -> int {
        return upload_ggml(static_cast<uint32_t>(ggml_type), data_dev, true, len, rows, cols, weight_scale, out_matrix);
    });
}

int vx_gguf_upload_matrix(const vx_gguf_t* g, const char* name, vx_matrix_t** out_matrix) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        size_t k, rows, cols;
        VX_TRY(find(g, name, &k));
        const TensorRec& t = g->tensors[k];
        VX_TRY(matrix_shape(t, &rows, &cols));
        float scale;
        VX_TRY(tensor_scale(g, t, &scale));
        return upload_ggml(t.type, payload(g, t), false, static_cast<size_t>(t.byte_len), rows, cols, scale, out_matrix);
    });
}

int vx_gguf_convert_q2_0(const vx_gguf_t* g, const char* name, uint8_t* planar, size_t planar_capacity,
                         uint16_t* scales_f16, size_t scales_capacity, size_t* out_rows, size_t* out_cols) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        size_t k, rows, cols;
        VX_TRY(find(g, name, &k));
        std::vector<uint8_t> p;
        std::vector<uint16_t> sc;
        VX_TRY(q2_0_convert(g, g->tensors[k], &p, &sc, &rows, &cols));
        if (out_rows) *out_rows = rows;
        if (out_cols) *out_cols = cols;
        if (planar_capacity < p.size() || scales_capacity < sc.size())
            VX_FAIL(VX_ERR_BUFFER_TOO_SMALL, "the planar bytes need %zu bytes and the scales %zu values", p.size(), sc.size());
        if (planar == nullptr || scales_f16 == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "planar or scales_f16 is NULL");
        std::memcpy(planar, p.data(), p.size());
        std::memcpy(scales_f16, sc.data(), sc.size() * 2);
        return VX_OK;
    });
}

int vx_gguf_upload_q2_matrix(const vx_gguf_t* g, const char* name, vx_matrix_t** out_matrix) {
    return guard([&]() -> int {
        VX_TRY(check_gguf(g));
        if (out_matrix == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "out_matrix is NULL");
        *out_matrix = nullptr;
        size_t k, rows, cols;
        VX_TRY(find(g, name, &k));
        std::vector<uint8_t> p;
        std::vector<uint16_t> sc;
        VX_TRY(q2_0_convert(g, g->tensors[k], &p, &sc, &rows, &cols));
        return vx_q2_matrix_create(p.data(), p.size(), sc.data(), sc.size(), rows, cols, out_matrix);
    });
}

int vx_decoder_open_gguf(const char* path, const vx_gpu_options_t* options, vx_decoder_t** out_decoder) {
    return guard([&]() -> int {
        if (path == nullptr || out_decoder == nullptr) VX_FAIL(VX_ERR_NULL_POINTER, "path or out_decoder is NULL");
        *out_decoder = nullptr;
        vx_gpu_options_t o{};
        if (options != nullptr) {
            if (options->struct_size != sizeof(vx_gpu_options_t))
                VX_FAIL(VX_ERR_INVALID_ARGUMENT, "options.struct_size is %u, expected %zu", options->struct_size, sizeof(vx_gpu_options_t));
            o = *options;
            if (o.flags != 0) VX_FAIL(VX_ERR_INVALID_ARGUMENT, "options.flags has unknown bits set: %#x", o.flags);
        }
        // The file is checked before the device, as the reference does (quintrit-c/src/runtime.rs:312-330).
        vx_gguf_t* g = nullptr;
        VX_TRY(vx_gguf_open(path, &g));
        vx_decoder_config_t c;
        int st = gguf_decoder_config(g, o.context_length, &c);
        int count = 0;
        if (st == VX_OK && (hipGetDeviceCount(&count) != hipSuccess || count <= 0)) {
            set_error(VX_ERR_UNSUPPORTED, "no GPU is visible");
            st = VX_ERR_UNSUPPORTED;
        } else if (st == VX_OK && o.device_index >= static_cast<uint32_t>(count)) {
            set_error(VX_ERR_INVALID_ARGUMENT, "device " + std::to_string(o.device_index) + " does not exist");
            st = VX_ERR_INVALID_ARGUMENT;
        }
        int prev = -1;
        vx_decoder_t* d = nullptr;
        if (st == VX_OK && (hipGetDevice(&prev) != hipSuccess || hipSetDevice(static_cast<int>(o.device_index)) != hipSuccess)) {
            set_error(VX_ERR_DEVICE, "cannot make device " + std::to_string(o.device_index) + " current");
            st = VX_ERR_DEVICE;
        } else if (st == VX_OK) {
            st = vx_decoder_create(&c, &d);
            if (st == VX_OK) st = gguf_load_decoder(g, d, c);
            (void)hipSetDevice(prev);
        }
        if (st != VX_OK) {
            // The clean-up calls clear the error slot: keep the first failure's message.
            const std::string msg = vx_last_error_message();
            if (d != nullptr) vx_decoder_free(d);
            vx_gguf_close(g);
            set_error(st, msg);
            return st;
        }
        vx_gguf_close(g);
        *out_decoder = d;
        return VX_OK;
    });
}

}  // extern "C"
