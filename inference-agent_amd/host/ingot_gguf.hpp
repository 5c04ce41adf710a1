// ingot_gguf.hpp — a GGUF model file on MI355X: the mmap'd file parsed into tensor views, the
// Llama model resolved from it, and the one-time upload of its weight bytes to device memory
// (header only; the upload needs the HIP runtime).
//
// Reference: the reader src/gguf.h:1-60 / src/gguf.cpp:178-231 (open + mmap + parse), the model
// table src/model.cpp:10-110 (Model::load), and the Metal backend's weight placement
// src/metal_backend.mm:213-255, which wraps the mmap'd file in GPU buffers without a copy
// (unified memory). On the MI355X the weights must be in HBM: DeviceWeights copies the span of
// the file that holds the model's tensors into one device allocation, staged through two pinned
// host buffers so reading the mapped pages overlaps the DMA, and hands back a HostModel whose
// tensor pointers are device addresses (HipBackend then uses them as they are).
//
// File format (little-endian): magic "GGUF" | version u32 (2 or 3) | n_tensors u64 | n_kv u64 |
// n_kv x (key string | type u32 | value) | n_tensors x (name string | n_dims u32 | ne u64[n_dims] |
// type u32 | offset u64) | padding to general.alignment (default 32) | tensor data. A string is
// a u64 length and its bytes. Errors throw std::runtime_error with the reference's messages (part
// of the interface); the parsing and model binding are this file's own.
#pragma once

#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <iterator>
#include <map>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

#include "ingot_hip_backend.hpp"

namespace ingot {
namespace gguf {

// Elements and bytes per block of every ggml type the reference knows (src/gguf.h:30-33).
inline bool type_block(uint32_t t, uint64_t& elems, uint64_t& bytes) {
    switch (t) {
        case 0: elems = 1; bytes = 4; return true;      // F32
        case 1: elems = 1; bytes = 2; return true;      // F16
        case 30: elems = 1; bytes = 2; return true;     // BF16
        case 2: elems = 32; bytes = 18; return true;    // Q4_0
        case 3: elems = 32; bytes = 20; return true;    // Q4_1
        case 6: elems = 32; bytes = 22; return true;    // Q5_0
        case 7: elems = 32; bytes = 24; return true;    // Q5_1
        case 8: elems = 32; bytes = 34; return true;    // Q8_0
        case 9: elems = 32; bytes = 36; return true;    // Q8_1
        case 10: elems = 256; bytes = 84; return true;  // Q2_K
        case 11: elems = 256; bytes = 110; return true; // Q3_K
        case 12: elems = 256; bytes = 144; return true; // Q4_K
        case 13: elems = 256; bytes = 176; return true; // Q5_K
        case 14: elems = 256; bytes = 210; return true; // Q6_K
        case 15: elems = 256; bytes = 292; return true; // Q8_K
        default: return false;
    }
}

// A metadata value: scalars keep both an integer and a floating view; strings their text; arrays
// their element type and count (the model needs no array contents beyond the token count).
struct Value {
    uint32_t type = 0;        // GGUF value type; 9 = array
    int64_t i = 0;
    double f = 0;
    std::string s;
    uint32_t elem_type = 0;   // arrays
    uint64_t count = 0;       // arrays
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> ne;
    uint32_t type = 0;
    uint64_t offset = 0;          // from the start of the data section
    const uint8_t* data = nullptr;
    uint64_t nbytes = 0;
};

namespace detail {

// Read-only mapping of a whole file; unmapped on destruction.
class Mapping {
public:
    Mapping() = default;
    explicit Mapping(const std::string& path) {
        const int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) throw std::runtime_error("gguf: cannot open " + path);
        struct stat st {};
        const bool sized = fstat(fd, &st) == 0 && st.st_size > 0;
        void* p = sized ? mmap(nullptr, size_t(st.st_size), PROT_READ, MAP_SHARED, fd, 0) : MAP_FAILED;
        ::close(fd);  // the mapping stays valid without the descriptor
        if (!sized) throw std::runtime_error("gguf: cannot stat " + path);
        if (p == MAP_FAILED) throw std::runtime_error("gguf: mmap failed for " + path);
        bytes_ = static_cast<const uint8_t*>(p);
        size_ = size_t(st.st_size);
    }
    Mapping(Mapping&& o) noexcept : bytes_(o.bytes_), size_(o.size_) { o.bytes_ = nullptr; o.size_ = 0; }
    Mapping& operator=(Mapping&& o) noexcept {
        std::swap(bytes_, o.bytes_);
        std::swap(size_, o.size_);
        return *this;
    }
    ~Mapping() {
        if (bytes_) munmap(const_cast<uint8_t*>(bytes_), size_);
    }
    const uint8_t* bytes() const { return bytes_; }
    size_t size() const { return size_; }

private:
    const uint8_t* bytes_ = nullptr;
    size_t size_ = 0;
};

// Width in bytes of a fixed-size GGUF scalar type (0 for strings, arrays and unknown types).
constexpr uint32_t scalar_width(uint32_t t) {
    constexpr uint8_t w[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    return t < 13 ? w[t] : 0;
}

// Decodes the little-endian header from a byte range; every read is bounds-checked against the
// end of the range.
class Decoder {
public:
    Decoder(const uint8_t* begin, const uint8_t* end) : at_(begin), begin_(begin), end_(end) {}
    size_t consumed() const { return size_t(at_ - begin_); }
    const uint8_t* take(uint64_t n) {
        if (n > uint64_t(end_ - at_)) throw std::runtime_error("gguf: file truncated while parsing header");
        const uint8_t* p = at_;
        at_ += n;
        return p;
    }
    template <typename T>
    T word() {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));
        return v;
    }
    std::string text() {
        const uint64_t n = word<uint64_t>();
        return std::string(reinterpret_cast<const char*>(take(n)), size_t(n));
    }
    // A scalar of type t into both views of v.
    void scalar(uint32_t t, Value& v) {
        if (t == 8) {
            v.s = text();
            return;
        }
        const uint32_t w = scalar_width(t);
        if (w == 0) throw std::runtime_error("gguf: unknown value type " + std::to_string(t));
        const uint8_t* p = take(w);
        switch (t) {
            case 6: { float x; std::memcpy(&x, p, 4); v.f = x; v.i = int64_t(x); return; }
            case 12: { std::memcpy(&v.f, p, 8); v.i = int64_t(v.f); return; }
            case 1: v.i = int8_t(p[0]); break;
            case 3: { int16_t x; std::memcpy(&x, p, 2); v.i = x; break; }
            case 5: { int32_t x; std::memcpy(&x, p, 4); v.i = x; break; }
            case 11: std::memcpy(&v.i, p, 8); break;
            case 7: v.i = p[0] != 0; break;
            default: {  // unsigned 1, 2, 4 or 8 bytes
                uint64_t x = 0;
                std::memcpy(&x, p, w);
                v.i = int64_t(x);
            }
        }
        v.f = double(v.i);
    }
    // Steps over an array of `count` elements of type t: one jump for fixed-size elements.
    void skip_array(uint32_t t, uint64_t count) {
        if (t == 8) {
            for (uint64_t j = 0; j < count; j++) take(word<uint64_t>());
        } else if (const uint32_t w = scalar_width(t)) {
            if (count > uint64_t(end_ - at_) / w) throw std::runtime_error("gguf: file truncated while parsing header");
            take(count * w);
        } else {
            throw std::runtime_error("gguf: unknown value type " + std::to_string(t));
        }
    }

private:
    const uint8_t* at_;
    const uint8_t* begin_;
    const uint8_t* end_;
};

}  // namespace detail

class File {
public:
    static File open(const std::string& path) {
        File f;
        f.path_ = path;
        f.map_ = detail::Mapping(path);
        f.index();
        return f;
    }

    uint32_t version() const { return version_; }
    const uint8_t* base() const { return map_.bytes(); }
    size_t size() const { return map_.size(); }
    bool has(const std::string& k) const { return meta_.count(k) != 0; }
    const Value& get(const std::string& k) const {
        const auto it = meta_.find(k);
        if (it == meta_.end()) throw std::runtime_error("gguf: missing metadata key " + k);
        return it->second;
    }
    int64_t get_int(const std::string& k) const { return get(k).i; }
    int64_t get_int(const std::string& k, int64_t def) const { return has(k) ? get(k).i : def; }
    double get_float(const std::string& k, double def) const { return has(k) ? get(k).f : def; }
    std::string get_str(const std::string& k, const std::string& def) const { return has(k) ? get(k).s : def; }
    const std::vector<Tensor>& tensors() const { return tensors_; }
    const Tensor* find_tensor(const std::string& name) const {
        const auto it = by_name_.find(name);
        return it == by_name_.end() ? nullptr : &tensors_[it->second];
    }
    const Tensor& tensor(const std::string& name) const {
        if (const Tensor* t = find_tensor(name)) return *t;
        throw std::runtime_error("gguf: missing tensor " + name);
    }

private:
    // The fixed 24-byte preamble: magic "GGUF", version, tensor count, metadata count.
    struct Preamble {
        uint32_t magic, version;
        uint64_t n_tensors, n_kv;
    };
    static_assert(sizeof(Preamble) == 24, "GGUF preamble");

    // Parses the header in one pass over the mapping, then validates and places every tensor.
    void index() {
        detail::Decoder dec(map_.bytes(), map_.bytes() + map_.size());
        Preamble pre;
        std::memcpy(&pre, dec.take(sizeof pre), sizeof pre);
        if (pre.magic != 0x46554747u) throw std::runtime_error("gguf: bad magic, not a GGUF file: " + path_);
        if (pre.version != 2 && pre.version != 3)
            throw std::runtime_error("gguf: unsupported version " + std::to_string(pre.version));
        version_ = pre.version;
        if (pre.n_tensors > (1u << 20) || pre.n_kv > (1u << 20)) throw std::runtime_error("gguf: implausible header counts");

        for (uint64_t k = 0; k < pre.n_kv; k++) {
            std::string key = dec.text();
            Value v;
            v.type = dec.word<uint32_t>();
            if (v.type == 9) {
                v.elem_type = dec.word<uint32_t>();
                v.count = dec.word<uint64_t>();
                if (v.elem_type == 9) throw std::runtime_error("gguf: nested arrays are not supported");
                if (v.count > map_.size()) throw std::runtime_error("gguf: array length larger than file");
                dec.skip_array(v.elem_type, v.count);
            } else {
                dec.scalar(v.type, v);
            }
            meta_.insert_or_assign(std::move(key), std::move(v));
        }

        tensors_.reserve(size_t(pre.n_tensors));
        for (uint64_t n = 0; n < pre.n_tensors; n++) {
            Tensor t;
            t.name = dec.text();
            const uint32_t n_dims = dec.word<uint32_t>();
            if (n_dims > 4)
                throw std::runtime_error("gguf: tensor " + t.name + " has " + std::to_string(n_dims) + " dims");
            t.ne.resize(n_dims);
            std::memcpy(t.ne.data(), dec.take(8ull * n_dims), 8ull * n_dims);
            t.type = dec.word<uint32_t>();
            t.offset = dec.word<uint64_t>();
            by_name_.emplace(t.name, tensors_.size());
            tensors_.push_back(std::move(t));
        }

        const uint64_t align = uint64_t(get_int("general.alignment", 32));
        if (align == 0 || (align & (align - 1)) != 0) throw std::runtime_error("gguf: alignment must be a power of two");
        const uint64_t data_start = (dec.consumed() + align - 1) & ~(align - 1);
        for (Tensor& t : tensors_) {
            uint64_t per_block, block_bytes;
            if (!type_block(t.type, per_block, block_bytes))
                throw std::runtime_error("gguf: tensor " + t.name + " has unknown type " + std::to_string(t.type));
            const uint64_t count = std::accumulate(t.ne.begin(), t.ne.end(), uint64_t(1), std::multiplies<uint64_t>());
            if (count % per_block != 0)
                throw std::runtime_error("gguf: tensor " + t.name + " size not a multiple of its block size");
            t.nbytes = count / per_block * block_bytes;
            const uint64_t room = map_.size() > data_start ? map_.size() - data_start : 0;
            if (t.offset > room || t.nbytes > room - t.offset)
                throw std::runtime_error("gguf: tensor " + t.name + " extends past end of file");
            t.data = map_.bytes() + data_start + t.offset;
        }
    }

    std::string path_;
    detail::Mapping map_;
    uint32_t version_ = 0;
    std::map<std::string, Value> meta_;
    std::vector<Tensor> tensors_;
    std::map<std::string, size_t> by_name_;
};

namespace detail {

// A small f32 vector from an F32, F16 or BF16 tensor of exactly n elements.
inline std::vector<float> dequant_vector(const File& f, const std::string& name, int64_t n) {
    const Tensor& t = f.tensor(name);
    if (t.ne.size() != 1 || int64_t(t.ne[0]) != n)
        throw std::runtime_error("model: " + name + " has unexpected shape (want [" + std::to_string(n) + "])");
    std::vector<float> out(static_cast<size_t>(n));
    const uint8_t* src = t.data;
    switch (t.type) {
        case 0:
            std::memcpy(out.data(), src, size_t(n) * 4);
            break;
        case 1:
        case 30:
            for (size_t i = 0; i < out.size(); i++) {
                uint16_t h;
                std::memcpy(&h, src + 2 * i, 2);
                out[i] = t.type == 1 ? float(__builtin_bit_cast(_Float16, h)) : __builtin_bit_cast(float, uint32_t(h) << 16);
            }
            break;
        default:
            throw std::runtime_error("model: " + name + " has unsupported type " + std::to_string(t.type));
    }
    return out;
}

// A weight matrix [n_in, n_out] of a type the linear kernels read.
inline HostTensor bind_matrix(const File& f, const std::string& name, int64_t n_in, int64_t n_out) {
    const Tensor& t = f.tensor(name);
    if (t.ne.size() != 2 || int64_t(t.ne[0]) != n_in || int64_t(t.ne[1]) != n_out)
        throw std::runtime_error("model: " + name + " has unexpected shape (want [" + std::to_string(n_in) + ", " +
                                 std::to_string(n_out) + "])");
    constexpr uint32_t kTypes[] = {0, 1, 30, 2, 3, 8, 14};  // F32 F16 BF16 Q4_0 Q4_1 Q8_0 Q6_K
    if (std::find(std::begin(kTypes), std::end(kTypes), t.type) == std::end(kTypes))
        throw std::runtime_error("model: " + name + " has unsupported type " + std::to_string(t.type));
    return HostTensor{t.type, t.ne[0], t.ne[1], t.data};
}

}  // namespace detail

// The Llama model of a GGUF file (what Model::load resolves, src/model.cpp:32-110): the config
// from the llama.* keys, every tensor bound through one table of (name, shape) per layer, the
// norm vectors dequantized, and the rotary frequencies — the iterated product
// theta^(-2/head_dim) per pair, divided by rope_freqs.weight where present, so that they equal
// the reference's bit for bit. Tensor pointers point into the mapping.
inline HostModel load_model(const File& f) {
    const std::string arch = f.get_str("general.architecture", "");
    if (arch != "llama") throw std::runtime_error("model: architecture '" + arch + "' not supported (only llama)");
    HostModel m;
    m.n_layer = int(f.get_int("llama.block_count"));
    m.n_embd = int(f.get_int("llama.embedding_length"));
    m.n_head = int(f.get_int("llama.attention.head_count"));
    m.n_ff = int(f.get_int("llama.feed_forward_length"));
    m.n_head_kv = int(f.get_int("llama.attention.head_count_kv", m.n_head));
    m.head_dim = int(f.get_int("llama.attention.key_length", m.n_embd / m.n_head));
    m.rms_eps = float(f.get_float("llama.attention.layer_norm_rms_epsilon", 1e-5));
    m.n_vocab = int(f.get_int("llama.vocab_size", int64_t(f.get("tokenizer.ggml.tokens").count)));
    const float theta = float(f.get_float("llama.rope.freq_base", 10000.0));
    if (m.n_head % m.n_head_kv != 0) throw std::runtime_error("model: head_count not divisible by head_count_kv");
    if (f.get_int("llama.attention.value_length", m.head_dim) != m.head_dim)
        throw std::runtime_error("model: value_length != key_length is not supported");
    if (f.get_int("llama.rope.dimension_count", m.head_dim) != m.head_dim)
        throw std::runtime_error("model: partial rotary dimensions are not supported");

    const int64_t embd = m.n_embd, ff = m.n_ff, vocab = m.n_vocab;
    const int64_t q_dim = int64_t(m.n_head) * m.head_dim, kv_dim = int64_t(m.n_head_kv) * m.head_dim;
    m.tok_embd = detail::bind_matrix(f, "token_embd.weight", embd, vocab);
    m.output = f.find_tensor("output.weight") ? detail::bind_matrix(f, "output.weight", embd, vocab) : m.tok_embd;
    m.output_norm = detail::dequant_vector(f, "output_norm.weight", embd);

    const size_t pairs = size_t(m.head_dim / 2);
    const std::vector<float> divisors =
        f.find_tensor("rope_freqs.weight") ? detail::dequant_vector(f, "rope_freqs.weight", int64_t(pairs))
                                           : std::vector<float>(pairs, 1.0f);
    const bool divided = f.find_tensor("rope_freqs.weight") != nullptr;
    const float ratio = powf(theta, -2.0f / float(m.head_dim));
    m.rope_inv_freq.resize(pairs);
    float base = 1.0f;
    for (size_t i = 0; i < pairs; i++, base *= ratio) m.rope_inv_freq[i] = divided ? base / divisors[i] : base;

    // One row per weight of a transformer block: GGUF suffix, shape [n_in, n_out], destination.
    struct Slot {
        const char* suffix;
        int64_t n_in, n_out;
        HostTensor HostLayer::*dst;
    };
    const Slot slots[] = {
        {"attn_q.weight", embd, q_dim, &HostLayer::wq},       {"attn_k.weight", embd, kv_dim, &HostLayer::wk},
        {"attn_v.weight", embd, kv_dim, &HostLayer::wv},      {"attn_output.weight", q_dim, embd, &HostLayer::wo},
        {"ffn_gate.weight", embd, ff, &HostLayer::w_gate},    {"ffn_up.weight", embd, ff, &HostLayer::w_up},
        {"ffn_down.weight", ff, embd, &HostLayer::w_down},
    };
    m.layers.resize(size_t(m.n_layer));
    for (int l = 0; l < m.n_layer; l++) {
        const std::string blk = "blk." + std::to_string(l) + ".";
        HostLayer& L = m.layers[size_t(l)];
        L.attn_norm = detail::dequant_vector(f, blk + "attn_norm.weight", embd);
        L.ffn_norm = detail::dequant_vector(f, blk + "ffn_norm.weight", embd);
        for (const Slot& s : slots) L.*s.dst = detail::bind_matrix(f, blk + s.suffix, s.n_in, s.n_out);
    }
    return m;
}

// The model's weight matrices copied into one device allocation. model() returns the host model
// with every matrix pointer moved to its device copy (HipBackend with device_weights = true).
class DeviceWeights {
public:
    DeviceWeights(const HostModel& host, hipStream_t stream = nullptr, size_t stage_bytes = size_t(64) << 20)
        : model_(host) {
        std::vector<HostTensor*> ts = {&model_.tok_embd, &model_.output};
        for (HostLayer& L : model_.layers)
            for (HostTensor* t : {&L.wq, &L.wk, &L.wv, &L.wo, &L.w_gate, &L.w_up, &L.w_down}) ts.push_back(t);
        // The byte span that holds every matrix: one allocation, one pass of large copies.
        const uint8_t *lo = nullptr, *hi = nullptr;
        for (HostTensor* t : ts) {
            const uint8_t* b = static_cast<const uint8_t*>(t->data);
            const uint8_t* e = b + bytes_of(*t);
            lo = lo && lo < b ? lo : b;
            hi = hi && hi > e ? hi : e;
        }
        bytes_ = size_t(hi - lo);
        check(hipMalloc(&dev_, bytes_), "weight allocation");
        void* stage[2] = {nullptr, nullptr};
        hipEvent_t done[2] = {nullptr, nullptr};
        try {
            for (int i = 0; i < 2; i++) {
                check(hipHostMalloc(&stage[i], stage_bytes, hipHostMallocDefault), "staging allocation");
                check(hipEventCreate(&done[i]), "event");
            }
            // Copy the mapped bytes into one pinned buffer while the other one's DMA runs.
            for (size_t off = 0, k = 0; off < bytes_; off += stage_bytes, k++) {
                const size_t n = std::min(stage_bytes, bytes_ - off);
                const int b = int(k & 1);
                if (k >= 2) check(hipEventSynchronize(done[b]), "staging");
                std::memcpy(stage[b], lo + off, n);
                check(hipMemcpyAsync(static_cast<uint8_t*>(dev_) + off, stage[b], n, hipMemcpyHostToDevice, stream),
                      "weight upload");
                check(hipEventRecord(done[b], stream), "event");
            }
            check(hipStreamSynchronize(stream), "weight upload");
        } catch (...) {
            release_stage(stage, done);
            (void)hipFree(dev_);
            throw;
        }
        release_stage(stage, done);
        for (HostTensor* t : ts) t->data = static_cast<uint8_t*>(dev_) + (static_cast<const uint8_t*>(t->data) - lo);
    }
    ~DeviceWeights() {
        if (dev_) (void)hipFree(dev_);
    }
    DeviceWeights(const DeviceWeights&) = delete;
    DeviceWeights& operator=(const DeviceWeights&) = delete;

    const HostModel& model() const { return model_; }
    size_t bytes() const { return bytes_; }

private:
    static size_t bytes_of(const HostTensor& t) {
        uint64_t elems, bytes;
        if (!gguf::type_block(t.type, elems, bytes)) throw std::runtime_error("hip: unknown tensor type");
        return size_t(t.ne0 * t.ne1 / elems * bytes);
    }
    static void check(hipError_t e, const char* what) {
        if (e != hipSuccess)
            throw std::runtime_error(std::string("hip: ") + what + " failed: " + hipGetErrorString(e));
    }
    static void release_stage(void* stage[2], hipEvent_t done[2]) {
        for (int i = 0; i < 2; i++) {
            if (done[i]) (void)hipEventDestroy(done[i]);
            if (stage[i]) (void)hipHostFree(stage[i]);
        }
    }

    HostModel model_;
    void* dev_ = nullptr;
    size_t bytes_ = 0;
};

}  // namespace gguf
}  // namespace ingot
