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
// a u64 length and its bytes. Errors throw std::runtime_error with the reference's messages.
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
#include <map>
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

struct Value {
    uint32_t type = 0;        // GGUF value type (scalars) or 9 (array)
    int64_t i = 0;            // integer / bool scalars, and the integer view of floats
    double f = 0;             // float scalars, and the float view of integers
    std::string s;            // string scalar
    uint32_t elem_type = 0;   // arrays: element type
    uint64_t count = 0;       // arrays: element count
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> ne;
    uint32_t type = 0;
    uint64_t offset = 0;          // from the start of the data section
    const uint8_t* data = nullptr;
    uint64_t nbytes = 0;
};

class File {
public:
    static File open(const std::string& path) {
        File f;
        f.path_ = path;
        f.fd_ = ::open(path.c_str(), O_RDONLY);
        if (f.fd_ < 0) throw std::runtime_error("gguf: cannot open " + path);
        struct stat st {};
        if (fstat(f.fd_, &st) != 0 || st.st_size <= 0) throw std::runtime_error("gguf: cannot stat " + path);
        f.size_ = size_t(st.st_size);
        void* p = mmap(nullptr, f.size_, PROT_READ, MAP_SHARED, f.fd_, 0);
        if (p == MAP_FAILED) throw std::runtime_error("gguf: mmap failed for " + path);
        f.base_ = static_cast<const uint8_t*>(p);
        f.parse();
        return f;
    }
    File() = default;
    File(File&& o) noexcept { *this = std::move(o); }
    File& operator=(File&& o) noexcept {
        if (this != &o) {
            close();
            path_ = std::move(o.path_);
            fd_ = o.fd_;
            base_ = o.base_;
            size_ = o.size_;
            version_ = o.version_;
            data_offset_ = o.data_offset_;
            kv_ = std::move(o.kv_);
            tensors_ = std::move(o.tensors_);
            o.fd_ = -1;
            o.base_ = nullptr;
            o.size_ = 0;
        }
        return *this;
    }
    ~File() { close(); }

    uint32_t version() const { return version_; }
    const uint8_t* base() const { return base_; }
    size_t size() const { return size_; }
    bool has(const std::string& k) const { return kv_.count(k) != 0; }
    const Value& get(const std::string& k) const {
        auto it = kv_.find(k);
        if (it == kv_.end()) throw std::runtime_error("gguf: missing metadata key " + k);
        return it->second;
    }
    int64_t get_int(const std::string& k) const { return get(k).i; }
    int64_t get_int(const std::string& k, int64_t def) const { return has(k) ? get(k).i : def; }
    double get_float(const std::string& k, double def) const { return has(k) ? get(k).f : def; }
    std::string get_str(const std::string& k, const std::string& def) const { return has(k) ? get(k).s : def; }
    const std::vector<Tensor>& tensors() const { return tensors_; }
    const Tensor* find_tensor(const std::string& name) const {
        for (const Tensor& t : tensors_)
            if (t.name == name) return &t;
        return nullptr;
    }
    const Tensor& tensor(const std::string& name) const {
        const Tensor* t = find_tensor(name);
        if (!t) throw std::runtime_error("gguf: missing tensor " + name);
        return *t;
    }

private:
    struct Reader {
        const uint8_t* p;
        size_t size, pos = 0;
        void need(uint64_t n) const {
            if (n > size - pos) throw std::runtime_error("gguf: file truncated while parsing header");
        }
        template <typename T>
        T get() {
            need(sizeof(T));
            T v;
            std::memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
            return v;
        }
        std::string str() {
            const uint64_t n = get<uint64_t>();
            need(n);
            std::string s(reinterpret_cast<const char*>(p + pos), size_t(n));
            pos += size_t(n);
            return s;
        }
        // One scalar of value type t into v (its integer and float views both set).
        void scalar(uint32_t t, Value& v) {
            switch (t) {
                case 0: v.i = get<uint8_t>(); break;
                case 1: v.i = get<int8_t>(); break;
                case 2: v.i = get<uint16_t>(); break;
                case 3: v.i = get<int16_t>(); break;
                case 4: v.i = get<uint32_t>(); break;
                case 5: v.i = get<int32_t>(); break;
                case 6: v.f = get<float>(); v.i = int64_t(v.f); return;
                case 7: v.i = get<uint8_t>() != 0; break;
                case 8: v.s = str(); return;
                case 10: v.i = int64_t(get<uint64_t>()); break;
                case 11: v.i = get<int64_t>(); break;
                case 12: v.f = get<double>(); v.i = int64_t(v.f); return;
                default: throw std::runtime_error("gguf: unknown value type " + std::to_string(t));
            }
            v.f = double(v.i);
        }
    };

    void parse() {
        Reader r{base_, size_};
        if (r.get<uint32_t>() != 0x46554747u) throw std::runtime_error("gguf: bad magic, not a GGUF file: " + path_);
        version_ = r.get<uint32_t>();
        if (version_ < 2 || version_ > 3)
            throw std::runtime_error("gguf: unsupported version " + std::to_string(version_));
        const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
        if (n_tensors > (1u << 20) || n_kv > (1u << 20)) throw std::runtime_error("gguf: implausible header counts");
        for (uint64_t k = 0; k < n_kv; k++) {
            std::string key = r.str();
            Value v;
            v.type = r.get<uint32_t>();
            if (v.type == 9) {
                v.elem_type = r.get<uint32_t>();
                v.count = r.get<uint64_t>();
                if (v.elem_type == 9) throw std::runtime_error("gguf: nested arrays are not supported");
                if (v.count > size_) throw std::runtime_error("gguf: array length larger than file");
                Value e;  // elements are read to advance; the model needs only the count
                for (uint64_t j = 0; j < v.count; j++) r.scalar(v.elem_type, e);
            } else {
                r.scalar(v.type, v);
            }
            kv_[key] = std::move(v);
        }
        tensors_.resize(size_t(n_tensors));
        for (Tensor& t : tensors_) {
            t.name = r.str();
            const uint32_t n_dims = r.get<uint32_t>();
            if (n_dims > 4)
                throw std::runtime_error("gguf: tensor " + t.name + " has " + std::to_string(n_dims) + " dims");
            for (uint32_t d = 0; d < n_dims; d++) t.ne.push_back(r.get<uint64_t>());
            t.type = r.get<uint32_t>();
            t.offset = r.get<uint64_t>();
        }
        const uint64_t align = uint64_t(get_int("general.alignment", 32));
        if (align == 0 || (align & (align - 1)) != 0) throw std::runtime_error("gguf: alignment must be a power of two");
        data_offset_ = (r.pos + align - 1) / align * align;
        for (Tensor& t : tensors_) {
            uint64_t elems, bytes, n = 1;
            if (!type_block(t.type, elems, bytes))
                throw std::runtime_error("gguf: tensor " + t.name + " has unknown type " + std::to_string(t.type));
            for (uint64_t d : t.ne) n *= d;
            if (n % elems != 0)
                throw std::runtime_error("gguf: tensor " + t.name + " size not a multiple of its block size");
            t.nbytes = n / elems * bytes;
            if (t.offset > size_ || data_offset_ + t.offset + t.nbytes > size_)
                throw std::runtime_error("gguf: tensor " + t.name + " extends past end of file");
            t.data = base_ + data_offset_ + t.offset;
        }
    }
    void close() {
        if (base_) munmap(const_cast<uint8_t*>(base_), size_);
        if (fd_ >= 0) ::close(fd_);
        base_ = nullptr;
        fd_ = -1;
    }

    std::string path_;
    int fd_ = -1;
    const uint8_t* base_ = nullptr;
    size_t size_ = 0;
    uint32_t version_ = 0;
    uint64_t data_offset_ = 0;
    std::map<std::string, Value> kv_;
    std::vector<Tensor> tensors_;
};

// Model::load (src/model.cpp:32-110): the Llama config keys, the tensor table with its shape and
// type checks, the small vectors dequantized, and the rotary frequencies (iterated multiply,
// optionally divided by rope_freqs.weight). Tensor pointers point into the mapped file.
inline HostModel load_model(const File& f) {
    const std::string arch = f.get_str("general.architecture", "");
    if (arch != "llama") throw std::runtime_error("model: architecture '" + arch + "' not supported (only llama)");
    HostModel m;
    m.n_layer = int(f.get_int("llama.block_count"));
    m.n_embd = int(f.get_int("llama.embedding_length"));
    m.n_head = int(f.get_int("llama.attention.head_count"));
    m.n_head_kv = int(f.get_int("llama.attention.head_count_kv", m.n_head));
    m.head_dim = int(f.get_int("llama.attention.key_length", m.n_embd / m.n_head));
    m.n_ff = int(f.get_int("llama.feed_forward_length"));
    const float theta = float(f.get_float("llama.rope.freq_base", 10000.0));
    m.rms_eps = float(f.get_float("llama.attention.layer_norm_rms_epsilon", 1e-5));
    m.n_vocab = int(f.get_int("llama.vocab_size", int64_t(f.get("tokenizer.ggml.tokens").count)));
    if (m.n_head % m.n_head_kv != 0) throw std::runtime_error("model: head_count not divisible by head_count_kv");
    if (int(f.get_int("llama.attention.value_length", m.head_dim)) != m.head_dim)
        throw std::runtime_error("model: value_length != key_length is not supported");
    if (int(f.get_int("llama.rope.dimension_count", m.head_dim)) != m.head_dim)
        throw std::runtime_error("model: partial rotary dimensions are not supported");
    const int64_t q_dim = int64_t(m.n_head) * m.head_dim, kv_dim = int64_t(m.n_head_kv) * m.head_dim;

    auto matrix = [&](const std::string& name, int64_t n_in, int64_t n_out) {
        const Tensor& t = f.tensor(name);
        if (t.ne.size() != 2 || int64_t(t.ne[0]) != n_in || int64_t(t.ne[1]) != n_out)
            throw std::runtime_error("model: " + name + " has unexpected shape (want [" + std::to_string(n_in) + ", " +
                                     std::to_string(n_out) + "])");
        const uint32_t ty = t.type;
        if (!(ty == 0 || ty == 1 || ty == 30 || ty == 2 || ty == 3 || ty == 8 || ty == 14))
            throw std::runtime_error("model: " + name + " has unsupported type " + std::to_string(ty));
        return HostTensor{t.type, t.ne[0], t.ne[1], t.data};
    };
    auto vec = [&](const std::string& name, int64_t n) {
        const Tensor& t = f.tensor(name);
        if (t.ne.size() != 1 || int64_t(t.ne[0]) != n)
            throw std::runtime_error("model: " + name + " has unexpected shape (want [" + std::to_string(n) + "])");
        std::vector<float> v(static_cast<size_t>(n));
        for (int64_t i = 0; i < n; i++) {
            if (t.type == 0) std::memcpy(&v[size_t(i)], t.data + 4 * i, 4);
            else if (t.type == 1 || t.type == 30) {
                uint16_t h;
                std::memcpy(&h, t.data + 2 * i, 2);
                if (t.type == 30) {
                    const uint32_t u = uint32_t(h) << 16;
                    std::memcpy(&v[size_t(i)], &u, 4);
                } else {
                    v[size_t(i)] = float(__builtin_bit_cast(_Float16, h));
                }
            } else {
                throw std::runtime_error("model: " + name + " has unsupported type " + std::to_string(t.type));
            }
        }
        return v;
    };

    m.tok_embd = matrix("token_embd.weight", m.n_embd, m.n_vocab);
    m.output = f.find_tensor("output.weight") ? matrix("output.weight", m.n_embd, m.n_vocab) : m.tok_embd;
    m.output_norm = vec("output_norm.weight", m.n_embd);
    std::vector<float> factors;
    if (f.find_tensor("rope_freqs.weight")) factors = vec("rope_freqs.weight", m.head_dim / 2);
    m.rope_inv_freq.resize(size_t(m.head_dim / 2));
    const float step = powf(theta, -2.0f / float(m.head_dim));
    float freq = 1.0f;
    for (int i = 0; i < m.head_dim / 2; i++) {
        m.rope_inv_freq[size_t(i)] = factors.empty() ? freq : freq / factors[size_t(i)];
        freq *= step;
    }
    for (int l = 0; l < m.n_layer; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        HostLayer L;
        L.attn_norm = vec(p + "attn_norm.weight", m.n_embd);
        L.ffn_norm = vec(p + "ffn_norm.weight", m.n_embd);
        L.wq = matrix(p + "attn_q.weight", m.n_embd, q_dim);
        L.wk = matrix(p + "attn_k.weight", m.n_embd, kv_dim);
        L.wv = matrix(p + "attn_v.weight", m.n_embd, kv_dim);
        L.wo = matrix(p + "attn_output.weight", q_dim, m.n_embd);
        L.w_gate = matrix(p + "ffn_gate.weight", m.n_embd, m.n_ff);
        L.w_up = matrix(p + "ffn_up.weight", m.n_embd, m.n_ff);
        L.w_down = matrix(p + "ffn_down.weight", m.n_ff, m.n_embd);
        m.layers.push_back(std::move(L));
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
