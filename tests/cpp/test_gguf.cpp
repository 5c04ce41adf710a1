// test_gguf.cpp — the GGUF path of the MI355X backend (host/ingot_gguf.hpp): a model file is
// written here from the published format (src/gguf.h:1-12), mapped and parsed by gguf::File,
// resolved by gguf::load_model (Model::load, src/model.cpp:32-110), its weight bytes uploaded by
// gguf::DeviceWeights, and run by HipBackend on the device copies. Checks: the config and the
// rotary frequencies; every tensor's bytes in the mapping and in device memory are the ones
// written; HipBackend over the file gives bit-identical logits to HipBackend over the in-memory
// model; and the reference's errors for a bad magic, an unsupported version, a truncated header
// and a tensor past the end of the file. Prints one line per check and "ALL PASSED".
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "ingot_gguf.hpp"
#include "synth_model.hpp"

namespace {

int g_fail = 0;

void expect(bool ok, const std::string& what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
    if (!ok) g_fail++;
}

struct Writer {
    std::vector<uint8_t> b;
    template <typename T>
    void put(T v) {
        const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
        b.insert(b.end(), p, p + sizeof(T));
    }
    void str(const std::string& s) {
        put<uint64_t>(s.size());
        b.insert(b.end(), s.begin(), s.end());
    }
    void kv_u32(const std::string& k, uint32_t v) { str(k); put<uint32_t>(4); put<uint32_t>(v); }
    void kv_f32(const std::string& k, float v) { str(k); put<uint32_t>(6); put<float>(v); }
    void kv_str(const std::string& k, const std::string& v) { str(k); put<uint32_t>(8); str(v); }
};

struct Entry {
    std::string name;
    std::vector<uint64_t> ne;
    uint32_t type;
    const void* data;
    size_t bytes;
};

// GGUF v3 with alignment 64; tensors in `es` order.
std::vector<uint8_t> write_gguf(const ingot::HostModel& m, const std::vector<Entry>& es, uint32_t version = 3) {
    Writer w;
    w.put<uint32_t>(0x46554747u);
    w.put<uint32_t>(version);
    w.put<uint64_t>(es.size());
    const uint64_t n_kv = 13;
    w.put<uint64_t>(n_kv);
    w.kv_str("general.architecture", "llama");
    w.kv_u32("general.alignment", 64);
    w.kv_u32("llama.block_count", uint32_t(m.n_layer));
    w.kv_u32("llama.embedding_length", uint32_t(m.n_embd));
    w.kv_u32("llama.attention.head_count", uint32_t(m.n_head));
    w.kv_u32("llama.attention.head_count_kv", uint32_t(m.n_head_kv));
    w.kv_u32("llama.feed_forward_length", uint32_t(m.n_ff));
    w.kv_f32("llama.rope.freq_base", 500000.f);
    w.kv_f32("llama.attention.layer_norm_rms_epsilon", m.rms_eps);
    // values the model does not use, of the other value types
    w.str("general.some_u64"); w.put<uint32_t>(10); w.put<uint64_t>(1ull << 40);
    w.str("general.flag"); w.put<uint32_t>(7); w.put<uint8_t>(1);
    w.str("general.ints"); w.put<uint32_t>(9); w.put<uint32_t>(5); w.put<uint64_t>(3);
    for (int32_t v : {1, -2, 3}) w.put<int32_t>(v);
    // the vocabulary, which fixes n_vocab
    w.str("tokenizer.ggml.tokens"); w.put<uint32_t>(9); w.put<uint32_t>(8); w.put<uint64_t>(uint64_t(m.n_vocab));
    for (int i = 0; i < m.n_vocab; i++) w.str("tok" + std::to_string(i));
    uint64_t off = 0;
    for (const Entry& e : es) {
        w.str(e.name);
        w.put<uint32_t>(uint32_t(e.ne.size()));
        for (uint64_t d : e.ne) w.put<uint64_t>(d);
        w.put<uint32_t>(e.type);
        w.put<uint64_t>(off);
        off = (off + e.bytes + 63) / 64 * 64;
    }
    while (w.b.size() % 64) w.b.push_back(0);
    for (const Entry& e : es) {
        const uint8_t* p = static_cast<const uint8_t*>(e.data);
        w.b.insert(w.b.end(), p, p + e.bytes);
        while (w.b.size() % 64) w.b.push_back(0);
    }
    return w.b;
}

std::string save(const std::vector<uint8_t>& bytes, const std::string& tag) {
    const std::string path = "/tmp/ingot_test_" + std::to_string(getpid()) + "_" + tag + ".gguf";
    std::ofstream(path, std::ios::binary).write(reinterpret_cast<const char*>(bytes.data()), std::streamsize(bytes.size()));
    return path;
}

template <typename F>
std::string error_of(F fn) {
    try {
        fn();
    } catch (const std::runtime_error& e) {
        return e.what();
    }
    return "";
}

}  // namespace

int main() {
    std::vector<std::string> files;
    try {
        synth::Owned own;
        const ingot::HostModel m = synth::make_model(own, 5);
        IngotLinearDesc d{0, 0, 0, 1, 0, 0, 0};
        auto mat = [&](const std::string& name, const ingot::HostTensor& t) {
            d.type = t.type; d.n_in = uint32_t(t.ne0); d.n_out = uint32_t(t.ne1);
            return Entry{name, {t.ne0, t.ne1}, t.type, t.data, ingot_linear_weight_bytes(&d)};
        };
        auto vec = [&](const std::string& name, const std::vector<float>& v) {
            return Entry{name, {v.size()}, 0, v.data(), v.size() * 4};
        };
        std::vector<Entry> es = {mat("token_embd.weight", m.tok_embd), vec("output_norm.weight", m.output_norm)};
        for (int l = 0; l < m.n_layer; l++) {
            const ingot::HostLayer& L = m.layers[size_t(l)];
            const std::string p = "blk." + std::to_string(l) + ".";
            es.push_back(vec(p + "attn_norm.weight", L.attn_norm));
            es.push_back(vec(p + "ffn_norm.weight", L.ffn_norm));
            es.push_back(mat(p + "attn_q.weight", L.wq));
            es.push_back(mat(p + "attn_k.weight", L.wk));
            es.push_back(mat(p + "attn_v.weight", L.wv));
            es.push_back(mat(p + "attn_output.weight", L.wo));
            es.push_back(mat(p + "ffn_gate.weight", L.w_gate));
            es.push_back(mat(p + "ffn_up.weight", L.w_up));
            es.push_back(mat(p + "ffn_down.weight", L.w_down));
        }
        const std::vector<uint8_t> bytes = write_gguf(m, es);
        files.push_back(save(bytes, "model"));

        ingot::gguf::File f = ingot::gguf::File::open(files.back());
        expect(f.version() == 3 && f.tensors().size() == es.size(), "header and tensor count");
        const ingot::HostModel fm = ingot::gguf::load_model(f);
        expect(fm.n_layer == m.n_layer && fm.n_embd == m.n_embd && fm.n_head == m.n_head &&
                   fm.n_head_kv == m.n_head_kv && fm.head_dim == 128 && fm.n_ff == m.n_ff &&
                   fm.n_vocab == m.n_vocab && fm.rms_eps == m.rms_eps,
               "config from the metadata (n_vocab from the token list)");
        expect(fm.output.data == fm.tok_embd.data, "no output.weight: tied embeddings");
        bool freq_ok = true;
        for (size_t i = 0; i < m.rope_inv_freq.size(); i++)
            freq_ok &= std::fabs(fm.rope_inv_freq[i] - m.rope_inv_freq[i]) <= 1e-7f * (1 + m.rope_inv_freq[i]);
        expect(freq_ok, "rotary frequencies");
        bool bytes_ok = fm.output_norm == m.output_norm;
        for (const Entry& e : es) {
            const ingot::gguf::Tensor& t = f.tensor(e.name);
            bytes_ok &= t.nbytes == e.bytes && std::memcmp(t.data, e.data, e.bytes) == 0 && t.type == e.type;
            bytes_ok &= (reinterpret_cast<uintptr_t>(t.data) - reinterpret_cast<uintptr_t>(f.base())) % 64 == 0;
        }
        expect(bytes_ok, "tensor bytes, types and 64-byte alignment in the mapping");

        ingot::gguf::DeviceWeights dw(fm, nullptr, 1 << 16);  // small stages: many double-buffered copies
        const ingot::HostModel& dm = dw.model();
        bool dev_ok = true;
        for (const ingot::HostTensor* t : {&dm.layers[1].w_down, &dm.layers[0].wq, &dm.tok_embd}) {
            const ingot::HostTensor& h = t == &dm.tok_embd ? fm.tok_embd : t == &dm.layers[0].wq ? fm.layers[0].wq
                                                                                                 : fm.layers[1].w_down;
            d.type = t->type; d.n_in = uint32_t(t->ne0); d.n_out = uint32_t(t->ne1);
            std::vector<uint8_t> back(ingot_linear_weight_bytes(&d));
            dev_ok &= hipMemcpy(back.data(), t->data, back.size(), hipMemcpyDeviceToHost) == hipSuccess;
            dev_ok &= std::memcmp(back.data(), h.data, back.size()) == 0;
        }
        expect(dev_ok, "device copies of the weights");

        ingot::HipBackend mem(m, 64, 16), file(dm, 64, 16, nullptr, /*device_weights=*/true);
        const int32_t toks[12] = {3, 17, 499, 0, 42, 42, 7, 300, 1, 2, 250, 64};
        std::vector<float> a(size_t(m.n_vocab));
        bool same = true;
        std::memcpy(a.data(), mem.forward_batch(toks, 9, 0), a.size() * 4);
        same &= std::memcmp(a.data(), file.forward_batch(toks, 9, 0), a.size() * 4) == 0;
        for (int p = 9; p < 12; p++) {
            std::memcpy(a.data(), mem.forward(toks[p], p), a.size() * 4);
            same &= std::memcmp(a.data(), file.forward(toks[p], p), a.size() * 4) == 0;
        }
        expect(same, "HipBackend over the file == over the in-memory model (bit-identical logits)");

        // malformed files
        std::vector<uint8_t> bad = bytes;
        bad[3] = 'X';
        files.push_back(save(bad, "magic"));
        expect(error_of([&] { ingot::gguf::File::open(files.back()); }).find("bad magic") != std::string::npos,
               "bad magic");
        bad = bytes;
        bad[4] = 1;
        files.push_back(save(bad, "version"));
        expect(error_of([&] { ingot::gguf::File::open(files.back()); }).find("unsupported version 1") != std::string::npos,
               "version 1");
        files.push_back(save(std::vector<uint8_t>(bytes.begin(), bytes.begin() + 300), "short"));
        expect(error_of([&] { ingot::gguf::File::open(files.back()); }).find("truncated") != std::string::npos,
               "truncated header");
        files.push_back(save(std::vector<uint8_t>(bytes.begin(), bytes.end() - 4096), "cut"));
        expect(error_of([&] { ingot::gguf::File::open(files.back()); }).find("extends past end of file") !=
                   std::string::npos,
               "tensor past the end");
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        g_fail++;
    }
    for (const std::string& p : files) std::remove(p.c_str());
    if (g_fail) {
        std::printf("%d FAILED\n", g_fail);
        return 1;
    }
    std::printf("ALL PASSED\n");
    return 0;
}
