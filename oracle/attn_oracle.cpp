// attn_oracle.cpp — CPU restatement of Ingot's attention, used ONLY as the checker.
//
// TEST INFRASTRUCTURE. Nothing on the product path (the HIP library under inference-agent_amd/)
// links, loads or calls this file. Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg use it, through liboracle.so and ctypes.
//
// What it restates (reference files under /root/reference, read as text, never compiled here):
//   - the attention block of CpuBackend::forward, src/cpu_backend.cpp:51-69:
//       kvh = h / group (line 53); s_t = (sum_i q_i k_t,i) * scale for t = 0..pos (lines 55-60);
//       softmax (line 61); out_h = sum_t p_t v_t (lines 62-68);
//   - ops::softmax, src/ops.cpp:234-241: max, x = expf(x - max) with a running sum, x *= 1/sum;
//   - ops::parallel_for, src/ops.h:16-19 (macOS GCD dispatch_apply_f over heads), replaced by a
//     std::thread fan-out over heads: each (token, head) result is computed by one thread with
//     the same sequential loop order, so the split does not change any rounding;
//   - Backend::forward_batch's default, src/backend.h:16-20: prefill of n tokens is n decode
//     steps at positions pos..pos+n-1, so query i attends to cache rows 0..pos+i;
//   - the f16 KV cache of the Metal backend (src/metal_backend.mm:197-198, 437) written with
//     half(x) (shaders/kernels.metal:280-281, 781): round-to-nearest-even binary16. The
//     reference CPU cache is f32 (src/cpu_backend.h:23); here it holds the same f16-rounded
//     values widened to f32, so the CPU and GPU paths see identical K/V;
//   - the step before attention: ops::rope, src/ops.cpp:243-255 (pairs (2i, 2i+1) of each head
//     rotated by angle float(pos) * inv_freq[i], cosf/sinf), applied to q and k
//     (src/cpu_backend.cpp:43-44), then K and V copied into the cache row of pos
//     (src/cpu_backend.cpp:46-49); in the f16 cache this is rope_k_to_cache + to_half
//     (shaders/kernels.metal:270-282, 779-782; src/metal_backend.mm:395-409);
//   - the rotary frequencies, src/model.cpp:59-68: an iterated multiply by
//     theta^(-2/head_dim) starting at 1, each optionally divided by rope_freqs.weight[i].
//
// Differences that do not affect results beyond f32 rounding: Apple clang contracts
// `s += q*k` into an FMA on arm64 (fp-contract=on); this file is built with
// -ffp-contract=off, so every multiply and add rounds separately, as the source reads.
//
// Parity status of each function is recorded in tests/test_oracle.py, which pins them
// against closed forms and numpy.
#include "attn_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

// IEEE binary16 -> binary32, exact (every half is representable as a float).
float half_to_float(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: value = man * 2^-24
            float v = std::ldexp(float(man), -24);
            uint32_t vb;
            std::memcpy(&vb, &v, 4);
            bits = sign | vb;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);  // inf / nan (payload kept)
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// IEEE binary32 -> binary16 with round-to-nearest-even, overflow to inf, NaN kept quiet.
uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) {  // inf or nan
        if (absx == 0x7f800000u) return sign | 0x7c00u;
        return uint16_t(sign | 0x7e00u | ((absx >> 13) & 0x3ffu));
    }
    if (absx >= 0x477ff000u) return sign | 0x7c00u;  // >= 65520 rounds to inf
    if (absx < 0x38800000u) {                          // below the smallest normal half (2^-14)
        if (absx < 0x33000000u) return sign;           // < 2^-25 rounds to zero (ties too)
        // subnormal half: value = round(|f| * 2^24)
        const uint32_t e = absx >> 23;                 // biased float exponent, 102..112
        const uint32_t m = (absx & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;               // 14..24: m >> shift = |f| * 2^24
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (r & 1u))) r++;
        return uint16_t(sign | r);
    }
    // normal half: rebias exponent, round the 13 dropped mantissa bits
    uint32_t r = ((absx >> 13) - (112u << 10));
    const uint32_t rem = absx & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;  // carry may roll into the exponent
    return uint16_t(sign | r);
}

// ops::softmax, src/ops.cpp:234-241.
void softmax(float* x, size_t n) {
    float mx = x[0];
    for (size_t i = 1; i < n; i++) mx = std::max(mx, x[i]);
    float sum = 0;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

// One (token, head) of src/cpu_backend.cpp:52-68 over an f16 cache; `n_keys` = pos + 1.
void attend_one(const float* qh, const uint16_t* kc, const uint16_t* vc, float* out, float* sc,
                int head_dim, size_t kv_stride, size_t kvh, int n_keys, float scale) {
    const int hd = head_dim;
    for (int t = 0; t < n_keys; t++) {
        const uint16_t* kt = kc + size_t(t) * kv_stride + kvh * hd;
        float s = 0;
        for (int i = 0; i < hd; i++) s += qh[i] * half_to_float(kt[i]);
        sc[t] = s * scale;
    }
    softmax(sc, size_t(n_keys));
    std::memset(out, 0, hd * sizeof(float));
    for (int t = 0; t < n_keys; t++) {
        const uint16_t* vt = vc + size_t(t) * kv_stride + kvh * hd;
        const float w = sc[t];
        for (int i = 0; i < hd; i++) out[i] += w * half_to_float(vt[i]);
    }
}

// Runs f(h) for every head h in [0, n) on up to n_threads std::threads (src/ops.h:16-19).
template <typename F>
void parallel_for(int n, int n_threads, F&& f) {
    if (n_threads <= 1 || n <= 1) {
        for (int h = 0; h < n; h++) f(h);
        return;
    }
    const int nt = std::min(n, n_threads);
    std::vector<std::thread> pool;
    pool.reserve(nt);
    for (int w = 0; w < nt; w++)
        pool.emplace_back([&, w] {
            for (int h = w; h < n; h += nt) f(h);
        });
    for (auto& t : pool) t.join();
}

// ops::rope, src/ops.cpp:243-255, on one row at position `pos`.
void rope_row(float* x, int n_heads, int head_dim, int pos, const float* inv_freq) {
    const int half = head_dim / 2;
    for (int h = 0; h < n_heads; h++) {
        float* v = x + size_t(h) * head_dim;
        for (int i = 0; i < half; i++) {
            const float angle = float(pos) * inv_freq[i];
            const float c = cosf(angle), s = sinf(angle);
            const float x0 = v[2 * i], x1 = v[2 * i + 1];
            v[2 * i] = x0 * c - x1 * s;
            v[2 * i + 1] = x0 * s + x1 * c;
        }
    }
}

}  // namespace

extern "C" {

void oracle_rope_inv_freq(float theta, int head_dim, const float* factors, float* out) {
    const float theta_scale = powf(theta, -2.0f / float(head_dim));
    float freq = 1.0f;
    for (int i = 0; i < head_dim / 2; i++) {
        out[i] = factors ? freq / factors[i] : freq;
        freq *= theta_scale;
    }
}

void oracle_rope(float* x, int n_tok, int row_stride, int n_heads, int head_dim, int pos,
                 const float* inv_freq) {
    for (int t = 0; t < n_tok; t++) rope_row(x + size_t(t) * row_stride, n_heads, head_dim, pos + t, inv_freq);
}

int oracle_rope_kv_store(float* q, int q_stride, int n_head, const float* k, const float* v,
                         int kv_stride, uint16_t* k_cache, uint16_t* v_cache, size_t dst_offset,
                         int n_head_kv, int head_dim, int pos, int n_tok, const float* inv_freq) {
    if (!k || !v || !k_cache || !v_cache || !inv_freq || n_head_kv <= 0 || head_dim <= 0 ||
        head_dim % 2 != 0 || pos < 0 || n_tok <= 0 || kv_stride < n_head_kv * head_dim)
        return -1;
    const size_t kv_dim = size_t(n_head_kv) * head_dim;
    std::vector<float> kr(kv_dim);
    for (int t = 0; t < n_tok; t++) {
        if (q) rope_row(q + size_t(t) * q_stride, n_head, head_dim, pos + t, inv_freq);
        std::memcpy(kr.data(), k + size_t(t) * kv_stride, kv_dim * sizeof(float));
        rope_row(kr.data(), n_head_kv, head_dim, pos + t, inv_freq);
        uint16_t* kd = k_cache + dst_offset + size_t(t) * kv_dim;
        uint16_t* vd = v_cache + dst_offset + size_t(t) * kv_dim;
        const float* vs = v + size_t(t) * kv_stride;
        for (size_t i = 0; i < kv_dim; i++) {
            kd[i] = float_to_half(kr[i]);
            vd[i] = float_to_half(vs[i]);
        }
    }
    return 0;
}

void oracle_f32_to_f16(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = float_to_half(in[i]);
}

void oracle_f16_to_f32(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = half_to_float(in[i]);
}

void oracle_softmax(float* x, size_t n) {
    if (n > 0) softmax(x, n);
}

int oracle_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                       int n_head, int n_head_kv, int head_dim, int n_keys, float scale,
                       int n_threads) {
    if (!q || !k_cache || !v_cache || !out || n_head <= 0 || n_head_kv <= 0 || head_dim <= 0 ||
        n_keys <= 0 || n_head % n_head_kv != 0)
        return -1;
    const int group = n_head / n_head_kv;  // src/cpu_backend.cpp:29
    const size_t kv_stride = size_t(n_head_kv) * head_dim;
    parallel_for(n_head, n_threads, [&](int h) {
        std::vector<float> sc(static_cast<size_t>(n_keys));
        attend_one(q + size_t(h) * head_dim, k_cache, v_cache, out + size_t(h) * head_dim, sc.data(),
                   head_dim, kv_stride, size_t(h / group), n_keys, scale);
    });
    return 0;
}

int oracle_attn_prefill(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                        int n_head, int n_head_kv, int head_dim, int pos, int n_tok, int q_stride,
                        float scale, int n_threads) {
    if (!q || !k_cache || !v_cache || !out || n_head <= 0 || n_head_kv <= 0 || head_dim <= 0 ||
        pos < 0 || n_tok <= 0 || n_head % n_head_kv != 0 || q_stride < n_head * head_dim)
        return -1;
    const int group = n_head / n_head_kv;
    const size_t kv_stride = size_t(n_head_kv) * head_dim;
    // forward_batch default (src/backend.h:16-20): token i runs as a decode step at pos + i.
    parallel_for(n_head, n_threads, [&](int h) {
        std::vector<float> sc(static_cast<size_t>(pos + n_tok));
        for (int i = 0; i < n_tok; i++) {
            const size_t row = size_t(i) * q_stride + size_t(h) * head_dim;
            attend_one(q + row, k_cache, v_cache, out + row, sc.data(), head_dim, kv_stride,
                       size_t(h / group), pos + i + 1, scale);
        }
    });
    return 0;
}

}  // extern "C"
