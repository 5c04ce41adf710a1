// linear_oracle.cpp — CPU restatement of Ingot's linear layer over GGUF weight layouts, used
// ONLY as the checker.
//
// TEST INFRASTRUCTURE. Nothing on the product path links, loads or calls this file; only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it (liboracle.so, ctypes).
//
// What it restates (reference files under /root/reference, read as text, never compiled here —
// src/ops.cpp includes <arm_neon.h> and cannot build for x86):
//   - dequantization, src/ops.cpp:23-87: F32 copy; F16 widen; BF16 as bits << 16;
//     Q8_0 = 34-byte blocks {f16 d, int8 q[32]}, value d*q (lines 34-40);
//     Q4_0 = 18-byte blocks {f16 d, 16 bytes}, element i is the low nibble of byte i and
//     element i+16 the high nibble, value d*(nibble-8) (lines 42-53);
//     Q4_1 = 20-byte blocks {f16 d, f16 m, 16 bytes}, value d*nibble + m (lines 55-65);
//     Q6_K = 210-byte blocks {ql[128], qh[64], int8 scales[16], f16 d} over 256 elements,
//     value d*scale*(q6-32), with the element order of lines 67-87;
//   - ops::dot_row, src/ops.cpp:199-215: F32/F16 rows as one f32 dot; Q8_0/Q4_0 as a per-block
//     dot of the integer values with x, times d, summed over blocks (dot_q8_0 / dot_q4_0, lines
//     153-187); the other types dequantized first and then one f32 dot (lines 208-213);
//   - ops::matvec, src/ops.cpp:218-225 (out[r] = dot_row(W, r, x)), per token; and the residual
//     add x += tmp after wo (src/cpu_backend.cpp:71-72) when `accumulate` is set.
// The NEON dots sum in 4 or 16 interleaved partial sums; this restatement sums left to right.
// The two orders differ by f32 rounding only (relative ~1e-7 * sqrt(n_in)).
//
// oracle_linear_f16 restates the Metal batched path instead (src/metal_backend.mm:298-309,
// 385-392): x rounded to f16 by to_half (shaders/kernels.metal:779-782), the weights
// dequantized to f16 by dequant16 (shaders/kernels.metal:728-776; each value rounded once from
// its f32 expression), products summed in f32.
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "attn_oracle.h"

namespace {

float h2f(uint16_t h) {
    float f;
    oracle_f16_to_f32(&h, &f, 1);
    return f;
}

float f16_round(float x) {
    uint16_t h;
    oracle_f32_to_f16(&x, &h, 1);
    return h2f(h);
}

uint16_t u16(const uint8_t* p) {
    uint16_t v;
    std::memcpy(&v, p, 2);
    return v;
}

int block_elems(int type) {
    switch (type) {
        case 0: case 1: case 30: return 1;
        case 8: case 2: case 3: return 32;
        case 14: return 256;
        default: return 0;
    }
}

int block_bytes(int type) {
    switch (type) {
        case 0: return 4;
        case 1: case 30: return 2;
        case 8: return 34;
        case 2: return 18;
        case 3: return 20;
        case 14: return 210;
        default: return 0;
    }
}

// src/ops.cpp:23-87, n a multiple of the block size.
void dequant(int type, const uint8_t* p, float* out, size_t n) {
    switch (type) {
        case 0: std::memcpy(out, p, n * 4); return;
        case 1: for (size_t i = 0; i < n; i++) out[i] = h2f(u16(p + 2 * i)); return;
        case 30:
            for (size_t i = 0; i < n; i++) {
                const uint32_t u = uint32_t(u16(p + 2 * i)) << 16;
                std::memcpy(out + i, &u, 4);
            }
            return;
        case 8:
            for (size_t b = 0; b < n / 32; b++, p += 34, out += 32) {
                const float d = h2f(u16(p));
                for (int i = 0; i < 32; i++) out[i] = d * float(int8_t(p[2 + i]));
            }
            return;
        case 2:
            for (size_t b = 0; b < n / 32; b++, p += 18, out += 32) {
                const float d = h2f(u16(p));
                for (int i = 0; i < 16; i++) {
                    out[i] = d * float(int(p[2 + i] & 0xF) - 8);
                    out[i + 16] = d * float(int(p[2 + i] >> 4) - 8);
                }
            }
            return;
        case 3:
            for (size_t b = 0; b < n / 32; b++, p += 20, out += 32) {
                const float d = h2f(u16(p)), m = h2f(u16(p + 2));
                for (int i = 0; i < 16; i++) {
                    out[i] = d * float(p[4 + i] & 0xF) + m;
                    out[i + 16] = d * float(p[4 + i] >> 4) + m;
                }
            }
            return;
        case 14:
            for (size_t b = 0; b < n / 256; b++, p += 210, out += 256) {
                const uint8_t* ql = p;
                const uint8_t* qh = p + 128;
                const int8_t* sc = reinterpret_cast<const int8_t*>(p + 192);
                const float d = h2f(u16(p + 208));
                float* y = out;
                for (int half = 0; half < 2; half++) {
                    for (int l = 0; l < 32; l++) {
                        const int is = l / 16;
                        const int q1 = int((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int q2 = int((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = int((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = int((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        y[l] = d * float(sc[is]) * float(q1);
                        y[l + 32] = d * float(sc[is + 2]) * float(q2);
                        y[l + 64] = d * float(sc[is + 4]) * float(q3);
                        y[l + 96] = d * float(sc[is + 6]) * float(q4);
                    }
                    y += 128;
                    ql += 64;
                    qh += 32;
                    sc += 8;
                }
            }
            return;
    }
}

// src/ops.cpp:199-215.
float dot_row(int type, const uint8_t* p, const float* x, size_t n, std::vector<float>& buf) {
    if (type == 8 || type == 2) {  // dot_q8_0 / dot_q4_0: integer values per block, then * d
        const size_t bytes = type == 8 ? 34 : 18;
        float acc = 0.f;
        for (size_t b = 0; b < n / 32; b++, p += bytes, x += 32) {
            const float d = h2f(u16(p));
            float blk = 0.f;
            for (int i = 0; i < 32; i++) {
                int q;
                if (type == 8) q = int8_t(p[2 + i]);
                else q = i < 16 ? int(p[2 + i] & 0xF) - 8 : int(p[2 + i - 16] >> 4) - 8;
                blk += float(q) * x[i];
            }
            acc += blk * d;
        }
        return acc;
    }
    buf.resize(n);
    dequant(type, p, buf.data(), n);
    float s = 0.f;
    for (size_t i = 0; i < n; i++) s += buf[i] * x[i];
    return s;
}

// Metal dequant16 (shaders/kernels.metal:728-776): one f16 rounding of each value's f32 form.
// For Q4_0 / Q4_1 the f32 form d*nibble + (-8d) / d*nibble + m equals the CPU's d*(nibble-8) /
// d*nibble + m here (the products are exact in f32).
void dequant_f16(int type, const uint8_t* p, float* out, size_t n) {
    dequant(type, p, out, n);
    if (type == 1) return;  // already f16
    for (size_t i = 0; i < n; i++) out[i] = f16_round(out[i]);
}

int linear_impl(int f16_path, int type, const uint8_t* w, const float* x, float* out, int n_in,
                int n_out, int n_tok, int accumulate, int n_threads) {
    const int be = block_elems(type);
    if (!w || !x || !out || be == 0 || n_in <= 0 || n_out <= 0 || n_tok <= 0 || n_in % be) return -1;
    const size_t row_bytes = size_t(n_in / be) * block_bytes(type);
    std::vector<float> xh;
    if (f16_path) {
        xh.resize(size_t(n_tok) * n_in);
        for (size_t i = 0; i < xh.size(); i++) xh[i] = f16_round(x[i]);
        x = xh.data();
    }
    if (n_threads < 1) n_threads = 1;
    auto work = [&](int t0) {
        std::vector<float> buf(n_in), wrow(n_in);
        for (int r = t0; r < n_out; r += n_threads) {
            const uint8_t* row = w + size_t(r) * row_bytes;
            if (f16_path) dequant_f16(type, row, wrow.data(), n_in);
            for (int t = 0; t < n_tok; t++) {
                const float* xt = x + size_t(t) * n_in;
                float s;
                if (f16_path) {
                    s = 0.f;
                    for (int i = 0; i < n_in; i++) s += wrow[i] * xt[i];
                } else {
                    s = dot_row(type, row, xt, n_in, buf);
                }
                float* o = out + size_t(t) * n_out + r;
                *o = accumulate ? *o + s : s;
            }
        }
    };
    std::vector<std::thread> pool;
    for (int i = 1; i < n_threads; i++) pool.emplace_back(work, i);
    work(0);
    for (auto& th : pool) th.join();
    return 0;
}

}  // namespace

extern "C" {

int oracle_dequant_row(int type, const uint8_t* row, float* out, int n) {
    const int be = block_elems(type);
    if (!row || !out || be == 0 || n <= 0 || n % be) return -1;
    dequant(type, row, out, size_t(n));
    return 0;
}

int oracle_linear(int type, const uint8_t* w, const float* x, float* out, int n_in, int n_out,
                  int n_tok, int accumulate, int n_threads) {
    return linear_impl(0, type, w, x, out, n_in, n_out, n_tok, accumulate, n_threads);
}

int oracle_linear_f16(int type, const uint8_t* w, const float* x, float* out, int n_in, int n_out,
                      int n_tok, int accumulate, int n_threads) {
    return linear_impl(1, type, w, x, out, n_in, n_out, n_tok, accumulate, n_threads);
}

}  // extern "C"
