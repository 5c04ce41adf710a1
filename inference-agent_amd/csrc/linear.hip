// linear.hip — out (+)= W·x over GGUF weight layouts, for gfx950.
//
// The projection right after attention (wo with the residual accumulate, src/metal_backend.mm:
// 446-447; src/cpu_backend.cpp:71-72) and every other linear layer of the forward pass
// (src/metal_backend.mm:282-310). W keeps its on-disk layout: ne = [n_in, n_out], row r holds
// n_in elements in blocks of the tensor type (src/ops.cpp:33-87 for the block formats).
// x is f32 [n_tok][n_in]; out is f32 [n_tok][n_out] starting at out + out_offset.
//
// One token (decode): linear_matvec_kernel. The op is HBM-bound (each weight byte used once).
// A workgroup copies the contiguous bytes of its rows into LDS with 16-byte loads (quantized
// blocks are only 2-byte aligned, so parsing them straight from HBM would need 2-byte loads),
// then every wave takes a quarter of the row length for all of the rows, with its slice of x in
// registers, and dequantizes 8 elements at a time from LDS in f32. Arithmetic is f32 throughout,
// like the CPU path (src/ops.cpp:199-224) and the Metal matvec kernels (shaders/kernels.metal:
// 73-226).
//
// Several tokens (prefill): linear_matmul_kernel on v_mfma_f32_32x32x16_f16. Like the Metal
// path (to_half + matmul_tiles, src/metal_backend.mm:385-392, shaders/kernels.metal:779-850)
// both x and the dequantized weights are rounded to f16 and products accumulate in f32. The
// MFMA B operand gives each lane 8 consecutive k of one column, i.e. 8 consecutive elements of
// one weight row — exactly one dequantization group — so each wave dequantizes its own 64 rows
// straight from global memory into registers (prefetched one 32-wide k step ahead) and only x,
// shared by the four waves, goes through LDS.
#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

typedef float float16v_ __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBufferFlags = 0x00020000;  // buffer descriptor word 3 (raw, 32-bit format)

// ---------------------------------------------------------------- block formats

// GGUF type ids (ggml's enum, src/gguf.h:30-33).
enum : int { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ8_0 = 8, kQ6_K = 14, kBF16 = 30 };

__device__ __forceinline__ float f16_bits(uint32_t h) {
    return float(__builtin_bit_cast(_Float16, uint16_t(h)));
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}
// 8 bytes from a 2-byte aligned address.
__device__ __forceinline__ void ld_8bytes(const uint8_t* p, uint32_t& lo, uint32_t& hi) {
    lo = ld_u16(p) | (ld_u16(p + 2) << 16);
    hi = ld_u16(p + 4) | (ld_u16(p + 6) << 16);
}
__device__ __forceinline__ uint32_t byte_of(uint32_t lo, uint32_t hi, int i) {
    return ((i < 4 ? lo : hi) >> (8 * (i & 3))) & 0xFF;
}

// Elements k..k+7 (k % 8 == 0) of the row starting at `row`, dequantized to f32.
// Q8_0 (34 B / 32): d·q.  Q4_0 (18 B / 32): byte j holds element j (low nibble) and j+16
// (high nibble), d·(nibble-8).  Q4_1 (20 B / 32): d·nibble + m.  Q6_K (210 B / 256): ql[128]
// low 4 bits, qh[64] high 2 bits, 16 int8 scales, f16 d; within each 128-element half, element
// 32g + l (g = 0..3, l = 0..31) takes the low (g < 2) or high nibble of ql[l + 32(g&1)] and
// bits 2g..2g+1 of qh[l], with scale index l/16 + 2g: d·scale·(q6-32).
template <int T>
__device__ __forceinline__ void deq8(const uint8_t* row, uint32_t k, float w[8]) {
    if constexpr (T == kF32) {
        const float4v a = *reinterpret_cast<const float4v*>(row + 4 * k);
        const float4v b = *reinterpret_cast<const float4v*>(row + 4 * k + 16);
        for (int i = 0; i < 4; i++) { w[i] = a[i]; w[i + 4] = b[i]; }
    } else if constexpr (T == kF16) {
        const half8 h = *reinterpret_cast<const half8*>(row + 2 * k);
        for (int i = 0; i < 8; i++) w[i] = float(h[i]);
    } else if constexpr (T == kBF16) {
        const u32x4 u = *reinterpret_cast<const u32x4*>(row + 2 * k);
        for (int i = 0; i < 4; i++) {
            w[2 * i] = __uint_as_float(u[i] << 16);
            w[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
        }
    } else if constexpr (T == kQ8_0) {
        const uint8_t* b = row + 34 * (k / 32);
        const float d = f16_bits(ld_u16(b));
        uint32_t lo, hi;
        ld_8bytes(b + 2 + k % 32, lo, hi);
        for (int i = 0; i < 8; i++) w[i] = d * float(int8_t(byte_of(lo, hi, i)));
    } else if constexpr (T == kQ4_0 || T == kQ4_1) {
        constexpr int kBytes = T == kQ4_0 ? 18 : 20, kQs = T == kQ4_0 ? 2 : 4;
        const uint8_t* b = row + kBytes * (k / 32);
        const uint32_t off = k % 32;
        const float d = f16_bits(ld_u16(b));
        const float m = T == kQ4_1 ? f16_bits(ld_u16(b + 2)) : -8.f * d;
        uint32_t lo, hi;
        ld_8bytes(b + kQs + (off & 15), lo, hi);
        const int sh = off >= 16 ? 4 : 0;
        for (int i = 0; i < 8; i++) w[i] = d * float((byte_of(lo, hi, i) >> sh) & 0xF) + m;
    } else if constexpr (T == kQ6_K) {
        const uint8_t* b = row + 210 * (k / 256);
        const uint32_t e = k % 256, h = e / 128, g = (e % 128) / 32, l = e % 32;
        const float d = f16_bits(ld_u16(b + 208));
        const float s = d * float(int8_t(b[192 + h * 8 + l / 16 + 2 * g]));
        uint32_t ql0, ql1, qh0, qh1;
        ld_8bytes(b + h * 64 + 32 * (g & 1) + l, ql0, ql1);
        ld_8bytes(b + 128 + h * 32 + l, qh0, qh1);
        const int shl = g >= 2 ? 4 : 0, shh = 2 * int(g);
        for (int i = 0; i < 8; i++) {
            const int q = int(((byte_of(ql0, ql1, i) >> shl) & 0xF) |
                              (((byte_of(qh0, qh1, i) >> shh) & 3) << 4));
            w[i] = s * float(q - 32);
        }
    }
}

template <int T> struct Fmt;
template <> struct Fmt<kF32>  { static constexpr uint32_t blk = 1,   bytes = 4; };
template <> struct Fmt<kF16>  { static constexpr uint32_t blk = 1,   bytes = 2; };
template <> struct Fmt<kBF16> { static constexpr uint32_t blk = 1,   bytes = 2; };
template <> struct Fmt<kQ8_0> { static constexpr uint32_t blk = 32,  bytes = 34; };
template <> struct Fmt<kQ4_0> { static constexpr uint32_t blk = 32,  bytes = 18; };
template <> struct Fmt<kQ4_1> { static constexpr uint32_t blk = 32,  bytes = 20; };
template <> struct Fmt<kQ6_K> { static constexpr uint32_t blk = 256, bytes = 210; };

__device__ __forceinline__ float wave_sum(float x) {
    x = row16_sum(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

// ---------------------------------------------------------------- one token

constexpr int kMvMaxRows = 8;
constexpr uint32_t kMvLdsRows = 32768;  // bytes of weight rows staged per workgroup (at most)

template <int T>
__global__ __launch_bounds__(256) void linear_matvec_kernel(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ out,
    uint32_t n_in, uint32_t n_out, uint32_t rows_per_wg, uint32_t row_bytes, uint64_t w_bytes,
    uint32_t accumulate) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const uint32_t row0 = blockIdx.x * rows_per_wg;
    const uint32_t nrows = min(rows_per_wg, n_out - row0);

    // Stage the rows' bytes [start, start + nrows*row_bytes) from a 16-byte aligned address.
    const uint64_t start = uint64_t(row0) * row_bytes;
    const uint64_t a0 = start & ~uint64_t(15);
    const uint32_t shift = uint32_t(start - a0);
    const uint32_t span = shift + nrows * row_bytes;
    const uint32_t nchunks = (span + 15) / 16;
    const uint64_t left = w_bytes - a0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(W + a0), 0, int(left < 0x7fffffffu ? left : 0x7fffffffu), kBufferFlags);
    for (uint32_t c = tid; c < nchunks; c += 256)
        *reinterpret_cast<u32x4*>(smem + 16 * c) =
            __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(16 * c), 0, 0));
    float* red = reinterpret_cast<float*>(smem + 16 * nchunks);  // [4 waves][kMvMaxRows]

    // This wave's share of the 8-element groups, and x for them, loaded while the copy lands.
    const uint32_t groups = n_in / 8, per_wave = (groups + 3) / 4;
    const uint32_t g_begin = wave * per_wave, g_end = min(groups, g_begin + per_wave);
    __syncthreads();

    float acc[kMvMaxRows];
#pragma unroll
    for (int r = 0; r < kMvMaxRows; r++) acc[r] = 0.f;
    const uint8_t* rows = smem + shift;
    for (uint32_t g = g_begin + lane; g < g_end; g += 64) {
        const float4v x0 = *reinterpret_cast<const float4v*>(x + 8 * g);
        const float4v x1 = *reinterpret_cast<const float4v*>(x + 8 * g + 4);
#pragma unroll
        for (int r = 0; r < kMvMaxRows; r++) {
            if (uint32_t(r) < nrows) {
                float w[8];
                deq8<T>(rows + r * row_bytes, 8 * g, w);
                float s = acc[r];
                for (int i = 0; i < 4; i++) s += w[i] * x0[i];
                for (int i = 0; i < 4; i++) s += w[i + 4] * x1[i];
                acc[r] = s;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kMvMaxRows; r++) {
        if (uint32_t(r) < nrows) {
            const float s = wave_sum(acc[r]);
            if (lane == 0) red[wave * kMvMaxRows + r] = s;
        }
    }
    __syncthreads();
    if (tid < nrows) {
        const float s = (red[tid] + red[kMvMaxRows + tid]) + (red[2 * kMvMaxRows + tid] + red[3 * kMvMaxRows + tid]);
        float* o = out + row0 + tid;
        *o = accumulate ? *o + s : s;
    }
}

// ---------------------------------------------------------------- several tokens

constexpr int kMmToks = 64;        // tokens per workgroup
constexpr int kMmRowsWave = 64;    // weight rows per wave
constexpr int kMmRows = 4 * kMmRowsWave;
constexpr int kMmK = 32;           // k per step
constexpr int kXPitch = kMmK + 8;  // f16 elements per staged token row (80 B: conflict-free b128 reads)

// Raw weight bytes of one lane for one k step: row-block j (rows 32j + lane%32 of the wave),
// elements k0 + 16s + 8h + i (h = lane/32, s = 0, 1; i = 0..7).
template <int T> struct Raw;
template <> struct Raw<kF32>  { float4v v[2][2][2]; };
template <> struct Raw<kF16>  { half8 v[2][2]; };
template <> struct Raw<kBF16> { u32x4 v[2][2]; };
template <> struct Raw<kQ8_0> { uint32_t d[2]; uint32_t q[2][2][2]; };
template <> struct Raw<kQ4_0> { uint32_t d[2]; uint32_t q[2][2]; };
template <> struct Raw<kQ4_1> { uint32_t d[2]; uint32_t m[2]; uint32_t q[2][2]; };
template <> struct Raw<kQ6_K> { uint32_t d[2]; uint32_t sc[2]; uint32_t ql[2][2][2]; uint32_t qh[2][2][2]; };

template <int T>
__device__ __forceinline__ void load_raw(Raw<T>& r, const uint8_t* const rows[2], uint32_t k0, uint32_t h) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint8_t* row = rows[j];
        if constexpr (T == kF32) {
            for (int s = 0; s < 2; s++) {
                const float4v* p = reinterpret_cast<const float4v*>(row + 4 * (k0 + 16 * s + 8 * h));
                r.v[j][s][0] = p[0];
                r.v[j][s][1] = p[1];
            }
        } else if constexpr (T == kF16 || T == kBF16) {
            for (int s = 0; s < 2; s++) {
                const uint8_t* p = row + 2 * (k0 + 16 * s + 8 * h);
                if constexpr (T == kF16) r.v[j][s] = *reinterpret_cast<const half8*>(p);
                else r.v[j][s] = *reinterpret_cast<const u32x4*>(p);
            }
        } else if constexpr (T == kQ8_0) {
            const uint8_t* b = row + 34 * (k0 / 32);
            r.d[j] = ld_u16(b);
            for (int s = 0; s < 2; s++) ld_8bytes(b + 2 + 16 * s + 8 * h, r.q[j][s][0], r.q[j][s][1]);
        } else if constexpr (T == kQ4_0 || T == kQ4_1) {
            constexpr int kBytes = T == kQ4_0 ? 18 : 20, kQs = T == kQ4_0 ? 2 : 4;
            const uint8_t* b = row + kBytes * (k0 / 32);
            r.d[j] = ld_u16(b);
            if constexpr (T == kQ4_1) r.m[j] = ld_u16(b + 2);
            ld_8bytes(b + kQs + 8 * h, r.q[j][0], r.q[j][1]);
        } else if constexpr (T == kQ6_K) {
            const uint8_t* b = row + 210 * (k0 / 256);
            const uint32_t e = k0 % 256, hh = e / 128, g = (e % 128) / 32;
            r.d[j] = ld_u16(b + 208);
            r.sc[j] = ld_u16(b + 192 + hh * 8 + 2 * g);  // scales for s = 0 (low byte) and 1
            for (int s = 0; s < 2; s++) {
                const uint32_t l = 16 * s + 8 * h;
                ld_8bytes(b + hh * 64 + 32 * (g & 1) + l, r.ql[j][s][0], r.ql[j][s][1]);
                ld_8bytes(b + 128 + hh * 32 + l, r.qh[j][s][0], r.qh[j][s][1]);
            }
        }
    }
}

// The f16 B fragment of row-block j, step s.
template <int T>
__device__ __forceinline__ half8 frag(const Raw<T>& r, int j, int s, uint32_t k0) {
    half8 o;
    if constexpr (T == kF16) {
        o = r.v[j][s];
    } else if constexpr (T == kF32) {
        for (int i = 0; i < 4; i++) {
            o[i] = _Float16(r.v[j][s][0][i]);
            o[i + 4] = _Float16(r.v[j][s][1][i]);
        }
    } else if constexpr (T == kBF16) {
        for (int i = 0; i < 4; i++) {
            o[2 * i] = _Float16(__uint_as_float(r.v[j][s][i] << 16));
            o[2 * i + 1] = _Float16(__uint_as_float(r.v[j][s][i] & 0xFFFF0000u));
        }
    } else if constexpr (T == kQ8_0) {
        const float d = f16_bits(r.d[j]);
        for (int i = 0; i < 8; i++) o[i] = _Float16(d * float(int8_t(byte_of(r.q[j][s][0], r.q[j][s][1], i))));
    } else if constexpr (T == kQ4_0 || T == kQ4_1) {
        const float d = f16_bits(r.d[j]);
        float m = -8.f * d;
        if constexpr (T == kQ4_1) m = f16_bits(r.m[j]);
        const int sh = 4 * s;  // elements 16..31 of the block are the high nibbles
        for (int i = 0; i < 8; i++) o[i] = _Float16(d * float((byte_of(r.q[j][0], r.q[j][1], i) >> sh) & 0xF) + m);
    } else if constexpr (T == kQ6_K) {
        const uint32_t g = (k0 % 128) / 32;
        const float sc = f16_bits(r.d[j]) * float(int8_t((r.sc[j] >> (8 * s)) & 0xFF));
        const int shl = g >= 2 ? 4 : 0, shh = 2 * int(g);
        for (int i = 0; i < 8; i++) {
            const int q = int(((byte_of(r.ql[j][s][0], r.ql[j][s][1], i) >> shl) & 0xF) |
                              (((byte_of(r.qh[j][s][0], r.qh[j][s][1], i) >> shh) & 3) << 4));
            o[i] = _Float16(sc * float(q - 32));
        }
    }
    return o;
}

template <int T>
__global__ __launch_bounds__(256) void linear_matmul_kernel(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ out,
    uint32_t n_in, uint32_t n_out, uint32_t n_tok, uint32_t row_bytes, uint32_t accumulate) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][kMmToks * kXPitch];
    const uint32_t tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const uint32_t n = lane % 32, h = lane / 32;
    const uint32_t tok0 = blockIdx.y * kMmToks;
    const uint32_t rowbase = blockIdx.x * kMmRows + wave * kMmRowsWave;

    // x staging: thread t converts 8 consecutive k of token t/4.
    const uint32_t st_tok = tid / 4, st_k = 8 * (tid % 4);
    const bool st_ok = tok0 + st_tok < n_tok;
    const float* xrow = x + size_t(st_ok ? tok0 + st_tok : 0) * n_in + st_k;
    float4v xa = {0.f, 0.f, 0.f, 0.f}, xb = xa;
    auto load_x = [&](uint32_t k0) {
        if (st_ok) {
            xa = *reinterpret_cast<const float4v*>(xrow + k0);
            xb = *reinterpret_cast<const float4v*>(xrow + k0 + 4);
        }
    };
    auto store_x = [&](int buf) {
        half8 v;
        for (int i = 0; i < 4; i++) { v[i] = _Float16(xa[i]); v[i + 4] = _Float16(xb[i]); }
        *reinterpret_cast<half8*>(&xs[buf][st_tok * kXPitch + st_k]) = v;
    };

    const uint8_t* rows[2];
    for (int j = 0; j < 2; j++)
        rows[j] = W + size_t(min(rowbase + 32 * j + n, n_out - 1)) * row_bytes;

    float16v_ acc[2][2];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

    Raw<T> raw;
    load_raw<T>(raw, rows, 0, h);
    load_x(0);
    store_x(0);
    __syncthreads();

    const uint32_t steps = n_in / kMmK;
    for (uint32_t t = 0; t < steps; t++) {
        const uint32_t k0 = t * kMmK;
        const int buf = t & 1;
        half8 b[2][2];
        for (int j = 0; j < 2; j++)
            for (int s = 0; s < 2; s++) b[j][s] = frag<T>(raw, j, s, k0);
        const bool more = t + 1 < steps;
        if (more) {
            load_raw<T>(raw, rows, k0 + kMmK, h);
            load_x(k0 + kMmK);
        }
#pragma unroll
        for (int s = 0; s < 2; s++) {
            half8 a[2];
            for (int i = 0; i < 2; i++)
                a[i] = *reinterpret_cast<const half8*>(&xs[buf][(32 * i + n) * kXPitch + 16 * s + 8 * h]);
            for (int i = 0; i < 2; i++)
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j][s], acc[i][j], 0, 0, 0);
        }
        if (more) store_x(buf ^ 1);
        __syncthreads();
    }

    // D[m][n] of a 32x32 tile: lane holds column n = lane%32, rows 8(e/4) + 4h + e%4.
    for (int j = 0; j < 2; j++) {
        const uint32_t row = rowbase + 32 * j + n;
        if (row >= n_out) continue;
        for (int i = 0; i < 2; i++) {
            for (int e = 0; e < 16; e++) {
                const uint32_t tok = tok0 + 32 * i + 8 * (e / 4) + 4 * h + e % 4;
                if (tok < n_tok) {
                    float* o = out + size_t(tok) * n_out + row;
                    *o = accumulate ? *o + acc[i][j][e] : acc[i][j][e];
                }
            }
        }
    }
}

template <int T>
int launch_t(const uint8_t* W, const float* x, float* out, uint32_t n_in, uint32_t n_out,
             uint32_t n_tok, uint32_t accumulate, hipStream_t stream) {
    const uint32_t row_bytes = n_in / Fmt<T>::blk * Fmt<T>::bytes;
    if (n_tok == 1) {
        uint32_t r = kMvLdsRows / row_bytes;
        r = r < 1 ? 1 : r > kMvMaxRows ? kMvMaxRows : r;
        // Keep at least ~3 workgroups per CU on the 256-CU part.
        const uint32_t fill = (n_out + 767) / 768;
        if (r > fill) r = fill < 1 ? 1 : fill;
        const uint32_t blocks = (n_out + r - 1) / r;
        const size_t lds = ((size_t(r) * row_bytes + 15 + 15) / 16) * 16 + 4 * kMvMaxRows * sizeof(float);
        hipLaunchKernelGGL(linear_matvec_kernel<T>, dim3(blocks), dim3(256), lds, stream, W, x, out,
                           n_in, n_out, r, row_bytes, uint64_t(n_out) * row_bytes, accumulate);
    } else {
        const dim3 grid((n_out + kMmRows - 1) / kMmRows, (n_tok + kMmToks - 1) / kMmToks);
        if (grid.y > 65535) return -1;
        hipLaunchKernelGGL(linear_matmul_kernel<T>, grid, dim3(256), 0, stream, W, x, out, n_in,
                           n_out, n_tok, row_bytes, accumulate);
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace

int launch_linear(uint32_t type, const void* W, const float* x, float* out, uint32_t n_in,
                  uint32_t n_out, uint32_t n_tok, uint32_t accumulate, hipStream_t stream) {
    const auto* w = static_cast<const uint8_t*>(W);
    switch (type) {
        case kF32:  return launch_t<kF32>(w, x, out, n_in, n_out, n_tok, accumulate, stream);
        case kF16:  return launch_t<kF16>(w, x, out, n_in, n_out, n_tok, accumulate, stream);
        case kBF16: return launch_t<kBF16>(w, x, out, n_in, n_out, n_tok, accumulate, stream);
        case kQ8_0: return launch_t<kQ8_0>(w, x, out, n_in, n_out, n_tok, accumulate, stream);
        case kQ4_0: return launch_t<kQ4_0>(w, x, out, n_in, n_out, n_tok, accumulate, stream);
        case kQ4_1: return launch_t<kQ4_1>(w, x, out, n_in, n_out, n_tok, accumulate, stream);
        case kQ6_K: return launch_t<kQ6_K>(w, x, out, n_in, n_out, n_tok, accumulate, stream);
        default: return -2;
    }
}

}  // namespace ingot
