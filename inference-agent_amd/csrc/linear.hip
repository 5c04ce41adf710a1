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
#include <type_traits>

#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

typedef float float16v_ __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

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

// dot(elements k..k+7 of the row, x0|x1) for the block types, without materializing each
// weight: the group's quants are converted a byte at a time (unsigned bytes, so Q8_0's int8 are
// biased by +128) and the block offset/scale applied once per group:
//   Q4_0  d * (sum q x - 8 sum x)      Q4_1  d * sum q x + m * sum x
//   Q8_0  d * (sum (q+128) x - 128 sum x)
// The same value as the per-element form up to f32 rounding (CPU dot_q4_0 / dot_q8_0 also sum
// the integer products per block and scale once, src/ops.cpp:153-187).
template <int T>
__device__ __forceinline__ float bytes_dot4(uint32_t w, const float4v& x) {
    float s = float(w & 0xFF) * x[0];
    s += float((w >> 8) & 0xFF) * x[1];
    s += float((w >> 16) & 0xFF) * x[2];
    s += float(w >> 24) * x[3];
    return s;
}

template <int T>
__device__ __forceinline__ float dot8(const uint8_t* row, uint32_t k, const float4v& x0, const float4v& x1) {
    const float sx = ((x0[0] + x0[1]) + (x0[2] + x0[3])) + ((x1[0] + x1[1]) + (x1[2] + x1[3]));
    if constexpr (T == kQ8_0) {
        const uint8_t* b = row + 34 * (k / 32);
        const float d = f16_bits(ld_u16(b));
        uint32_t lo, hi;
        ld_8bytes(b + 2 + k % 32, lo, hi);
        const float s = bytes_dot4<T>(lo ^ 0x80808080u, x0) + bytes_dot4<T>(hi ^ 0x80808080u, x1);
        return d * (s - 128.f * sx);
    } else {
        constexpr int kBytes = T == kQ4_0 ? 18 : 20, kQs = T == kQ4_0 ? 2 : 4;
        const uint8_t* b = row + kBytes * (k / 32);
        const uint32_t off = k % 32;
        const float d = f16_bits(ld_u16(b));
        uint32_t lo, hi;
        ld_8bytes(b + kQs + (off & 15), lo, hi);
        const uint32_t sh = off >= 16 ? 4 : 0;
        const float s = bytes_dot4<T>((lo >> sh) & 0x0F0F0F0Fu, x0) + bytes_dot4<T>((hi >> sh) & 0x0F0F0F0Fu, x1);
        if constexpr (T == kQ4_0) return d * (s - 8.f * sx);
        else return d * s + f16_bits(ld_u16(b + 2)) * sx;
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

constexpr uint32_t kMvLdsBytes = 160 * 1024;  // weight rows + x staged per workgroup (at most)
constexpr int kMvChunks = 8;  // 16-byte staging loads per thread per round (one round up to 32 KB)

// What happens to x before the products, and to the row sums after (ingot_proj):
//   prologue kProNone: x as given; kProRmsNorm: x * (1/sqrt(mean(x^2) + eps)) * aux, the
//     rmsnorm that precedes q/k/v and gate/up (the same arithmetic, in the same order, as
//     rmsnorm_kernel, so the fused and the separate sequence give identical results);
//   epilogue kEpiStore / kEpiAccumulate: out = s or out += s per matrix; kEpiSiluGate: two
//     matrices (gate, up) over the same rows, out0 = silu(s_gate) * s_up with
//     silu(g) = g / (1 + exp(-g)), as silu_mul_kernel.
enum : int { kProNone = 0, kProRmsNorm = 1 };
enum : int { kEpiStore = 0, kEpiAccumulate = 1, kEpiSiluGate = 2, kEpiRopeKv = 3 };
//   kEpiRopeKv: matrices q, k, v of one decode token: q and k rotated by RoPE (pairs (2i, 2i+1)
//     of each head, angle pos * inv_freq[i], rotated as rope_kv_store_kernel does), q stored in
//     f32, K and V rounded to f16 into their cache rows (ingot_rope_kv_store's work).

// Up to three matrices of one type sharing n_in and x (q/k/v, gate/up), launched as one grid:
// blocks [blk_end[m-1], blk_end[m]) take matrix m's rows, R per block.
struct MvArgs {
    const uint8_t* W[3];
    float* out[3];
    uint32_t n_out[3];
    uint32_t blk_end[3];
    const float* x;
    const float* aux;  // rmsnorm weights [n_in]
    uint32_t n_in, row_bytes;
    float eps;
    // kEpiRopeKv
    const float* inv_freq;
    _Float16* cache[2];  // K and V rows of the token
    uint32_t head_dim, pos;
};

// R weight rows per matrix per workgroup of 4 waves (2R for the gate/up pair); each wave takes a
// quarter of the 8-element groups of all rows, reads x for a group once and applies it to every
// row (x dominates the LDS reads otherwise: 32 bytes per group against ~10 for a Q4_0 row). x
// (and the rmsnorm weights), and for the block-quantized types the rows' bytes, are staged in
// LDS by one pass of 16-byte loads, all issued before the first wait; rows of plain
// F32/F16/BF16 elements (every group a 16- or 32-byte aligned piece) are read straight from
// memory. Rows past n_out are computed from a clamped row and not written.
template <int T>
constexpr bool kMvStageW = !(T == kF32 || T == kF16 || T == kBF16);

template <int T, int R, int PRO, int EPI>
__global__ __launch_bounds__(256) void linear_matvec_kernel(const MvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int NS = EPI == kEpiSiluGate ? 2 : 1;  // row sets: (gate, up) or one matrix
    constexpr int NR = NS * R;
    const uint32_t tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    uint32_t m = 0, blk = blockIdx.x;
    if constexpr (EPI != kEpiSiluGate) {
        if (blk >= a.blk_end[0]) m = blk >= a.blk_end[1] ? 2 : 1;
        if (m > 0) blk -= a.blk_end[m - 1];
    }
    const uint32_t n_in = a.n_in, row_bytes = a.row_bytes;
    const uint32_t n_out = a.n_out[m];
    const uint32_t row0 = blk * R;
    const uint32_t nrows = min(uint32_t(R), n_out - row0);

    // LDS: x ([n_in] f32, 16-byte chunks), the rmsnorm weights, then each set's rows' bytes
    // from a 16-byte aligned start.
    const uint32_t xchunks = n_in / 4;
    const uint32_t achunks = PRO == kProRmsNorm ? xchunks : 0;
    const uint64_t start = uint64_t(row0) * row_bytes;
    const uint64_t a0 = start & ~uint64_t(15);
    const uint32_t shift = uint32_t(start - a0);
    const uint32_t wchunks = kMvStageW<T> ? (shift + nrows * row_bytes + 15) / 16 : 0;
    const uint32_t nchunks = xchunks + achunks + NS * wchunks;
    const uint64_t w_bytes = uint64_t(n_out) * row_bytes;
    // Bytes from a0 to the end of the matrix, rounded up to whole dwords: buffer loads drop
    // every dword that reaches past num_records, and a row may end mid-dword (an odd number of
    // 18-, 34- or 210-byte rows); the dword holding the last byte never crosses a page.
    const uint64_t left = (w_bytes - a0 + 3) & ~uint64_t(3);
    const int wrec = int(left < 0x7fffffffu ? left : 0x7fffffffu);
    __amdgpu_buffer_rsrc_t ws[NS];
#pragma unroll
    for (int s = 0; s < NS; s++)
        ws[s] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.W[m + s] + a0), 0, wrec, kBufferFlags);
    const __amdgpu_buffer_rsrc_t xs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.x), 0,
                                                                        int(4 * n_in), kBufferFlags);
    const __amdgpu_buffer_rsrc_t as = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(PRO == kProRmsNorm ? a.aux : a.x), 0, int(4 * n_in), kBufferFlags);
    // The staging rounds walk the regions x | norm weights | row set 0 | row set 1, each padded
    // to a multiple of 256 chunks, so that a load's source (its buffer descriptor) is uniform
    // across the workgroup: a descriptor chosen per lane makes the compiler loop over the
    // distinct descriptors of a wave.
    const uint32_t px = (xchunks + 255) & ~255u, pa = (achunks + 255) & ~255u, pw = (wchunks + 255) & ~255u;
    const uint32_t nvirt = px + pa + NS * pw;
    for (uint32_t base = 0; base < nvirt; base += 256 * kMvChunks) {
        u32x4 st[kMvChunks];
        uint32_t dst[kMvChunks];
#pragma unroll
        for (int i = 0; i < kMvChunks; i++) {
            const uint32_t v0 = base + 256u * i;  // workgroup-uniform
            if (v0 >= nvirt) break;
            // region of this round slot, its chunk count, LDS chunk offset and descriptor
            uint32_t start, count, lds0;
            __amdgpu_buffer_rsrc_t src;
            if (v0 < px) {
                start = 0; count = xchunks; lds0 = 0; src = xs;
            } else if (v0 < px + pa) {
                start = px; count = achunks; lds0 = xchunks; src = as;
            } else if (NS == 1 || v0 < px + pa + pw) {
                start = px + pa; count = wchunks; lds0 = xchunks + achunks; src = ws[0];
            } else {
                start = px + pa + pw; count = wchunks; lds0 = xchunks + achunks + wchunks; src = ws[NS - 1];
            }
            const uint32_t local = v0 - start + tid;
            st[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(src, int(16 * min(local, count - 1)), 0, 0));
            dst[i] = local < count ? lds0 + local : ~0u;
        }
#pragma unroll
        for (int i = 0; i < kMvChunks; i++) {
            if (base + 256u * i >= nvirt) break;
            if (dst[i] != ~0u) *reinterpret_cast<u32x4*>(smem + 16 * dst[i]) = st[i];
        }
    }
    float* red = reinterpret_cast<float*>(smem + 16 * nchunks);  // [4 waves][NR]
    __syncthreads();

    float* xl = reinterpret_cast<float*>(smem);
    if constexpr (PRO == kProRmsNorm) {
        // rmsnorm_kernel's reduction: float4 per thread strided by 1024 elements, row sums,
        // then the four wave partials in fixed order; each thread then rescales the elements
        // it summed.
        const float* wl = xl + n_in;
        float ss = 0.f;
        for (uint32_t i = 4 * tid; i < n_in; i += 1024) {
            const float4v v = *reinterpret_cast<const float4v*>(xl + i);
            ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
        }
        ss = row16_sum(ss);
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        const float total = (red[0] + red[1]) + (red[2] + red[3]);
        const float scale = 1.0f / sqrtf(total / float(n_in) + a.eps);
        for (uint32_t i = 4 * tid; i < n_in; i += 1024) {
            const float4v v = *reinterpret_cast<const float4v*>(xl + i);
            const float4v g = *reinterpret_cast<const float4v*>(wl + i);
            *reinterpret_cast<float4v*>(xl + i) = v * scale * g;
        }
        __syncthreads();
    }

    const uint32_t groups = n_in / 8, per_wave = (groups + 3) / 4;
    const uint32_t g_begin = wave * per_wave, g_end = min(groups, g_begin + per_wave);
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) acc[r] = 0.f;
    if constexpr (kMvStageW<T>) {
        const uint8_t* rows = smem + 16 * (xchunks + achunks) + shift;
        for (uint32_t g = g_begin + lane; g < g_end; g += 64) {
            const float4v x0 = *reinterpret_cast<const float4v*>(xl + 8 * g);
            const float4v x1 = *reinterpret_cast<const float4v*>(xl + 8 * g + 4);
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const uint8_t* row = rows + (r / R) * 16 * wchunks + min(uint32_t(r % R), nrows - 1) * row_bytes;
                if constexpr (T == kQ8_0 || T == kQ4_0 || T == kQ4_1) {
                    acc[r] += dot8<T>(row, 8 * g, x0, x1);
                } else {
                    float w[8];
                    deq8<T>(row, 8 * g, w);
                    float s = 0.f;
                    for (int i = 0; i < 4; i++) s += w[i] * x0[i];
                    for (int i = 0; i < 4; i++) s += w[i + 4] * x1[i];
                    acc[r] += s;
                }
            }
        }
    } else {
        constexpr uint32_t GB = T == kF32 ? 32 : 16;  // bytes per 8-element group
        __amdgpu_buffer_rsrc_t rs[NS];
#pragma unroll
        for (int s = 0; s < NS; s++)
            rs[s] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.W[m + s] + start), 0,
                                                      int(nrows * row_bytes), kBufferFlags);
        for (uint32_t g = g_begin + lane; g < g_end; g += 64) {
            u32x4 raw[NR][GB / 16];
#pragma unroll
            for (int r = 0; r < NR; r++)
                for (uint32_t q = 0; q < GB / 16; q++)
                    raw[r][q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                             rs[r / R], int(min(uint32_t(r % R), nrows - 1) * row_bytes + g * GB + 16 * q), 0, 0));
            const float4v x0 = *reinterpret_cast<const float4v*>(xl + 8 * g);
            const float4v x1 = *reinterpret_cast<const float4v*>(xl + 8 * g + 4);
#pragma unroll
            for (int r = 0; r < NR; r++) {
                float w[8];
                deq8<T>(reinterpret_cast<const uint8_t*>(&raw[r][0]), 0, w);
                float s = 0.f;
                for (int i = 0; i < 4; i++) s += w[i] * x0[i];
                for (int i = 0; i < 4; i++) s += w[i + 4] * x1[i];
                acc[r] += s;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const float s = wave_sum(acc[r]);
        if (lane == 0) red[wave * NR + r] = s;
    }
    __syncthreads();
    if (tid < nrows) {
        auto total = [&](int r) { return (red[r] + red[NR + r]) + (red[2 * NR + r] + red[3 * NR + r]); };
        float* o = a.out[m] + row0 + tid;
        if constexpr (EPI == kEpiSiluGate) {
            const float g = total(tid), u = total(R + tid);
            *o = g / (1.0f + expf(-g)) * u;
        } else {
            const float s = total(tid);
            *o = EPI == kEpiAccumulate ? *o + s : s;
        }
    }
}

// ---------------------------------------------------------------- one token, streamed rows

// The block types with 32-element blocks and the 16-bit float types take a second one-token
// kernel that reads weight rows straight from memory into registers (no LDS staging, no
// barrier between the loads and the arithmetic): x (after the rmsnorm prologue) is staged in
// LDS once per workgroup; a half-wave (32 lanes) owns RPH rows and walks their 32-element
// columns, lane l taking columns l, l+32, ..., with the next column's loads issued before the
// current column's arithmetic. A quantized block is only 2-byte aligned, so a lane loads the
// dword-aligned window around it (5 dwords for Q4_0 / Q4_1, 9 for Q8_0) and realigns it with
// v_alignbyte. Each x column is read from LDS once per lane and applied to all RPH rows.
template <int T> struct Col;
template <> struct Col<kQ4_0> { static constexpr int ndw = 5, bytes = 18; };
template <> struct Col<kQ4_1> { static constexpr int ndw = 5, bytes = 20; };
template <> struct Col<kQ8_0> { static constexpr int ndw = 9, bytes = 34; };
template <> struct Col<kF16>  { static constexpr int ndw = 16, bytes = 64; };
template <> struct Col<kBF16> { static constexpr int ndw = 16, bytes = 64; };
// Q6_K: column c is the 32-element group (h, g) = ((c % 8) / 4, c % 4) of 210-byte block c / 8;
// the lane loads the windows of its 32 low-bit bytes, its 32 high-bit bytes, its two scales and
// the block's d.
template <> struct Col<kQ6_K> { static constexpr int ndw = 20; };

template <int T>
constexpr bool kStreamed = T == kQ4_0 || T == kQ4_1 || T == kQ8_0 || T == kF16 || T == kBF16 || T == kQ6_K;

// Byte offset of column c from the row start.
template <int T>
__device__ __forceinline__ uint32_t col_offset(uint32_t c) {
    if constexpr (T == kQ6_K) return 210 * (c >> 3);
    else return c * Col<T>::bytes;
}

// The window of the column at byte offset off (relative to a 16-byte aligned buffer base).
template <int T>
__device__ __forceinline__ void col_load(const __amdgpu_buffer_rsrc_t& rs, uint32_t off, uint32_t (&w)[Col<T>::ndw],
                                         uint32_t c = 0) {
    auto ld4 = [&](uint32_t o, int at) {
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(o), 0, 0));
        w[at] = v[0]; w[at + 1] = v[1]; w[at + 2] = v[2]; w[at + 3] = v[3];
    };
    if constexpr (T == kQ6_K) {
        const uint32_t h = (c >> 2) & 1, g = c & 3;
        const uint32_t pl = (off + 64 * h + 32 * (g & 1)) & ~3u, ph = (off + 128 + 32 * h) & ~3u;
        ld4(pl, 0);
        ld4(pl + 16, 4);
        w[8] = __builtin_amdgcn_raw_buffer_load_b32(rs, int(pl + 32), 0, 0);
        ld4(ph, 9);
        ld4(ph + 16, 13);
        w[17] = __builtin_amdgcn_raw_buffer_load_b32(rs, int(ph + 32), 0, 0);
        w[18] = __builtin_amdgcn_raw_buffer_load_b32(rs, int((off + 192 + 8 * h + 2 * g) & ~3u), 0, 0);
        w[19] = __builtin_amdgcn_raw_buffer_load_b32(rs, int((off + 208) & ~3u), 0, 0);
    } else if constexpr (T == kF16 || T == kBF16) {
        for (int i = 0; i < 4; i++) ld4(off + 16 * i, 4 * i);
    } else {
        const uint32_t p = off & ~3u;
        ld4(p, 0);
        if constexpr (T == kQ8_0) ld4(p + 16, 4);
        w[Col<T>::ndw - 1] = __builtin_amdgcn_raw_buffer_load_b32(rs, int(p + 4 * (Col<T>::ndw - 1)), 0, 0);
    }
}

// s + sum_k byte_k(q) * x[k], one fma per element (v_cvt_f32_ubyte0..3 read the bytes in place).
__device__ __forceinline__ float fma_u8x4(uint32_t q, const float4v& x, float s) {
    s = fmaf(float(q & 0xFF), x[0], s);
    s = fmaf(float((q >> 8) & 0xFF), x[1], s);
    s = fmaf(float((q >> 16) & 0xFF), x[2], s);
    return fmaf(float(q >> 24), x[3], s);
}

// The low / high nibbles of each byte of w, as bytes. The mask is applied in inline asm so the
// optimizer cannot fold it into the byte extraction of fma_u8x4 (it would turn each
// v_cvt_f32_ubyteN into a bit-field extract plus a conversion).
__device__ __forceinline__ uint32_t lo_nibbles(uint32_t w) {
    uint32_t r;
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(w));
    return r;
}
__device__ __forceinline__ uint32_t hi_nibbles(uint32_t w) {
    uint32_t r;
    asm("v_lshrrev_b32 %0, 4, %1\n\tv_and_b32 %0, 0x0f0f0f0f, %0" : "=&v"(r) : "v"(w));
    return r;
}

// W-row column · x column (32 elements; sx = sum of the x column, shared by the rows).
template <int T>
__device__ __forceinline__ float col_dot(const uint32_t (&w)[Col<T>::ndw], uint32_t off, const float4v (&x)[8], float sx,
                                         uint32_t c = 0, float sx_hi = 0.f) {
    if constexpr (T == kQ6_K) {
        // q = (4 low bits from ql: the low nibble for g < 2, else the high one) | (2 bits of qh
        // at 2g) << 4, an unsigned 0..63 byte; each 16 elements share an int8 scale:
        // d * (sc_lo * (sum_lo q x - 32 sum_lo x) + sc_hi * (sum_hi q x - 32 sum_hi x)).
        const uint32_t h = (c >> 2) & 1, g = c & 3;
        const uint32_t shl_ = (off + 64 * h + 32 * (g & 1)) & 3, shh_ = (off + 128 + 32 * h) & 3;
        const uint32_t nib = g >= 2 ? 4 : 0, hb = 2 * g;
        float s_lo = 0.f, s_hi = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t ql = __builtin_amdgcn_alignbyte(w[i + 1], w[i], shl_);
            const uint32_t qh = __builtin_amdgcn_alignbyte(w[9 + i + 1], w[9 + i], shh_);
            uint32_t q = ((ql >> nib) & 0x0F0F0F0Fu) | (((qh >> hb) & 0x03030303u) << 4);
            asm("" : "+v"(q));  // keep the byte conversions as v_cvt_f32_ubyteN
            if (i < 4) s_lo = fma_u8x4(q, x[i], s_lo);
            else s_hi = fma_u8x4(q, x[i], s_hi);
        }
        const uint32_t scw = w[18] >> (8 * ((off + 192 + 8 * h + 2 * g) & 3));
        const float sc_lo = float(int8_t(scw & 0xFF)), sc_hi = float(int8_t((scw >> 8) & 0xFF));
        const float d = f16_bits((w[19] >> (8 * ((off + 208) & 3))) & 0xFFFF);
        const float t = fmaf(sc_lo, fmaf(-32.f, sx, s_lo), __fmul_rn(sc_hi, fmaf(-32.f, sx_hi, s_hi)));
        return __fmul_rn(d, t);
    } else if constexpr (T == kF16 || T == kBF16) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t u = w[2 * i + e];
                float lo, hi;
                if constexpr (T == kF16) {
                    lo = f16_bits(u & 0xFFFF);
                    hi = f16_bits(u >> 16);
                } else {
                    lo = __uint_as_float(u << 16);
                    hi = __uint_as_float(u & 0xFFFF0000u);
                }
                s = fmaf(lo, x[i][2 * e], s);
                s = fmaf(hi, x[i][2 * e + 1], s);
            }
        }
        return s;
    } else if constexpr (T == kQ4_1) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s = fma_u8x4(lo_nibbles(w[1 + i]), x[i], s);
            s = fma_u8x4(hi_nibbles(w[1 + i]), x[4 + i], s);
        }
        return fmaf(f16_bits(w[0] & 0xFFFF), s, __fmul_rn(f16_bits(w[0] >> 16), sx));
    } else {
        // the block starts at byte 0 or 2 of the window; its quants at byte 2 or 4
        const bool odd = (off & 2) != 0;
        const float d = f16_bits((odd ? w[0] >> 16 : w[0]) & 0xFFFF);
        constexpr int NQ = T == kQ8_0 ? 8 : 4;
        uint32_t q[NQ];
#pragma unroll
        for (int i = 0; i < NQ; i++) q[i] = odd ? w[i + 1] : __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
        float s = 0.f;
        if constexpr (T == kQ8_0) {
#pragma unroll
            for (int i = 0; i < 8; i++) s = fma_u8x4(q[i] ^ 0x80808080u, x[i], s);
            return __fmul_rn(d, fmaf(-128.f, sx, s));
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                s = fma_u8x4(lo_nibbles(q[i]), x[i], s);
                s = fma_u8x4(hi_nibbles(q[i]), x[4 + i], s);
            }
            return __fmul_rn(d, fmaf(-8.f, sx, s));
        }
    }
}

// x chunk (16 bytes) i of the staged x -> its LDS slot: column c = i / 8 keeps its 8 chunks,
// permuted by (c / 2) % 8, so that the 16 lanes of one LDS read phase (consecutive columns,
// same chunk) hit 16 different 16-byte bank groups.
__device__ __forceinline__ uint32_t xslot(uint32_t i) {
    const uint32_t c = i >> 3;
    return (c << 3) | ((i & 7) ^ ((c >> 1) & 7));
}

template <int T, int RPH, int PRO, int EPI, int NT>
__global__ __launch_bounds__(NT) void linear_stream_kernel(const MvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int NDW = Col<T>::ndw;
    constexpr int RPM = EPI == kEpiSiluGate ? RPH / 2 : RPH;  // rows of each matrix per half-wave
    const uint32_t tid = threadIdx.x, lane = tid % 64, hw = tid / 32, l32 = tid % 32;
    uint32_t m = 0, blk = blockIdx.x;
    if constexpr (EPI != kEpiSiluGate) {
        if (blk >= a.blk_end[0]) m = blk >= a.blk_end[1] ? 2 : 1;
        if (m > 0) blk -= a.blk_end[m - 1];
    }
    const uint32_t n_in = a.n_in, row_bytes = a.row_bytes, n_out = a.n_out[m];
    constexpr uint32_t NHW = NT / 32;  // half-waves
    const uint32_t row0 = blk * NHW * RPM;  // the workgroup's first row of matrix m

    // This half-wave's rows: RPM of matrix m (and the same RPM of matrix m + 1 for the gate/up
    // pair); rows past n_out read the last row and are not written.
    const uint64_t wbase = (uint64_t(row0) * row_bytes) & ~uint64_t(15);
    uint32_t roff[RPH];
#pragma unroll
    for (int i = 0; i < RPH; i++) {
        const uint32_t r = min(row0 + hw * RPM + uint32_t(i % RPM), n_out - 1);
        roff[i] = uint32_t(uint64_t(r) * row_bytes - wbase);
    }
    const uint64_t left = (uint64_t(n_out) * row_bytes - wbase + 3) & ~uint64_t(3);
    const int nrec = int(left < 0x7fffffffu ? left : 0x7fffffffu);
    __amdgpu_buffer_rsrc_t rs[EPI == kEpiSiluGate ? 2 : 1];
    rs[0] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.W[m] + wbase), 0, nrec, kBufferFlags);
    if constexpr (EPI == kEpiSiluGate)
        rs[1] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.W[1] + wbase), 0, nrec, kBufferFlags);

    const uint32_t ncols = n_in / 32, last = ncols - 1;
    const uint32_t nsteps = (ncols + 31) / 32;
    uint32_t b0[RPH][NDW], b1[RPH][NDW], b2[RPH][NDW];
    auto load = [&](uint32_t step, uint32_t (&b)[RPH][NDW]) {
        const uint32_t c = min(step * 32 + l32, last);
#pragma unroll
        for (int i = 0; i < RPH; i++) col_load<T>(rs[i / RPM], roff[i] + col_offset<T>(c), b[i], c);
    };
    // x (and the norm weights, unpermuted after it) into LDS. The loads of x's first round go
    // out first, then the first three columns of the rows (they do not depend on x), then x is
    // stored: the row data streams in while x is staged and normalized.
    const uint32_t xchunks = n_in / 4;
    const uint32_t nchunks = PRO == kProRmsNorm ? 2 * xchunks : xchunks;
    float4v* xl = reinterpret_cast<float4v*>(smem);
    const __amdgpu_buffer_rsrc_t xs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.x), 0,
                                                                        int(4 * n_in), kBufferFlags);
    const __amdgpu_buffer_rsrc_t as = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(PRO == kProRmsNorm ? a.aux : a.x), 0, int(4 * n_in), kBufferFlags);
    auto stage_round = [&](uint32_t base, bool prefetch) {
        float4v st[kMvChunks];
        // (x chunks and norm-weight chunks come from two descriptors; the choice is made per
        // load from the workgroup-uniform round position, never per lane, which would make the
        // compiler loop over the distinct descriptors of a wave)
#pragma unroll
        for (int i = 0; i < kMvChunks; i++) {
            if (base + NT * i >= nchunks) break;  // workgroup-uniform
            const uint32_t c = min(base + tid + NT * i, nchunks - 1);
            const uint32_t cx = min(c, xchunks - 1);
            const float4v vx = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(xs, int(16 * cx), 0, 0));
            if (PRO == kProRmsNorm && base + NT * i + NT - 1 >= xchunks) {
                const uint32_t ca = c >= xchunks ? c - xchunks : 0;
                const float4v va = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(as, int(16 * ca), 0, 0));
                st[i] = c < xchunks ? vx : va;
            } else {
                st[i] = vx;
            }
        }
        if (prefetch) {
            load(0, b0);
            load(1, b1);
            load(2, b2);
        }
#pragma unroll
        for (int i = 0; i < kMvChunks; i++) {
            if (base + NT * i >= nchunks) break;
            const uint32_t c = base + tid + NT * i;
            if (c < nchunks) xl[c < xchunks ? xslot(c) : c] = st[i];
        }
    };
    stage_round(0, false);
    for (uint32_t base = NT * kMvChunks; base < nchunks; base += NT * kMvChunks) stage_round(base, false);
    float* part = reinterpret_cast<float*>(smem + 16 * nchunks);  // [4] wave partials
    __syncthreads();
    load(0, b0);
    load(1, b1);
    load(2, b2);
    if constexpr (PRO == kProRmsNorm) {
        // rmsnorm_kernel's arithmetic and order: its 256 threads' float4 sums strided by 1024
        // elements (the first four waves here), row sums, the four wave partials in fixed
        // order; then the elementwise rescale by every thread.
        if (tid < 256) {
            float ss = 0.f;
            for (uint32_t i = tid; i < xchunks; i += 256) {
                const float4v v = xl[xslot(i)];
                ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
            }
            ss = row16_sum(ss);
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            if (lane == 0) part[tid / 64] = ss;
        }
        __syncthreads();
        const float total = (part[0] + part[1]) + (part[2] + part[3]);
        const float scale = 1.0f / sqrtf(total / float(n_in) + a.eps);
        for (uint32_t i = tid; i < xchunks; i += NT) xl[xslot(i)] = xl[xslot(i)] * scale * xl[xchunks + i];
        __syncthreads();
    }

    float acc[RPH];
#pragma unroll
    for (int i = 0; i < RPH; i++) acc[i] = 0.f;
    auto compute = [&](uint32_t step, const uint32_t (&b)[RPH][NDW]) {
        const uint32_t c0 = step * 32 + l32;
        const uint32_t c = min(c0, last);
        float4v xv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) xv[j] = xl[(c << 3) | (j ^ ((c >> 1) & 7))];
        float sx = 0.f, sx_hi = 0.f;
        if constexpr (T == kQ4_0 || T == kQ4_1 || T == kQ8_0) {
#pragma unroll
            for (int j = 0; j < 8; j++) sx += (xv[j][0] + xv[j][1]) + (xv[j][2] + xv[j][3]);
        } else if constexpr (T == kQ6_K) {  // the two 16-element halves separately
#pragma unroll
            for (int j = 0; j < 4; j++) sx += (xv[j][0] + xv[j][1]) + (xv[j][2] + xv[j][3]);
#pragma unroll
            for (int j = 4; j < 8; j++) sx_hi += (xv[j][0] + xv[j][1]) + (xv[j][2] + xv[j][3]);
        }
        const bool valid = c0 < ncols;
#pragma unroll
        for (int i = 0; i < RPH; i++) {
            // explicit roundings: every instantiation (rows per half-wave, prologue, epilogue)
            // sums a row in exactly the same way
            const float v = col_dot<T>(b[i], roff[i] + col_offset<T>(c), xv, sx, c, sx_hi);
            acc[i] = __fadd_rn(acc[i], valid ? v : 0.f);
        }
    };
    // three columns in flight (all of a 3072-long row), refilled as each is computed; the
    // last three buffered columns are computed without refills
    uint32_t st = 0;
    for (; st + 3 < nsteps; st += 3) {
        compute(st, b0);
        load(st + 3, b0);
        compute(st + 1, b1);
        load(st + 4, b1);
        compute(st + 2, b2);
        load(st + 5, b2);
    }
    compute(st, b0);
    compute(st + 1, b1);
    compute(st + 2, b2);

    // Row sums over the half-wave; lane i writes row i.
    float tot[RPH];
#pragma unroll
    for (int i = 0; i < RPH; i++) {
        float t = row16_sum(acc[i]);
        tot[i] = t + __shfl_xor(t, 16);
    }
    if constexpr (EPI == kEpiRopeKv) {
        // RPM is even and row0 + hw * RPM is even: each rotary pair is in one half-wave
        static_assert(RPM % 2 == 0, "rotary pairs stay in one half-wave");
        if (l32 < uint32_t(RPM)) {
            const uint32_t r = row0 + hw * RPM + l32;
            float val = tot[0];
#pragma unroll
            for (int i = 1; i < RPM; i++) val = l32 == uint32_t(i) ? tot[i] : val;
            if (m < 2) {
                // partner of the pair
                float x0 = tot[0], x1 = tot[1];
#pragma unroll
                for (int i = 2; i < RPM; i += 2) {
                    x0 = (l32 >> 1) == uint32_t(i / 2) ? tot[i] : x0;
                    x1 = (l32 >> 1) == uint32_t(i / 2) ? tot[i + 1] : x1;
                }
                const uint32_t pair = (r % a.head_dim) / 2;
                float sn, cs;
                sincosf(float(a.pos) * a.inv_freq[pair], &sn, &cs);
                val = (l32 & 1) ? rope_odd(x0, x1, cs, sn) : rope_even(x0, x1, cs, sn);
            }
            if (r < n_out) {
                if (m == 0) a.out[0][r] = val;
                else a.cache[m - 1][r] = _Float16(val);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < RPM; i++) {
            const uint32_t r = row0 + hw * RPM + i;
            if (l32 == uint32_t(i) && r < n_out) {
                float* o = a.out[m] + r;
                if constexpr (EPI == kEpiSiluGate) {
                    const float g = tot[i], u = tot[RPM + i];
                    *o = g / (1.0f + expf(-g)) * u;
                } else {
                    *o = EPI == kEpiAccumulate ? *o + tot[i] : tot[i];
                }
            }
        }
    }
}

template <int T, int RPH, int PRO, int EPI, int NT>
int launch_st(const MvArgs& a, uint32_t blocks, size_t lds, hipStream_t stream) {
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&linear_stream_kernel<T, RPH, PRO, EPI, NT>),
        hipFuncAttributeMaxDynamicSharedMemorySize, int(kMvLdsBytes));
    if (attr != hipSuccess) return -4;
    hipLaunchKernelGGL((linear_stream_kernel<T, RPH, PRO, EPI, NT>), dim3(blocks), dim3(NT), lds, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <int T, int RPH, int PRO, int NT>
int launch_st_epi(const MvArgs& a, int epi, uint32_t blocks, size_t lds, hipStream_t stream) {
    switch (epi) {
        case kEpiStore: return launch_st<T, RPH, PRO, kEpiStore, NT>(a, blocks, lds, stream);
        case kEpiAccumulate: return launch_st<T, RPH, PRO, kEpiAccumulate, NT>(a, blocks, lds, stream);
        case kEpiRopeKv:
            if constexpr (RPH >= 2) return launch_st<T, RPH, PRO, kEpiRopeKv, NT>(a, blocks, lds, stream);
            return -2;
        default:
            if constexpr (RPH >= 2) return launch_st<T, RPH, PRO, kEpiSiluGate, NT>(a, blocks, lds, stream);
            return -2;
    }
}

// Workgroup shape: many rows per workgroup (x is staged once per workgroup, and its staging
// traffic otherwise rivals the weights' for the smaller matrices) while the grid still fills the
// 256 CUs: 512 threads with 4, 2 or 1 rows per half-wave when that gives 128..256 workgroups,
// else 256 threads with the most rows per half-wave that still gives >= 256 workgroups (the
// gate/up pair: at least 2, one of each matrix). F16/BF16 windows are 16 dwords: at most 2.
template <int T>
int launch_stream_t(MvArgs a, uint32_t n_mats, int pro, int epi, hipStream_t stream) {
    const bool silu = epi == kEpiSiluGate;
    // (Q6_K: 20-dword windows; two rows per half-wave only where an epilogue needs row pairs,
    // and then in 256-thread workgroups, whose register budget holds them without spilling)
    constexpr int kMaxRph = T == kQ6_K ? 1 : T == kF16 || T == kBF16 ? 2 : 4;
    const int min_rph = silu || epi == kEpiRopeKv ? 2 : 1;
    auto count = [&](int nt, int rph, bool set) {
        const uint32_t rpw = uint32_t(nt / 32) * uint32_t(silu ? rph / 2 : rph);  // rows per workgroup
        uint32_t blocks = 0;
        for (uint32_t m = 0; m < 3; m++) {
            if (m < n_mats && !(silu && m > 0)) blocks += (a.n_out[m] + rpw - 1) / rpw;
            if (set) a.blk_end[m] = blocks;
        }
        return blocks;
    };
    // (measured: a CU holds one 512-thread workgroup of this kernel at a time, so those are
    // used only when one round of at most 256 of them covers the rows)
    int nt = 0, rph = min_rph;
    for (int r = kMaxRph; r >= min_rph && !nt; r /= 2) {
        const uint32_t b = count(512, r, false);
        if (b >= 128 && b <= 256) { nt = 512; rph = r; }
    }
    for (int r = kMaxRph; r >= min_rph && !nt; r /= 2)
        if (count(256, r, false) >= 256 || r == min_rph) { nt = 256; rph = r; }
    if (!nt) { nt = 256; rph = min_rph; }  // (Q6_K pairs: min_rph above kMaxRph)
    const uint32_t blocks = count(nt, rph, true);
    const size_t lds = size_t(a.n_in) * 4 * (pro == kProRmsNorm ? 2 : 1) + 16;
    if (lds > kMvLdsBytes) return -2;
    auto go = [&](auto pro_tag, auto nt_tag) -> int {
        constexpr int P = decltype(pro_tag)::value, N = decltype(nt_tag)::value;
        switch (rph) {
            case 4: if constexpr (kMaxRph >= 4) return launch_st_epi<T, 4, P, N>(a, epi, blocks, lds, stream); return -2;
            case 2: if constexpr (kMaxRph >= 2 || N == 256) return launch_st_epi<T, 2, P, N>(a, epi, blocks, lds, stream); return -2;
            default: return launch_st_epi<T, 1, P, N>(a, epi, blocks, lds, stream);
        }
    };
    using R = std::integral_constant<int, kProRmsNorm>;
    using X = std::integral_constant<int, kProNone>;
    using N5 = std::integral_constant<int, 512>;
    using N2 = std::integral_constant<int, 256>;
    if (pro == kProRmsNorm) return nt == 512 ? go(R{}, N5{}) : go(R{}, N2{});
    return nt == 512 ? go(X{}, N5{}) : go(X{}, N2{});
}

// Bytes of LDS a matvec workgroup stages (x, norm weights, rows) plus its reduction slots.
template <int T>
size_t matvec_lds(uint32_t n_in, uint32_t row_bytes, int R, int pro, int epi) {
    const int ns = epi == kEpiSiluGate ? 2 : 1;
    const size_t x = size_t(n_in) * 4 * (pro == kProRmsNorm ? 2 : 1);
    const size_t w = kMvStageW<T> ? (size_t(R) * row_bytes + 15 + 15) / 16 * 16 : 0;
    return x + ns * w + 4 * size_t(ns) * R * sizeof(float);
}

template <int T, int R, int PRO, int EPI>
int launch_mv(const MvArgs& a, uint32_t blocks, size_t lds, hipStream_t stream) {
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&linear_matvec_kernel<T, R, PRO, EPI>),
        hipFuncAttributeMaxDynamicSharedMemorySize, int(kMvLdsBytes));
    if (attr != hipSuccess) return -4;
    hipLaunchKernelGGL((linear_matvec_kernel<T, R, PRO, EPI>), dim3(blocks), dim3(256), lds, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <int T, int R, int PRO>
int launch_mv_epi(const MvArgs& a, int epi, uint32_t blocks, size_t lds, hipStream_t stream) {
    switch (epi) {
        case kEpiStore: return launch_mv<T, R, PRO, kEpiStore>(a, blocks, lds, stream);
        case kEpiAccumulate: return launch_mv<T, R, PRO, kEpiAccumulate>(a, blocks, lds, stream);
        default:
            if constexpr (R <= 4) return launch_mv<T, R, PRO, kEpiSiluGate>(a, blocks, lds, stream);
            return -2;
    }
}

// One token through up to three matrices (n_mats) of type T: out[m] (+)= W[m]·x'.
template <int T>
int launch_matvec_t(MvArgs a, uint32_t n_mats, int pro, int epi, hipStream_t stream) {
    const uint32_t n_in = a.n_in;
    a.row_bytes = n_in / Fmt<T>::blk * Fmt<T>::bytes;
    if constexpr (kStreamed<T>) return launch_stream_t<T>(a, n_mats, pro, epi, stream);
    uint32_t rows = 0;
    for (uint32_t m = 0; m < n_mats; m++) rows = max(rows, a.n_out[m]);
    // Eight rows per matrix per workgroup when that still leaves >= 3 workgroups per CU
    // (measured: fewer, larger workgroups are slower here; more rows per workgroup only pay
    // for x traffic, which is not the limit) and the rows fit the staging buffer; four
    // otherwise. The gate/up pair takes four of each.
    // (One row per workgroup when four do not fit: long rows, e.g. a 28672-wide down projection.)
    int R = 4;
    if (epi != kEpiSiluGate && rows / 8 >= 768 && matvec_lds<T>(n_in, a.row_bytes, 8, pro, epi) <= kMvLdsBytes) R = 8;
    if (matvec_lds<T>(n_in, a.row_bytes, R, pro, epi) > kMvLdsBytes) R = 1;
    const size_t lds = matvec_lds<T>(n_in, a.row_bytes, R, pro, epi);
    if (lds > kMvLdsBytes) return -2;  // rows too long to stage
    uint32_t blocks = 0;
    for (uint32_t m = 0; m < 3; m++) {
        if (m < n_mats) blocks += (a.n_out[m] + R - 1) / R;
        a.blk_end[m] = blocks;
    }
    if (epi == kEpiSiluGate) blocks = a.blk_end[0];
    if (pro == kProRmsNorm)
        return R == 8 ? launch_mv_epi<T, 8, kProRmsNorm>(a, epi, blocks, lds, stream)
             : R == 4 ? launch_mv_epi<T, 4, kProRmsNorm>(a, epi, blocks, lds, stream)
                      : launch_mv_epi<T, 1, kProRmsNorm>(a, epi, blocks, lds, stream);
    return R == 8 ? launch_mv_epi<T, 8, kProNone>(a, epi, blocks, lds, stream)
         : R == 4 ? launch_mv_epi<T, 4, kProNone>(a, epi, blocks, lds, stream)
                  : launch_mv_epi<T, 1, kProNone>(a, epi, blocks, lds, stream);
}

// ---------------------------------------------------------------- several tokens

constexpr int kMmWaves = 8;
constexpr int kMmToks = 64;        // tokens per workgroup
constexpr int kMmRowsWave = 32;    // weight rows per wave (one 32-wide MFMA column block)
constexpr int kMmRows = kMmWaves * kMmRowsWave;
constexpr int kMmK = 32;           // k per step
constexpr int kXPitch = kMmK + 8;  // f16 elements per staged token row (80 B: conflict-free b128 reads)

// Raw weight bytes of one lane for one k step: row rowbase + lane%32 of the wave, elements
// k0 + 16s + 8h + i (h = lane/32, s = 0, 1; i = 0..7) — the B operands of the step's two
// 32x32x16 MFMAs.
template <int T> struct Raw;
template <> struct Raw<kF32>  { float4v v[2][2]; };
template <> struct Raw<kF16>  { half8 v[2]; };
template <> struct Raw<kBF16> { u32x4 v[2]; };
template <> struct Raw<kQ8_0> { uint32_t d; uint32_t q[2][2]; };
template <> struct Raw<kQ4_0> { uint32_t d; uint32_t q[2]; };
template <> struct Raw<kQ4_1> { uint32_t d; uint32_t m; uint32_t q[2]; };
template <> struct Raw<kQ6_K> { uint32_t d; uint32_t sc; uint32_t ql[2][2]; uint32_t qh[2][2]; };

template <int T>
__device__ __forceinline__ void load_raw(Raw<T>& r, const uint8_t* row, uint32_t k0, uint32_t h) {
    if constexpr (T == kF32) {
        for (int s = 0; s < 2; s++) {
            const float4v* p = reinterpret_cast<const float4v*>(row + 4 * (k0 + 16 * s + 8 * h));
            r.v[s][0] = p[0];
            r.v[s][1] = p[1];
        }
    } else if constexpr (T == kF16 || T == kBF16) {
        for (int s = 0; s < 2; s++) {
            const uint8_t* p = row + 2 * (k0 + 16 * s + 8 * h);
            if constexpr (T == kF16) r.v[s] = *reinterpret_cast<const half8*>(p);
            else r.v[s] = *reinterpret_cast<const u32x4*>(p);
        }
    } else if constexpr (T == kQ8_0) {
        const uint8_t* b = row + 34 * (k0 / 32);
        r.d = ld_u16(b);
        for (int s = 0; s < 2; s++) ld_8bytes(b + 2 + 16 * s + 8 * h, r.q[s][0], r.q[s][1]);
    } else if constexpr (T == kQ4_0 || T == kQ4_1) {
        constexpr int kBytes = T == kQ4_0 ? 18 : 20, kQs = T == kQ4_0 ? 2 : 4;
        const uint8_t* b = row + kBytes * (k0 / 32);
        r.d = ld_u16(b);
        if constexpr (T == kQ4_1) r.m = ld_u16(b + 2);
        ld_8bytes(b + kQs + 8 * h, r.q[0], r.q[1]);
    } else if constexpr (T == kQ6_K) {
        const uint8_t* b = row + 210 * (k0 / 256);
        const uint32_t e = k0 % 256, hh = e / 128, g = (e % 128) / 32;
        r.d = ld_u16(b + 208);
        r.sc = ld_u16(b + 192 + hh * 8 + 2 * g);  // scales for s = 0 (low byte) and 1
        for (int s = 0; s < 2; s++) {
            const uint32_t l = 16 * s + 8 * h;
            ld_8bytes(b + hh * 64 + 32 * (g & 1) + l, r.ql[s][0], r.ql[s][1]);
            ld_8bytes(b + 128 + hh * 32 + l, r.qh[s][0], r.qh[s][1]);
        }
    }
}

// The f16 B fragment of step half s.
// load_raw from a row staged in LDS. A quantized block is only 2-byte aligned, so the 8 or 16
// quant bytes are read as dword-aligned dwords and realigned with v_alignbyte (an 8-byte LDS
// read at a 2-byte aligned address stalls on the unaligned access).
// 8 bytes at a 2-byte aligned LDS address, as two dwords.
__device__ __forceinline__ void lds_8bytes(const uint8_t* a, uint32_t& lo, uint32_t& hi) {
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(a)) & 3;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(a - sh);
    const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
    lo = __builtin_amdgcn_alignbyte(w1, w0, sh);
    hi = __builtin_amdgcn_alignbyte(w2, w1, sh);
}

template <int T>
__device__ __forceinline__ void load_raw_lds(Raw<T>& r, const uint8_t* row, uint32_t k0, uint32_t h) {
    if constexpr (T == kQ4_0) {
        const uint8_t* b = row + 18 * (k0 / 32);
        r.d = ld_u16(b);
        lds_8bytes(b + 2 + 8 * h, r.q[0], r.q[1]);
    } else if constexpr (T == kQ8_0) {
        const uint8_t* b = row + 34 * (k0 / 32);
        r.d = ld_u16(b);
        for (int s = 0; s < 2; s++) lds_8bytes(b + 2 + 16 * s + 8 * h, r.q[s][0], r.q[s][1]);
    } else if constexpr (T == kQ6_K) {  // `row` is the block (a stage holds one)
        const uint32_t e = k0 % 256, hh = e / 128, g = (e % 128) / 32;
        r.d = ld_u16(row + 208);
        r.sc = ld_u16(row + 192 + hh * 8 + 2 * g);
        for (int s = 0; s < 2; s++) {
            const uint32_t l = 16 * s + 8 * h;
            lds_8bytes(row + hh * 64 + 32 * (g & 1) + l, r.ql[s][0], r.ql[s][1]);
            lds_8bytes(row + 128 + hh * 32 + l, r.qh[s][0], r.qh[s][1]);
        }
    } else {
        load_raw<T>(r, row, k0, h);
    }
}

// Block types whose B fragments hold their 8 k values in the order 0,2,1,3,4,6,5,7: two
// elements two bytes apart share a 32-bit word, so one masked word gives a packed half pair.
template <int T>
constexpr bool kFragSwap13 = T == kQ4_0 || T == kQ8_0;

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    return (a & m) | c;  // v_and_or_b32
}

template <int T>
__device__ __forceinline__ half8 frag(const Raw<T>& r, int s, uint32_t k0) {
    half8 o;
    if constexpr (T == kF16) {
        o = r.v[s];
    } else if constexpr (T == kF32) {
        for (int i = 0; i < 4; i++) {
            o[i] = _Float16(r.v[s][0][i]);
            o[i + 4] = _Float16(r.v[s][1][i]);
        }
    } else if constexpr (T == kBF16) {
        for (int i = 0; i < 4; i++) {
            o[2 * i] = _Float16(__uint_as_float(r.v[s][i] << 16));
            o[2 * i + 1] = _Float16(__uint_as_float(r.v[s][i] & 0xFFFF0000u));
        }
    } else if constexpr (T == kQ8_0) {
        // Packed f16, k order 0,2,1,3 per word: the byte q ^ 0x80 = q + 128 becomes the half
        // 1024 + q + 128 (exact), minus 1152 gives q, times d rounds once — d*q rounded to half,
        // as when formed in f32.
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const _Float16 dh = __builtin_bit_cast(_Float16, uint16_t(r.d));
        const h2 dd = {dh, dh}, off = {_Float16(-1152.f), _Float16(-1152.f)};
        for (int w = 0; w < 2; w++) {
            const uint32_t q = r.q[s][w] ^ 0x80808080u;
            const h2 a = (__builtin_bit_cast(h2, and_or(q, 0x00FF00FFu, 0x64006400u)) + off) * dd;
            const h2 b = (__builtin_bit_cast(h2, and_or(q >> 8, 0x00FF00FFu, 0x64006400u)) + off) * dd;
            o[4 * w] = a[0];      // k 4w
            o[4 * w + 1] = a[1];  // k 4w + 2
            o[4 * w + 2] = b[0];  // k 4w + 1
            o[4 * w + 3] = b[1];  // k 4w + 3
        }
    } else if constexpr (T == kQ4_0) {
        // Packed f16, k order 0,2,1,3 per word: the nibble n becomes the half 1024 + n (bits
        // 0x6400 | n), minus 1032 gives n - 8 exactly, times d rounds once — the same value as
        // d*(n-8) formed in f32 and rounded to half.
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const _Float16 dh = __builtin_bit_cast(_Float16, uint16_t(r.d));
        const h2 dd = {dh, dh}, off = {_Float16(-1032.f), _Float16(-1032.f)};
        const uint32_t sh = 4 * s;  // elements 16..31 of the block are the high nibbles
        for (int w = 0; w < 2; w++) {
            const uint32_t q = r.q[w] >> sh;
            const h2 a = (__builtin_bit_cast(h2, and_or(q, 0x000F000Fu, 0x64006400u)) + off) * dd;
            const h2 b = (__builtin_bit_cast(h2, and_or(q >> 8, 0x000F000Fu, 0x64006400u)) + off) * dd;
            o[4 * w] = a[0];      // k 4w
            o[4 * w + 1] = a[1];  // k 4w + 2
            o[4 * w + 2] = b[0];  // k 4w + 1
            o[4 * w + 3] = b[1];  // k 4w + 3
        }
    } else if constexpr (T == kQ4_1) {
        const float d = f16_bits(r.d);
        const float m = f16_bits(r.m);
        const int sh = 4 * s;  // elements 16..31 of the block are the high nibbles
        for (int i = 0; i < 8; i++) o[i] = _Float16(d * float((byte_of(r.q[0], r.q[1], i) >> sh) & 0xF) + m);
    } else if constexpr (T == kQ6_K) {
        // Four 6-bit values per word (low nibbles from ql, two high bits from qh, byte-wise),
        // each converted from its byte; sc*(q - 32) is formed as fma(sc, q, -32*sc): -32*sc is
        // exact and the fma rounds the exact sc*q - 32*sc once, the same f32 value.
        const uint32_t g = (k0 % 128) / 32;
        const float sc = f16_bits(r.d) * float(int8_t((r.sc >> (8 * s)) & 0xFF));
        const float c = -32.f * sc;
        const uint32_t shl = g >= 2 ? 4 : 0, shh = 2 * g;
        for (int w = 0; w < 2; w++) {
            const uint32_t q = ((r.ql[s][w] >> shl) & 0x0F0F0F0Fu) | (((r.qh[s][w] >> shh) & 0x03030303u) << 4);
            for (int b = 0; b < 4; b++) o[4 * w + b] = _Float16(__builtin_fmaf(sc, float((q >> (8 * b)) & 0xFF), c));
        }
    }
    return o;
}

// Split-K bookkeeping: one counter per output tile (own 64-byte line), then the partial tiles.
constexpr int kScDevice = 16;                 // buffer cache-policy bits: sc1 = device scope
constexpr uint32_t kTileFloats = kMmToks * kMmRows;
constexpr uint32_t kMaxSplits = 8;
// Output transpose: one 32-token half of a wave's 64 x 32 tile at a time, rows of 32 floats
// at a pitch of 40 (the two token groups of a write instruction land in opposite bank halves).
constexpr int kOutPitch = 40;
constexpr int kOutStage = 32 * kOutPitch;

// W staged through LDS (LW kernels): a stage is `ks` elements of every row of the tile, `bytes`
// per row (a whole number of 16-byte chunks, so lanes load full cache lines), stored at a row
// pitch that keeps the B-operand reads free of bank conflicts.
// `win`: the stage's bytes do not start on a 16-byte boundary (Q6_K: 210-byte blocks, rows of
// 210 * n_in / 256 bytes), so each row's stage is loaded as the 16-byte aligned window that holds
// it (14 chunks hold the 210 bytes at any even shift) and read at the row's shift within it. The
// pitch of 232 bytes (58 dwords: 32 rows on distinct banks) is 8-byte aligned, so a window chunk
// goes to LDS as two 8-byte writes.
template <int T> struct Stage { static constexpr uint32_t ks = 0, bytes = 0, pitch = 0; static constexpr bool swz = false, win = false; };
template <> struct Stage<kF32>  { static constexpr uint32_t ks = 32,  bytes = 128, pitch = 128; static constexpr bool swz = true, win = false; };
template <> struct Stage<kF16>  { static constexpr uint32_t ks = 64,  bytes = 128, pitch = 128; static constexpr bool swz = true, win = false; };
template <> struct Stage<kBF16> { static constexpr uint32_t ks = 64,  bytes = 128, pitch = 128; static constexpr bool swz = true, win = false; };
template <> struct Stage<kQ8_0> { static constexpr uint32_t ks = 256, bytes = 272, pitch = 272; static constexpr bool swz = false, win = false; };
template <> struct Stage<kQ4_0> { static constexpr uint32_t ks = 256, bytes = 144, pitch = 144; static constexpr bool swz = false, win = false; };
template <> struct Stage<kQ4_1> { static constexpr uint32_t ks = 256, bytes = 160, pitch = 176; static constexpr bool swz = false, win = false; };
template <> struct Stage<kQ6_K> { static constexpr uint32_t ks = 256, bytes = 224, pitch = 232; static constexpr bool swz = false, win = true; };

// 16-byte chunk swizzles of the LDS stages (XOR of the chunk index with a function of the row)
// so that the 16-row b128 reads and the 2-row (b128) or 4-row (b64) write groups each touch 64
// distinct banks. 128-byte rows (two rows per 64 banks): rows of one parity take the 8 chunk
// positions in the order of g3(r >> 1), whose bit 2 alternates between consecutive pairs.
__device__ __forceinline__ uint32_t g3(uint32_t m) { return ((m & 1) << 2) | ((m >> 1) & 3); }
__device__ __forceinline__ uint32_t swz128(uint32_t r) { return g3((r >> 1) & 7); }
// x rows of XK halves: 64 B (four rows per 64 banks), 128 B, 256 B (one row per 64 banks).
template <uint32_t XK>
__device__ __forceinline__ uint32_t swz_x(uint32_t r) {
    if constexpr (XK == 32) return (r >> 2) & 3;
    else if constexpr (XK == 64) return swz128(r);
    else return ((r & 3) << 2) | ((r >> 2) & 3);
}

// Up to three matrices of one type sharing n_in and x (q/k/v of a chunk) in one launch: their
// row tiles are numbered one after another, matrix m taking tiles [tile_end[m-1], tile_end[m]);
// out[m] is [n_tok][n_out[m]].
struct MmMats {
    const uint8_t* W[3];
    float* out[3];
    uint32_t n_out[3];
    uint32_t tile_end[2];
};

// PAIR: the gate/up projections of the feed-forward block in one launch: a row tile is 128 rows
// of matrix 0 (gate, waves 0-3) and the same 128 rows of matrix 1 (up, waves 4-7), and the
// output is silu(gate) * up (unsplit, no accumulate).
template <int T, bool LW, bool PAIR = false, int TT = 1>
__global__ __launch_bounds__(512) void linear_matmul_kernel(
    const MmMats mats, const float* __restrict__ x,
    uint32_t n_in, uint32_t n_tok, uint32_t row_bytes, uint32_t accumulate,
    uint32_t tiles_n, uint32_t tiles_m, uint32_t splits, uint32_t k_per_split, uint32_t per_xcd,
    float* __restrict__ part, unsigned int* __restrict__ counters) {
    // Register rings: W raw bytes DW steps ahead, x DX steps ahead of its LDS double buffer.
    // A wait for the x of step t+1 (issued at step t+1-DX, before that step's W load) leaves
    // every later load in flight, so both streams keep DX-1 or more steps of slack.
    constexpr int DW = 8, DX = 8;
    // Ring slots are indexed by the unrolled position d, equal to t mod DX and t mod 2 only
    // when DW is a multiple of both.
    static_assert(DW % DX == 0 && DW % 2 == 0, "ring depths");
    const uint32_t tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const uint32_t n = lane % 32, h = lane / 32;

    // Workgroup b runs on XCD b % 8; give each XCD a contiguous run of (row tile, token tile,
    // split) ids, split fastest, so the splits of a tile and the token tiles that share weight
    // rows share one L2.
    const uint32_t L = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    const uint32_t total = tiles_n * tiles_m * splits;
    if (L >= total) return;
    const uint32_t split = L % splits, tt = (L / splits) % tiles_m, rt = L / splits / tiles_m;
    // This row tile's matrix (selected without indexing the argument arrays, which would put
    // them in scratch) and its tile index within that matrix; with PAIR the wave's matrix.
    constexpr uint32_t RT = PAIR ? kMmRows / 2 : kMmRows;  // rows of one matrix per tile
    const uint32_t mat = PAIR ? wave / 4 : rt < mats.tile_end[0] ? 0u : rt < mats.tile_end[1] ? 1u : 2u;
    const uint8_t* __restrict__ const W = mat == 0 ? mats.W[0] : mat == 1 ? mats.W[1] : mats.W[2];
    float* __restrict__ const out = PAIR || mat == 0 ? mats.out[0] : mat == 1 ? mats.out[1] : mats.out[2];
    const uint32_t n_out = PAIR || mat == 0 ? mats.n_out[0] : mat == 1 ? mats.n_out[1] : mats.n_out[2];
    const uint32_t rtl = PAIR ? rt : rt - (mat == 0 ? 0u : mat == 1 ? mats.tile_end[0] : mats.tile_end[1]);
    const uint32_t kbeg = split * k_per_split;
    const uint32_t steps = (min(n_in, kbeg + k_per_split) - kbeg) / kMmK;
    // TT token halves of 64 per tile: with TT = 2 a wave covers 64 tokens x 64 rows (NB = 2
    // row blocks of 32) instead of 64 x 32, so each A operand read from LDS feeds two MFMAs.
    static_assert(TT == 1 || (TT == 2 && LW), "two token halves on the LDS-staged path only");
    constexpr uint32_t NB = TT, TM = kMmToks * TT;
    const uint32_t th = TT == 1 ? 0u : PAIR ? (wave >> 1) & 1 : wave & 1;   // token half
    const uint32_t rg = TT == 1 ? (PAIR ? wave % 4 : wave) : PAIR ? wave & 1 : wave >> 1;  // row group
    const uint32_t tok0 = tt * TM;
    const uint32_t wtok0 = tok0 + 64 * th;  // the wave's first token
    const uint32_t rowbase = rtl * RT + rg * kMmRowsWave * NB;
    const uint32_t lrow0 = (PAIR ? mat * RT : 0) + rg * kMmRowsWave * NB;  // its first row in a stage
    const bool writer = !PAIR || wave < 4;  // the waves that write the output

    // x staging: thread t converts 4 consecutive k of token t/8. Loads are unconditional (rows
    // past n_tok read the last token, steps past the split re-read its last step; neither
    // reaches an output) so the rings stay in registers with exact wait counts.
    const uint32_t st_tok = tid / 8, st_k = 4 * (tid % 8);
    // A buffer load (wave-uniform descriptor over the workgroup's token rows, per-lane offset)
    // keeps the compiler from moving these prefetches next to their use.
    const uint32_t x_rows = min(n_tok - tok0, TM);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + size_t(tok0) * n_in), 0, int(4 * x_rows * n_in), kBufferFlags);
    float16v_ acc[2 * NB];  // [token block i][row block j] at i * NB + j
    for (int i = 0; i < 2 * int(NB); i++)
        for (int e = 0; e < 16; e++) acc[i][e] = 0.f;
    // LDS for the output transpose (kOutStage floats per wave): the W buffers once the loop
    // is done (LW), else an array of its own.
    __shared__ __attribute__((aligned(16))) float ost_direct[LW ? 4 : kMmWaves * kOutStage];
    float* ost = ost_direct;

    if constexpr (LW) {
        // W and x through LDS, one stage (`ks` elements of k) at a time, one barrier per stage:
        // thread t loads 16-byte chunks t, t+512, ... of the W stage (row-major, so 8-10
        // consecutive lanes cover one row's piece: whole cache lines), two stages ahead in
        // registers, and x's float4s k = 32i + 4(t%8) of token t/8, one stage ahead; both are
        // written to the idle LDS buffers at the end of a stage (x as f16). Each wave then
        // builds its B operands from its 32 rows in LDS and reads its A operands from the x
        // stage: P steps of 4 MFMAs between barriers.
        constexpr uint32_t KS = Stage<T>::ks, P = KS / kMmK, SB = Stage<T>::bytes;
        constexpr uint32_t PITCH = Stage<T>::pitch, CH = SB / 16;
        constexpr uint32_t NM = PAIR ? 2 : 1;                // matrices staged per tile
        constexpr uint32_t NCH = (RT * CH + 511) / 512;      // chunks per thread per matrix
        // x stages of XK elements (NXS per W stage), as large as the LDS left by the W double
        // buffer allows
        constexpr uint32_t XK = T == kQ8_0 || (TT == 2 && (T == kQ4_0 || T == kQ6_K)) ? 64 : (KS < 128 ? KS : 128);
        constexpr uint32_t NXS = KS / XK, PX = XK / kMmK;  // x stages per W stage, steps per x stage
        constexpr uint32_t XP = XK;        // halves per token row of an x stage (chunks swizzled)
        constexpr uint32_t XF4 = XK / 32;  // float4 x loads per thread per x stage
        static_assert(KS % XK == 0 && XK % kMmK == 0 && kMmToks * XK == 512 * 4 * XF4, "stage shape");
        static_assert(2 * kMmRows * PITCH + 2 * TM * XP * 2 <= 160 * 1024, "LDS");
        __shared__ __attribute__((aligned(16))) _Float16 xst[2][TM * XP];
        extern __shared__ __attribute__((aligned(16))) uint8_t wsm[];  // [2][kMmRows][PITCH]
        static_assert(kMmWaves * kOutStage * 4 <= 2 * kMmRows * PITCH, "output staging fits");
        ost = reinterpret_cast<float*>(wsm);
        const uint32_t nst = steps / P;
        // One descriptor per staged matrix (a load instruction never mixes them: a per-lane
        // choice would make the compiler loop over the wave's distinct descriptors).
        const uint32_t rows_here = min(n_out - rtl * RT, RT);
        // WIN: each descriptor starts at the 16-byte boundary at or below its tile's first row,
        // a0[m] bytes before it, and ends at the 16-byte boundary at or above its last byte: a
        // 16-byte load that crosses the end of the range returns zeros as a whole, and the
        // chunk that holds the tile's last byte lies in that byte's page.
        constexpr bool WIN = Stage<T>::win;
        __amdgpu_buffer_rsrc_t wrs[NM];
        uint32_t a0[NM];
        for (uint32_t m = 0; m < NM; m++) {
            const uint8_t* wb = (PAIR ? (m == 0 ? mats.W[0] : mats.W[1]) : W) + size_t(rtl) * RT * row_bytes;
            a0[m] = WIN ? uint32_t(reinterpret_cast<uintptr_t>(wb)) & 15u : 0u;
            const uint32_t span = rows_here * row_bytes + a0[m];
            wrs[m] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wb - a0[m]), 0,
                                                       int(WIN ? (span + 15) & ~15u : span), kBufferFlags);
        }
        const uint32_t kbyte0 = kbeg / Fmt<T>::blk * Fmt<T>::bytes;
        // goff: the chunk's byte offset in the tile (WIN: of its row's stage 0, the chunk's own
        // 16 * o in o16; the window start is aligned per stage)
        uint32_t goff[NCH], loff[NCH], o16[NCH];
        for (uint32_t i = 0; i < NCH; i++) {
            const uint32_t c = min(tid + 512 * i, RT * CH - 1);
            const uint32_t r = c / CH, o = c % CH;
            goff[i] = min(r, rows_here - 1) * row_bytes + kbyte0 + (WIN ? 0u : 16 * o);
            o16[i] = 16 * o;
            loff[i] = r * PITCH + 16 * (Stage<T>::swz ? o ^ swz128(r) : o);  // matrix m's rows follow at m * RT * PITCH
        }
        // WIN: the shift of the wave's rows (row block jb, lane row n) within their windows at
        // stage 0; a block is 210 = 13 * 16 + 2 bytes, so stage j adds 2j (mod 16).
        uint32_t wsh0[NB];
        for (uint32_t jb = 0; jb < NB; jb++) {
            const uint32_t tr = min(lrow0 - (PAIR ? mat * RT : 0u) + 32 * jb + n, rows_here - 1);
            wsh0[jb] = WIN ? (a0[PAIR ? mat : 0] + tr * row_bytes + kbyte0) & 15u : 0u;
        }
        u32x4 wr[2][NM][NCH];
        // The tile's 128-token group g walks its stages starting at stage g * nst / groups and
        // wrapping, so the tiles that share these rows read different W lines at any one time
        // (all starting at stage 0, they queued on the same L2 lines: wo F16 27.9 -> 26.9 us,
        // Q8_0 37.1 -> 34.6 us). The order depends on the 128-token group, not on the tile
        // height, so both tile heights sum every output in the same order.
        const uint32_t groups = (n_tok + 127) / 128;
        const uint32_t rot = uint32_t(__builtin_amdgcn_readfirstlane(int(tok0 / 128 * nst / groups % nst)));
        auto phys = [&](uint32_t j) { j = min(j, nst - 1) + rot; return j >= nst ? j - nst : j; };
        auto load_w = [&](int slot, uint32_t j) {
            const uint32_t sb = phys(j) * (WIN ? Fmt<T>::bytes : SB);
            for (uint32_t m = 0; m < NM; m++)
                for (uint32_t i = 0; i < NCH; i++) {
                    const uint32_t off = WIN ? ((a0[m] + goff[i] + sb) & ~15u) + o16[i] : goff[i] + sb;
                    wr[slot][m][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                   wrs[m], int(off), 0, 0));
                }
        };
        auto store_w = [&](int slot) {
            uint8_t* base = wsm + slot * (kMmRows * PITCH);
            for (uint32_t m = 0; m < NM; m++)
                for (uint32_t i = 0; i < NCH; i++)
                    if (tid + 512 * i < RT * CH) {
                        uint8_t* dst = base + m * RT * PITCH + loff[i];
                        if constexpr (WIN) {
                            const u32x4 v = wr[slot][m][i];
                            *reinterpret_cast<u32x2*>(dst) = u32x2{v[0], v[1]};
                            *reinterpret_cast<u32x2*>(dst + 8) = u32x2{v[2], v[3]};
                        } else {
                            *reinterpret_cast<u32x4*>(dst) = wr[slot][m][i];
                        }
                    }
        };
        const uint32_t xk = 4 * (tid % 8);
        uint32_t xso[TT];
        for (uint32_t q = 0; q < TT; q++) xso[q] = 4 * (min(st_tok + 64 * q, x_rows - 1) * n_in + kbeg + xk);
        float4v xq[TT][XF4];
        const uint32_t nxs = nst * NXS;  // x stages
        auto load_xs = [&](uint32_t j) {  // x stage j of the walk (NXS per W stage)
            j = min(j, nxs - 1);
            const uint32_t kb = (phys(j / NXS) * NXS + j % NXS) * XK;
#pragma unroll
            for (uint32_t q = 0; q < TT; q++)
#pragma unroll
                for (uint32_t i = 0; i < XF4; i++)
                    xq[q][i] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                               xrs, int(xso[q] + 4 * (kb + 32 * i)), 0, 0));
        };
        auto store_xs = [&](int buf) {
            typedef _Float16 half4_ __attribute__((ext_vector_type(4)));
#pragma unroll
            for (uint32_t q = 0; q < TT; q++)
#pragma unroll
            for (uint32_t i = 0; i < XF4; i++) {
                const float4v v = xq[q][i];
                const half4_ hv = kFragSwap13<T>
                    ? half4_{_Float16(v[0]), _Float16(v[2]), _Float16(v[1]), _Float16(v[3])}
                    : half4_{_Float16(v[0]), _Float16(v[1]), _Float16(v[2]), _Float16(v[3])};
                const uint32_t xr = st_tok + 64 * q;
                const uint32_t ch = (4 * i + (tid % 8) / 2) ^ swz_x<XK>(xr);
                *reinterpret_cast<half4_*>(&xst[buf][xr * XP + 8 * ch + 4 * (tid & 1)]) = hv;
            }
        };

        load_xs(0);
        load_w(0, 0);
        load_w(1, 1);
        store_xs(0);
        store_w(0);
        load_xs(1);
        __syncthreads();

        for (uint32_t j0 = 0; j0 < nst; j0 += 2) {
#pragma unroll
            for (uint32_t jj = 0; jj < 2; jj++) {
                const uint32_t j = j0 + jj;
                if (j >= nst) break;
                const uint8_t* wrow = wsm + jj * (kMmRows * PITCH) + (lrow0 + n) * PITCH;
                const uint32_t wsh_j = WIN ? 2 * phys(j) : 0u;  // (before load_w's phys(j + 2))
                load_w(jj, j + 2);  // this slot's stage j is already in LDS
                // Issue the prefetch here: left to the scheduler, these loads sink below the
                // stage's MFMAs and the next stage waits for them.
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (uint32_t xs_i = 0; xs_i < NXS; xs_i++) {
                    const uint32_t xb = (jj * NXS + xs_i) & 1;  // x buffer of x stage j*NXS + xs_i
                    const _Float16* xsb = &xst[xb][0];
#pragma unroll
                    for (uint32_t v = 0; v < PX; v++) {
                        const uint32_t u = xs_i * PX + v;  // step within the W stage
                        const uint32_t t = j * P + u;
                        half8 b[NB][2];
#pragma unroll
                        for (uint32_t jb = 0; jb < NB; jb++) {
                            const uint8_t* wr_j = wrow + 32 * jb * PITCH + (WIN ? (wsh0[jb] + wsh_j) & 15u : 0u);
                            Raw<T> r;
                            if constexpr (Stage<T>::swz) {
                                const uint32_t sw = swz128(lrow0 + 32 * jb + n);
                                if constexpr (T == kF32) {
                                    for (int s = 0; s < 2; s++)
                                        for (int e = 0; e < 2; e++)
                                            r.v[s][e] = *reinterpret_cast<const float4v*>(wr_j + 16 * ((8 * u + 4 * s + 2 * h + e) ^ sw));
                                } else {
                                    for (int s = 0; s < 2; s++)
                                        r.v[s] = *reinterpret_cast<const std::remove_reference_t<decltype(r.v[0])>*>(wr_j + 16 * ((4 * u + 2 * s + h) ^ sw));
                                }
                            } else {
                                load_raw_lds<T>(r, wr_j, u * kMmK, h);
                            }
                            for (int s = 0; s < 2; s++) b[jb][s] = frag<T>(r, s, kbeg + t * kMmK);
                        }
#pragma unroll
                        for (int s = 0; s < 2; s++) {
                            for (int i = 0; i < 2; i++) {
                                const uint32_t xr = 64 * th + 32 * i + n;
                                const half8 a = *reinterpret_cast<const half8*>(&xsb[xr * XP + 8 * ((4 * v + 2 * s + h) ^ swz_x<XK>(xr))]);
#pragma unroll
                                for (uint32_t jb = 0; jb < NB; jb++)
                                    acc[i * NB + jb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b[jb][s], acc[i * NB + jb], 0, 0, 0);
                            }
                        }
                    }
                    // The stage's MFMAs before its LDS writes (hoisted above them, the writes would
                    // wait for x loads issued just before the previous barrier).
                    __builtin_amdgcn_sched_barrier(0);
                    store_xs(xb ^ 1);  // x of the next x stage
                    if (xs_i == NXS - 1) store_w(jj ^ 1);  // W of stage j+1
                    load_xs(j * NXS + xs_i + 2);
                    __syncthreads();
                }
            }
        }
    } else {
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][kMmToks * kXPitch];
    const uint32_t xoff = 4 * (min(st_tok, x_rows - 1) * n_in + kbeg + st_k);
    float4v xr[DX];
    auto load_x = [&](int slot, uint32_t t) {
        xr[slot] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                   xrs, int(xoff + 4 * min(t, steps - 1) * kMmK), 0, 0));
    };
    // (for the block types whose fragments come out in the k order 0,2,1,3 within each group of
    // four, x is staged in the same order: the MFMA pairs A and B elements by position)
    auto store_x = [&](int slot, int buf) {
        typedef _Float16 half4_ __attribute__((ext_vector_type(4)));
        const half4_ v = kFragSwap13<T>
            ? half4_{_Float16(xr[slot][0]), _Float16(xr[slot][2]), _Float16(xr[slot][1]), _Float16(xr[slot][3])}
            : half4_{_Float16(xr[slot][0]), _Float16(xr[slot][1]), _Float16(xr[slot][2]), _Float16(xr[slot][3])};
        *reinterpret_cast<half4_*>(&xs[buf][st_tok * kXPitch + st_k]) = v;
    };

    const uint8_t* row = W + size_t(min(rowbase + n, n_out - 1)) * row_bytes;
    const uint32_t k_last = kbeg + (steps - 1) * kMmK;

#pragma unroll
    for (int d = 0; d < DX; d++) load_x(d, d);
    Raw<T> raw[DW];
#pragma unroll
    for (int d = 0; d < DW; d++) load_raw<T>(raw[d], row, min(kbeg + d * kMmK, k_last), h);
    store_x(0, 0);
    __syncthreads();

    for (uint32_t t0 = 0; t0 < steps; t0 += DW) {
#pragma unroll
        for (int d = 0; d < DW; d++) {
            const uint32_t t = t0 + d;
            if (t >= steps) break;
            const uint32_t k0 = kbeg + t * kMmK;
            const int buf = d & 1;  // == t & 1 (DW is even)
            load_x(d % DX, t + DX);  // the slot of step t, whose x is already in LDS
            half8 b[2];
            for (int s = 0; s < 2; s++) b[s] = frag<T>(raw[d], s, k0);
            load_raw<T>(raw[d], row, min(k0 + DW * kMmK, k_last), h);
#pragma unroll
            for (int s = 0; s < 2; s++) {
                for (int i = 0; i < 2; i++) {
                    const half8 a = *reinterpret_cast<const half8*>(&xs[buf][(32 * i + n) * kXPitch + 16 * s + 8 * h]);
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b[s], acc[i], 0, 0, 0);
                }
            }
            store_x((d + 1) % DX, buf ^ 1);  // x of step t+1
            __syncthreads();
        }
    }
    }

    // D[m][n] of a 32x32 tile: lane holds column n = lane%32, rows 8(e/4) + 4h + e%4.
    if (TT == 1 && splits > 1) {  // (two token halves are launched unsplit)
        // Publish this split's partial tile (16-byte device-scope stores), count the arrival;
        // the last split of the tile sums the partials in split order and writes the output.
        const uint32_t tile = rt * tiles_m + tt;
        const uint32_t tile_bytes = kTileFloats * 4;
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
            part, 0, int(tiles_n * tiles_m * splits * tile_bytes), kBufferFlags);
        auto off = [&](uint32_t sp, int i, int q) {
            return int((tile * splits + sp) * tile_bytes + ((((wave * 2 + i) * 4 + q) * 64 + lane) * 16));
        };
        for (int i = 0; i < 2; i++)
            for (int q = 0; q < 4; q++) {
                const float4v v = {acc[i][4 * q], acc[i][4 * q + 1], acc[i][4 * q + 2], acc[i][4 * q + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs, off(split, i, q), 0, kScDevice);
            }
        // The partial's device-scope (write-through) stores are acknowledged by memory before the
        // arrival is counted, and the last split reads the partials with device-scope loads, which
        // do not take a clean L2 line: the hand-off needs no release/acquire pair, whose L2
        // writeback and invalidate around the atomic would cost more than the whole tail.
        // Compiler-only fences on both sides of the wait keep the optimizer from moving the
        // stores past it or the counter increment before it; the hardware order comes from the
        // wait and the barrier.
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);  // the partial has reached device scope
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        __shared__ unsigned int last;
        if (tid == 0) {
            const unsigned prev = __hip_atomic_fetch_add(counters + tile * 16, 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            last = prev == splits - 1;
        }
        __syncthreads();
        if (!last) return;
        // Sum the partials in split order (this split's own from registers, the others'
        // loaded); all loads of a partial are issued together and the next partial's loads are
        // in flight while the current one is added.
        float16v_ own[2] = {acc[0], acc[1]};
        for (int i = 0; i < 2; i++)
            for (int e = 0; e < 16; e++) acc[i][e] = 0.f;
        float4v pv[2][8];
        auto load_part = [&](int slot, uint32_t sp) {
            if (sp == split) return;
            for (int i = 0; i < 2; i++)
                for (int q = 0; q < 4; q++)
                    pv[slot][i * 4 + q] = __builtin_bit_cast(
                        float4v, __builtin_amdgcn_raw_buffer_load_b128(prs, off(sp, i, q), 0, kScDevice));
        };
        auto add_part = [&](int slot, uint32_t sp) {
            for (int i = 0; i < 2; i++)
                for (int q = 0; q < 4; q++)
                    for (int e = 0; e < 4; e++)
                        acc[i][4 * q + e] += sp == split ? own[i][4 * q + e] : pv[slot][i * 4 + q][e];
        };
        load_part(0, 0);
        for (uint32_t sp = 0; sp < splits; sp += 2) {
            if (sp + 1 < splits) load_part(1, sp + 1);
            add_part(0, sp);
            if (sp + 1 >= splits) break;
            if (sp + 2 < splits) load_part(0, sp + 2);
            add_part(1, sp + 1);
        }
        if (tid == 0)  // leave the workspace ready for the next call
            __hip_atomic_store(counters + tile * 16, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if constexpr (PAIR) {
        // The up waves hand their tiles to the gate waves of the same rows through LDS (16
        // floats per lane per pass, lane-minor), which form silu(gate) * up as silu_mul_kernel.
        for (int i = 0; i < 2 * int(NB); i++) {
            __syncthreads();  // the LDS is free (loop reads, or the previous pass)
            float* xb = ost + (wave % 4) * (16 * 64) + lane;
            if (!writer)
                for (int e = 0; e < 16; e++) xb[e * 64] = acc[i][e];
            __syncthreads();
            if (writer)
                for (int e = 0; e < 16; e++) {
                    const float g = acc[i][e];
                    acc[i][e] = g / (1.0f + expf(-g)) * xb[e * 64];
                }
        }
    }
    // Output: out[tok][row] = prev + acc for the wave's 64 tokens x 32 rows. With 16-byte
    // aligned rows the tile is transposed through LDS, 32 tokens at a time, so that each lane
    // loads and stores 16 contiguous bytes (8 lanes per token row: 8 instructions each way
    // instead of 32 scattered 4-byte ones); all previous values are read before any store.
    const bool vec = ((reinterpret_cast<uintptr_t>(out) | (size_t(n_out) * 4)) & 15) == 0;
    if (vec) {
        const uint32_t tr = lane / 8, c4 = 4 * (lane % 8);  // token row within 8, first row
        float* st = ost + wave * kOutStage;
        for (uint32_t jb = 0; jb < NB; jb++) {
            const uint32_t row0 = rowbase + 32 * jb + c4;
            float4v prev[2][4];
            for (int i = 0; i < 2; i++)
                for (int k = 0; k < 4; k++) {
                    const uint32_t tok = wtok0 + 32 * i + 8 * k + tr;
                    prev[i][k] = accumulate && tok < n_tok && row0 < n_out
                        ? *reinterpret_cast<const float4v*>(out + size_t(tok) * n_out + row0)
                        : float4v{0.f, 0.f, 0.f, 0.f};
                }
            for (int i = 0; i < 2; i++) {
                __syncthreads();  // the staging area is free (loop reads, or the previous pass)
                for (int e = 0; e < 16; e++)
                    st[(8 * (e / 4) + 4 * h + e % 4) * kOutPitch + n] = acc[i * NB + jb][e];
                __syncthreads();
                for (int k = 0; k < 4; k++) {
                    const uint32_t tok = wtok0 + 32 * i + 8 * k + tr;
                    const float4v v = *reinterpret_cast<const float4v*>(st + (8 * k + tr) * kOutPitch + c4);
                    if (writer && tok < n_tok && row0 < n_out)
                        *reinterpret_cast<float4v*>(out + size_t(tok) * n_out + row0) = prev[i][k] + v;
                }
            }
        }
        return;
    }
    for (uint32_t jb = 0; jb < NB; jb++) {
        const uint32_t orow = rowbase + 32 * jb + n;
        if (writer && orow < n_out) {
            float prev[2][16];
            for (int i = 0; i < 2; i++)
                for (int e = 0; e < 16; e++) {
                    const uint32_t tok = wtok0 + 32 * i + 8 * (e / 4) + 4 * h + e % 4;
                    prev[i][e] = accumulate && tok < n_tok ? out[size_t(tok) * n_out + orow] : 0.f;
                }
            for (int i = 0; i < 2; i++)
                for (int e = 0; e < 16; e++) {
                    const uint32_t tok = wtok0 + 32 * i + 8 * (e / 4) + 4 * h + e % 4;
                    if (tok < n_tok) out[size_t(tok) * n_out + orow] = prev[i][e] + acc[i * NB + jb][e];
                }
        }
    }
}

// The batched kernel over mats (n_mats matrices; W, out and n_out set) with `splits`-way
// split-K (partials and counters in the workspace when splits > 1).
// pair: mats holds (gate, up) with equal n_out and out[0] receives silu(gate) * up (no split,
// no accumulate).
template <int T>
int launch_mm_t(MmMats mats, uint32_t n_mats, const float* x, uint32_t n_in, uint32_t n_tok,
                uint32_t accumulate, uint32_t splits, void* workspace, hipStream_t stream,
                bool pair = false) {
    const uint32_t row_bytes = n_in / Fmt<T>::blk * Fmt<T>::bytes;
    uint32_t tiles_n = 0;
    if (pair) {
        if (n_mats != 2 || mats.n_out[0] != mats.n_out[1] || accumulate || splits != 1) return -1;
        tiles_n = (mats.n_out[0] + kMmRows / 2 - 1) / (kMmRows / 2);
    } else {
        for (uint32_t m = 0; m < 3; m++) {
            if (m < n_mats) tiles_n += (mats.n_out[m] + kMmRows - 1) / kMmRows;
            if (m < 2) mats.tile_end[m] = tiles_n;
        }
    }
    // LDS-staged W when rows split into whole 16-byte stage pieces.
    constexpr uint32_t KS = Stage<T>::ks;
    const bool lw = KS != 0 && (Stage<T>::win || row_bytes % 16 == 0) && n_in % (KS != 0 ? KS : 1) == 0;
    // Tiles of 128 tokens (two halves; waves of 64 x 64: each A operand read from LDS feeds two
    // MFMAs and each W stage serves twice the tokens) for unsplit calls when they take fewer
    // rounds of 256 workgroups: a 128-token tile costs ~1.8x a 64-token one (Q4_0 gate/up at
    // 512 tokens: 256 tiles in 80.0 us against 512 in 89.3; q/k/v at 2048 tokens, 320 tiles in
    // 2 rounds against 640 in 3: 137.9 against 125.3 us). Q8_0's stages leave no LDS for the
    // larger x stage.
    const uint64_t rounds1 = (uint64_t(tiles_n) * ((n_tok + 63) / 64) + 255) / 256;
    const uint64_t rounds2 = (uint64_t(tiles_n) * ((n_tok + 127) / 128) + 255) / 256;
    const bool tt2 = T != kQ8_0 && lw && splits == 1 && 9 * rounds2 < 5 * rounds1;
    const uint32_t tiles_m = (n_tok + kMmToks * (tt2 ? 2 : 1) - 1) / (kMmToks * (tt2 ? 2 : 1));
    const uint32_t gran = lw ? KS : kMmK;
    const uint32_t units = n_in / gran;
    const uint32_t k_per_split = (units + splits - 1) / splits * gran;
    splits = (n_in + k_per_split - 1) / k_per_split;  // never more than requested
    const uint64_t total = uint64_t(tiles_n) * tiles_m * splits;
    const uint64_t per_xcd = (total + 7) / 8;
    if (per_xcd * 8 > 0x7fffffffu) return -1;
    auto* counters = static_cast<unsigned int*>(workspace);
    auto* part = splits > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kLinearCounterBytes)
                            : nullptr;
    const dim3 grid(uint32_t(per_xcd * 8)), block(kMmWaves * 64);
    auto go = [&](auto lw_c, auto pair_c, auto tt_c) {
        constexpr bool LWc = decltype(lw_c)::value, PAIRc = decltype(pair_c)::value;
        constexpr int TTc = decltype(tt_c)::value;
        const size_t lds = LWc ? size_t(2) * kMmRows * Stage<T>::pitch : 0;
        if (LWc) {
            static const hipError_t attr = hipFuncSetAttribute(
                reinterpret_cast<const void*>(&linear_matmul_kernel<T, LWc, PAIRc, TTc>),
                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
            if (attr != hipSuccess) return -4;
        }
        hipLaunchKernelGGL((linear_matmul_kernel<T, LWc, PAIRc, TTc>), grid, block, lds, stream, mats, x,
                           n_in, n_tok, row_bytes, accumulate, tiles_n, tiles_m, splits,
                           k_per_split, uint32_t(per_xcd), part, counters);
        return hipGetLastError() == hipSuccess ? 0 : -4;
    };
    using yes = std::true_type;
    using no = std::false_type;
    using one = std::integral_constant<int, 1>;
    using two = std::integral_constant<int, 2>;
    if constexpr (Stage<T>::ks != 0) {
        if constexpr (T != kQ8_0)
            if (lw && tt2) return pair ? go(yes{}, yes{}, two{}) : go(yes{}, no{}, two{});
        if (lw) return pair ? go(yes{}, yes{}, one{}) : go(yes{}, no{}, one{});
    }
    return pair ? go(no{}, yes{}, one{}) : go(no{}, no{}, one{});
}

template <int T>
int launch_t(const uint8_t* W, const float* x, float* out, uint32_t n_in, uint32_t n_out,
             uint32_t n_tok, uint32_t accumulate, uint32_t n_splits, void* workspace,
             size_t workspace_bytes, hipStream_t stream) {
    if (n_tok == 1) {
        MvArgs a{};
        a.W[0] = W;
        a.out[0] = out;
        a.n_out[0] = n_out;
        a.x = x;
        a.n_in = n_in;
        return launch_matvec_t<T>(a, 1, kProNone, accumulate ? kEpiAccumulate : kEpiStore, stream);
    }
    MmMats mats{};
    mats.W[0] = W;
    mats.out[0] = out;
    mats.n_out[0] = n_out;
    const uint32_t splits = workspace ? linear_splits(n_in, n_out, n_tok, n_splits, workspace_bytes) : 1;
    return launch_mm_t<T>(mats, 1, x, n_in, n_tok, accumulate, splits, workspace, stream);
}

}  // namespace

uint32_t linear_splits(uint32_t n_in, uint32_t n_out, uint32_t n_tok, uint32_t requested,
                       size_t workspace_bytes) {
    if (n_tok <= 1 || requested == 1) return 1;
    const uint32_t tiles = ((n_out + kMmRows - 1) / kMmRows) * ((n_tok + kMmToks - 1) / kMmToks);
    if (tiles > kLinearMaxTiles) return 1;
    const uint32_t steps = n_in / kMmK;
    // At least 8 k steps (256 elements) per split, at most kMaxSplits.
    uint32_t cap = steps / 8;
    if (cap > kMaxSplits) cap = kMaxSplits;
    uint32_t s = 1;
    if (requested > 1) {
        s = requested < cap ? requested : cap;
    } else {
        // One workgroup per CU saturates a CU (a second co-resident one adds no throughput),
        // and every split adds a partial tile to write and sum: take the largest split that
        // still fits the tiles x splits workgroups on the 256 CUs in one round.
        s = 256 / tiles;
        if (s > cap) s = cap;
    }
    if (s < 2) return 1;
    // No split may be empty.
    const uint32_t per = (steps + s - 1) / s;
    while (s > 1 && (s - 1) * per >= steps) s--;
    if (kLinearCounterBytes + size_t(tiles) * s * kTileFloats * 4 > workspace_bytes) return 1;
    return s;
}

size_t linear_workspace_size(uint32_t n_in, uint32_t n_out, uint32_t n_tok, uint32_t requested) {
    const uint32_t s = linear_splits(n_in, n_out, n_tok, requested, ~size_t(0));
    const uint32_t tiles = ((n_out + kMmRows - 1) / kMmRows) * ((n_tok + kMmToks - 1) / kMmToks);
    return kLinearCounterBytes + (s > 1 ? size_t(tiles) * s * kTileFloats * 4 : 0);
}

int launch_proj(uint32_t type, const void* const* W, const float* x, const float* aux,
                float* const* out, uint32_t n_in, const uint32_t* n_out, uint32_t n_mats,
                int pro, int epi, float eps, hipStream_t stream, const ProjRope* rope, uint32_t n_tok) {
    if (n_tok > 1) {  // a chunk: the batched kernel over every matrix's rows, no split-K
        // Epilogues: store, accumulate, or silu(gate) * up over two matrices (one launch with
        // gate and up rows paired in each tile).
        const bool pair = epi == kEpiSiluGate;
        if (pro != kProNone || rope) return -2;
        if (epi != kEpiStore && epi != kEpiAccumulate && !pair) return -2;
        if (pair && (n_mats != 2 || n_out[0] != n_out[1])) return -1;
        MmMats mats{};
        for (uint32_t m = 0; m < n_mats; m++) {
            mats.W[m] = static_cast<const uint8_t*>(W[m]);
            mats.out[m] = pair ? out[0] : out[m];
            mats.n_out[m] = n_out[m];
        }
        const uint32_t acc = epi == kEpiAccumulate ? 1u : 0u;
        switch (type) {
            case kF32:  return launch_mm_t<kF32>(mats, n_mats, x, n_in, n_tok, acc, 1, nullptr, stream, pair);
            case kF16:  return launch_mm_t<kF16>(mats, n_mats, x, n_in, n_tok, acc, 1, nullptr, stream, pair);
            case kBF16: return launch_mm_t<kBF16>(mats, n_mats, x, n_in, n_tok, acc, 1, nullptr, stream, pair);
            case kQ8_0: return launch_mm_t<kQ8_0>(mats, n_mats, x, n_in, n_tok, acc, 1, nullptr, stream, pair);
            case kQ4_0: return launch_mm_t<kQ4_0>(mats, n_mats, x, n_in, n_tok, acc, 1, nullptr, stream, pair);
            case kQ4_1: return launch_mm_t<kQ4_1>(mats, n_mats, x, n_in, n_tok, acc, 1, nullptr, stream, pair);
            case kQ6_K: return launch_mm_t<kQ6_K>(mats, n_mats, x, n_in, n_tok, acc, 1, nullptr, stream, pair);
            default:    return -2;
        }
    }
    MvArgs a{};
    if (epi == kEpiRopeKv) {
        if (!rope || n_mats != 3) return -2;
        if (!(type == kQ4_0 || type == kQ4_1 || type == kQ8_0 || type == kF16 || type == kBF16 || type == kQ6_K)) return -2;
        a.inv_freq = rope->inv_freq;
        a.cache[0] = rope->k_row;
        a.cache[1] = rope->v_row;
        a.head_dim = rope->head_dim;
        a.pos = rope->pos;
    }
    for (uint32_t m = 0; m < n_mats; m++) {
        a.W[m] = static_cast<const uint8_t*>(W[m]);
        a.n_out[m] = n_out[m];
        a.out[m] = epi == kEpiSiluGate || epi == kEpiRopeKv ? out[0] : out[m];
    }
    a.x = x;
    a.aux = aux;
    a.n_in = n_in;
    a.eps = eps;
    switch (type) {
        case kF32:  return launch_matvec_t<kF32>(a, n_mats, pro, epi, stream);
        case kF16:  return launch_matvec_t<kF16>(a, n_mats, pro, epi, stream);
        case kBF16: return launch_matvec_t<kBF16>(a, n_mats, pro, epi, stream);
        case kQ8_0: return launch_matvec_t<kQ8_0>(a, n_mats, pro, epi, stream);
        case kQ4_0: return launch_matvec_t<kQ4_0>(a, n_mats, pro, epi, stream);
        case kQ4_1: return launch_matvec_t<kQ4_1>(a, n_mats, pro, epi, stream);
        case kQ6_K: return launch_matvec_t<kQ6_K>(a, n_mats, pro, epi, stream);
        default:    return -2;
    }
}

int launch_linear(uint32_t type, const void* W, const float* x, float* out, uint32_t n_in,
                  uint32_t n_out, uint32_t n_tok, uint32_t accumulate, uint32_t n_splits,
                  void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const auto* w = static_cast<const uint8_t*>(W);
    switch (type) {
        case kF32:  return launch_t<kF32>(w, x, out, n_in, n_out, n_tok, accumulate, n_splits, workspace, workspace_bytes, stream);
        case kF16:  return launch_t<kF16>(w, x, out, n_in, n_out, n_tok, accumulate, n_splits, workspace, workspace_bytes, stream);
        case kBF16: return launch_t<kBF16>(w, x, out, n_in, n_out, n_tok, accumulate, n_splits, workspace, workspace_bytes, stream);
        case kQ8_0: return launch_t<kQ8_0>(w, x, out, n_in, n_out, n_tok, accumulate, n_splits, workspace, workspace_bytes, stream);
        case kQ4_0: return launch_t<kQ4_0>(w, x, out, n_in, n_out, n_tok, accumulate, n_splits, workspace, workspace_bytes, stream);
        case kQ4_1: return launch_t<kQ4_1>(w, x, out, n_in, n_out, n_tok, accumulate, n_splits, workspace, workspace_bytes, stream);
        case kQ6_K: return launch_t<kQ6_K>(w, x, out, n_in, n_out, n_tok, accumulate, n_splits, workspace, workspace_bytes, stream);
        default: return -2;
    }
}

}  // namespace ingot
