// attn_prefill.hip — causal tiled (flash) prefill attention on f16 MFMA for gfx950.
//
// For a chunk of n_tok queries at absolute positions pos..pos+n_tok-1, query i of head h
// attends to cache rows 0..pos+i of KV head h / G: the semantics of n_tok successive decode
// steps (src/backend.h:16-20, src/cpu_backend.cpp:51-69) and of the reference's attn_prefill
// (shaders/kernels.metal:518-633, mask `key <= pos+tok`, line 578), re-designed for CDNA4:
//
//   - Head size HD = 64, 128 or 256 (a template parameter: row bytes, swizzles, k steps).
//   - A workgroup = 8 waves over one unit (G <= 3 query heads of one KV head; 1 at HD 256) and
//     64 queries: 4 query waves x 2 key groups. A wave owns 16 queries and the unit's G heads
//     (48 score columns for G = 3);
//     the two key groups take alternate key tiles (each with its own double-buffered LDS
//     stages) and are merged through LDS at the end, which gives 2 waves per SIMD without
//     splitting the key range across workgroups. Every K/V operand read from LDS feeds G MFMAs
//     (v_mfma_f32_16x16x32_f16), so the GQA sharing happens at register level, on top of the
//     workgroup-level sharing of each LDS tile.
//   - K/V tiles (64 keys; 32 at HD 256) are copied HBM -> LDS with buffer_load ... lds (no
//     VGPRs, no VALU) into a
//     double buffer: the next tile streams in while the current one is computed. 16-byte
//     chunks are XOR-swizzled per row so that every LDS read below is bank-conflict free.
//   - S^T = K Q^T: the A operand is a 16-byte LDS read of a K row, B is Q^T held in registers
//     (pre-scaled by scale*log2(e) and rounded to f16, as the reference rounds Q*scale to half,
//     shaders/kernels.metal:543). A lane owns one query column, so the online-softmax max/sum
//     are lane-local plus two exchanges.
//   - O^T += V^T P^T: P^T comes straight out of the S^T accumulator (rounded to f16, as at
//     shaders/kernels.metal:588); V^T is read with ds_read_b64_tr_b16 (transposing LDS read),
//     whose 4-consecutive-key runs match the accumulator's key order, so nothing is shuffled.
//   - Causal tile skipping per wave; tiles straddling the diagonal are masked per element.
//   - Split-KV for short chunks (few waves): each split writes (o, m, l) partials and
//     attn_prefill_combine merges them (log-sum-exp rule of attn_combine,
//     shaders/kernels.metal:501-516).
//
// MFMA 16x16x32 f16 register layouts (wave64, lane l, i = l%16, g = l/16):
//   A (16 x 32): lane holds A[i][8g + e];  B (32 x 16): lane holds B[8g + e][i];
//   D (16 x 16): lane holds D[4g + j][i], j = 0..3.
// ds_read_b64_tr_b16 (per 16-lane group; lane r supplies an address, lane i receives 4 halves):
//   out[i][j] = halves[4j + i/4][i%4], where halves[r][0..3] are the 4 halves at lane r's address.
#include <type_traits>

#include "attn_common.h"
#include "attn_internal.h"

namespace ingot {

namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x4 __attribute__((__vector_size__(8)));  // operand type of ds_read_tr16_b64
typedef __attribute__((address_space(3))) fp16x4 lds_fp16x4;
typedef __attribute__((address_space(3))) half8 lds_half8;

// Keys per tile: 64, or 32 for head_dim 256 (four 64 KB stages would not fit the LDS).
template <int HD> constexpr int kBN = HD == 256 ? 32 : 64;
constexpr float kLazy = 8.f;                   // base-2 headroom before the reference max moves
constexpr int kBufferFlags = 0x00020000;       // buffer descriptor word 3 (raw, 32-bit format)
constexpr int kScDevice = 16;                  // buffer cache-policy bits: sc1 = device scope
// LDS geometry for head size HD: a K/V row of HD halves (no padding), 16-byte chunks per row,
// a K or V tile of kBN rows, a stage = K tile + V tile (HD 128: 256 B, 16, 16 KB, 32 KB).
template <int HD> constexpr int kRowBytes = HD * 2;
template <int HD> constexpr int kChunks = HD / 8;
template <int HD> constexpr int kTileBytes = kBN<HD> * kRowBytes<HD>;
template <int HD> constexpr int kStageBytes = 2 * kTileBytes<HD>;

// Max over the 4 lanes l, l^16, l^32, l^48 (the lanes that hold one query column) with the
// gfx950 lane-swap instructions: with both operands equal to x, the two results of
// v_permlane16_swap are {x_l, x_(l^16)} and those of v_permlane32_swap {x_l, x_(l^32)}.
__device__ __forceinline__ float max_lanes4(float x) {
    unsigned u = __float_as_uint(x);
    auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    u = __float_as_uint(x);
    r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// XOR swizzles of the 16-byte chunk index inside a row, chosen so that the 16 lanes of a
// 16-byte K read (16 rows, one logical chunk) and the 32 lanes of a transposing V read (8 rows,
// a 32-byte chunk pair each) cover all 64 banks once. A 256-byte row spans the 64 banks, so
// the chunk (pair) index alone must differ (a 512-byte row: its low bits); a 128-byte row spans
// half of them, so rows of the same parity must differ, hence row >> 1.
template <int HD> __device__ __forceinline__ int swz_k(int row) {
    return HD == 64 ? (row >> 1) & 7 : row & 15;
}
template <int HD> __device__ __forceinline__ int swz_v(int row) {
    return HD == 64 ? ((row >> 1) & 3) << 1 : (row & 7) << 1;
}

template <int HD, int G, int QW, int KG>
__global__ __launch_bounds__(64 * QW * KG) __attribute__((amdgpu_waves_per_eu(2)))
void attn_prefill_kernel(const float* __restrict__ q, const _Float16* __restrict__ K,
                         const _Float16* __restrict__ V, float* __restrict__ out,
                         char* __restrict__ part, uint32_t pos, uint32_t n_tok, uint32_t q_stride,
                         uint32_t n_head_kv, uint32_t kv_div, uint32_t tps, float qscale) {
    constexpr int BN = kBN<HD>, RB = kRowBytes<HD>, CPR = kChunks<HD>, TB = kTileBytes<HD>, SB = kStageBytes<HD>;
    constexpr int HALVES = BN / 32;  // 32-key halves per tile
    constexpr int PB = HD * 2 + 16;  // bytes per split record: o[HD] / l as f16, then {m, l, 0, 0}
    constexpr int NIT = TB / 1024;  // 1 KB copy instructions per K (or V) tile
    constexpr int RPI = 1024 / RB;  // rows per copy instruction
    constexpr int KS = HD / 32;     // 32-wide k steps of a score MFMA chain
    constexpr int ND = HD / 16;     // 16-dim blocks of O
    // LDS: one object per (key group, buffer) stage, so the compiler can tell that the reads of
    // the current stage do not touch the stage being filled by the DMA (with one array it waits
    // for every copy in flight before each transposing read), and the (m, l) fields of the
    // key-group merge.
    __shared__ __attribute__((aligned(16))) char sg00[SB];
    __shared__ __attribute__((aligned(16))) char sg01[SB];
    __shared__ __attribute__((aligned(16))) char sg10[KG > 1 ? SB : 16];
    __shared__ __attribute__((aligned(16))) char sg11[KG > 1 ? SB : 16];
    __shared__ __attribute__((aligned(16))) float4v mlx[KG > 1 ? G : 1][QW][64];
    auto stage_of = [&](uint32_t g_, int b) -> char* {
        return b == 0 ? (g_ != 0 ? sg10 : sg00) : (g_ != 0 ? sg11 : sg01);
    };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int qw = wave % QW, kg = wave / QW;  // query sub-block, key group
    const int li = lane & 15, g = lane >> 4;
    // 1-D grid: workgroup b serves KV head b % n_head_kv, so with 8 KV heads each XCD (b % 8)
    // holds one head's K/V and Q in its L2 for all of that head's query blocks and splits.
    // b / n_head_kv enumerates (query block, key split) pairs, the longest query blocks first:
    // block j sees ntiles_j key tiles and is split into n_splits_j = ceil(ntiles_j / tps)
    // near-equal key ranges, so no workgroup walks more than tps tiles (the causal chunk's last
    // block no longer sets the critical path alone).
    // With kv_div > 1 the G query heads of a unit are a 1/kv_div share of a KV head's group
    // (n_head_kv counts units, kv_div of them per KV head): the group's heads run in separate
    // workgroups, each reading the same K/V.
    const uint32_t kvh = blockIdx.x % n_head_kv;
    const size_t kv_dim = size_t(n_head_kv / kv_div) * HD;
    uint32_t qblk = (n_tok + 16 * QW - 1) / (16 * QW), split = blockIdx.x / n_head_kv, n_splits = 1;
    uint32_t ntiles = 0;
    while (qblk > 0) {
        qblk--;
        ntiles = (pos + min(n_tok, (qblk + 1) * 16 * QW) + BN - 1) / BN;
        n_splits = (ntiles + tps - 1) / tps;
        if (split < n_splits) break;
        split -= n_splits;
    }
    if (split >= n_splits) return;  // past the enumerated pairs (the host never launches these)
    const uint32_t qblk0 = qblk * 16 * QW;
    const uint32_t q0 = qblk0 + 16 * qw;

    // Keys [0, kend) are visible to some query of this workgroup.
    const uint32_t qlast_wg = min(n_tok, qblk0 + 16 * QW) - 1;
    const uint32_t kend = pos + qlast_wg + 1;
    const uint32_t t_begin = uint32_t((uint64_t(split) * ntiles) / n_splits);
    const uint32_t t_end = uint32_t((uint64_t(split + 1) * ntiles) / n_splits);
    // Keys [0, kend_w) are visible to some query of this wave; 0 if the wave has no queries.
    const uint32_t kend_w = q0 < n_tok ? pos + min(n_tok, q0 + 16) : 0;
    const uint32_t qpos = pos + q0 + li;  // this lane's query position

    const _Float16* Kg = K + size_t(kvh / kv_div) * HD;
    const _Float16* Vg = V + size_t(kvh / kv_div) * HD;

    // Tile copy HBM -> LDS: 2*NIT buffer_load ... lds instructions of 1 KB (RPI rows) per tile
    // (HD 128: 32 of 4 rows), spread over the waves of the key group and issued in two groups
    // between the compute phases of the current tile, so that the CU's address unit never
    // receives all of them at once (a burst stalls every wave at the issue). Lane l of
    // instruction i fills physical chunk l%CPR of row RPI*(i%NIT) + l/CPR, so it fetches the
    // logical chunk (l%CPR) ^ swizzle(row). The
    // per-lane byte offsets do not change from tile to tile; the buffer resource is rebased per
    // tile and its size covers only the visible rows, so rows past kend read as zeros (finite;
    // those keys are masked, so their P is exactly 0) with no clamping arithmetic.
    constexpr int kInstPerWave = 2 * NIT / QW;  // each key group copies its own tiles
    const uint32_t row_bytes = uint32_t(kv_dim) * 2;
    uint32_t dma_off[kInstPerWave];
#pragma unroll
    for (int k = 0; k < kInstPerWave; k++) {
        const int i = qw + k * QW;
        const int isv = i / NIT;
        const int row = RPI * (i % NIT) + lane / CPR;
        const int logical = (lane % CPR) ^ (isv ? swz_v<HD>(row) : swz_k<HD>(row));
        dma_off[k] = uint32_t(row) * row_bytes + 16u * uint32_t(logical);
    }
    // Copy instruction k (0 .. kInstPerWave-1) of this wave for tile t into buffer `buf`.
    auto issue_inst = [&](uint32_t t, int buf, int k) {
        const uint32_t kb = t * BN;
        char* stage = stage_of(kg, buf);
        const uint32_t nrec = min(kend - kb, uint32_t(BN)) * row_bytes;
        const int i = qw + k * QW;  // wave-uniform
        const int isv = i / NIT;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<_Float16*>((isv ? Vg : Kg) + size_t(kb) * kv_dim), 0, int(nrec), kBufferFlags);
        char* dst = stage + isv * TB + (RPI * (i % NIT)) * RB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 16, int(dma_off[k]), 0, 0, 0);
    };

    // Q is loaded once per workgroup: every thread converts part of the workgroup's
    // QW*16 queries x G heads (times scale*log2(e), to f16) into the second stage of each key
    // group, which the first tile's copy does not touch: queries 0..31 in key group 0's, 32..63
    // in key group 1's, as rows [query][head][HD dims] with the 16-byte chunk c of a row stored
    // at c ^ (query % CPR), so that the B-operand reads below are (nearly) bank-conflict free.
    // All of the thread's Q loads are issued first, then the first tile's copy: loads complete
    // in order, so the conversion waits only for Q, and the tile streams in meanwhile.
    static_assert(QW * 16 == 64 && G * 32 * RB <= SB, "Q staging fits the free stages");
    constexpr int QF4 = HD / 4;            // float4 chunks of one (query, head) row
    constexpr int kF4 = QW * 16 * G * QF4;  // float4 chunks of the workgroup's Q
    constexpr int NT = 64 * QW * KG;
    constexpr int kQIt = (kF4 + NT - 1) / NT;
    float4v qx[kQIt];
    {
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(q + size_t(qblk0) * q_stride + size_t(kvh) * G * HD), 0,
            0x7fffffff, kBufferFlags);
#pragma unroll
        for (int it = 0; it < kQIt; it++) {
            const int idx = min(tid + it * NT, kF4 - 1);
            const int ql = idx / (G * QF4), rem = idx % (G * QF4);
            const uint32_t row = min(qblk0 + ql, n_tok - 1) - qblk0;
            qx[it] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(
                qr, int(4 * (row * q_stride + (rem / QF4) * HD + 4 * (rem % QF4))), 0, 0));
        }
    }
    uint32_t t_first = t_begin + kg;
    if (t_begin < t_end && t_first < t_end)
#pragma unroll
        for (int k = 0; k < kInstPerWave; k++) issue_inst(t_first, 0, k);
#pragma unroll
    for (int it = 0; it < kQIt; it++) {
        const int idx = tid + it * NT;
        if (kF4 % NT != 0 && idx >= kF4) break;
        const int ql = idx / (G * QF4), rem = idx % (G * QF4);
        const int h = rem / QF4, c4 = rem % QF4;
        half4 y;
#pragma unroll
        for (int e = 0; e < 4; e++) y[e] = _Float16(qx[it][e] * qscale);
        char* qs = stage_of(ql >> 5, 1);
        const int chunk = (c4 >> 1) ^ (ql % CPR);
        *reinterpret_cast<half4*>(qs + ((ql & 31) * G + h) * RB + 16 * chunk + 8 * (c4 & 1)) = y;
    }
    __syncthreads();
    // B operand Q^T per head: lane holds Q[q0 + li][32*ks + 8*g + e] * scale*log2(e), as f16.
    half8 qb[G][KS];
    {
        const int ql = 16 * qw + li;
        const char* qs = stage_of(ql >> 5, 1) + (ql & 31) * G * RB;
#pragma unroll
        for (int h = 0; h < G; h++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
                qb[h][ks] = *reinterpret_cast<const lds_half8*>(
                    (const lds_void*)(qs + h * RB + 16 * ((4 * ks + g) ^ (ql % CPR))));
    }

    // Online-softmax state per head: reference max m (base 2), lane-partial row sum l, O^T.
    // Scores are produced already shifted (S' = s - m: the MFMA accumulator starts at -m), and
    // m only moves when some score exceeds it by more than kLazy (or for the first visible
    // keys), so P = 2^S' <= 2^kLazy and the O rescale is rare. O/l does not depend on the
    // reference, so this is exact.
    float4v O[G][ND];
    float m[G], l[G];
    float4v negm[G];  // {-m, -m, -m, -m}: the C operand of the first score MFMA of each tile
    bool started[G];
    bool all_started = false;  // wave-uniform: every lane has seen a key for every head
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = 0.f;
        l[h] = 0.f;
        negm[h] = float4v{0.f, 0.f, 0.f, 0.f};
        started[h] = false;
#pragma unroll
        for (int d = 0; d < ND; d++) O[h][d] = float4v{0.f, 0.f, 0.f, 0.f};
    }

    // `dma(k)` issues copy instruction k of the next tile (k < kInstPerWave).
    auto compute_tile = [&](uint32_t t, auto bufc, auto&& dma) {
        constexpr int buf = decltype(bufc)::value;
        const uint32_t kb = t * BN;
        if (kb >= kend_w) {  // every key of this tile is in this wave's future
#pragma unroll
            for (int k = 0; k < kInstPerWave; k++) dma(k);
            return;
        }
        const char* Ks = stage_of(kg, buf);
        const char* Vs = Ks + TB;

        // Halves of 32 keys (scores, online-softmax update, P*V each), so only 32 keys' worth
        // of S and P is live at a time.
        float4v S[2][G];
        half8 P[G];
        auto scores = [&](int hs) {
#pragma unroll
            for (int T = 0; T < 2; T++) {
                const int row = 32 * hs + 16 * T + li;
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const int chunk = (4 * ks + g) ^ swz_k<HD>(row);
                    const half8 a = *reinterpret_cast<const lds_half8*>((const lds_void*)(Ks + row * RB + 16 * chunk));
#pragma unroll
                    for (int h = 0; h < G; h++)
                        S[T][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qb[h][ks], ks == 0 ? negm[h] : S[T][h], 0, 0, 0);
                }
            }
        };
        auto softmax = [&](int hs) {
            const uint32_t kh = kb + 32 * hs;
            // Causal mask where these keys reach past the wave's first query position.
            if (kh + 31 > pos + q0) {
#pragma unroll
                for (int T = 0; T < 2; T++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t key = kh + 16 * T + 4 * g + j;
                        if (key > qpos) {
#pragma unroll
                            for (int h = 0; h < G; h++) S[T][h][j] = -__builtin_inff();
                        }
                    }
            }
            // Does a reference max have to move? In steady state (every lane started) one
            // max over all G*8 scores of the lane and a ballot decide; the exact per-head
            // cross-lane max is computed only when something moves or some lane has not seen
            // a key yet.
            bool need = true;
            if (all_started) {
                float x = -__builtin_inff();
#pragma unroll
                for (int h = 0; h < G; h++)
#pragma unroll
                    for (int T = 0; T < 2; T++)
                        x = fmaxf(x, fmaxf(fmaxf(S[T][h][0], S[T][h][1]), fmaxf(S[T][h][2], S[T][h][3])));
                need = __builtin_amdgcn_ballot_w64(x > kLazy) != 0;
            }
            if (need) {  // wave-uniform, rare after warm-up
                bool pending = false;
#pragma unroll
                for (int h = 0; h < G; h++) {
                    float x = fmaxf(fmaxf(fmaxf(S[0][h][0], S[0][h][1]), fmaxf(S[0][h][2], S[0][h][3])),
                                    fmaxf(fmaxf(S[1][h][0], S[1][h][1]), fmaxf(S[1][h][2], S[1][h][3])));
                    x = max_lanes4(x);  // max over the 4 lanes of a query
                    const bool grow = started[h] ? (x > kLazy) : (x > -__builtin_inff());
                    const float delta = grow ? x : 0.f;
                    const float alpha = fast_exp2(-delta);
                    m[h] += delta;
                    negm[h] = float4v{-m[h], -m[h], -m[h], -m[h]};
                    l[h] *= alpha;
                    started[h] |= grow;
                    pending |= !started[h];
#pragma unroll
                    for (int T = 0; T < 2; T++) S[T][h] -= delta;
#pragma unroll
                    for (int d = 0; d < ND; d++) O[h][d] *= alpha;
                }
                all_started = __builtin_amdgcn_ballot_w64(pending) == 0;
            }
            // P = 2^S' in f16 (P^T B operand: element 4T + j is key kh+16T+4g+j); row sums from
            // the same f16 values with v_dot2_f32_f16.
#pragma unroll
            for (int h = 0; h < G; h++) {
#pragma unroll
                for (int T = 0; T < 2; T++)
#pragma unroll
                    for (int j = 0; j < 4; j++) P[h][4 * T + j] = _Float16(fast_exp2(S[T][h][j]));
                const half2v one = {_Float16(1.f), _Float16(1.f)};
                float ls = l[h];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    ls = __builtin_amdgcn_fdot2(half2v{P[h][2 * e], P[h][2 * e + 1]}, one, ls, false);
                l[h] = ls;
            }
        };
        auto pv = [&](int hs, const half8 (&Pp)[G]) {
            // O^T (128 dims x (G x 16 queries)) += V^T (128 x 32) P^T (32 x 16) per head.
#pragma unroll
            for (int d = 0; d < ND; d++) {
                half4 part_[2];
#pragma unroll
                for (int half_ = 0; half_ < 2; half_++) {
                    // this 16-lane group reads keys key0..key0+3 x dims 16d..16d+15
                    const int key0 = 32 * hs + 16 * half_ + 4 * g;
                    const int row = key0 + (li >> 2);
                    const int byte = 32 * d + 8 * (li & 3);
                    const int chunk = (byte >> 4) ^ swz_v<HD>(row);
                    lds_fp16x4* src = (lds_fp16x4*)(lds_void*)const_cast<char*>(Vs + row * RB + 16 * chunk + (byte & 15));
                    part_[half_] = __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(src));
                }
                const half8 a = __builtin_shufflevector(part_[0], part_[1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int h = 0; h < G; h++)
                    O[h][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, Pp[h], O[h][d], 0, 0, 0);
            }
        };

        // The wave's priority is raised for its MFMA blocks and dropped for the softmax: the
        // switches break the lockstep of the two waves on a SIMD (which the per-tile barrier
        // restores), so one wave's VALU work lines up more often with the other's matrix work
        // (measured: C5 187.8 -> 182.6 us; which phase gets the priority makes no difference).
        // The next tile's copy goes out in two groups of instructions: after the first P*V
        // half and after the second half's scores. The compiler waits for every copy in flight
        // before a transposing LDS read (it cannot tell them apart), so no copy may be issued
        // before or among the first half's reads; these have the second half's softmax (and
        // scores) to land before its P*V, and the next tile's start is not held up. (Copies
        // issued among the P*V reads made C5 1.9x slower; all of them after the first half
        // measured like this split within 1%.) A one-half tile (head_dim 256) issues them
        // before its scores and softmax, and its P*V waits for them.
        static_assert(kInstPerWave % 2 == 0, "two groups of copies");
        if constexpr (HALVES == 1) {
#pragma unroll
            for (int k = 0; k < kInstPerWave / 2; k++) dma(k);
            __builtin_amdgcn_s_setprio(1);
            scores(0);
            __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int k = kInstPerWave / 2; k < kInstPerWave; k++) dma(k);
            softmax(0);
            __builtin_amdgcn_s_setprio(1);
            pv(0, P);
            __builtin_amdgcn_s_setprio(0);
        } else {
            __builtin_amdgcn_s_setprio(1);
            scores(0);
            __builtin_amdgcn_s_setprio(0);
            softmax(0);
            __builtin_amdgcn_s_setprio(1);
            pv(0, P);
            __builtin_amdgcn_s_setprio(0);
#pragma unroll
            for (int k = 0; k < kInstPerWave / 2; k++) dma(k);
            if (kb + 32 < kend_w) {
                __builtin_amdgcn_s_setprio(1);
                scores(1);
                __builtin_amdgcn_s_setprio(0);
#pragma unroll
                for (int k = kInstPerWave / 2; k < kInstPerWave; k++) dma(k);
                softmax(1);
                __builtin_amdgcn_s_setprio(1);
                pv(1, P);
                __builtin_amdgcn_s_setprio(0);
            } else {
#pragma unroll
                for (int k = kInstPerWave / 2; k < kInstPerWave; k++) dma(k);
            }
        }
    };

    // Key group kg takes tiles t_begin + kg, t_begin + kg + KG, ...; all groups step together
    // (one barrier per step).
    if (t_begin < t_end) {
        const uint32_t steps = (t_end - t_begin + KG - 1) / KG;
        __builtin_amdgcn_s_waitcnt(0);  // this wave's Q reads and first-tile copies are done
        __syncthreads();                // ... and everyone's: the Q staging may be overwritten
        // One step: tile t from buffer `buf` while the next tile of this key group streams into
        // the other buffer (two steps per iteration, so the buffers are fixed in the code).
        auto step = [&](uint32_t t, auto bufc) {
            constexpr int buf = decltype(bufc)::value;
            const bool next = t + KG < t_end;
            auto dma = [&](int k) {
                if (next) issue_inst(t + KG, buf ^ 1, k);
            };
            if (t < t_end) compute_tile(t, bufc, dma);
            else {
#pragma unroll
                for (int k = 0; k < kInstPerWave; k++) dma(k);
            }
            __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of the next tile have landed
            __syncthreads();                // ... and everyone's; this tile is no longer read
        };
        uint32_t t = t_first;
        for (uint32_t st = 0; st < steps; st += 2, t += 2 * KG) {
            step(t, std::integral_constant<int, 0>{});
            if (st + 1 < steps) step(t + KG, std::integral_constant<int, 1>{});
        }
    }

    if (KG == 2) {
        // Merge the two key groups through LDS (the tiles are no longer read): group 1 stores
        // its (O, m, l, started) per lane for every head, one barrier, group 0 folds them in
        // with the log-sum-exp rule. O field f = h*ND + d (16 bytes per lane, QW waves x 64
        // lanes, lane-minor: conflict-free) goes to stage object f / FPS, slot f % FPS; (m, l)
        // to mlx.
        constexpr int FPS = SB / (QW * 64 * 16);  // O fields per stage object
        static_assert(G * ND <= 4 * FPS, "merge buffers");
        auto field = [&](int h, int d) -> float4v* {
            const int f = h * ND + d;
            return reinterpret_cast<float4v*>(stage_of((f / FPS) >> 1, (f / FPS) & 1)) +
                   ((f % FPS) * QW + qw) * 64 + lane;
        };
        {
            if (kg == 1) {
#pragma unroll
                for (int h = 0; h < G; h++) {
#pragma unroll
                    for (int d = 0; d < ND; d++) *field(h, d) = O[h][d];
                    mlx[h][qw][lane] = float4v{m[h], l[h], started[h] ? 1.f : 0.f, 0.f};
                }
            }
            __syncthreads();
            if (kg == 0) {
#pragma unroll
                for (int h = 0; h < G; h++) {
                    const float4v ml = mlx[h][qw][lane];
                    const float m1 = ml[0], l1 = ml[1];
                    const bool s1 = ml[2] != 0.f;
                    const float M = started[h] ? (s1 ? fmaxf(m[h], m1) : m[h]) : m1;
                    const float a0 = started[h] ? fast_exp2(m[h] - M) : 0.f;
                    const float a1 = s1 ? fast_exp2(m1 - M) : 0.f;
#pragma unroll
                    for (int d = 0; d < ND; d++) O[h][d] = O[h][d] * a0 + *field(h, d) * a1;
                    l[h] = l[h] * a0 + l1 * a1;
                    m[h] = (started[h] || s1) ? M : m[h];
                    started[h] = started[h] || s1;
                }
            }
        }
    }
    const bool owner = kg == 0;  // the waves holding the workgroup's merged O (wave-uniform)

    // Row sums: the 4 lane groups g hold partial sums of the same query (same m).
    if (owner) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            l[h] += __shfl_xor(l[h], 16);
            l[h] += __shfl_xor(l[h], 32);
        }
    }
    const uint32_t row = q0 + li;
    const bool live = row < n_tok;
    if (n_splits == 1) {  // the whole key range: write the output
        if (!owner || !live) return;
        // Write-through (sc1) stores: the output leaves no dirty lines in the L2 for the
        // end-of-dispatch write-back (measured: C2 11.75 -> 11.19 us, C4 39.8 -> 38.5; a
        // nontemporal store gained less).
        const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
            out + size_t(qblk0) * q_stride, 0, int(min(uint64_t(64) * q_stride * 4, uint64_t(0x7fffffff))),
            kBufferFlags);
#pragma unroll
        for (int h = 0; h < G; h++) {
            const uint32_t head = kvh * G + h;
            const float inv = l[h] > 0.f ? 1.f / l[h] : 0.f;
            const int off = int(4 * ((row - qblk0) * q_stride + head * HD + 4 * g));
#pragma unroll
            for (int d = 0; d < ND; d++)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, O[h][d] * inv), ors, off + 64 * d, 0,
                                                       kScDevice);
        }
        return;
    }

    // A key split: its record per (query, head) is o / l rounded to f16 (each output element
    // becomes a weighted mean of the splits' values, so the rounding is relative to the output:
    // ~2^-12), then (m, l) as f32; a query that saw no key in this split reports m = -inf-like
    // and l = 0. attn_prefill_combine merges the records. (Merging them in this kernel, by the
    // last split of each query block to finish, measured slower: C4 50.7 us against 38.3.)
    if (!owner || !live) return;
    const uint32_t n_head = n_head_kv * G;
#pragma unroll
    for (int h = 0; h < G; h++) {
        char* dst = part + ((size_t(split) * n_tok + row) * n_head + kvh * G + h) * PB;
        const float inv = l[h] > 0.f ? 1.f / l[h] : 0.f;
#pragma unroll
        for (int d = 0; d < ND; d++) {
            const float4v v = O[h][d] * inv;
            // device-scope (write-through) 8-byte stores, like the output (C4 39.6 -> 38.7 us)
            __hip_atomic_store(reinterpret_cast<unsigned long long*>(dst + 2 * (16 * d + 4 * g)),
                               __builtin_bit_cast(unsigned long long,
                                                  half4{_Float16(v[0]), _Float16(v[1]), _Float16(v[2]), _Float16(v[3])}),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (g == 0)
            __hip_atomic_store(reinterpret_cast<unsigned long long*>(dst + 2 * HD),
                               __builtin_bit_cast(unsigned long long, float2{started[h] ? m[h] : kNoMax, l[h]}),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// out[tok][h][d] = sum_s o_s[d] 2^(m_s - M) / sum_s l_s 2^(m_s - M); 0 if the sum is 0 — the
// log-sum-exp merge of attn_combine (shaders/kernels.metal:501-516) over the split records, whose
// o is stored divided by l (so o_s[d] = l_s * rec_s[d]). HD/4 threads per (token, head) record,
// each owning 4 dims; the loads of 4 splits are in flight at once and folded in online (clamped
// indices keep them unconditional, masked entries get weight 0).
constexpr int kCombineThreads = 256;
constexpr uint32_t kQBlock = 64;  // queries per prefill workgroup (16 x kQW)
template <int HD>
__global__ __launch_bounds__(kCombineThreads) void attn_prefill_combine(
    const char* __restrict__ part, float* __restrict__ out, uint32_t pos, uint32_t n_tok,
    uint32_t n_head, uint32_t q_stride, uint32_t tps) {
    constexpr int TPR = HD / 4;      // threads per record
    constexpr int PB = HD * 2 + 16;  // bytes per record
    const uint32_t rec = blockIdx.x * (kCombineThreads / TPR) + threadIdx.x / TPR;
    if (rec >= n_tok * n_head) return;
    const uint32_t row = rec / n_head, h = rec % n_head;
    // The split count of this token's query block, as the prefill kernel enumerates it; blocks
    // of one split wrote their output directly.
    const uint32_t blk_end = min(n_tok, (row / kQBlock + 1) * kQBlock);
    const uint32_t n_splits = ((pos + blk_end + kBN<HD> - 1) / kBN<HD> + tps - 1) / tps;
    if (n_splits == 1) return;
    const int d = 4 * (threadIdx.x % TPR);
    const size_t sstride = size_t(n_tok) * n_head * PB;
    const char* src = part + size_t(rec) * PB;
    float M = kNoMax, L = 0.f;
    float4v O = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t s0 = 0; s0 < n_splits; s0 += 4) {
        float ms[4], ls[4];
        half4 os[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const char* ps = src + min(s0 + u, n_splits - 1) * sstride;
            const float2 ml = *reinterpret_cast<const float2*>(ps + 2 * HD);
            ms[u] = s0 + u < n_splits ? ml.x : kNoMax;
            ls[u] = ml.y;
            os[u] = *reinterpret_cast<const half4*>(ps + 2 * d);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float Mn = fmaxf(M, ms[u]);
            const float a0 = fast_exp2(M - Mn), a1 = ls[u] * fast_exp2(ms[u] - Mn);
            L = L * a0 + a1;
            O = O * a0 + float4v{float(os[u][0]), float(os[u][1]), float(os[u][2]), float(os[u][3])} * a1;
            M = Mn;
        }
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    __builtin_nontemporal_store(O * inv, reinterpret_cast<float4v*>(out + size_t(row) * q_stride + size_t(h) * HD + d));
}

constexpr int kQW = 4;  // query waves per workgroup (16 queries x G heads each)
constexpr int kKG = 2;  // key groups per workgroup (alternate tiles, merged through LDS)

template <int HD, int G>
int launch_prefill_g(const float* q, const _Float16* k, const _Float16* v, float* out, char* part,
                     uint32_t pos, uint32_t n_tok, uint32_t q_stride, uint32_t n_head_kv,
                     uint32_t kv_div, uint32_t n_splits, float qscale, hipStream_t stream) {
    static_assert(16 * kQW == kQBlock, "query block size");
    constexpr uint32_t BN = kBN<HD>;
    const uint32_t max_tiles = (pos + n_tok + BN - 1) / BN;
    const uint32_t tps = (max_tiles + n_splits - 1) / n_splits;  // tiles per split at most
    uint32_t pairs = 0;  // (query block, split) pairs: the kernel's enumeration
    for (uint32_t b = 0; b * kQBlock < n_tok; b++) {
        const uint32_t nt = (pos + min(n_tok, (b + 1) * kQBlock) + BN - 1) / BN;
        pairs += (nt + tps - 1) / tps;
    }
    if (uint64_t(pairs) * n_head_kv > 0x7fffffffu) return -1;
    const dim3 grid(pairs * n_head_kv);
    hipLaunchKernelGGL((attn_prefill_kernel<HD, G, kQW, kKG>), grid, dim3(64 * kQW * kKG), 0, stream,
                       q, k, v, out, part, pos, n_tok, q_stride, n_head_kv, kv_div, tps, qscale);
    if (hipGetLastError() != hipSuccess) return -4;
    if (n_splits > 1) {
        const uint32_t n_head = n_head_kv * G;
        const uint32_t per_block = kCombineThreads / (HD / 4);
        hipLaunchKernelGGL(attn_prefill_combine<HD>, dim3((n_tok * n_head + per_block - 1) / per_block),
                           dim3(kCombineThreads), 0, stream, part,
                           out, pos, n_tok, n_head, q_stride, tps);
        if (hipGetLastError() != hipSuccess) return -4;
    }
    return 0;
}

}  // namespace

uint32_t prefill_unit_heads(uint32_t group, uint32_t head_dim) {
    // At most 3 heads per unit (1 for head_dim 256): more O accumulators than that need more
    // than the 256 registers two waves per SIMD leave and spill (4 heads of 128 measured 163
    // TFLOP/s at 32 Q / 8 KV heads, C4 shape, against 600 for 3), so a group of 4 runs as two
    // units of 2.
    const uint32_t cap = head_dim == 256 ? 1 : 3;
    for (uint32_t g = group < cap ? group : cap; g > 1; g--)
        if (group % g == 0) return g;
    return 1;
}

uint32_t prefill_splits(uint32_t pos, uint32_t n_tok, uint32_t n_head_kv, uint32_t head_dim,
                        uint32_t requested) {
    const uint32_t BN = head_dim == 256 ? kBN<256> : kBN<128>;
    const uint32_t max_tiles = (pos + n_tok + BN - 1) / BN;
    const uint32_t cap = min(max_tiles, kMaxPrefillSplits);
    // (query block, split) workgroups for at most s splits per block (the kernel's enumeration)
    auto workgroups = [&](uint32_t s) {
        const uint32_t tps = (max_tiles + s - 1) / s;
        uint64_t pairs = 0;
        for (uint32_t b = 0; b * kQBlock < n_tok; b++)
            pairs += ((pos + min(n_tok, (b + 1) * kQBlock) + BN - 1) / BN + tps - 1) / tps;
        return pairs * n_head_kv;
    };
    uint32_t s = min(requested, cap);
    if (requested == 0) {
        // The shortest per-workgroup key walk whose workgroups still fit one round of 8-wave
        // workgroups on the 256 CUs (one per CU: 128 KB of LDS each), with >= 8 tiles per
        // split: each split adds a record write (~3 us at C4's 26 MB) and the combine launch,
        // which shorter walks do not pay back (measured with all G heads per workgroup: C2
        // 20.0 us unsplit, 22.0 us with 4 splits of <= 2 tiles; unsplit chunks now take the
        // head split of launch_prefill, 11.9 us).
        constexpr uint32_t kMinSplitTiles = 8;
        s = 1;
        for (uint32_t c = 2; c <= cap; c++) {
            if ((max_tiles + c - 1) / c < kMinSplitTiles) break;
            if (workgroups(c) <= 256) s = c;
        }
    }
    s = max(1u, s);
    // The largest per-block split count that this many tiles per split gives.
    const uint32_t tps = (max_tiles + s - 1) / s;
    return (max_tiles + tps - 1) / tps;
}

namespace {

template <int HD>
int launch_prefill_hd(const float* q, const _Float16* k, const _Float16* v, float* out, char* part,
                      uint32_t pos, uint32_t n_tok, uint32_t q_stride, uint32_t n_head_kv,
                      uint32_t group, uint32_t n_splits, float scale, hipStream_t stream) {
    const float qscale = scale * kLog2e;
    // A chunk that gives fewer workgroups than the chip has CUs and needs no key split runs
    // every query head of a group in its own workgroup (G = 1 over n_head_kv * group units):
    // 3x the workgroups at G = 3, each walking its keys with a third of the MFMA and softmax
    // work per tile, so the causal chunk's longest key walk, which sets the kernel's duration,
    // is shorter (the K/V tile is then read from L2 once per head instead of once per group).
    const uint32_t blocks = (n_tok + kQBlock - 1) / kQBlock;
    if (group > 1 && n_splits == 1 && uint64_t(blocks) * n_head_kv * group <= 256)
        return launch_prefill_g<HD, 1>(q, k, v, out, part, pos, n_tok, q_stride, n_head_kv * group,
                                       group, 1, qscale, stream);
    // Groups above 3 run as units of gs heads (the largest divisor of the group up to 3), kv_div of
    // them per KV head, each reading that head's K/V.
    const uint32_t gs = prefill_unit_heads(group, HD), kv_div = group / gs, units = n_head_kv * kv_div;
    switch (gs) {
        case 1: return launch_prefill_g<HD, 1>(q, k, v, out, part, pos, n_tok, q_stride, units, kv_div, n_splits, qscale, stream);
        case 2:
            if constexpr (HD != 256)
                return launch_prefill_g<HD, 2>(q, k, v, out, part, pos, n_tok, q_stride, units, kv_div, n_splits, qscale, stream);
            return -2;
        case 3:
            if constexpr (HD != 256)
                return launch_prefill_g<HD, 3>(q, k, v, out, part, pos, n_tok, q_stride, units, kv_div, n_splits, qscale, stream);
            return -2;
        default: return -2;
    }
}

}  // namespace

int launch_prefill(const float* q, const _Float16* k, const _Float16* v, float* out, char* part,
                   uint32_t pos, uint32_t n_tok, uint32_t q_stride, uint32_t n_head_kv,
                   uint32_t group, uint32_t head_dim, uint32_t n_splits, float scale,
                   hipStream_t stream) {
    switch (head_dim) {
        case 64: return launch_prefill_hd<64>(q, k, v, out, part, pos, n_tok, q_stride, n_head_kv, group, n_splits, scale, stream);
        case 128: return launch_prefill_hd<128>(q, k, v, out, part, pos, n_tok, q_stride, n_head_kv, group, n_splits, scale, stream);
        case 256: return launch_prefill_hd<256>(q, k, v, out, part, pos, n_tok, q_stride, n_head_kv, group, n_splits, scale, stream);
        default: return -2;
    }
}

}  // namespace ingot
