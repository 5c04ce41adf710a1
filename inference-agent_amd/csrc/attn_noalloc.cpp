// attn_noalloc.cpp — ingot_attn_decode_noalloc: the decode entry point for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). It has no counterpart in the reference.
//
// The decode kernels need a workspace (completion counters and split records). Here it is a
// file-scope device array, `scratch`, of INGOT_ATTN_NOALLOC_SCRATCH_BYTES (enough for up to 64
// query heads at any split count); every GPU the library runs on holds its own copy until the
// process ends. Host code never passes the array's name to a kernel (on the host it is only a
// stand-in): the first call on a device, with that device current, resolves the device address
// with hipGetSymbolAddress and keeps it per device, then clears the array with a fill kernel on
// the caller's stream. (A __device__ array starts zero-filled when the code object loads, which
// is what the decode hand-off needs: counters and records at zero, and every call leaves them at
// zero again. The clear re-establishes that explicitly; under HIP graph capture it is recorded
// into the graph instead of run, and the array's load-time zeros still hold.) After that a call
// only launches the decode kernels: no hipMalloc, hipFree or allocating library call. All calls on one GPU share that GPU's array, so calls that overlap on
// one GPU race: order them on one stream.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "../../include/ingot_attn.h"
#include "attn_internal.h"

namespace {

constexpr size_t kScratchBytes = INGOT_ATTN_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes == ingot::kCounterBytes + 64 * ingot::kDecodeHeadRecordBytes,
              "the scratch holds the decode workspace of 64 query heads");

static __device__ __attribute__((aligned(256))) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device, once resolved

__global__ __launch_bounds__(256) void clear_scratch(uint4* p, size_t n16) {
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n16; i += size_t(gridDim.x) * 256)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The current device's scratch address; resolved and cleared (on `stream`) on first use.
int device_scratch(void** out, hipStream_t stream) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return INGOT_ATTN_EHIP;
    if (dev < 0 || dev >= kMaxDevices) return INGOT_ATTN_EUNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_scratch[dev] == nullptr) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return INGOT_ATTN_EHIP;
        hipLaunchKernelGGL(clear_scratch, dim3(256), dim3(256), 0, stream, static_cast<uint4*>(p),
                           kScratchBytes / 16);
        if (hipGetLastError() != hipSuccess) return INGOT_ATTN_EHIP;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return INGOT_ATTN_OK;
}

}  // namespace

extern "C" int ingot_attn_decode_noalloc(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                         float* out, const IngotAttnDecodeDesc* d, void* stream) {
    // Validate before the scratch is claimed: an invalid descriptor has size 0, and
    // ingot_attn_decode then rejects it with its own code without touching the device.
    const size_t need = ingot_attn_decode_workspace_size(d);
    if (need == 0) return ingot_attn_decode(q, k_cache, v_cache, out, nullptr, 0, d, stream);
    if (need > kScratchBytes) return INGOT_ATTN_EWORKSPACE;
    void* ws = nullptr;
    const int rc = device_scratch(&ws, static_cast<hipStream_t>(stream));
    if (rc) return rc;
    return ingot_attn_decode(q, k_cache, v_cache, out, ws, kScratchBytes, d, stream);
}
