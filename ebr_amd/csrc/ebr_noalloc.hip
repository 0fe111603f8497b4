// ebr_attn_bwd_bwd_noalloc: the backward of the backward for callers that cannot allocate device memory (code under
// HIP graph capture, serving loops, harnesses that forbid hipMalloc). It runs exactly the kernels of
// ebr_attn_bwd_bwd; the fp32 row-statistics scratch those kernels exchange for L > 128 or D > 128 ([3, B, H, L]:
// Dr, E, T)
// lives in a fixed device array of this library instead of a caller buffer.
//
// The array is a file-scope __device__ variable: every GPU the library runs on holds its own copy, at its own address,
// until the process ends. Host code never passes the array's name to a kernel (on the host that name is a stand-in,
// not a device address); it passes the address hipGetSymbolAddress returns for the current device, looked up once per
// device on the entry point's first call there. That first call may come inside HIP stream capture (a caller
// recording a graph): the lookup enqueues nothing, and it runs with this thread's capture mode switched to relaxed,
// so a capture in global or thread-local mode neither rejects it nor is invalidated by it. The per-device address
// table is the library's only mutable host state. Every call on one GPU shares that GPU's copy and leaves the last
// call's contents in it: calls that overlap on one GPU (two streams, two threads) race. Nothing has to start at zero:
// the row kernel writes every statistic the column kernel reads.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/ebr_attn.h"

namespace {

constexpr int64_t SCRATCH_FLOATS = EBR_NOALLOC_SCRATCH_BYTES / 4;
static_assert(EBR_NOALLOC_SCRATCH_BYTES % 256 == 0, "whole 256-byte blocks");

__device__ __align__(256) float scratch[SCRATCH_FLOATS];

constexpr int MAX_DEVICES = 64;
std::atomic<float*> scratch_of[MAX_DEVICES];  // the device address of ``scratch`` on each device, once looked up

// Address of the current device's copy of ``scratch`` (looked up on the first call on that device), or an error.
int device_scratch(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return EBR_ERR_HIP_BASE + (int)e;
    if (dev < 0 || dev >= MAX_DEVICES) return EBR_ERR_SHAPE;
    float* p = scratch_of[dev].load(std::memory_order_acquire);
    if (!p) {
        void* addr = nullptr;
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        e = hipThreadExchangeStreamCaptureMode(&mode);  // relaxed for the lookup; the caller's mode comes back below
        if (e != hipSuccess) return EBR_ERR_HIP_BASE + (int)e;
        e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        const hipError_t e2 = hipThreadExchangeStreamCaptureMode(&mode);
        if (e == hipSuccess && e2 != hipSuccess) e = e2;
        if (e != hipSuccess || !addr) return EBR_ERR_HIP_BASE + (int)(e != hipSuccess ? e : hipErrorInvalidSymbol);
        p = static_cast<float*>(addr);
        scratch_of[dev].store(p, std::memory_order_release);  // every thread that races here stores the same value
    }
    *out = p;
    return EBR_OK;
}

}  // namespace

extern "C" {

int ebr_attn_bwd_bwd_noalloc(int dtype, int B, int H, int L, int D, float scale, const void* q,
                             const int64_t q_str[3], const void* k, const int64_t k_str[3], const void* v,
                             const int64_t v_str[3], const void* o, const void* lse, const void* dO,
                             const int64_t dO_str[3], const void* gq, const int64_t gq_str[3], const void* gk,
                             const int64_t gk_str[3], const void* gv, const int64_t gv_str[3], void* hq, void* hk,
                             void* hv, void* hdo, void* stream) {
    const int64_t need = dtype == EBR_DTYPE_F64 ? 0 : ebr_attn_scratch_bytes(EBR_OP_BWD_BWD, B, H, L, D);
    if (need > EBR_NOALLOC_SCRATCH_BYTES) return EBR_ERR_NOALLOC_SIZE;
    float* ptr = nullptr;
    if (need > 0) {
        const int rc = device_scratch(&ptr);
        if (rc) return rc;
    }
    return ebr_attn_bwd_bwd(dtype, B, H, L, D, scale, q, q_str, k, k_str, v, v_str, o, lse, dO, dO_str, gq, gq_str,
                            gk, gk_str, gv, gv_str, hq, hk, hv, hdo, ptr, stream);
}

}  // extern "C"
