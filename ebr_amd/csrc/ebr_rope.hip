// Fused 2D-RoPE split and merge for gfx950 (C ABI: include/ebr_rope.h).
//
// Both are HBM-bound elementwise passes. A thread moves VW consecutive elements of one row: the quarter swap maps a
// VW-aligned chunk of a quarter onto a VW-aligned chunk of the partner quarter when VW divides D / 4, so a thread
// reads its chunk and its partner chunk with two vector loads (the partner's bytes are the neighbouring lanes' own,
// so they come from the cache). Work is flattened with the output's fastest dimensions innermost, so the stores of a
// wave are contiguous: the split writes [B, H, N, D] rows, the merge writes [B, N, 3*H*D] rows.
//
// Arithmetic is fp32 with contraction off: every product and sum is rounded as the dense formula's separate
// operations are (reference models/fused_attn/rope_split.py:40-44, 58-61), then rounded once to the tensor dtype.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ebr_rope.h"

namespace ebr_rope {

template <typename T, int VW> using Vec = T __attribute__((ext_vector_type(VW)));  // aligned to its size

template <typename T> __device__ __forceinline__ float f32(T x) { return (float)x; }

template <typename T> __device__ __forceinline__ T narrow(float x) { return (T)x; }  // round to nearest even

// An fp32 product kept opaque, so that narrowing it rounds twice (to fp32, then to T) as the dense formula does; for
// fp16 the compiler would otherwise fuse multiply and narrowing into one mixed-precision op that rounds once.
__device__ __forceinline__ float mul_f32(float a, float b) {
    float p = a * b;
    asm volatile("" : "+v"(p));
    return p;
}

struct SplitArgs {
    const void* qkv;
    int64_t sb, sn;
    const float* cos;
    const float* sin;
    const float* qs;
    void *q, *k, *v;
    int B, N, H, D;
    int64_t total;  // B * H * N * (D / VW) threads
};

struct MergeArgs {
    const void *dq, *dk, *dv;
    int64_t sq[3], sk[3], sv[3];
    const float* cos;
    const float* sin;
    const float* qs;
    void* g;
    int B, H, N, D;
    int64_t total;  // B * N * H * (D / VW) threads
};

// Partner chunk start of the quarter swap: quarter (d / Q) ^ 1, same offset inside the quarter.
__device__ __forceinline__ int swap_start(int d0, int Q) { return ((d0 / Q) ^ 1) * Q + d0 % Q; }

template <typename T, int VW> __global__ __launch_bounds__(256) void k_rope_split(SplitArgs a) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= a.total) return;
    const int cpr = a.D / VW;
    int64_t r = t / cpr;
    const int c = (int)(t - r * cpr);
    const int n = (int)(r % a.N);
    r /= a.N;
    const int h = (int)(r % a.H);
    const int b = (int)(r / a.H);
    const int d0 = c * VW;
    const int p0 = swap_start(d0, a.D >> 2);
    using V = Vec<T, VW>;
    using F = Vec<float, VW>;
    const int64_t hd = (int64_t)a.H * a.D;
    const T* row = reinterpret_cast<const T*>(a.qkv) + (int64_t)b * a.sb + (int64_t)n * a.sn + (int64_t)h * a.D;
    const V xq = *reinterpret_cast<const V*>(row + d0);
    const V xqs = *reinterpret_cast<const V*>(row + p0);
    const V xk = *reinterpret_cast<const V*>(row + hd + d0);
    const V xks = *reinterpret_cast<const V*>(row + hd + p0);
    const V xv = *reinterpret_cast<const V*>(row + 2 * hd + d0);
    const F cs = *reinterpret_cast<const F*>(a.cos + (int64_t)n * a.D + d0);
    const F sn = *reinterpret_cast<const F*>(a.sin + (int64_t)n * a.D + d0);
    V oq, ok;
#pragma unroll
    for (int e = 0; e < VW; ++e) {
        oq[e] = narrow<T>(f32(xq[e]) * cs[e] + f32(xqs[e]) * sn[e]);
        ok[e] = narrow<T>(f32(xk[e]) * cs[e] + f32(xks[e]) * sn[e]);
    }
    if (a.qs) {  // per-head temperature after the rotation: round(round(R q) * t)
        const float tq = a.qs[h];
#pragma unroll
        for (int e = 0; e < VW; ++e) oq[e] = narrow<T>(mul_f32(f32(oq[e]), tq));
    }
    const int64_t out = (((int64_t)b * a.H + h) * a.N + n) * a.D + d0;
    *reinterpret_cast<V*>(reinterpret_cast<T*>(a.q) + out) = oq;
    *reinterpret_cast<V*>(reinterpret_cast<T*>(a.k) + out) = ok;
    *reinterpret_cast<V*>(reinterpret_cast<T*>(a.v) + out) = xv;
}

template <typename T, int VW> __global__ __launch_bounds__(256) void k_rope_merge(MergeArgs a) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= a.total) return;
    const int cpr = a.D / VW;
    int64_t r = t / cpr;
    const int c = (int)(t - r * cpr);
    const int h = (int)(r % a.H);
    r /= a.H;
    const int n = (int)(r % a.N);
    const int b = (int)(r / a.N);
    const int d0 = c * VW;
    const int p0 = swap_start(d0, a.D >> 2);
    using V = Vec<T, VW>;
    using F = Vec<float, VW>;
    const T* qr = reinterpret_cast<const T*>(a.dq) + (int64_t)b * a.sq[0] + (int64_t)h * a.sq[1] + (int64_t)n * a.sq[2];
    const T* kr = reinterpret_cast<const T*>(a.dk) + (int64_t)b * a.sk[0] + (int64_t)h * a.sk[1] + (int64_t)n * a.sk[2];
    const T* vr = reinterpret_cast<const T*>(a.dv) + (int64_t)b * a.sv[0] + (int64_t)h * a.sv[1] + (int64_t)n * a.sv[2];
    const V gq = *reinterpret_cast<const V*>(qr + d0);
    const V gqs = *reinterpret_cast<const V*>(qr + p0);
    const V gk = *reinterpret_cast<const V*>(kr + d0);
    const V gks = *reinterpret_cast<const V*>(kr + p0);
    const V gv = *reinterpret_cast<const V*>(vr + d0);
    const F cs = *reinterpret_cast<const F*>(a.cos + (int64_t)n * a.D + d0);
    const F sp = *reinterpret_cast<const F*>(a.sin + (int64_t)n * a.D + p0);
    float fq[VW], fqs[VW];
#pragma unroll
    for (int e = 0; e < VW; ++e) {
        fq[e] = f32(gq[e]);
        fqs[e] = f32(gqs[e]);
    }
    if (a.qs) {  // adjoint of the temperature first, rounded as the dtype's multiply is
        const float tq = a.qs[h];
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            fq[e] = f32(narrow<T>(mul_f32(fq[e], tq)));
            fqs[e] = f32(narrow<T>(mul_f32(fqs[e], tq)));
        }
    }
    V oq, ok;
#pragma unroll
    for (int e = 0; e < VW; ++e) {
        oq[e] = narrow<T>(fq[e] * cs[e] + fqs[e] * sp[e]);
        ok[e] = narrow<T>(f32(gk[e]) * cs[e] + f32(gks[e]) * sp[e]);
    }
    const int64_t hd = (int64_t)a.H * a.D;
    T* out = reinterpret_cast<T*>(a.g) + ((int64_t)b * a.N + n) * 3 * hd + (int64_t)h * a.D + d0;
    *reinterpret_cast<V*>(out) = oq;
    *reinterpret_cast<V*>(out + hd) = ok;
    *reinterpret_cast<V*>(out + 2 * hd) = gv;
}

// ---------------------------------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------------------------------

constexpr int THREADS = 256;

static int es_of(int dtype) { return dtype == EBR_DTYPE_F32 ? 4 : 2; }

static int check_common(int dtype, int B, int N, int H, int D) {
    if (dtype != EBR_DTYPE_F32 && dtype != EBR_DTYPE_BF16 && dtype != EBR_DTYPE_F16) return EBR_ERR_DTYPE;
    if (B < 1 || N < 1 || H < 1 || D < 4 || D > 256 || D % 4) return EBR_ERR_SHAPE;
    if ((int64_t)B * N * H * D >= ((int64_t)1 << 40)) return EBR_ERR_SHAPE;
    return EBR_OK;
}

static bool aligned(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

// Widest vector (elements) such that it divides D / 4, fits 16 bytes, and every row start and table row is aligned.
static int pick_vw(int es, int D, const void* const* ptrs, int nptr, const int64_t* strides, int nstr,
                   const float* cos, const float* sin) {
    for (int vw = 16 / es; vw > 1; vw >>= 1) {
        if ((D / 4) % vw) continue;
        const int vb = vw * es;
        bool ok = aligned(cos, vw * 4) && aligned(sin, vw * 4) && (D * 4) % (vw * 4) == 0;
        for (int i = 0; i < nptr && ok; ++i) ok = aligned(ptrs[i], vb);
        for (int i = 0; i < nstr && ok; ++i) ok = (strides[i] * es) % vb == 0;
        if (ok) return vw;
    }
    return 1;
}

static int rc_launch() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? EBR_OK : EBR_ERR_HIP_BASE + (int)e;
}

template <typename T, int VW> static int launch_split(SplitArgs a, hipStream_t s) {
    a.total = (int64_t)a.B * a.H * a.N * (a.D / VW);
    const int64_t blocks = (a.total + THREADS - 1) / THREADS;
    if (blocks >= ((int64_t)1 << 31)) return EBR_ERR_SHAPE;
    hipLaunchKernelGGL((k_rope_split<T, VW>), dim3((unsigned)blocks), dim3(THREADS), 0, s, a);
    return rc_launch();
}

template <typename T, int VW> static int launch_merge(MergeArgs a, hipStream_t s) {
    a.total = (int64_t)a.B * a.N * a.H * (a.D / VW);
    const int64_t blocks = (a.total + THREADS - 1) / THREADS;
    if (blocks >= ((int64_t)1 << 31)) return EBR_ERR_SHAPE;
    hipLaunchKernelGGL((k_rope_merge<T, VW>), dim3((unsigned)blocks), dim3(THREADS), 0, s, a);
    return rc_launch();
}

template <typename T> static int split_vw(int vw, SplitArgs a, hipStream_t s) {
    if constexpr (sizeof(T) == 2) {
        if (vw == 8) return launch_split<T, 8>(a, s);
    }
    if (vw == 4) return launch_split<T, 4>(a, s);
    if (vw == 2) return launch_split<T, 2>(a, s);
    return launch_split<T, 1>(a, s);
}

template <typename T> static int merge_vw(int vw, MergeArgs a, hipStream_t s) {
    if constexpr (sizeof(T) == 2) {
        if (vw == 8) return launch_merge<T, 8>(a, s);
    }
    if (vw == 4) return launch_merge<T, 4>(a, s);
    if (vw == 2) return launch_merge<T, 2>(a, s);
    return launch_merge<T, 1>(a, s);
}

}  // namespace ebr_rope

using namespace ebr_rope;

extern "C" {

int ebr_rope_split(int dtype, int B, int N, int H, int D, const void* qkv, int64_t qkv_sb, int64_t qkv_sn,
                   const float* cos, const float* sin, const float* qscale, void* q, void* k, void* v,
                   void* stream) {
    int rc = check_common(dtype, B, N, H, D);
    if (rc) return rc;
    if (!qkv || !cos || !sin || !q || !k || !v) return EBR_ERR_NULL;
    if (qkv_sb < 0 || qkv_sn < 0) return EBR_ERR_SHAPE;
    const int es = es_of(dtype);
    SplitArgs a = {};
    a.qkv = qkv;
    a.sb = qkv_sb;
    a.sn = qkv_sn;
    a.cos = cos;
    a.sin = sin;
    a.qs = qscale;
    a.q = q;
    a.k = k;
    a.v = v;
    a.B = B;
    a.N = N;
    a.H = H;
    a.D = D;
    const void* ptrs[4] = {qkv, q, k, v};
    const int64_t strides[2] = {qkv_sb, qkv_sn};
    const int vw = pick_vw(es, D, ptrs, 4, strides, 2, cos, sin);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (dtype == EBR_DTYPE_F32) return split_vw<float>(vw, a, s);
    if (dtype == EBR_DTYPE_BF16) return split_vw<__bf16>(vw, a, s);
    return split_vw<_Float16>(vw, a, s);
}

int ebr_rope_merge(int dtype, int B, int H, int N, int D, const void* dq, const int64_t dq_str[3], const void* dk,
                   const int64_t dk_str[3], const void* dv, const int64_t dv_str[3], const float* cos,
                   const float* sin, const float* qscale, void* g, void* stream) {
    int rc = check_common(dtype, B, N, H, D);
    if (rc) return rc;
    if (!dq || !dk || !dv || !dq_str || !dk_str || !dv_str || !cos || !sin || !g) return EBR_ERR_NULL;
    MergeArgs a = {};
    for (int i = 0; i < 3; ++i) {
        if (dq_str[i] < 0 || dk_str[i] < 0 || dv_str[i] < 0) return EBR_ERR_SHAPE;
        a.sq[i] = dq_str[i];
        a.sk[i] = dk_str[i];
        a.sv[i] = dv_str[i];
    }
    const int es = es_of(dtype);
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.cos = cos;
    a.sin = sin;
    a.qs = qscale;
    a.g = g;
    a.B = B;
    a.H = H;
    a.N = N;
    a.D = D;
    const void* ptrs[4] = {dq, dk, dv, g};
    const int64_t strides[9] = {dq_str[0], dq_str[1], dq_str[2], dk_str[0], dk_str[1],
                                dk_str[2], dv_str[0], dv_str[1], dv_str[2]};
    const int vw = pick_vw(es, D, ptrs, 4, strides, 9, cos, sin);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (dtype == EBR_DTYPE_F32) return merge_vw<float>(vw, a, s);
    if (dtype == EBR_DTYPE_BF16) return merge_vw<__bf16>(vw, a, s);
    return merge_vw<_Float16>(vw, a, s);
}

}  // extern "C"
