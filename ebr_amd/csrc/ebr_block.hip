// Fused pointwise work of the energy network's blocks on gfx950 (C ABI: include/ebr_block.h): rms_norm over the last
// dimension and the SwiGLU activation silu(gate) * up, each with its backward and the backward of that backward (the
// graded descent differentiates the energy twice). All are HBM-bound; arithmetic is fp32 (fp64 for fp64 tensors) and
// each output is rounded once to the tensor dtype, where eager autograd chains several rounded kernels.
//
// rms_norm (reference models/layers.py:37-42): y = x r, r = (mean(x^2) + eps)^-1/2 per row of C; one wave per row.
//   backward:  dx = r dy - (r^3 / C) x Sdx                                   Sdx = sum dy x
//   backward2 (cotangent c of dx):
//     gdy = r c - (r^3 / C) x Scx                                            Scx = sum c x
//     gx  = -(r^3 / C) Scdy x + (3 r^5 / C^2) Scx Sdx x - (r^3 / C) Sdx c - (r^3 / C) Scx dy,   Scdy = sum c dy
// SwiGLU (reference models/layers.py:74-84, gate and up the two halves of one [.., 2I] projection):
//   y = silu(g) u;  dg = dy u silu'(g), du = dy silu(g);
//   backward2 (cotangents cg, cu of dg, du): gg = cg dy u silu''(g) + cu dy silu'(g), gu = cg dy silu'(g),
//   gdy = cg u silu'(g) + cu silu(g); with s = sigmoid(g): silu' = s (1 + g (1 - s)),
//   silu'' = s (1 - s) (2 + g (1 - 2 s)).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ebr_block.h"

namespace ebr_block {

template <typename T> struct Acc { using type = float; };
template <> struct Acc<double> { using type = double; };

template <typename T, typename A> __device__ __forceinline__ A wide(T x) { return (A)x; }
template <typename T, typename A> __device__ __forceinline__ T narrow(A x) { return (T)x; }

template <typename A> __device__ __forceinline__ A wave_sum(A v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

template <typename A> __device__ __forceinline__ A rsqrt_of(A x);
template <> __device__ __forceinline__ float rsqrt_of(float x) { return 1.f / __builtin_sqrtf(x); }
template <> __device__ __forceinline__ double rsqrt_of(double x) { return 1.0 / sqrt(x); }

constexpr int ROWS_PER_BLOCK = 4;  // one wave per row

struct NormArgs {
    const void *x, *dy, *c;
    void *y, *gx, *gdy;
    int64_t rows;
    int C;
    float eps;
};

// mode 0: y = rms_norm(x); 1: y = dx given dy; 2: gx, gdy given dy and c.
template <typename T, int MODE> __global__ __launch_bounds__(64 * ROWS_PER_BLOCK) void k_rmsnorm(NormArgs a) {
#pragma clang fp contract(off)
    using A = typename Acc<T>::type;
    const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= a.rows) return;  // wave-uniform
    const int C = a.C;
    const T* x = reinterpret_cast<const T*>(a.x) + row * C;
    const T* dy = MODE >= 1 ? reinterpret_cast<const T*>(a.dy) + row * C : nullptr;
    const T* c = MODE == 2 ? reinterpret_cast<const T*>(a.c) + row * C : nullptr;
    A sxx = 0, sdx = 0, scx = 0, scd = 0;
    for (int k = lane; k < C; k += 64) {
        const A xv = wide<T, A>(x[k]);
        sxx += xv * xv;
        if constexpr (MODE >= 1) sdx += wide<T, A>(dy[k]) * xv;
        if constexpr (MODE == 2) {
            const A cv = wide<T, A>(c[k]);
            scx += cv * xv;
            scd += cv * wide<T, A>(dy[k]);
        }
    }
    const A r = rsqrt_of<A>(wave_sum(sxx) / (A)C + (A)a.eps);
    if constexpr (MODE == 0) {
        T* y = reinterpret_cast<T*>(a.y) + row * C;
        for (int k = lane; k < C; k += 64) y[k] = narrow<T, A>(wide<T, A>(x[k]) * r);
        return;
    }
    sdx = wave_sum(sdx);
    const A r3c = r * r * r / (A)C;
    if constexpr (MODE == 1) {
        T* dx = reinterpret_cast<T*>(a.y) + row * C;
        for (int k = lane; k < C; k += 64) dx[k] = narrow<T, A>(r * wide<T, A>(dy[k]) - r3c * sdx * wide<T, A>(x[k]));
        return;
    }
    scx = wave_sum(scx);
    scd = wave_sum(scd);
    const A kx = -r3c * scd + (A)3 * r3c * r * r / (A)C * scx * sdx;
    T* gx = reinterpret_cast<T*>(a.gx) + row * C;
    T* gdy = reinterpret_cast<T*>(a.gdy) + row * C;
    for (int k = lane; k < C; k += 64) {
        const A xv = wide<T, A>(x[k]), cv = wide<T, A>(c[k]), dv = wide<T, A>(dy[k]);
        gx[k] = narrow<T, A>(kx * xv - r3c * sdx * cv - r3c * scx * dv);
        gdy[k] = narrow<T, A>(r * cv - r3c * scx * xv);
    }
}

struct GluArgs {
    const void *gu, *dy, *c;
    void *y, *ggu, *gdy;
    int64_t n;  // rows
    int I;      // half width
};

template <typename A> __device__ __forceinline__ A sigmoid_of(A g) { return (A)1 / ((A)1 + exp(-g)); }

// mode 0: y = silu(g) u; 1: dgu = [dg | du] given dy; 2: ggu = [gg | gu], gdy given dy and c = [cg | cu].
template <typename T, int MODE> __global__ __launch_bounds__(256) void k_swiglu(GluArgs a) {
#pragma clang fp contract(off)
    using A = typename Acc<T>::type;
    const int64_t total = a.n * a.I;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = e / a.I;
        const int j = (int)(e - row * a.I);
        const T* gu = reinterpret_cast<const T*>(a.gu) + row * 2 * a.I;
        const A g = wide<T, A>(gu[j]), u = wide<T, A>(gu[a.I + j]);
        const A s = sigmoid_of(g);
        const A silu = g * s;
        if constexpr (MODE == 0) {
            // eager: silu rounded to T, then the product rounded to T
            reinterpret_cast<T*>(a.y)[e] = narrow<T, A>(wide<T, A>(narrow<T, A>(silu)) * u);
            continue;
        }
        const A d1 = s * ((A)1 + g * ((A)1 - s));  // silu'
        const A dy = wide<T, A>(reinterpret_cast<const T*>(a.dy)[e]);
        if constexpr (MODE == 1) {
            T* out = reinterpret_cast<T*>(a.y) + row * 2 * a.I;
            // eager: d(silu) = round(dy u), dg = round(d(silu) silu'); du = round(dy round(silu))
            out[j] = narrow<T, A>(wide<T, A>(narrow<T, A>(dy * u)) * d1);
            out[a.I + j] = narrow<T, A>(dy * wide<T, A>(narrow<T, A>(silu)));
            continue;
        }
        const T* c = reinterpret_cast<const T*>(a.c) + row * 2 * a.I;
        const A cg = wide<T, A>(c[j]), cu = wide<T, A>(c[a.I + j]);
        const A d2 = s * ((A)1 - s) * ((A)2 + g * ((A)1 - (A)2 * s));  // silu''
        T* out = reinterpret_cast<T*>(a.ggu) + row * 2 * a.I;
        out[j] = narrow<T, A>(cg * dy * u * d2 + cu * dy * d1);
        out[a.I + j] = narrow<T, A>(cg * dy * d1);
        reinterpret_cast<T*>(a.gdy)[e] = narrow<T, A>(cg * u * d1 + cu * silu);
    }
}

static int rc_launch() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? EBR_OK : EBR_ERR_HIP_BASE + (int)e;
}

static int check(int dtype, int64_t rows, int64_t width) {
    if (dtype != EBR_DTYPE_F32 && dtype != EBR_DTYPE_BF16 && dtype != EBR_DTYPE_F16 && dtype != EBR_DTYPE_F64)
        return EBR_ERR_DTYPE;
    if (rows < 1 || width < 1 || rows * width >= ((int64_t)1 << 40) || width > (1 << 30)) return EBR_ERR_SHAPE;
    return EBR_OK;
}

template <int MODE> static void launch_norm(int dtype, hipStream_t s, const NormArgs& a) {
    const dim3 grid((unsigned)((a.rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK)), block(64 * ROWS_PER_BLOCK);
    if (dtype == EBR_DTYPE_F32) hipLaunchKernelGGL((k_rmsnorm<float, MODE>), grid, block, 0, s, a);
    else if (dtype == EBR_DTYPE_BF16) hipLaunchKernelGGL((k_rmsnorm<__bf16, MODE>), grid, block, 0, s, a);
    else if (dtype == EBR_DTYPE_F16) hipLaunchKernelGGL((k_rmsnorm<_Float16, MODE>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_rmsnorm<double, MODE>), grid, block, 0, s, a);
}

template <int MODE> static void launch_glu(int dtype, hipStream_t s, const GluArgs& a) {
    const int64_t total = a.n * a.I;
    const int64_t want = (total + 255) / 256;
    const dim3 grid((unsigned)(want < 65536 ? want : 65536)), block(256);
    if (dtype == EBR_DTYPE_F32) hipLaunchKernelGGL((k_swiglu<float, MODE>), grid, block, 0, s, a);
    else if (dtype == EBR_DTYPE_BF16) hipLaunchKernelGGL((k_swiglu<__bf16, MODE>), grid, block, 0, s, a);
    else if (dtype == EBR_DTYPE_F16) hipLaunchKernelGGL((k_swiglu<_Float16, MODE>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_swiglu<double, MODE>), grid, block, 0, s, a);
}

}  // namespace ebr_block

using namespace ebr_block;

extern "C" {

int ebr_block_rmsnorm(int dtype, int64_t rows, int C, float eps, const void* x, void* y, void* stream) {
    int rc = check(dtype, rows, C);
    if (rc) return rc;
    if (!x || !y) return EBR_ERR_NULL;
    NormArgs a = {x, nullptr, nullptr, y, nullptr, nullptr, rows, C, eps};
    launch_norm<0>(dtype, (hipStream_t)stream, a);
    return rc_launch();
}

int ebr_block_rmsnorm_bwd(int dtype, int64_t rows, int C, float eps, const void* x, const void* dy, void* dx,
                          void* stream) {
    int rc = check(dtype, rows, C);
    if (rc) return rc;
    if (!x || !dy || !dx) return EBR_ERR_NULL;
    NormArgs a = {x, dy, nullptr, dx, nullptr, nullptr, rows, C, eps};
    launch_norm<1>(dtype, (hipStream_t)stream, a);
    return rc_launch();
}

int ebr_block_rmsnorm_bwd2(int dtype, int64_t rows, int C, float eps, const void* x, const void* dy, const void* c,
                           void* gx, void* gdy, void* stream) {
    int rc = check(dtype, rows, C);
    if (rc) return rc;
    if (!x || !dy || !c || !gx || !gdy) return EBR_ERR_NULL;
    NormArgs a = {x, dy, c, nullptr, gx, gdy, rows, C, eps};
    launch_norm<2>(dtype, (hipStream_t)stream, a);
    return rc_launch();
}

int ebr_block_swiglu(int dtype, int64_t rows, int I, const void* gu, void* y, void* stream) {
    int rc = check(dtype, rows, I);
    if (rc) return rc;
    if (!gu || !y) return EBR_ERR_NULL;
    GluArgs a = {gu, nullptr, nullptr, y, nullptr, nullptr, rows, I};
    launch_glu<0>(dtype, (hipStream_t)stream, a);
    return rc_launch();
}

int ebr_block_swiglu_bwd(int dtype, int64_t rows, int I, const void* gu, const void* dy, void* dgu, void* stream) {
    int rc = check(dtype, rows, I);
    if (rc) return rc;
    if (!gu || !dy || !dgu) return EBR_ERR_NULL;
    GluArgs a = {gu, dy, nullptr, dgu, nullptr, nullptr, rows, I};
    launch_glu<1>(dtype, (hipStream_t)stream, a);
    return rc_launch();
}

int ebr_block_swiglu_bwd2(int dtype, int64_t rows, int I, const void* gu, const void* dy, const void* c, void* ggu,
                          void* gdy, void* stream) {
    int rc = check(dtype, rows, I);
    if (rc) return rc;
    if (!gu || !dy || !c || !ggu || !gdy) return EBR_ERR_NULL;
    GluArgs a = {gu, dy, c, nullptr, ggu, gdy, rows, I};
    launch_glu<2>(dtype, (hipStream_t)stream, a);
    return rc_launch();
}

}  // extern "C"
