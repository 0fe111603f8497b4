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

// 16 bytes of consecutive elements: one global load or store instruction per lane.
template <typename T> struct alignas(16) Vec {
    static constexpr int N = 16 / (int)sizeof(T);
    T e[N];
};
template <typename T> __device__ __forceinline__ Vec<T> ldv(const T* p) {
    Vec<T> v;
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    __builtin_memcpy(&v, &raw, 16);
    return v;
}
template <typename T> __device__ __forceinline__ void stv(T* p, const Vec<T>& v) {
    uint4 raw;
    __builtin_memcpy(&raw, &v, 16);
    *reinterpret_cast<uint4*>(p) = raw;
}

constexpr int WAVES_PER_BLOCK = 4;

struct NormArgs {
    const void *x, *dy, *c;
    void *y, *gx, *gdy;
    int64_t rows;
    int C;
    float eps;
};

// Per-row factors of the three rms_norm modes, from the row sums (already reduced over the wave).
template <typename A> struct NormRow {
    A r, r3c, sdx, scx, kx;
};
template <typename A, int MODE> __device__ __forceinline__ NormRow<A> norm_row(A sxx, A sdx, A scx, A scd, int C,
                                                                                 float eps) {
#pragma clang fp contract(off)
    NormRow<A> f;
    f.r = rsqrt_of<A>(sxx / (A)C + (A)eps);
    f.r3c = f.r * f.r * f.r / (A)C;
    f.sdx = sdx;
    f.scx = scx;
    f.kx = MODE == 2 ? -f.r3c * scd + (A)3 * f.r3c * f.r * f.r / (A)C * scx * sdx : (A)0;
    return f;
}

// mode 0: o0 = y; 1: o0 = dx; 2: o0 = gx, o1 = gdy.
template <typename T, typename A, int MODE>
__device__ __forceinline__ void norm_out(const NormRow<A>& f, A xv, A dv, A cv, T& o0, T& o1) {
#pragma clang fp contract(off)
    if constexpr (MODE == 0) o0 = narrow<T, A>(xv * f.r);
    if constexpr (MODE == 1) o0 = narrow<T, A>(f.r * dv - f.r3c * f.sdx * xv);
    if constexpr (MODE == 2) {
        o0 = narrow<T, A>(f.kx * xv - f.r3c * f.sdx * cv - f.r3c * f.scx * dv);
        o1 = narrow<T, A>(f.r * cv - f.r3c * f.scx * xv);
    }
}

// Any C and alignment: one wave per row, the row streamed twice (sums, then outputs).
template <typename T, int MODE> __global__ __launch_bounds__(64 * WAVES_PER_BLOCK) void k_rmsnorm(NormArgs a) {
#pragma clang fp contract(off)
    using A = typename Acc<T>::type;
    const int64_t row = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
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
    const NormRow<A> f = norm_row<A, MODE>(wave_sum(sxx), MODE >= 1 ? wave_sum(sdx) : (A)0,
                                           MODE == 2 ? wave_sum(scx) : (A)0, MODE == 2 ? wave_sum(scd) : (A)0, C,
                                           a.eps);
    T* o0 = reinterpret_cast<T*>(MODE == 2 ? a.gx : a.y) + row * C;
    T* o1 = MODE == 2 ? reinterpret_cast<T*>(a.gdy) + row * C : nullptr;
    for (int k = lane; k < C; k += 64) {
        T r0, r1;
        norm_out<T, A, MODE>(f, wide<T, A>(x[k]), MODE >= 1 ? wide<T, A>(dy[k]) : (A)0,
                             MODE == 2 ? wide<T, A>(c[k]) : (A)0, r0, r1);
        o0[k] = r0;
        if constexpr (MODE == 2) o1[k] = r1;
    }
}

// C a multiple of the 16-byte vector, 16-byte-aligned rows, C <= NV * 64 vectors: each wave owns RPW consecutive
// rows, issues every load of them before the first use (a row index past the end is clamped to the last row and a
// vector past C to the row's first, so no load is conditional; their values are masked out of the sums and never
// stored), and writes the outputs from registers. HBM traffic is the algorithmic bytes.
template <typename T, int MODE, int NV, int RPW>
__global__ __launch_bounds__(64 * WAVES_PER_BLOCK) void k_rmsnorm_vec(NormArgs a) {
#pragma clang fp contract(off)
    using A = typename Acc<T>::type;
    constexpr int VEC = Vec<T>::N;
    const int lane = threadIdx.x & 63;
    const int64_t row0 = ((int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6)) * RPW;
    if (row0 >= a.rows) return;  // wave-uniform
    const int C = a.C;
    const T* X = reinterpret_cast<const T*>(a.x);
    const T* DY = reinterpret_cast<const T*>(a.dy);
    const T* CC = reinterpret_cast<const T*>(a.c);
    Vec<T> xv[RPW][NV], dv[RPW][NV], cv[RPW][NV];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int64_t row = row0 + r < a.rows ? row0 + r : a.rows - 1;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int k = (v * 64 + lane) * VEC;
            const int64_t off = row * C + (k < C ? k : 0);
            xv[r][v] = ldv(X + off);
            if constexpr (MODE >= 1) dv[r][v] = ldv(DY + off);
            if constexpr (MODE == 2) cv[r][v] = ldv(CC + off);
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        A sxx = 0, sdx = 0, scx = 0, scd = 0;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            if ((v * 64 + lane) * VEC >= C) continue;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const A xe = wide<T, A>(xv[r][v].e[e]);
                sxx += xe * xe;
                if constexpr (MODE >= 1) sdx += wide<T, A>(dv[r][v].e[e]) * xe;
                if constexpr (MODE == 2) {
                    const A ce = wide<T, A>(cv[r][v].e[e]);
                    scx += ce * xe;
                    scd += ce * wide<T, A>(dv[r][v].e[e]);
                }
            }
        }
        const NormRow<A> f = norm_row<A, MODE>(wave_sum(sxx), MODE >= 1 ? wave_sum(sdx) : (A)0,
                                               MODE == 2 ? wave_sum(scx) : (A)0, MODE == 2 ? wave_sum(scd) : (A)0, C,
                                               a.eps);
        if (row0 + r >= a.rows) break;  // wave-uniform
        const int64_t base = (row0 + r) * C;
        T* O0 = reinterpret_cast<T*>(MODE == 2 ? a.gx : a.y) + base;
        T* O1 = MODE == 2 ? reinterpret_cast<T*>(a.gdy) + base : nullptr;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int k = (v * 64 + lane) * VEC;
            if (k >= C) continue;
            Vec<T> r0, r1;
#pragma unroll
            for (int e = 0; e < VEC; ++e)
                norm_out<T, A, MODE>(f, wide<T, A>(xv[r][v].e[e]), MODE >= 1 ? wide<T, A>(dv[r][v].e[e]) : (A)0,
                                     MODE == 2 ? wide<T, A>(cv[r][v].e[e]) : (A)0, r0.e[e], r1.e[e]);
            stv(O0 + k, r0);
            if constexpr (MODE == 2) stv(O1 + k, r1);
        }
    }
}

struct GluArgs {
    const void *gu, *dy, *c;
    void *y, *ggu, *gdy;
    int64_t n;  // rows
    int I;      // half width
};

template <typename A> __device__ __forceinline__ A sigmoid_of(A g) { return (A)1 / ((A)1 + exp(-g)); }

// One element of SwiGLU. mode 0: o0 = y = silu(g) u; 1: o0 = dg, o1 = du given dy; 2: o0 = gg, o1 = gu, o2 = gdy
// given dy and the cotangents (cg, cu) of (dg, du). The 16-bit roundings of modes 0 and 1 are where eager autograd
// rounds: silu is rounded before the product; dg = round(round(dy u) silu'), du = round(dy round(silu)).
template <typename T, typename A, int MODE>
__device__ __forceinline__ void glu_elem(A g, A u, A dy, A cg, A cu, T& o0, T& o1, T& o2) {
#pragma clang fp contract(off)
    const A s = sigmoid_of(g);
    const A silu = g * s;
    if constexpr (MODE == 0) {
        o0 = narrow<T, A>(wide<T, A>(narrow<T, A>(silu)) * u);
        return;
    }
    const A d1 = s * ((A)1 + g * ((A)1 - s));  // silu'
    if constexpr (MODE == 1) {
        o0 = narrow<T, A>(wide<T, A>(narrow<T, A>(dy * u)) * d1);
        o1 = narrow<T, A>(dy * wide<T, A>(narrow<T, A>(silu)));
        return;
    }
    const A d2 = s * ((A)1 - s) * ((A)2 + g * ((A)1 - (A)2 * s));  // silu''
    o0 = narrow<T, A>(cg * dy * u * d2 + cu * dy * d1);
    o1 = narrow<T, A>(cg * dy * d1);
    o2 = narrow<T, A>(cg * u * d1 + cu * silu);
}

// Any I and alignment: grid-stride over elements (row, j).
template <typename T, int MODE> __global__ __launch_bounds__(256) void k_swiglu(GluArgs a) {
    using A = typename Acc<T>::type;
    const int64_t total = a.n * a.I;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = e / a.I;
        const int j = (int)(e - row * a.I);
        const T* gu = reinterpret_cast<const T*>(a.gu) + row * 2 * a.I;
        const A dy = MODE >= 1 ? wide<T, A>(reinterpret_cast<const T*>(a.dy)[e]) : (A)0;
        const T* c = MODE == 2 ? reinterpret_cast<const T*>(a.c) + row * 2 * a.I : nullptr;
        T o0, o1, o2;
        glu_elem<T, A, MODE>(wide<T, A>(gu[j]), wide<T, A>(gu[a.I + j]), dy, MODE == 2 ? wide<T, A>(c[j]) : (A)0,
                             MODE == 2 ? wide<T, A>(c[a.I + j]) : (A)0, o0, o1, o2);
        if constexpr (MODE == 0) reinterpret_cast<T*>(a.y)[e] = o0;
        if constexpr (MODE == 1) {
            T* out = reinterpret_cast<T*>(a.y) + row * 2 * a.I;
            out[j] = o0;
            out[a.I + j] = o1;
        }
        if constexpr (MODE == 2) {
            T* out = reinterpret_cast<T*>(a.ggu) + row * 2 * a.I;
            out[j] = o0;
            out[a.I + j] = o1;
            reinterpret_cast<T*>(a.gdy)[e] = o2;
        }
    }
}

// I a multiple of the 16-byte vector and 16-byte-aligned tensors: grid-stride over vectors, each thread loading
// 16 bytes of gate and of up (and of dy and the cotangents) per step. IDX is the index type (32-bit when the
// vector count fits, which keeps the row division cheap).
template <typename T, int MODE, typename IDX> __global__ __launch_bounds__(256) void k_swiglu_vec(GluArgs a) {
    using A = typename Acc<T>::type;
    constexpr int VEC = Vec<T>::N;
    const IDX IV = (IDX)(a.I / VEC), total = (IDX)a.n * IV, I = (IDX)a.I;
    for (IDX v = (IDX)blockIdx.x * blockDim.x + threadIdx.x; v < total; v += (IDX)gridDim.x * blockDim.x) {
        const IDX row = v / IV;
        const IDX j = (v - row * IV) * VEC;
        const T* gu = reinterpret_cast<const T*>(a.gu) + (int64_t)row * 2 * I + j;
        const Vec<T> gv = ldv(gu), uv = ldv(gu + I);
        Vec<T> dyv, cgv, cuv, r0, r1, r2;
        if constexpr (MODE >= 1) dyv = ldv(reinterpret_cast<const T*>(a.dy) + (int64_t)v * VEC);
        if constexpr (MODE == 2) {
            const T* c = reinterpret_cast<const T*>(a.c) + (int64_t)row * 2 * I + j;
            cgv = ldv(c);
            cuv = ldv(c + I);
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e)
            glu_elem<T, A, MODE>(wide<T, A>(gv.e[e]), wide<T, A>(uv.e[e]), MODE >= 1 ? wide<T, A>(dyv.e[e]) : (A)0,
                                 MODE == 2 ? wide<T, A>(cgv.e[e]) : (A)0, MODE == 2 ? wide<T, A>(cuv.e[e]) : (A)0,
                                 r0.e[e], r1.e[e], r2.e[e]);
        if constexpr (MODE == 0) stv(reinterpret_cast<T*>(a.y) + (int64_t)v * VEC, r0);
        if constexpr (MODE >= 1) {
            T* out = reinterpret_cast<T*>(MODE == 1 ? a.y : a.ggu) + (int64_t)row * 2 * I + j;
            stv(out, r0);
            stv(out + I, r1);
        }
        if constexpr (MODE == 2) stv(reinterpret_cast<T*>(a.gdy) + (int64_t)v * VEC, r2);
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

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

constexpr int NORM_NV_MAX = 4;  // register-resident rows of up to 4 vectors per lane (2048 16-bit elements)

template <typename T, int MODE, int NV>
static void launch_norm_nv(hipStream_t s, const NormArgs& a) {
    constexpr int RPW = NV == 1 ? 4 : NV == 2 ? 2 : 1;
    const int64_t per_block = (int64_t)WAVES_PER_BLOCK * RPW;
    const dim3 grid((unsigned)((a.rows + per_block - 1) / per_block)), block(64 * WAVES_PER_BLOCK);
    hipLaunchKernelGGL((k_rmsnorm_vec<T, MODE, NV, RPW>), grid, block, 0, s, a);
}

template <typename T, int MODE> static void launch_norm_t(hipStream_t s, const NormArgs& a, bool vec_ok) {
    constexpr int VEC = 16 / (int)sizeof(T);
    const int nv = (a.C + 64 * VEC - 1) / (64 * VEC);
    if (vec_ok && a.C % VEC == 0 && nv <= NORM_NV_MAX) {
        if (nv == 1) launch_norm_nv<T, MODE, 1>(s, a);
        else if (nv == 2) launch_norm_nv<T, MODE, 2>(s, a);
        else if (nv == 3) launch_norm_nv<T, MODE, 3>(s, a);
        else launch_norm_nv<T, MODE, 4>(s, a);
        return;
    }
    const dim3 grid((unsigned)((a.rows + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK)), block(64 * WAVES_PER_BLOCK);
    hipLaunchKernelGGL((k_rmsnorm<T, MODE>), grid, block, 0, s, a);
}

template <int MODE> static void launch_norm(int dtype, hipStream_t s, const NormArgs& a) {
    const bool vec_ok = aligned16(a.x) && (MODE < 1 || aligned16(a.dy)) && (MODE < 2 || aligned16(a.c)) &&
                        (MODE == 2 ? aligned16(a.gx) && aligned16(a.gdy) : aligned16(a.y));
    if (dtype == EBR_DTYPE_F32) launch_norm_t<float, MODE>(s, a, vec_ok);
    else if (dtype == EBR_DTYPE_BF16) launch_norm_t<__bf16, MODE>(s, a, vec_ok);
    else if (dtype == EBR_DTYPE_F16) launch_norm_t<_Float16, MODE>(s, a, vec_ok);
    else launch_norm_t<double, MODE>(s, a, vec_ok);
}

constexpr int64_t GLU_MAX_BLOCKS = 8192;

template <typename T, int MODE> static void launch_glu_t(hipStream_t s, const GluArgs& a, bool vec_ok) {
    constexpr int VEC = 16 / (int)sizeof(T);
    if (vec_ok && a.I % VEC == 0) {
        const int64_t total = a.n * (a.I / VEC);
        const int64_t want = (total + 255) / 256;
        const dim3 grid((unsigned)(want < GLU_MAX_BLOCKS ? want : GLU_MAX_BLOCKS)), block(256);
        // 32-bit indices when every element offset (2 I per row) fits
        if (a.n * 2 * (int64_t)a.I < ((int64_t)1 << 31)) hipLaunchKernelGGL((k_swiglu_vec<T, MODE, uint32_t>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((k_swiglu_vec<T, MODE, int64_t>), grid, block, 0, s, a);
        return;
    }
    const int64_t want = (a.n * a.I + 255) / 256;
    const dim3 grid((unsigned)(want < 65536 ? want : 65536)), block(256);
    hipLaunchKernelGGL((k_swiglu<T, MODE>), grid, block, 0, s, a);
}

template <int MODE> static void launch_glu(int dtype, hipStream_t s, const GluArgs& a) {
    const bool vec_ok = aligned16(a.gu) && (MODE < 1 || aligned16(a.dy)) && (MODE < 2 || aligned16(a.c)) &&
                        (MODE == 2 ? aligned16(a.ggu) && aligned16(a.gdy) : aligned16(a.y));
    if (dtype == EBR_DTYPE_F32) launch_glu_t<float, MODE>(s, a, vec_ok);
    else if (dtype == EBR_DTYPE_BF16) launch_glu_t<__bf16, MODE>(s, a, vec_ok);
    else if (dtype == EBR_DTYPE_F16) launch_glu_t<_Float16, MODE>(s, a, vec_ok);
    else launch_glu_t<double, MODE>(s, a, vec_ok);
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
