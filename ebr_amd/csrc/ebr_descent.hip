// Fused latent-descent wrapper for gfx950 (C ABI: include/ebr_descent.h): the pointwise passes around every descent
// microstep, z -> sphere(rms_norm(z) + noise - alpha dE/dz), and their gradients. All are HBM-bound.
//
// noisy point: one wave per token row of C elements (RMS over the last dim, wave reduction), a thread moving VW
//              consecutive elements per access.
// step/project: one workgroup per board row of N = L * C elements (the sphere's RMS is over the whole row): a first
//              pass forms u = v - round(alpha g) and its sum of squares (workgroup reduction through LDS), a second
//              pass recomputes u (its bytes come back from the cache) and writes u / rms; the backward does the same
//              with the sum of dout * y.
// Arithmetic is fp32 with contraction off; values the eager formula holds in the tensor dtype are rounded to it where
// it rounds them (reference models/layers.py:37-42, models/energy.py:219-241).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "../../include/ebr_descent.h"

namespace ebr_descent {

template <typename T, int VW> using Vec = T __attribute__((ext_vector_type(VW)));

template <typename T> __device__ __forceinline__ float f32(T x) { return (float)x; }
template <typename T> __device__ __forceinline__ T narrow(float x) { return (T)x; }

// An fp32 product kept opaque, so that narrowing it rounds twice (to fp32, then to T) as the eager formula does.
__device__ __forceinline__ float mul_f32(float a, float b) {
    float p = a * b;
    asm volatile("" : "+v"(p));
    return p;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

constexpr int TOK_WAVES = 4;   // token rows per workgroup of the noisy-point kernels (one wave each)
constexpr int ROW_THREADS = 1024;  // threads per board row of the step/project kernels
constexpr int STREAM_K = 4;       // vectors in flight per thread in the streaming step/project passes
constexpr int RES_MAX = 8;        // most vectors per thread a register-resident row takes

// Sum over the workgroup (ROW_THREADS threads); every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < ROW_THREADS / 64; ++i) t += red[i];
    __syncthreads();
    return t;
}

struct TokArgs {
    const void *z, *noise, *dv;
    const float* sigma;
    void* out;
    int B, L, C;
    float eps;
};

// 1 / sqrt(mean + eps), correctly rounded square root and division (as the eager rsqrt of fp32).
__device__ __forceinline__ float inv_rms(float sumsq, int C, float eps) { return 1.f / __builtin_sqrtf(sumsq / C + eps); }

template <typename T, int VW> __global__ __launch_bounds__(64 * TOK_WAVES) void k_noisy_point(TokArgs a) {
#pragma clang fp contract(off)
    const int tok = blockIdx.x * TOK_WAVES + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (tok >= a.B * a.L) return;  // wave-uniform
    using V = Vec<T, VW>;
    const int nc = a.C / VW;
    const T* zr = reinterpret_cast<const T*>(a.z) + (int64_t)tok * a.C;
    float ss = 0.f;
    for (int c = lane; c < nc; c += 64) {
        const V x = *reinterpret_cast<const V*>(zr + c * VW);
#pragma unroll
        for (int e = 0; e < VW; ++e) ss += f32(x[e]) * f32(x[e]);
    }
    const float r = inv_rms(wave_sum(ss), a.C, a.eps);
    const T* nr = a.noise ? reinterpret_cast<const T*>(a.noise) + (int64_t)tok * a.C : nullptr;
    const float sg = a.sigma ? a.sigma[tok / a.L] : 0.f;
    T* vr = reinterpret_cast<T*>(a.out) + (int64_t)tok * a.C;
    for (int c = lane; c < nc; c += 64) {
        const V x = *reinterpret_cast<const V*>(zr + c * VW);
        V y;
#pragma unroll
        for (int e = 0; e < VW; ++e) y[e] = narrow<T>(mul_f32(f32(x[e]), r));
        if (nr) {
            const V n = *reinterpret_cast<const V*>(nr + c * VW);
#pragma unroll
            for (int e = 0; e < VW; ++e) {
                const T add = a.sigma ? narrow<T>(mul_f32(f32(n[e]), sg)) : n[e];
                y[e] = narrow<T>(f32(y[e]) + f32(add));
            }
        }
        *reinterpret_cast<V*>(vr + c * VW) = y;
    }
}

// y = x r, r = (mean(x^2) + eps)^-1/2:  dx = r dy - x r^3 mean(dy x).
template <typename T, int VW> __global__ __launch_bounds__(64 * TOK_WAVES) void k_noisy_point_bwd(TokArgs a) {
#pragma clang fp contract(off)
    const int tok = blockIdx.x * TOK_WAVES + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (tok >= a.B * a.L) return;
    using V = Vec<T, VW>;
    const int nc = a.C / VW;
    const T* zr = reinterpret_cast<const T*>(a.z) + (int64_t)tok * a.C;
    const T* gr = reinterpret_cast<const T*>(a.dv) + (int64_t)tok * a.C;
    float ss = 0.f, sd = 0.f;
    for (int c = lane; c < nc; c += 64) {
        const V x = *reinterpret_cast<const V*>(zr + c * VW);
        const V g = *reinterpret_cast<const V*>(gr + c * VW);
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            ss += f32(x[e]) * f32(x[e]);
            sd += f32(g[e]) * f32(x[e]);
        }
    }
    ss = wave_sum(ss);
    sd = wave_sum(sd);
    const float r = inv_rms(ss, a.C, a.eps);
    const float k = r * r * r * (sd / a.C);
    T* dr = reinterpret_cast<T*>(a.out) + (int64_t)tok * a.C;
    for (int c = lane; c < nc; c += 64) {
        const V x = *reinterpret_cast<const V*>(zr + c * VW);
        const V g = *reinterpret_cast<const V*>(gr + c * VW);
        V o;
#pragma unroll
        for (int e = 0; e < VW; ++e) o[e] = narrow<T>(r * f32(g[e]) - f32(x[e]) * k);
        *reinterpret_cast<V*>(dr + c * VW) = o;
    }
}

struct RowArgs {
    const void *v, *g, *z, *dout;
    const float* alpha;
    const uint8_t* active;
    float* rms;
    void *out, *dv, *dg, *dz;
    int B;
    int64_t N;
    float eps;
};

// u = v - round(alpha g), in the dtype. The rounded 16-bit product is kept opaque too: without it the SLP vectoriser
// pairs the widened products into a vector the gfx950 backend cannot select with packed fp32 disabled.
template <typename T, int VW>
__device__ __forceinline__ void step_u(const Vec<T, VW>& v, const Vec<T, VW>& g, float al, float (&u)[VW]) {
#pragma unroll
    for (int e = 0; e < VW; ++e) {
        T q = narrow<T>(mul_f32(al, f32(g[e])));
        if constexpr (sizeof(T) == 2) asm volatile("" : "+v"(q));
        u[e] = f32(narrow<T>(f32(v[e]) - f32(q)));
    }
}

// KB vectors per thread at vector indices c0 + k ROW_THREADS. Indices past the row's end are clamped to its last
// vector (loaded, never used), so every load is unconditional and all KB are in flight before the first use.
template <typename V, int KB>
__device__ __forceinline__ void load_k(const V* row, int64_t c0, int64_t nc, V (&x)[KB]) {
#pragma unroll
    for (int k = 0; k < KB; ++k) x[k] = row[min(c0 + (int64_t)k * ROW_THREADS, nc - 1)];
}

// Step and projection of one board row per workgroup. KRES > 0: the row stays in registers (each thread holds KRES
// vectors, so a row of up to KRES * VW * ROW_THREADS elements is read once); KRES == 0: two streaming passes over the
// row, STREAM_K vectors in flight per thread (the second pass re-reads v and g, mostly from cache).
template <typename T, int VW, int KRES> __global__ __launch_bounds__(ROW_THREADS) void k_step_project(RowArgs a) {
#pragma clang fp contract(off)
    __shared__ float red[ROW_THREADS / 64];
    using V = Vec<T, VW>;
    constexpr int KB = KRES > 0 ? KRES : STREAM_K;
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t nc = a.N / VW;
    const int64_t base = (int64_t)b * a.N;
    const V* vr = reinterpret_cast<const V*>(reinterpret_cast<const T*>(a.v) + base);
    const V* gr = reinterpret_cast<const V*>(reinterpret_cast<const T*>(a.g) + base);
    V* orow = reinterpret_cast<V*>(reinterpret_cast<T*>(a.out) + base);
    const bool moves = a.active == nullptr || a.active[b] != 0;  // workgroup-uniform
    if (!moves) {
        const V* zr = reinterpret_cast<const V*>(reinterpret_cast<const T*>(a.z) + base);
        for (int64_t c = tid; c < nc; c += ROW_THREADS) orow[c] = zr[c];
        if (tid == 0) a.rms[b] = 1.f;
        return;
    }
    const float al = a.alpha[b];
    float ss = 0.f;
    float u[KB][VW];
    for (int64_t c0 = tid; c0 < (KRES > 0 ? tid + 1 : nc); c0 += (int64_t)KB * ROW_THREADS) {
        V xv[KB], xg[KB];
        load_k<V, KB>(vr, c0, nc, xv);
        load_k<V, KB>(gr, c0, nc, xg);
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            step_u<T, VW>(xv[k], xg[k], al, u[k]);
            if (c0 + (int64_t)k * ROW_THREADS < nc) {
#pragma unroll
                for (int e = 0; e < VW; ++e) ss += u[k][e] * u[k][e];
            }
        }
    }
    ss = block_sum(ss, red);
    const float r = fmaxf(__builtin_sqrtf(ss / (float)a.N), a.eps);
    if (tid == 0) a.rms[b] = r;
    for (int64_t c0 = tid; c0 < (KRES > 0 ? tid + 1 : nc); c0 += (int64_t)KB * ROW_THREADS) {
        if constexpr (KRES == 0) {
            V xv[KB], xg[KB];
            load_k<V, KB>(vr, c0, nc, xv);
            load_k<V, KB>(gr, c0, nc, xg);
#pragma unroll
            for (int k = 0; k < KB; ++k) step_u<T, VW>(xv[k], xg[k], al, u[k]);
        }
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const int64_t c = c0 + (int64_t)k * ROW_THREADS;
            if (c < nc) {
                V o;
#pragma unroll
                for (int e = 0; e < VW; ++e) o[e] = narrow<T>(u[k][e] / r);
                orow[c] = o;
            }
        }
    }
}

// y = u / r with r = max(sqrt(mean(u^2)), eps): du = dy / r - u sum(dy u) / (N r^3), the second term absent where the
// clamp holds. The eager formula reads u through two separate fp32 casts (one for the RMS, one for the division), so
// autograd rounds each term's gradient to the dtype before adding them in the dtype; so does this kernel.
// KRES as in k_step_project.
template <typename T, int VW, int KRES> __global__ __launch_bounds__(ROW_THREADS) void k_step_project_bwd(RowArgs a) {
#pragma clang fp contract(off)
    __shared__ float red[ROW_THREADS / 64];
    using V = Vec<T, VW>;
    constexpr int KB = KRES > 0 ? KRES : STREAM_K;
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t nc = a.N / VW;
    const int64_t base = (int64_t)b * a.N;
    const V* dyr = reinterpret_cast<const V*>(reinterpret_cast<const T*>(a.dout) + base);
    V* dvr = reinterpret_cast<V*>(reinterpret_cast<T*>(a.dv) + base);
    V* dgr = reinterpret_cast<V*>(reinterpret_cast<T*>(a.dg) + base);
    V* dzr = a.dz ? reinterpret_cast<V*>(reinterpret_cast<T*>(a.dz) + base) : nullptr;  // NULL only if every row moves
    const V zero = V(narrow<T>(0.f));
    const bool moves = a.active == nullptr || a.active[b] != 0;
    if (!moves) {
        for (int64_t c = tid; c < nc; c += ROW_THREADS) {
            dzr[c] = dyr[c];
            dvr[c] = zero;
            dgr[c] = zero;
        }
        return;
    }
    const V* vr = reinterpret_cast<const V*>(reinterpret_cast<const T*>(a.v) + base);
    const V* gr = reinterpret_cast<const V*>(reinterpret_cast<const T*>(a.g) + base);
    const float al = a.alpha[b];
    const float r = a.rms[b];
    const bool clamped = !(r > a.eps);  // workgroup-uniform
    float u[KB][VW];
    V dy[KB];
    float k2 = 0.f;  // du's second term is k2 u
    if (!clamped) {
        float sd = 0.f;
        for (int64_t c0 = tid; c0 < (KRES > 0 ? tid + 1 : nc); c0 += (int64_t)KB * ROW_THREADS) {
            V xv[KB], xg[KB];
            load_k<V, KB>(vr, c0, nc, xv);
            load_k<V, KB>(gr, c0, nc, xg);
            load_k<V, KB>(dyr, c0, nc, dy);
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                step_u<T, VW>(xv[k], xg[k], al, u[k]);
                if (c0 + (int64_t)k * ROW_THREADS < nc) {
#pragma unroll
                    for (int e = 0; e < VW; ++e) sd += f32(dy[k][e]) * u[k][e];
                }
            }
        }
        k2 = -(block_sum(sd, red) / (r * r)) / (2.f * r) / (float)a.N * 2.f;
    }
    for (int64_t c0 = tid; c0 < (KRES > 0 ? tid + 1 : nc); c0 += (int64_t)KB * ROW_THREADS) {
        if (KRES == 0 || clamped) {
            load_k<V, KB>(dyr, c0, nc, dy);
            if (!clamped) {
                V xv[KB], xg[KB];
                load_k<V, KB>(vr, c0, nc, xv);
                load_k<V, KB>(gr, c0, nc, xg);
#pragma unroll
                for (int k = 0; k < KB; ++k) step_u<T, VW>(xv[k], xg[k], al, u[k]);
            }
        }
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const int64_t c = c0 + (int64_t)k * ROW_THREADS;
            if (c < nc) {
                V dvv, dgv;
#pragma unroll
                for (int e = 0; e < VW; ++e) {
                    const float t1 = f32(narrow<T>(f32(dy[k][e]) / r));
                    const T dut = clamped ? narrow<T>(t1) : narrow<T>(t1 + f32(narrow<T>(mul_f32(k2, u[k][e]))));
                    dvv[e] = dut;
                    dgv[e] = narrow<T>(mul_f32(-f32(dut), al));
                }
                dvr[c] = dvv;
                dgr[c] = dgv;
                if (dzr) dzr[c] = zero;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------------------------------

static int rc_launch() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? EBR_OK : EBR_ERR_HIP_BASE + (int)e;
}

static bool aligned(const void* p, int bytes) { return p == nullptr || ((uintptr_t)p % (uintptr_t)bytes) == 0; }

// Widest access (elements, at most 16 bytes) dividing ``len`` with every pointer aligned to it.
static int pick_vw(int es, int64_t len, std::initializer_list<const void*> ptrs) {
    for (int vw = 16 / es; vw > 1; vw >>= 1) {
        if (len % vw) continue;
        bool ok = true;
        for (const void* p : ptrs) ok = ok && aligned(p, vw * es);
        if (ok) return vw;
    }
    return 1;
}

static int check(int dtype, int B, int64_t n) {
    if (dtype != EBR_DTYPE_F32 && dtype != EBR_DTYPE_BF16 && dtype != EBR_DTYPE_F16) return EBR_ERR_DTYPE;
    if (B < 1 || n < 1 || (int64_t)B * n >= ((int64_t)1 << 40)) return EBR_ERR_SHAPE;
    return EBR_OK;
}

#define EBR_DESCENT_DISPATCH(KERNEL, GRID, BLOCK, ARGS)                                                             \
    do {                                                                                                             \
        hipStream_t s_ = reinterpret_cast<hipStream_t>(stream);                                                      \
        if (dtype == EBR_DTYPE_F32) {                                                                                \
            if (vw == 4) hipLaunchKernelGGL((KERNEL<float, 4>), GRID, BLOCK, 0, s_, ARGS);                          \
            else if (vw == 2) hipLaunchKernelGGL((KERNEL<float, 2>), GRID, BLOCK, 0, s_, ARGS);                     \
            else hipLaunchKernelGGL((KERNEL<float, 1>), GRID, BLOCK, 0, s_, ARGS);                                  \
        } else if (dtype == EBR_DTYPE_BF16) {                                                                        \
            if (vw == 8) hipLaunchKernelGGL((KERNEL<__bf16, 8>), GRID, BLOCK, 0, s_, ARGS);                         \
            else if (vw == 4) hipLaunchKernelGGL((KERNEL<__bf16, 4>), GRID, BLOCK, 0, s_, ARGS);                    \
            else if (vw == 2) hipLaunchKernelGGL((KERNEL<__bf16, 2>), GRID, BLOCK, 0, s_, ARGS);                    \
            else hipLaunchKernelGGL((KERNEL<__bf16, 1>), GRID, BLOCK, 0, s_, ARGS);                                 \
        } else {                                                                                                     \
            if (vw == 8) hipLaunchKernelGGL((KERNEL<_Float16, 8>), GRID, BLOCK, 0, s_, ARGS);                       \
            else if (vw == 4) hipLaunchKernelGGL((KERNEL<_Float16, 4>), GRID, BLOCK, 0, s_, ARGS);                  \
            else if (vw == 2) hipLaunchKernelGGL((KERNEL<_Float16, 2>), GRID, BLOCK, 0, s_, ARGS);                  \
            else hipLaunchKernelGGL((KERNEL<_Float16, 1>), GRID, BLOCK, 0, s_, ARGS);                               \
        }                                                                                                            \
    } while (0)

// Launchers of the row kernels, so that one dispatch picks dtype, vector width and register residency for both.
template <typename T, int VW, int KRES> struct StepFwd {
    static constexpr int KMAX = RES_MAX;
    static void launch(unsigned rows, hipStream_t s, const RowArgs& a) {
        hipLaunchKernelGGL((k_step_project<T, VW, KRES>), dim3(rows), dim3(ROW_THREADS), 0, s, a);
    }
};
template <typename T, int VW, int KRES> struct StepBwd {
    static constexpr int KMAX = 6;  // the row plus dout in registers: 8 vectors per thread would spill
    static void launch(unsigned rows, hipStream_t s, const RowArgs& a) {
        hipLaunchKernelGGL((k_step_project_bwd<T, VW, KRES>), dim3(rows), dim3(ROW_THREADS), 0, s, a);
    }
};

// Vectors per thread a register-resident row takes (1, 2, 4, 6 or 8, at most kmax), or 0 when the row is streamed:
// residency is used at the full 16-byte width only.
static int pick_kres(int vw, int es, int64_t N, int kmax) {
    if (vw * es != 16) return 0;
    const int64_t need = (N / vw + ROW_THREADS - 1) / ROW_THREADS;
    for (int k : {1, 2, 4, 6, RES_MAX})
        if (need <= k && k <= kmax) return k;
    return 0;
}

template <template <typename, int, int> class L, typename T>
static void launch_rows(int vw, int kres, unsigned rows, hipStream_t s, const RowArgs& a) {
    constexpr int W = 16 / (int)sizeof(T);
    if (vw == W) {
        switch (kres) {
            case 1: L<T, W, 1>::launch(rows, s, a); return;
            case 2: L<T, W, 2>::launch(rows, s, a); return;
            case 4: L<T, W, 4>::launch(rows, s, a); return;
            case 6: L<T, W, 6>::launch(rows, s, a); return;
            default: break;
        }
        if constexpr (L<T, W, 0>::KMAX >= RES_MAX) {
            if (kres == RES_MAX) {
                L<T, W, RES_MAX>::launch(rows, s, a);
                return;
            }
        }
        L<T, W, 0>::launch(rows, s, a);
        return;
    }
    if constexpr (W >= 8) {
        if (vw == 4) {
            L<T, 4, 0>::launch(rows, s, a);
            return;
        }
    }
    if (vw == 2) L<T, 2, 0>::launch(rows, s, a);
    else L<T, 1, 0>::launch(rows, s, a);
}

template <template <typename, int, int> class L>
static void launch_rows_dtype(int dtype, int vw, int64_t N, unsigned rows, void* stream, const RowArgs& a) {
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    constexpr int kmax = L<float, 4, 0>::KMAX;
    if (dtype == EBR_DTYPE_F32) launch_rows<L, float>(vw, pick_kres(vw, 4, N, kmax), rows, s, a);
    else if (dtype == EBR_DTYPE_BF16) launch_rows<L, __bf16>(vw, pick_kres(vw, 2, N, kmax), rows, s, a);
    else launch_rows<L, _Float16>(vw, pick_kres(vw, 2, N, kmax), rows, s, a);
}

}  // namespace ebr_descent

using namespace ebr_descent;

extern "C" {

int ebr_descent_noisy_point(int dtype, int B, int L, int C, float eps, const void* z, const void* noise,
                            const float* sigma, void* v, void* stream) {
    int rc = check(dtype, B, (int64_t)L * C);
    if (rc) return rc;
    if (L < 1 || C < 1) return EBR_ERR_SHAPE;
    if (!z || !v || (sigma && !noise)) return EBR_ERR_NULL;
    const int es = dtype == EBR_DTYPE_F32 ? 4 : 2;
    TokArgs a = {z, noise, nullptr, sigma, v, B, L, C, eps};
    const int vw = pick_vw(es, C, {z, noise, v});
    const dim3 grid((unsigned)(((int64_t)B * L + TOK_WAVES - 1) / TOK_WAVES)), block(64 * TOK_WAVES);
    EBR_DESCENT_DISPATCH(k_noisy_point, grid, block, a);
    return rc_launch();
}

int ebr_descent_noisy_point_bwd(int dtype, int B, int L, int C, float eps, const void* z, const void* dv, void* dz,
                                void* stream) {
    int rc = check(dtype, B, (int64_t)L * C);
    if (rc) return rc;
    if (L < 1 || C < 1) return EBR_ERR_SHAPE;
    if (!z || !dv || !dz) return EBR_ERR_NULL;
    const int es = dtype == EBR_DTYPE_F32 ? 4 : 2;
    TokArgs a = {z, nullptr, dv, nullptr, dz, B, L, C, eps};
    const int vw = pick_vw(es, C, {z, dv, dz});
    const dim3 grid((unsigned)(((int64_t)B * L + TOK_WAVES - 1) / TOK_WAVES)), block(64 * TOK_WAVES);
    EBR_DESCENT_DISPATCH(k_noisy_point_bwd, grid, block, a);
    return rc_launch();
}

int ebr_descent_step_project(int dtype, int B, int64_t N, float eps, const void* v, const void* g,
                             const float* alpha, const void* z, const uint8_t* active, void* out, float* rms,
                             void* stream) {
    int rc = check(dtype, B, N);
    if (rc) return rc;
    if (!v || !g || !alpha || !out || !rms || (active && !z)) return EBR_ERR_NULL;
    const int es = dtype == EBR_DTYPE_F32 ? 4 : 2;
    RowArgs a = {};
    a.v = v;
    a.g = g;
    a.z = z;
    a.alpha = alpha;
    a.active = active;
    a.rms = rms;
    a.out = out;
    a.B = B;
    a.N = N;
    a.eps = eps;
    const int vw = pick_vw(es, N, {v, g, z, out});
    launch_rows_dtype<StepFwd>(dtype, vw, N, (unsigned)B, stream, a);
    return rc_launch();
}

int ebr_descent_step_project_bwd(int dtype, int B, int64_t N, float eps, const void* v, const void* g,
                                 const float* alpha, const uint8_t* active, const float* rms, const void* dout,
                                 void* dv, void* dg, void* dz, void* stream) {
    int rc = check(dtype, B, N);
    if (rc) return rc;
    if (!v || !g || !alpha || !rms || !dout || !dv || !dg || (active && !dz)) return EBR_ERR_NULL;
    const int es = dtype == EBR_DTYPE_F32 ? 4 : 2;
    RowArgs a = {};
    a.v = v;
    a.g = g;
    a.alpha = alpha;
    a.active = active;
    a.rms = const_cast<float*>(rms);
    a.dout = dout;
    a.dv = dv;
    a.dg = dg;
    a.dz = dz;
    a.B = B;
    a.N = N;
    a.eps = eps;
    const int vw = pick_vw(es, N, {v, g, dout, dv, dg, dz});
    launch_rows_dtype<StepBwd>(dtype, vw, N, (unsigned)B, stream, a);
    return rc_launch();
}

}  // extern "C"
