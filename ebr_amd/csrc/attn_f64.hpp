// fp64 kernels of the three attention ops, for the reference's fp64 contract (reference reference.py:10-16: compute in
// fp64, lse in fp64; the Triton path takes fp64 for gradcheck shapes, triton_kernels.py:34-37). MI355X runs fp64 on
// the vector ALUs at the same peak as its fp64 matrix cores, so these are plain VALU kernels: exact fp64 arithmetic,
// any D in [1, 128], element-aligned strided inputs. They favour simplicity over speed (gradcheck shapes).
// Included inside namespace ebr by ebr_attn.hip.
//
// A workgroup of 256 threads owns F64_ROWS rows of one (b, h) slice and streams the other side through LDS in tiles
// of F64_TILE rows. Thread t pairs own row t / 16 with tile row t % 16 for the scores, and accumulates own row t / 16
// at d = t % 16 + 16 k for the D-wide outputs. Per-row sums over the 16 threads of a row use lane shuffles.
//   fwd:     two sweeps over the keys (row maximum and sum, then P V with P = exp(s - lse)).
//   bwd:     row kernel dQ (own = queries), col kernel dK, dV (own = keys); rowsum(dO o O) from the stored O.
//   bwd_bwd: a row-statistics sweep writes E = rowsum(P o G) and T = rowsum(P o Gp) of every query row into
//            element 0 of its hQ and hdO rows; the col kernel reads them for hK, hV; the row kernel then recomputes
//            them for its own rows and overwrites hQ, hdO with the results (the launches are stream-ordered).
// The formulas are the reference's dense closed forms (reference.py:32-91).

constexpr int F64_ROWS = 16;
constexpr int F64_TILE = 16;
constexpr int F64_THREADS = 256;
constexpr int F64_DMAX = DMAX_F64;
constexpr int F64_NACC = F64_DMAX / 16;  // D-wide accumulators per thread

// Rows [r0, r0 + 16) of a strided slice into LDS (pitch D); rows past L are 0.
__device__ __forceinline__ void f64_load_rows(double* dst, const double* slice, int64_t srow, int r0, int L, int D) {
    for (int e = threadIdx.x; e < 16 * D; e += F64_THREADS) {
        const int x = e / D, d = e - x * D;
        const int row = r0 + x;
        dst[e] = row < L ? slice[(int64_t)row * srow + d] : 0.0;
    }
}

__device__ __forceinline__ double f64_dot(const double* a, const double* b, int D) {
    double s = 0.0;
    for (int d = 0; d < D; ++d) s = fma(a[d], b[d], s);
    return s;
}

// Sum / max over the 16 consecutive lanes that share an own row.
__device__ __forceinline__ double f64_rowsum(double v) {
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, 16);
    return v;
}
__device__ __forceinline__ double f64_rowmax(double v) {
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) v = fmax(v, __shfl_xor(v, m, 16));
    return v;
}

// acc[k] (own row orow, d = dcol + 16 k) += sum_j W[orow][j] X[j][d]  (W row pitch 16, X pitch D); trans: W[j][orow].
template <bool TRANS>
__device__ __forceinline__ void f64_accum(double (&acc)[F64_NACC], const double* W, const double* X, int orow,
                                          int dcol, int D) {
#pragma unroll
    for (int k = 0; k < F64_NACC; ++k) {
        const int d = dcol + 16 * k;
        if (d < D) {
            double s = acc[k];
            for (int j = 0; j < F64_TILE; ++j) s = fma(TRANS ? W[j * 16 + orow] : W[orow * 16 + j], X[j * D + d], s);
            acc[k] = s;
        }
    }
}

__device__ __forceinline__ void f64_zero(double (&acc)[F64_NACC]) {
#pragma unroll
    for (int k = 0; k < F64_NACC; ++k) acc[k] = 0.0;
}

__device__ __forceinline__ void f64_store(void* out, int64_t row_base, int row, int L, const double (&acc)[F64_NACC],
                                          double mul, int dcol, int D) {
    if (row >= L) return;
    double* p = reinterpret_cast<double*>(out) + (row_base + row) * D;
#pragma unroll
    for (int k = 0; k < F64_NACC; ++k) {
        const int d = dcol + 16 * k;
        if (d < D) p[d] = acc[k] * mul;
    }
}

__device__ __forceinline__ const double* f64_slice(const Strided& t, int b, int h) {
    return reinterpret_cast<const double*>(t.p) + (int64_t)b * t.sb + (int64_t)h * t.sh;
}

// ---------------------------------------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(F64_THREADS) void k64_fwd(Args a) {
    __shared__ double Qo[16 * F64_DMAX], Kt[16 * F64_DMAX], Vt[16 * F64_DMAX], W[16 * 16];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, i0 = (blockIdx.x - bh * a.nblk) * F64_ROWS;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pi = threadIdx.x >> 4, pj = threadIdx.x & 15;
    const double sc = (double)a.scale;
    const double* Kg = f64_slice(a.k, b, h);
    const double* Vg = f64_slice(a.v, b, h);
    f64_load_rows(Qo, f64_slice(a.q, b, h), a.q.sl, i0, L, D);
    double m = -INFINITY, l = 0.0;
    for (int j0 = 0; j0 < L; j0 += F64_TILE) {
        __syncthreads();
        f64_load_rows(Kt, Kg, a.k.sl, j0, L, D);
        __syncthreads();
        const double s = j0 + pj < L ? f64_dot(Qo + pi * D, Kt + pj * D, D) * sc : -INFINITY;
        const double mn = fmax(m, f64_rowmax(s));  // the tile's first key is below L: finite
        l = l * exp(m - mn) + f64_rowsum(exp(s - mn));
        m = mn;
    }
    const double lse = m + log(l);
    double acc[F64_NACC];
    f64_zero(acc);
    for (int j0 = 0; j0 < L; j0 += F64_TILE) {
        __syncthreads();
        f64_load_rows(Kt, Kg, a.k.sl, j0, L, D);
        f64_load_rows(Vt, Vg, a.v.sl, j0, L, D);
        __syncthreads();
        W[pi * 16 + pj] = j0 + pj < L ? exp(f64_dot(Qo + pi * D, Kt + pj * D, D) * sc - lse) : 0.0;
        __syncthreads();
        f64_accum<false>(acc, W, Vt, pi, pj, D);
    }
    const int64_t rb = (int64_t)bh * L;
    f64_store(a.out0, rb, i0 + pi, L, acc, 1.0, pj, D);
    if (pj == 0 && i0 + pi < L) reinterpret_cast<double*>(a.lse_out)[rb + i0 + pi] = lse;
}

// ---------------------------------------------------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------------------------------------------------

__global__ __launch_bounds__(F64_THREADS) void k64_bwd_row(Args a) {
    __shared__ double Qo[16 * F64_DMAX], dOo[16 * F64_DMAX], Kt[16 * F64_DMAX], Vt[16 * F64_DMAX], W[16 * 16];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, i0 = (blockIdx.x - bh * a.nblk) * F64_ROWS;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pi = threadIdx.x >> 4, pj = threadIdx.x & 15;
    const double sc = (double)a.scale;
    const int64_t rb = (int64_t)bh * L;
    const int i = i0 + pi, ic = i < L ? i : L - 1;
    f64_load_rows(Qo, f64_slice(a.q, b, h), a.q.sl, i0, L, D);
    f64_load_rows(dOo, f64_slice(a.dO, b, h), a.dO.sl, i0, L, D);
    f64_load_rows(Kt, reinterpret_cast<const double*>(a.o) + rb * D, D, i0, L, D);  // O rows, for rowsum(dO o O)
    __syncthreads();
    const double Di = f64_dot(dOo + pi * D, Kt + pi * D, D);
    const double lse = reinterpret_cast<const double*>(a.lse)[rb + ic];
    const double* Kg = f64_slice(a.k, b, h);
    const double* Vg = f64_slice(a.v, b, h);
    double acc[F64_NACC];
    f64_zero(acc);
    for (int j0 = 0; j0 < L; j0 += F64_TILE) {
        __syncthreads();
        f64_load_rows(Kt, Kg, a.k.sl, j0, L, D);
        f64_load_rows(Vt, Vg, a.v.sl, j0, L, D);
        __syncthreads();
        double ds = 0.0;
        if (j0 + pj < L) {
            const double p = exp(f64_dot(Qo + pi * D, Kt + pj * D, D) * sc - lse);
            ds = p * (f64_dot(dOo + pi * D, Vt + pj * D, D) - Di);
        }
        W[pi * 16 + pj] = ds;
        __syncthreads();
        f64_accum<false>(acc, W, Kt, pi, pj, D);
    }
    f64_store(a.out0, rb, i, L, acc, sc, pj, D);
}

// Query-tile statistics of the col kernels: lse and rowsum(dO o O) of tile rows [i0, i0 + 16) (0 past L).
__device__ __forceinline__ void f64_tile_stats(double* lse_t, double* d_t, const Args& a, int64_t rb, int i0,
                                               const double* dOt, const double* Ot) {
    const int t = threadIdx.x;
    if (t < 16) {
        const int i = i0 + t;
        lse_t[t] = i < a.L ? reinterpret_cast<const double*>(a.lse)[rb + i] : 0.0;
        d_t[t] = f64_dot(dOt + t * a.D, Ot + t * a.D, a.D);
    }
}

__global__ __launch_bounds__(F64_THREADS) void k64_bwd_col(Args a) {
    __shared__ double Ko[16 * F64_DMAX], Vo[16 * F64_DMAX], Qt[16 * F64_DMAX], dOt[16 * F64_DMAX],
        Ot[16 * F64_DMAX], Wp[16 * 16], Wds[16 * 16], lse_t[16], d_t[16];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, j0 = (blockIdx.x - bh * a.nblk) * F64_ROWS;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pk = threadIdx.x >> 4, pq = threadIdx.x & 15;  // own key row, query tile row
    const double sc = (double)a.scale;
    const int64_t rb = (int64_t)bh * L;
    f64_load_rows(Ko, f64_slice(a.k, b, h), a.k.sl, j0, L, D);
    f64_load_rows(Vo, f64_slice(a.v, b, h), a.v.sl, j0, L, D);
    const double* Qg = f64_slice(a.q, b, h);
    const double* dOg = f64_slice(a.dO, b, h);
    const double* Og = reinterpret_cast<const double*>(a.o) + rb * D;
    double ak[F64_NACC], av[F64_NACC];
    f64_zero(ak);
    f64_zero(av);
    for (int i0 = 0; i0 < L; i0 += F64_TILE) {
        __syncthreads();
        f64_load_rows(Qt, Qg, a.q.sl, i0, L, D);
        f64_load_rows(dOt, dOg, a.dO.sl, i0, L, D);
        f64_load_rows(Ot, Og, D, i0, L, D);
        __syncthreads();
        f64_tile_stats(lse_t, d_t, a, rb, i0, dOt, Ot);
        __syncthreads();
        double p = 0.0, ds = 0.0;
        if (i0 + pq < L) {
            p = exp(f64_dot(Qt + pq * D, Ko + pk * D, D) * sc - lse_t[pq]);
            ds = p * (f64_dot(dOt + pq * D, Vo + pk * D, D) - d_t[pq]);
        }
        Wp[pq * 16 + pk] = p;
        Wds[pq * 16 + pk] = ds;
        __syncthreads();
        f64_accum<true>(ak, Wds, Qt, pk, pq, D);
        f64_accum<true>(av, Wp, dOt, pk, pq, D);
    }
    f64_store(a.out1, rb, j0 + pk, L, ak, sc, pq, D);
    f64_store(a.out2, rb, j0 + pk, L, av, 1.0, pq, D);
}

// ---------------------------------------------------------------------------------------------------------------------
// Backward of the backward (reference reference.py:61-91):
//   G = s (gQ K^T + Q gK^T), R = dO gV^T, dP = dO V^T, dS = P o (dP - D),
//   E = rowsum(P o G), A = P o (G - E), Gp = (dP - D) o G - E dP + R, T = rowsum(P o Gp), Gs = P o (Gp - T),
//   hQ = s (Gs K + dS gK), hK = s (Gs^T Q + dS^T gQ), hV = A^T dO, hdO = A V + P gV.
// T is formed as rowsum(P o (dP - D) o G) + rowsum(P o R) - E rowsum(P o dP), one sweep with E.
// ---------------------------------------------------------------------------------------------------------------------

struct F64Pair {  // the per-(query, key) values of one score
    double p, g, r, dp;
};

// STATS: write E, T of the own rows to element 0 of their hQ, hdO rows; else compute hQ, hdO.
template <bool STATS> __global__ __launch_bounds__(F64_THREADS) void k64_bb_row(Args a) {
    __shared__ double Qo[16 * F64_DMAX], gQo[16 * F64_DMAX], dOo[16 * F64_DMAX], Kt[16 * F64_DMAX],
        gKt[16 * F64_DMAX], Vt[16 * F64_DMAX], gVt[16 * F64_DMAX], Wgs[16 * 16], Wds[16 * 16], Wa[16 * 16],
        Wp[16 * 16];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, i0 = (blockIdx.x - bh * a.nblk) * F64_ROWS;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pi = threadIdx.x >> 4, pj = threadIdx.x & 15;
    const double sc = (double)a.scale;
    const int64_t rb = (int64_t)bh * L;
    const int i = i0 + pi, ic = i < L ? i : L - 1;
    f64_load_rows(Qo, f64_slice(a.q, b, h), a.q.sl, i0, L, D);
    f64_load_rows(gQo, f64_slice(a.gq, b, h), a.gq.sl, i0, L, D);
    f64_load_rows(dOo, f64_slice(a.dO, b, h), a.dO.sl, i0, L, D);
    f64_load_rows(Kt, reinterpret_cast<const double*>(a.o) + rb * D, D, i0, L, D);  // O rows
    __syncthreads();
    const double Di = f64_dot(dOo + pi * D, Kt + pi * D, D);
    const double lse = reinterpret_cast<const double*>(a.lse)[rb + ic];
    const double* Kg = f64_slice(a.k, b, h);
    const double* gKg = f64_slice(a.gk, b, h);
    const double* Vg = f64_slice(a.v, b, h);
    const double* gVg = f64_slice(a.gv, b, h);
    auto pair = [&](int j0) {
        F64Pair x = {0.0, 0.0, 0.0, 0.0};
        if (j0 + pj < L) {
            const double* qi = Qo + pi * D;
            x.p = exp(f64_dot(qi, Kt + pj * D, D) * sc - lse);
            x.g = (f64_dot(gQo + pi * D, Kt + pj * D, D) + f64_dot(qi, gKt + pj * D, D)) * sc;
            x.r = f64_dot(dOo + pi * D, gVt + pj * D, D);
            x.dp = f64_dot(dOo + pi * D, Vt + pj * D, D);
        }
        return x;
    };
    auto load_tiles = [&](int j0) {
        __syncthreads();
        f64_load_rows(Kt, Kg, a.k.sl, j0, L, D);
        f64_load_rows(gKt, gKg, a.gk.sl, j0, L, D);
        f64_load_rows(Vt, Vg, a.v.sl, j0, L, D);
        f64_load_rows(gVt, gVg, a.gv.sl, j0, L, D);
        __syncthreads();
    };
    double e = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    for (int j0 = 0; j0 < L; j0 += F64_TILE) {
        load_tiles(j0);
        const F64Pair x = pair(j0);
        e += x.p * x.g;
        s1 += x.p * (x.dp - Di) * x.g;
        s2 += x.p * x.r;
        s3 += x.p * x.dp;
    }
    e = f64_rowsum(e);
    const double T = f64_rowsum(s1) + f64_rowsum(s2) - e * f64_rowsum(s3);
    if constexpr (STATS) {
        if (pj == 0 && i < L) {
            reinterpret_cast<double*>(a.out0)[(rb + i) * D] = e;
            reinterpret_cast<double*>(a.out3)[(rb + i) * D] = T;
        }
        return;
    }
    double aq[F64_NACC], ad[F64_NACC];
    f64_zero(aq);
    f64_zero(ad);
    for (int j0 = 0; j0 < L; j0 += F64_TILE) {
        load_tiles(j0);
        const F64Pair x = pair(j0);
        const double ds = x.p * (x.dp - Di);
        const double gp = (x.dp - Di) * x.g - e * x.dp + x.r;
        Wgs[pi * 16 + pj] = x.p * (gp - T);
        Wds[pi * 16 + pj] = ds;
        Wa[pi * 16 + pj] = x.p * (x.g - e);
        Wp[pi * 16 + pj] = x.p;
        __syncthreads();
        f64_accum<false>(aq, Wgs, Kt, pi, pj, D);
        f64_accum<false>(aq, Wds, gKt, pi, pj, D);
        f64_accum<false>(ad, Wa, Vt, pi, pj, D);
        f64_accum<false>(ad, Wp, gVt, pi, pj, D);
    }
    f64_store(a.out0, rb, i, L, aq, sc, pj, D);
    f64_store(a.out3, rb, i, L, ad, 1.0, pj, D);
}

__global__ __launch_bounds__(F64_THREADS) void k64_bb_col(Args a) {
    __shared__ double Ko[16 * F64_DMAX], gKo[16 * F64_DMAX], Vo[16 * F64_DMAX], gVo[16 * F64_DMAX],
        Qt[16 * F64_DMAX], gQt[16 * F64_DMAX], dOt[16 * F64_DMAX], Ot[16 * F64_DMAX], Wgs[16 * 16], Wds[16 * 16],
        Wa[16 * 16], lse_t[16], d_t[16], e_t[16], t_t[16];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, j0 = (blockIdx.x - bh * a.nblk) * F64_ROWS;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pk = threadIdx.x >> 4, pq = threadIdx.x & 15;
    const double sc = (double)a.scale;
    const int64_t rb = (int64_t)bh * L;
    f64_load_rows(Ko, f64_slice(a.k, b, h), a.k.sl, j0, L, D);
    f64_load_rows(gKo, f64_slice(a.gk, b, h), a.gk.sl, j0, L, D);
    f64_load_rows(Vo, f64_slice(a.v, b, h), a.v.sl, j0, L, D);
    f64_load_rows(gVo, f64_slice(a.gv, b, h), a.gv.sl, j0, L, D);
    const double* Qg = f64_slice(a.q, b, h);
    const double* gQg = f64_slice(a.gq, b, h);
    const double* dOg = f64_slice(a.dO, b, h);
    const double* Og = reinterpret_cast<const double*>(a.o) + rb * D;
    const double* Eg = reinterpret_cast<const double*>(a.out0);  // E, T from k64_bb_row<true>
    const double* Tg = reinterpret_cast<const double*>(a.out3);
    double ak[F64_NACC], av[F64_NACC];
    f64_zero(ak);
    f64_zero(av);
    for (int i0 = 0; i0 < L; i0 += F64_TILE) {
        __syncthreads();
        f64_load_rows(Qt, Qg, a.q.sl, i0, L, D);
        f64_load_rows(gQt, gQg, a.gq.sl, i0, L, D);
        f64_load_rows(dOt, dOg, a.dO.sl, i0, L, D);
        f64_load_rows(Ot, Og, D, i0, L, D);
        __syncthreads();
        f64_tile_stats(lse_t, d_t, a, rb, i0, dOt, Ot);
        if (threadIdx.x < 16) {
            const int i = i0 + threadIdx.x;
            e_t[threadIdx.x] = i < L ? Eg[(rb + i) * D] : 0.0;
            t_t[threadIdx.x] = i < L ? Tg[(rb + i) * D] : 0.0;
        }
        __syncthreads();
        double gs = 0.0, ds = 0.0, av_w = 0.0;
        if (i0 + pq < L) {
            const double* qi = Qt + pq * D;
            const double p = exp(f64_dot(qi, Ko + pk * D, D) * sc - lse_t[pq]);
            const double g = (f64_dot(gQt + pq * D, Ko + pk * D, D) + f64_dot(qi, gKo + pk * D, D)) * sc;
            const double r = f64_dot(dOt + pq * D, gVo + pk * D, D);
            const double dp = f64_dot(dOt + pq * D, Vo + pk * D, D);
            const double Di = d_t[pq], E = e_t[pq];
            ds = p * (dp - Di);
            gs = p * (((dp - Di) * g - E * dp + r) - t_t[pq]);
            av_w = p * (g - E);
        }
        Wgs[pq * 16 + pk] = gs;
        Wds[pq * 16 + pk] = ds;
        Wa[pq * 16 + pk] = av_w;
        __syncthreads();
        f64_accum<true>(ak, Wgs, Qt, pk, pq, D);
        f64_accum<true>(ak, Wds, gQt, pk, pq, D);
        f64_accum<true>(av, Wa, dOt, pk, pq, D);
    }
    f64_store(a.out1, rb, j0 + pk, L, ak, sc, pq, D);
    f64_store(a.out2, rb, j0 + pk, L, av, 1.0, pq, D);
}

// Host launchers (grid: one workgroup per 16 own rows of each (b, h)).
static int f64_fwd(Args a, hipStream_t s) {
    a.nblk = (a.L + F64_ROWS - 1) / F64_ROWS;
    hipLaunchKernelGGL(k64_fwd, dim3((unsigned)((int64_t)a.B * a.H * a.nblk)), dim3(F64_THREADS), 0, s, a);
    return launch_rc();
}

static int f64_bwd(Args a, hipStream_t s) {
    a.nblk = (a.L + F64_ROWS - 1) / F64_ROWS;
    const dim3 grid((unsigned)((int64_t)a.B * a.H * a.nblk)), block(F64_THREADS);
    hipLaunchKernelGGL(k64_bwd_row, grid, block, 0, s, a);
    int rc = launch_rc();
    if (rc) return rc;
    hipLaunchKernelGGL(k64_bwd_col, grid, block, 0, s, a);
    return launch_rc();
}

static int f64_bwd_bwd(Args a, hipStream_t s) {
    a.nblk = (a.L + F64_ROWS - 1) / F64_ROWS;
    const dim3 grid((unsigned)((int64_t)a.B * a.H * a.nblk)), block(F64_THREADS);
    hipLaunchKernelGGL(k64_bb_row<true>, grid, block, 0, s, a);
    int rc = launch_rc();
    if (rc) return rc;
    hipLaunchKernelGGL(k64_bb_col, grid, block, 0, s, a);
    if ((rc = launch_rc())) return rc;
    hipLaunchKernelGGL(k64_bb_row<false>, grid, block, 0, s, a);
    return launch_rc();
}
