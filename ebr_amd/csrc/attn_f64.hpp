// fp64 kernels of the three attention ops, for the reference's fp64 contract (reference reference.py:10-16: compute in
// fp64, lse in fp64; the Triton path takes fp64 for gradcheck shapes, triton_kernels.py:34-37). MI355X runs fp64 on
// the vector ALUs at the same peak as its fp64 matrix cores, so these are plain VALU kernels: exact fp64 arithmetic,
// any D in [1, 256], element-aligned strided inputs. They favour simplicity over speed (gradcheck shapes).
// Included inside namespace ebr by ebr_attn.hip.
//
// A workgroup of R x R threads owns R rows of one (b, h) slice and streams the other side through LDS in tiles of R
// rows: R = 16 (256 threads) for D <= 128, R = 8 (64 threads) for D <= 256, so that the eight [R, D] LDS arrays of
// the col kernel of the backward of the backward stay within 128 KB. Thread t pairs own row t / R with tile row
// t % R for the scores, and accumulates own row t / R at d = t % R + R k for the D-wide outputs. Per-row sums over
// the R threads of a row use lane shuffles.
//   fwd:     two sweeps over the keys (row maximum and sum, then P V with P = exp(s - lse)).
//   bwd:     row kernel dQ (own = queries), col kernel dK, dV (own = keys); rowsum(dO o O) from the stored O.
//   bwd_bwd: a row-statistics sweep writes E = rowsum(P o G) and T = rowsum(P o Gp) of every query row into
//            element 0 of its hQ and hdO rows; the col kernel reads them for hK, hV; the row kernel then recomputes
//            them for its own rows and overwrites hQ, hdO with the results (the launches are stream-ordered).
// The formulas are the reference's dense closed forms (reference.py:32-91).

// Tile rows R and widest D of one instantiation.
template <int R_, int DM_> struct F64Cfg {
    static constexpr int R = R_, DM = DM_, THREADS = R * R, NACC = DM / R;
    static_assert((R & (R - 1)) == 0 && R <= 16 && DM % R == 0, "R a power of two, D range a multiple of R");
};
using F64Narrow = F64Cfg<16, 128>;
using F64Wide = F64Cfg<8, DMAX_F64>;

// Rows [r0, r0 + R) of a strided slice into LDS (pitch D); rows past L are 0.
template <class C>
__device__ __forceinline__ void f64_load_rows(double* dst, const double* slice, int64_t srow, int r0, int L, int D) {
    for (int e = threadIdx.x; e < C::R * D; e += C::THREADS) {
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

// Sum / max over the R consecutive lanes that share an own row.
template <class C> __device__ __forceinline__ double f64_rowsum(double v) {
#pragma unroll
    for (int m = C::R / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, C::R);
    return v;
}
template <class C> __device__ __forceinline__ double f64_rowmax(double v) {
#pragma unroll
    for (int m = C::R / 2; m >= 1; m >>= 1) v = fmax(v, __shfl_xor(v, m, C::R));
    return v;
}

// acc[k] (own row orow, d = dcol + R k) += sum_j W[orow][j] X[j][d]  (W row pitch R, X pitch D); trans: W[j][orow].
template <class C, bool TRANS>
__device__ __forceinline__ void f64_accum(double (&acc)[C::NACC], const double* W, const double* X, int orow,
                                          int dcol, int D) {
#pragma unroll
    for (int k = 0; k < C::NACC; ++k) {
        const int d = dcol + C::R * k;
        if (d < D) {
            double s = acc[k];
            for (int j = 0; j < C::R; ++j) s = fma(TRANS ? W[j * C::R + orow] : W[orow * C::R + j], X[j * D + d], s);
            acc[k] = s;
        }
    }
}

template <class C> __device__ __forceinline__ void f64_zero(double (&acc)[C::NACC]) {
#pragma unroll
    for (int k = 0; k < C::NACC; ++k) acc[k] = 0.0;
}

template <class C>
__device__ __forceinline__ void f64_store(void* out, int64_t row_base, int row, int L, const double (&acc)[C::NACC],
                                          double mul, int dcol, int D) {
    if (row >= L) return;
    double* p = reinterpret_cast<double*>(out) + (row_base + row) * D;
#pragma unroll
    for (int k = 0; k < C::NACC; ++k) {
        const int d = dcol + C::R * k;
        if (d < D) p[d] = acc[k] * mul;
    }
}

__device__ __forceinline__ const double* f64_slice(const Strided& t, int b, int h) {
    return reinterpret_cast<const double*>(t.p) + (int64_t)b * t.sb + (int64_t)h * t.sh;
}

// ---------------------------------------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------------------------------------

template <class C> __global__ __launch_bounds__(C::THREADS) void k64_fwd(Args a) {
    __shared__ double Qo[C::R * C::DM], Kt[C::R * C::DM], Vt[C::R * C::DM], W[C::R * C::R];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, i0 = (blockIdx.x - bh * a.nblk) * C::R;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pi = threadIdx.x / C::R, pj = threadIdx.x % C::R;
    const double sc = (double)a.scale;
    const double* Kg = f64_slice(a.k, b, h);
    const double* Vg = f64_slice(a.v, b, h);
    f64_load_rows<C>(Qo, f64_slice(a.q, b, h), a.q.sl, i0, L, D);
    double m = -INFINITY, l = 0.0;
    for (int j0 = 0; j0 < L; j0 += C::R) {
        __syncthreads();
        f64_load_rows<C>(Kt, Kg, a.k.sl, j0, L, D);
        __syncthreads();
        const double s = j0 + pj < L ? f64_dot(Qo + pi * D, Kt + pj * D, D) * sc : -INFINITY;
        const double mn = fmax(m, f64_rowmax<C>(s));  // the tile's first key is below L: finite
        l = l * exp(m - mn) + f64_rowsum<C>(exp(s - mn));
        m = mn;
    }
    const double lse = m + log(l);
    double acc[C::NACC];
    f64_zero<C>(acc);
    for (int j0 = 0; j0 < L; j0 += C::R) {
        __syncthreads();
        f64_load_rows<C>(Kt, Kg, a.k.sl, j0, L, D);
        f64_load_rows<C>(Vt, Vg, a.v.sl, j0, L, D);
        __syncthreads();
        W[pi * C::R + pj] = j0 + pj < L ? exp(f64_dot(Qo + pi * D, Kt + pj * D, D) * sc - lse) : 0.0;
        __syncthreads();
        f64_accum<C, false>(acc, W, Vt, pi, pj, D);
    }
    const int64_t rb = (int64_t)bh * L;
    f64_store<C>(a.out0, rb, i0 + pi, L, acc, 1.0, pj, D);
    if (pj == 0 && i0 + pi < L) reinterpret_cast<double*>(a.lse_out)[rb + i0 + pi] = lse;
}

// ---------------------------------------------------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------------------------------------------------

template <class C> __global__ __launch_bounds__(C::THREADS) void k64_bwd_row(Args a) {
    __shared__ double Qo[C::R * C::DM], dOo[C::R * C::DM], Kt[C::R * C::DM], Vt[C::R * C::DM], W[C::R * C::R];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, i0 = (blockIdx.x - bh * a.nblk) * C::R;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pi = threadIdx.x / C::R, pj = threadIdx.x % C::R;
    const double sc = (double)a.scale;
    const int64_t rb = (int64_t)bh * L;
    const int i = i0 + pi, ic = i < L ? i : L - 1;
    f64_load_rows<C>(Qo, f64_slice(a.q, b, h), a.q.sl, i0, L, D);
    f64_load_rows<C>(dOo, f64_slice(a.dO, b, h), a.dO.sl, i0, L, D);
    f64_load_rows<C>(Kt, reinterpret_cast<const double*>(a.o) + rb * D, D, i0, L, D);  // O rows, for rowsum(dO o O)
    __syncthreads();
    const double Di = f64_dot(dOo + pi * D, Kt + pi * D, D);
    const double lse = reinterpret_cast<const double*>(a.lse)[rb + ic];
    const double* Kg = f64_slice(a.k, b, h);
    const double* Vg = f64_slice(a.v, b, h);
    double acc[C::NACC];
    f64_zero<C>(acc);
    for (int j0 = 0; j0 < L; j0 += C::R) {
        __syncthreads();
        f64_load_rows<C>(Kt, Kg, a.k.sl, j0, L, D);
        f64_load_rows<C>(Vt, Vg, a.v.sl, j0, L, D);
        __syncthreads();
        double ds = 0.0;
        if (j0 + pj < L) {
            const double p = exp(f64_dot(Qo + pi * D, Kt + pj * D, D) * sc - lse);
            ds = p * (f64_dot(dOo + pi * D, Vt + pj * D, D) - Di);
        }
        W[pi * C::R + pj] = ds;
        __syncthreads();
        f64_accum<C, false>(acc, W, Kt, pi, pj, D);
    }
    f64_store<C>(a.out0, rb, i, L, acc, sc, pj, D);
}

// Query-tile statistics of the col kernels: lse and rowsum(dO o O) of tile rows [i0, i0 + R) (0 past L).
template <class C>
__device__ __forceinline__ void f64_tile_stats(double* lse_t, double* d_t, const Args& a, int64_t rb, int i0,
                                               const double* dOt, const double* Ot) {
    const int t = threadIdx.x;
    if (t < C::R) {
        const int i = i0 + t;
        lse_t[t] = i < a.L ? reinterpret_cast<const double*>(a.lse)[rb + i] : 0.0;
        d_t[t] = f64_dot(dOt + t * a.D, Ot + t * a.D, a.D);
    }
}

template <class C> __global__ __launch_bounds__(C::THREADS) void k64_bwd_col(Args a) {
    __shared__ double Ko[C::R * C::DM], Vo[C::R * C::DM], Qt[C::R * C::DM], dOt[C::R * C::DM],
        Ot[C::R * C::DM], Wp[C::R * C::R], Wds[C::R * C::R], lse_t[C::R], d_t[C::R];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, j0 = (blockIdx.x - bh * a.nblk) * C::R;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pk = threadIdx.x / C::R, pq = threadIdx.x % C::R;  // own key row, query tile row
    const double sc = (double)a.scale;
    const int64_t rb = (int64_t)bh * L;
    f64_load_rows<C>(Ko, f64_slice(a.k, b, h), a.k.sl, j0, L, D);
    f64_load_rows<C>(Vo, f64_slice(a.v, b, h), a.v.sl, j0, L, D);
    const double* Qg = f64_slice(a.q, b, h);
    const double* dOg = f64_slice(a.dO, b, h);
    const double* Og = reinterpret_cast<const double*>(a.o) + rb * D;
    double ak[C::NACC], av[C::NACC];
    f64_zero<C>(ak);
    f64_zero<C>(av);
    for (int i0 = 0; i0 < L; i0 += C::R) {
        __syncthreads();
        f64_load_rows<C>(Qt, Qg, a.q.sl, i0, L, D);
        f64_load_rows<C>(dOt, dOg, a.dO.sl, i0, L, D);
        f64_load_rows<C>(Ot, Og, D, i0, L, D);
        __syncthreads();
        f64_tile_stats<C>(lse_t, d_t, a, rb, i0, dOt, Ot);
        __syncthreads();
        double p = 0.0, ds = 0.0;
        if (i0 + pq < L) {
            p = exp(f64_dot(Qt + pq * D, Ko + pk * D, D) * sc - lse_t[pq]);
            ds = p * (f64_dot(dOt + pq * D, Vo + pk * D, D) - d_t[pq]);
        }
        Wp[pq * C::R + pk] = p;
        Wds[pq * C::R + pk] = ds;
        __syncthreads();
        f64_accum<C, true>(ak, Wds, Qt, pk, pq, D);
        f64_accum<C, true>(av, Wp, dOt, pk, pq, D);
    }
    f64_store<C>(a.out1, rb, j0 + pk, L, ak, sc, pq, D);
    f64_store<C>(a.out2, rb, j0 + pk, L, av, 1.0, pq, D);
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
template <class C, bool STATS> __global__ __launch_bounds__(C::THREADS) void k64_bb_row(Args a) {
    __shared__ double Qo[C::R * C::DM], gQo[C::R * C::DM], dOo[C::R * C::DM], Kt[C::R * C::DM],
        gKt[C::R * C::DM], Vt[C::R * C::DM], gVt[C::R * C::DM], Wgs[C::R * C::R], Wds[C::R * C::R], Wa[C::R * C::R],
        Wp[C::R * C::R];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, i0 = (blockIdx.x - bh * a.nblk) * C::R;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pi = threadIdx.x / C::R, pj = threadIdx.x % C::R;
    const double sc = (double)a.scale;
    const int64_t rb = (int64_t)bh * L;
    const int i = i0 + pi, ic = i < L ? i : L - 1;
    f64_load_rows<C>(Qo, f64_slice(a.q, b, h), a.q.sl, i0, L, D);
    f64_load_rows<C>(gQo, f64_slice(a.gq, b, h), a.gq.sl, i0, L, D);
    f64_load_rows<C>(dOo, f64_slice(a.dO, b, h), a.dO.sl, i0, L, D);
    f64_load_rows<C>(Kt, reinterpret_cast<const double*>(a.o) + rb * D, D, i0, L, D);  // O rows
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
        f64_load_rows<C>(Kt, Kg, a.k.sl, j0, L, D);
        f64_load_rows<C>(gKt, gKg, a.gk.sl, j0, L, D);
        f64_load_rows<C>(Vt, Vg, a.v.sl, j0, L, D);
        f64_load_rows<C>(gVt, gVg, a.gv.sl, j0, L, D);
        __syncthreads();
    };
    double e = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    for (int j0 = 0; j0 < L; j0 += C::R) {
        load_tiles(j0);
        const F64Pair x = pair(j0);
        e += x.p * x.g;
        s1 += x.p * (x.dp - Di) * x.g;
        s2 += x.p * x.r;
        s3 += x.p * x.dp;
    }
    e = f64_rowsum<C>(e);
    const double T = f64_rowsum<C>(s1) + f64_rowsum<C>(s2) - e * f64_rowsum<C>(s3);
    if constexpr (STATS) {
        if (pj == 0 && i < L) {
            reinterpret_cast<double*>(a.out0)[(rb + i) * D] = e;
            reinterpret_cast<double*>(a.out3)[(rb + i) * D] = T;
        }
        return;
    }
    double aq[C::NACC], ad[C::NACC];
    f64_zero<C>(aq);
    f64_zero<C>(ad);
    for (int j0 = 0; j0 < L; j0 += C::R) {
        load_tiles(j0);
        const F64Pair x = pair(j0);
        const double ds = x.p * (x.dp - Di);
        const double gp = (x.dp - Di) * x.g - e * x.dp + x.r;
        Wgs[pi * C::R + pj] = x.p * (gp - T);
        Wds[pi * C::R + pj] = ds;
        Wa[pi * C::R + pj] = x.p * (x.g - e);
        Wp[pi * C::R + pj] = x.p;
        __syncthreads();
        f64_accum<C, false>(aq, Wgs, Kt, pi, pj, D);
        f64_accum<C, false>(aq, Wds, gKt, pi, pj, D);
        f64_accum<C, false>(ad, Wa, Vt, pi, pj, D);
        f64_accum<C, false>(ad, Wp, gVt, pi, pj, D);
    }
    f64_store<C>(a.out0, rb, i, L, aq, sc, pj, D);
    f64_store<C>(a.out3, rb, i, L, ad, 1.0, pj, D);
}

template <class C> __global__ __launch_bounds__(C::THREADS) void k64_bb_col(Args a) {
    __shared__ double Ko[C::R * C::DM], gKo[C::R * C::DM], Vo[C::R * C::DM], gVo[C::R * C::DM],
        Qt[C::R * C::DM], gQt[C::R * C::DM], dOt[C::R * C::DM], Ot[C::R * C::DM], Wgs[C::R * C::R], Wds[C::R * C::R],
        Wa[C::R * C::R], lse_t[C::R], d_t[C::R], e_t[C::R], t_t[C::R];
    const int L = a.L, D = a.D;
    const int bh = blockIdx.x / a.nblk, j0 = (blockIdx.x - bh * a.nblk) * C::R;
    const int b = bh / a.H, h = bh - b * a.H;
    const int pk = threadIdx.x / C::R, pq = threadIdx.x % C::R;
    const double sc = (double)a.scale;
    const int64_t rb = (int64_t)bh * L;
    f64_load_rows<C>(Ko, f64_slice(a.k, b, h), a.k.sl, j0, L, D);
    f64_load_rows<C>(gKo, f64_slice(a.gk, b, h), a.gk.sl, j0, L, D);
    f64_load_rows<C>(Vo, f64_slice(a.v, b, h), a.v.sl, j0, L, D);
    f64_load_rows<C>(gVo, f64_slice(a.gv, b, h), a.gv.sl, j0, L, D);
    const double* Qg = f64_slice(a.q, b, h);
    const double* gQg = f64_slice(a.gq, b, h);
    const double* dOg = f64_slice(a.dO, b, h);
    const double* Og = reinterpret_cast<const double*>(a.o) + rb * D;
    const double* Eg = reinterpret_cast<const double*>(a.out0);  // E, T from k64_bb_row<true>
    const double* Tg = reinterpret_cast<const double*>(a.out3);
    double ak[C::NACC], av[C::NACC];
    f64_zero<C>(ak);
    f64_zero<C>(av);
    for (int i0 = 0; i0 < L; i0 += C::R) {
        __syncthreads();
        f64_load_rows<C>(Qt, Qg, a.q.sl, i0, L, D);
        f64_load_rows<C>(gQt, gQg, a.gq.sl, i0, L, D);
        f64_load_rows<C>(dOt, dOg, a.dO.sl, i0, L, D);
        f64_load_rows<C>(Ot, Og, D, i0, L, D);
        __syncthreads();
        f64_tile_stats<C>(lse_t, d_t, a, rb, i0, dOt, Ot);
        if (threadIdx.x < C::R) {
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
        Wgs[pq * C::R + pk] = gs;
        Wds[pq * C::R + pk] = ds;
        Wa[pq * C::R + pk] = av_w;
        __syncthreads();
        f64_accum<C, true>(ak, Wgs, Qt, pk, pq, D);
        f64_accum<C, true>(ak, Wds, gQt, pk, pq, D);
        f64_accum<C, true>(av, Wa, dOt, pk, pq, D);
    }
    f64_store<C>(a.out1, rb, j0 + pk, L, ak, sc, pq, D);
    f64_store<C>(a.out2, rb, j0 + pk, L, av, 1.0, pq, D);
}

// Host launchers (grid: one workgroup per R own rows of each (b, h); R = 16 up to D = 128, 8 above).
template <class C> static int f64_fwd_c(Args a, hipStream_t s) {
    a.nblk = (a.L + C::R - 1) / C::R;
    hipLaunchKernelGGL((k64_fwd<C>), dim3((unsigned)((int64_t)a.B * a.H * a.nblk)), dim3(C::THREADS), 0, s, a);
    return launch_rc();
}

template <class C> static int f64_bwd_c(Args a, hipStream_t s) {
    a.nblk = (a.L + C::R - 1) / C::R;
    const dim3 grid((unsigned)((int64_t)a.B * a.H * a.nblk)), block(C::THREADS);
    hipLaunchKernelGGL((k64_bwd_row<C>), grid, block, 0, s, a);
    int rc = launch_rc();
    if (rc) return rc;
    hipLaunchKernelGGL((k64_bwd_col<C>), grid, block, 0, s, a);
    return launch_rc();
}

template <class C> static int f64_bwd_bwd_c(Args a, hipStream_t s) {
    a.nblk = (a.L + C::R - 1) / C::R;
    const dim3 grid((unsigned)((int64_t)a.B * a.H * a.nblk)), block(C::THREADS);
    hipLaunchKernelGGL((k64_bb_row<C, true>), grid, block, 0, s, a);
    int rc = launch_rc();
    if (rc) return rc;
    hipLaunchKernelGGL((k64_bb_col<C>), grid, block, 0, s, a);
    if ((rc = launch_rc())) return rc;
    hipLaunchKernelGGL((k64_bb_row<C, false>), grid, block, 0, s, a);
    return launch_rc();
}

static int f64_fwd(Args a, hipStream_t s) {
    return a.D <= F64Narrow::DM ? f64_fwd_c<F64Narrow>(a, s) : f64_fwd_c<F64Wide>(a, s);
}
static int f64_bwd(Args a, hipStream_t s) {
    return a.D <= F64Narrow::DM ? f64_bwd_c<F64Narrow>(a, s) : f64_bwd_c<F64Wide>(a, s);
}
static int f64_bwd_bwd(Args a, hipStream_t s) {
    return a.D <= F64Narrow::DM ? f64_bwd_bwd_c<F64Narrow>(a, s) : f64_bwd_bwd_c<F64Wide>(a, s);
}
