// One-workgroup-per-(b, h) kernels for 16-bit inputs with L <= 128 and D a supported width (32, 64, 128).
// Included inside namespace ebr by ebr_attn.hip (uses Args, WaveIds, slice, store_rows and attn_tiles.hpp).
//
// Every row of a pass's "other side" tensors sits in LDS at once, in natural [row][d] layout without padding; the
// 16-byte chunks of row x are XOR-swizzled (chunk c at position c ^ swz(x)) so that the 16 rows an MFMA A-operand
// read touches fall in distinct banks. Rows are loaded with buffer_load ... lds (global -> LDS, no registers, one
// 1 KB block per wave instruction; reads past the slice return 0), so a pass waits for memory once.
//   d-contraction A operand:   ds_read_b128 of row (tile + l16), chunk 4 c + g.
//   seq-contraction A operand: two ds_read_b64_tr_b16 (16-lane groups transpose a 4 x 16 block of 16-bit values:
//                              lane 4 k + j addresses row k, columns 4 j .. 4 j + 3; lane i receives column i), which
//                              yields, in lane (d = l16, group g), X[x0 + 16 h + 4 g + k][d] in k-slot 4 h + k - the
//                              slot order of the accumulator-derived B operand (attn_tiles.hpp).
// So no transposed copy of any input exists, and the chunk loops run without barriers.

typedef __attribute__((ext_vector_type(4))) short s16x4;
#define EBR_LDS __attribute__((address_space(3)))

constexpr uint32_t BUF_RSRC_WORD3 = 0x00020000;  // raw buffer, dword data format (gfx9 family)

template <int DP> struct Sw {
    static constexpr int NCK = DP / 8;   // 16-byte chunks per row
    static constexpr int ROWB = DP * 2;  // bytes per row
    static constexpr int RPI = 64 / NCK; // rows moved by one 64-lane x 16-byte load
    static __device__ __forceinline__ int swz(int x) {
        if constexpr (DP == 32) {
            return (x >> 2) & 3;
        } else if constexpr (DP == 64) {
            return (x ^ (x >> 3)) & 7;
        } else {
            return x & 15;
        }
    }
    static __device__ __forceinline__ int off(int x, int c) { return x * ROWB + 16 * (c ^ swz(x)); }
};

// Issue the loads of rows [0, Lp) of one (b, h) slice into ``region`` (Lp * ROWB bytes); waves split the 1 KB blocks.
template <typename T, int DP>
__device__ __forceinline__ void async_rows(unsigned char* region, const T* slice, int64_t srow, int L, int Lp, int wave,
                                           int nw, int lane) {
    using S = Sw<DP>;
    const uint32_t nbytes = (uint32_t)(((int64_t)(L - 1) * srow + DP) * (int64_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)slice, (short)0, (int)nbytes, (int)BUF_RSRC_WORD3);
    const uint32_t rowb = (uint32_t)(srow * (int64_t)sizeof(T));
    const int nq = Lp / S::RPI;
    for (int q = wave; q < nq; q += nw) {
        const int x = q * S::RPI + lane / S::NCK;
        const int c = (lane % S::NCK) ^ S::swz(x);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (EBR_LDS void*)(region + q * 1024), 16,
                                                 (uint32_t)x * rowb + 16u * (uint32_t)c, 0, 0, 0);
    }
}

__device__ __forceinline__ void async_wait() { __builtin_amdgcn_s_waitcnt(0); }

// Own-side B fragment from a swizzled region (row = own index).
template <typename T, int DP>
__device__ __forceinline__ void own_from_lds(OwnFrag<T, DP>& f, const unsigned char* region, int row, int g) {
#pragma unroll
    for (int c = 0; c < Lay<T, DP>::NC; ++c)
        f.v[c] = *reinterpret_cast<const u32x4*>(region + Sw<DP>::off(row, 4 * c + g));
}

// acc[m = x][n = own] += sum_d X[x][d] Own[own][d] for the 16 rows starting at ``row0`` of a swizzled region.
template <typename T, int DP>
__device__ __forceinline__ void mma_d_sw(f32x4& acc, const unsigned char* region, int row0, const OwnFrag<T, DP>& f,
                                         int l16, int g) {
    const int row = row0 + l16;
#pragma unroll
    for (int c = 0; c < Lay<T, DP>::NC; ++c) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(region + Sw<DP>::off(row, 4 * c + g));
        acc = ET<T>::mma(a, f.v[c], acc);
    }
}

// Seq-contraction A operand of d tile t for the 32 rows starting at x0, read transposed from the natural region.
template <typename T, int DP>
__device__ __forceinline__ SeqA<T> seqa_tr(const unsigned char* region, int x0, int t, int l16, int g) {
    const int k = l16 >> 2, j = l16 & 3;
    const int d = 16 * t + 4 * j;
    const int c = d >> 3, inb = (d & 7) * 2;
    const int xa = x0 + 4 * g + k;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EBR_LDS s16x4*)(region + Sw<DP>::off(xa, c) + inb));
    const s16x4 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((EBR_LDS s16x4*)(region + Sw<DP>::off(xa + 16, c) + inb));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
    SeqA<T> a;
    a.v = u32x4{l2[0], l2[1], h2[0], h2[1]};
    return a;
}

template <int N> struct StatArrays {
    float* s;
    __device__ __forceinline__ void defaults(int tid, int nthr) {
        for (int i = tid; i < STAT_MAX; i += nthr) {
            s[i] = INFINITY;
#pragma unroll
            for (int k = 1; k < N; ++k) s[k * STAT_MAX + i] = 0.f;
        }
    }
};

// =====================================================================================================================
// Forward
// =====================================================================================================================

template <typename T, int DP> struct FwdRes {
    static constexpr int SMEM = 2 * STAT_MAX * Sw<DP>::ROWB;  // K and V, up to 128 rows
};

template <typename T, int DP> __global__ __launch_bounds__(512) void k_fwd_res(Args a) {
    using LY = Lay<T, DP>;
    __shared__ __align__(1024) unsigned char smem[FwdRes<T, DP>::SMEM];
    const WaveIds w = wave_ids();
    const int nw = w.nthr >> 6;
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    const int Lp = (L + CH - 1) / CH * CH;
    unsigned char* Kr = smem;
    unsigned char* Vr = smem + Lp * Sw<DP>::ROWB;
    async_rows<T, DP>(Kr, slice<T>(a.k, b, h), a.k.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(Vr, slice<T>(a.v, b, h), a.v.sl, L, Lp, w.wave, nw, w.lane);
    const int row0 = w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    OwnFrag<T, DP> qf;
    load_own<T, DP>(qf, slice<T>(a.q, b, h), a.q.sl, own, L, DP, w.g);
    async_wait();
    __syncthreads();
    if (!active) return;
    const float sc = a.scale;
    float m = -INFINITY, lsum = 0.f;
    f32x4 acc[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int x0 = 0; x0 < L; x0 += CH) {
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
        mma_d_sw<T, DP>(s0, Kr, x0, qf, w.l16, w.g);
        mma_d_sw<T, DP>(s1, Kr, x0 + 16, qf, w.l16, w.g);
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int x = x0 + 4 * w.g + r;
            s0[r] = (x < L) ? s0[r] * sc : -INFINITY;
            s1[r] = (x + 16 < L) ? s1[r] * sc : -INFINITY;
            mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
        }
        const float mnew = fmaxf(m, xmax4(mx));
        const float alpha = fast_exp2((m - mnew) * LOG2E);
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s0[r] = fast_exp2((s0[r] - mnew) * LOG2E);
            s1[r] = fast_exp2((s1[r] - mnew) * LOG2E);
            ps += s0[r] + s1[r];
        }
        lsum = lsum * alpha + ps;
        const SeqB<T> pb = make_seqb<T>(s0, s1);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) acc[t] = mma_seq<T>(acc[t] * alpha, seqa_tr<T, DP>(Vr, x0, t, w.l16, w.g), pb);
        m = mnew;
    }
    lsum = xsum4(lsum);
    if (own < L) {
        const int64_t r = (int64_t)bh * L + own;
        store_rows<T, DP>(a.out0, r * DP, acc, 1.f / lsum, DP, w.g);
        if (w.g == 0) a.lse_out[r] = m + logf(lsum);
    }
}

// =====================================================================================================================
// Backward: row pass (dQ) then col pass (dK, dV) on one slice.
// =====================================================================================================================

template <typename T, int DP> struct BwdRes {
    static constexpr int REGION = STAT_MAX * Sw<DP>::ROWB;           // one tensor, up to 128 rows
    static constexpr bool SEP = 4 * REGION <= 64 * 1024;              // K, V, Q, dO all resident at once
    static constexpr int SMEM = (SEP ? 4 : 2) * REGION;
};

template <typename T, int DP> __global__ __launch_bounds__(512) void k_bwd_res(Args a) {
    using LY = Lay<T, DP>;
    using R = BwdRes<T, DP>;
    __shared__ __align__(1024) unsigned char smem[R::SMEM];
    __shared__ __align__(16) float st[2 * STAT_MAX];
    const WaveIds w = wave_ids();
    const int nw = w.nthr >> 6;
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    const int Lp = (L + CH - 1) / CH * CH;
    const int rb = Lp * Sw<DP>::ROWB;
    unsigned char* Kr = smem;
    unsigned char* Vr = smem + rb;
    unsigned char* Qr = R::SEP ? smem + 2 * rb : smem;
    unsigned char* Or = R::SEP ? smem + 3 * rb : smem + rb;  // dO
    const T* Qg = slice<T>(a.q, b, h);
    const T* Og = slice<T>(a.dO, b, h);
    async_rows<T, DP>(Kr, slice<T>(a.k, b, h), a.k.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(Vr, slice<T>(a.v, b, h), a.v.sl, L, Lp, w.wave, nw, w.lane);
    if constexpr (R::SEP) {
        async_rows<T, DP>(Qr, Qg, a.q.sl, L, Lp, w.wave, nw, w.lane);
        async_rows<T, DP>(Or, Og, a.dO.sl, L, Lp, w.wave, nw, w.lane);
    }
    StatArrays<2>{st}.defaults(w.tid, w.nthr);
    const float sc = a.scale;
    const int row0 = w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;

    // ---- row pass: own = queries
    {
        OwnFrag<T, DP> qf, df, of;
        load_own<T, DP>(qf, Qg, a.q.sl, own, L, DP, w.g);
        load_own<T, DP>(df, Og, a.dO.sl, own, L, DP, w.g);
        load_own<T, DP>(of, reinterpret_cast<const T*>(a.o) + (int64_t)bh * L * DP, DP, own, L, DP, w.g);
        const float lse = (own < L) ? a.lse[(int64_t)bh * L + own] : 0.f;
        const float dr = xsum4(frag_dot<T, DP>(df, of));
        async_wait();
        __syncthreads();  // regions loaded, statistics defaults written
        if (active) {
            if (w.g == 0) {
                st[own] = (own < L) ? lse : INFINITY;
                st[STAT_MAX + own] = (own < L) ? dr : 0.f;
            }
            f32x4 acc[LY::NT];
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            for (int x0 = 0; x0 < L; x0 += CH) {
                f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = p0, d1 = p0;
                mma_d_sw<T, DP>(p0, Kr, x0, qf, w.l16, w.g);
                mma_d_sw<T, DP>(p1, Kr, x0 + 16, qf, w.l16, w.g);
                mma_d_sw<T, DP>(d0, Vr, x0, df, w.l16, w.g);
                mma_d_sw<T, DP>(d1, Vr, x0 + 16, df, w.l16, w.g);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int x = x0 + 4 * w.g + r;
                    p0[r] = (x < L) ? fast_exp2(fmaf(p0[r], sc, -lse) * LOG2E) : 0.f;
                    p1[r] = (x + 16 < L) ? fast_exp2(fmaf(p1[r], sc, -lse) * LOG2E) : 0.f;
                    d0[r] = p0[r] * (d0[r] - dr);
                    d1[r] = p1[r] * (d1[r] - dr);
                }
                const SeqB<T> dsb = make_seqb<T>(d0, d1);
#pragma unroll
                for (int t = 0; t < LY::NT; ++t)
                    acc[t] = mma_seq<T>(acc[t], seqa_tr<T, DP>(Kr, x0, t, w.l16, w.g), dsb);
            }
            if (own < L) store_rows<T, DP>(a.out0, ((int64_t)bh * L + own) * DP, acc, sc, DP, w.g);
        }
    }
    __syncthreads();  // statistics published; K, V no longer read by the row pass

    // ---- col pass: own = keys
    OwnFrag<T, DP> kf, vf;
    if (active) {
        own_from_lds<T, DP>(kf, Kr, own, w.g);
        own_from_lds<T, DP>(vf, Vr, own, w.g);
    }
    if constexpr (!R::SEP) {
        __syncthreads();  // every wave holds its K, V rows before Q, dO overwrite them
        async_rows<T, DP>(Qr, Qg, a.q.sl, L, Lp, w.wave, nw, w.lane);
        async_rows<T, DP>(Or, Og, a.dO.sl, L, Lp, w.wave, nw, w.lane);
        async_wait();
        __syncthreads();
    }
    if (!active) return;
    f32x4 ak[LY::NT], av[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) ak[t] = av[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int x0 = 0; x0 < L; x0 += CH) {
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(st + x0 + 4 * w.g);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(st + x0 + 16 + 4 * w.g);
        const f32x4 r0 = *reinterpret_cast<const f32x4*>(st + STAT_MAX + x0 + 4 * w.g);
        const f32x4 r1 = *reinterpret_cast<const f32x4*>(st + STAT_MAX + x0 + 16 + 4 * w.g);
        f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = p0, d1 = p0;
        mma_d_sw<T, DP>(p0, Qr, x0, kf, w.l16, w.g);
        mma_d_sw<T, DP>(p1, Qr, x0 + 16, kf, w.l16, w.g);
        mma_d_sw<T, DP>(d0, Or, x0, vf, w.l16, w.g);
        mma_d_sw<T, DP>(d1, Or, x0 + 16, vf, w.l16, w.g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p0[r] = fast_exp2(fmaf(p0[r], sc, -l0[r]) * LOG2E);
            p1[r] = fast_exp2(fmaf(p1[r], sc, -l1[r]) * LOG2E);
            d0[r] = p0[r] * (d0[r] - r0[r]);
            d1[r] = p1[r] * (d1[r] - r1[r]);
        }
        const SeqB<T> pb = make_seqb<T>(p0, p1);
        const SeqB<T> dsb = make_seqb<T>(d0, d1);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) {
            av[t] = mma_seq<T>(av[t], seqa_tr<T, DP>(Or, x0, t, w.l16, w.g), pb);
            ak[t] = mma_seq<T>(ak[t], seqa_tr<T, DP>(Qr, x0, t, w.l16, w.g), dsb);
        }
    }
    if (own < L) {
        const int64_t r = ((int64_t)bh * L + own) * DP;
        store_rows<T, DP>(a.out1, r, ak, sc, DP, w.g);
        store_rows<T, DP>(a.out2, r, av, 1.f, DP, w.g);
    }
}

// =====================================================================================================================
// Backward of the backward: register-resident row pass, then the col pass.
// Row pass, phase 1: the wave's 16 query rows x all keys of P, dS, M1 = dS A + P Bm and PA = P A, kept as packed
// 16-bit MFMA operands, and the exact E = rowsum(PA), T = rowsum(M1). Phase 2: dS2 = M1 - E dS - T P and
// Pa = PA - E P, then hQ = s (dS2 K + dS gK) and hdO = Pa V + P gV directly (9 GEMM units on the row side).
// =====================================================================================================================

template <typename T, int DP, int NCH> struct BbRes {
    static constexpr int SMEM = 4 * NCH * CH * Sw<DP>::ROWB;  // K, gK, V, gV; later Q, gQ, dO in the same space
};

template <typename T, int DP, int NCH> __global__ __launch_bounds__(512) void k_bb_res(Args a) {
    using LY = Lay<T, DP>;
    __shared__ __align__(1024) unsigned char smem[BbRes<T, DP, NCH>::SMEM];
    __shared__ __align__(16) float st[4 * STAT_MAX];
    const WaveIds w = wave_ids();
    const int nw = w.nthr >> 6;
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    constexpr int Lp = NCH * CH;
    constexpr int rb = Lp * Sw<DP>::ROWB;
    unsigned char* Kr = smem;
    unsigned char* gKr = smem + rb;
    unsigned char* Vr = smem + 2 * rb;
    unsigned char* gVr = smem + 3 * rb;
    unsigned char* Qr = smem;
    unsigned char* gQr = smem + rb;
    unsigned char* Or = smem + 2 * rb;  // dO
    const T* Qg = slice<T>(a.q, b, h);
    const T* gQg = slice<T>(a.gq, b, h);
    const T* Og = slice<T>(a.dO, b, h);
    async_rows<T, DP>(Kr, slice<T>(a.k, b, h), a.k.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(gKr, slice<T>(a.gk, b, h), a.gk.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(Vr, slice<T>(a.v, b, h), a.v.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(gVr, slice<T>(a.gv, b, h), a.gv.sl, L, Lp, w.wave, nw, w.lane);
    StatArrays<4>{st}.defaults(w.tid, w.nthr);
    const float sc = a.scale;
    const int row0 = w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;

    // ---- row pass: own = queries
    {
        OwnFrag<T, DP> qf, gqf, df, of;
        load_own<T, DP>(qf, Qg, a.q.sl, own, L, DP, w.g);
        load_own<T, DP>(gqf, gQg, a.gq.sl, own, L, DP, w.g);
        load_own<T, DP>(df, Og, a.dO.sl, own, L, DP, w.g);
        load_own<T, DP>(of, reinterpret_cast<const T*>(a.o) + (int64_t)bh * L * DP, DP, own, L, DP, w.g);
        const float lse = (own < L) ? a.lse[(int64_t)bh * L + own] : 0.f;
        const float dr = xsum4(frag_dot<T, DP>(df, of));
        async_wait();
        __syncthreads();
        if (active) {
            SeqB<T> m1b[NCH], dsb[NCH], pb[NCH], pab[NCH];
            float e_acc = 0.f, t_acc = 0.f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int x0 = c * CH;
                f32x4 p[2], dp[2], at[2], bm[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    p[hh] = dp[hh] = at[hh] = bm[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
                    const int r0 = x0 + 16 * hh;
                    mma_d_sw<T, DP>(p[hh], Kr, r0, qf, w.l16, w.g);
                    mma_d_sw<T, DP>(at[hh], Kr, r0, gqf, w.l16, w.g);
                    mma_d_sw<T, DP>(at[hh], gKr, r0, qf, w.l16, w.g);
                    mma_d_sw<T, DP>(dp[hh], Vr, r0, df, w.l16, w.g);
                    mma_d_sw<T, DP>(bm[hh], gVr, r0, df, w.l16, w.g);
                }
                f32x4 ds[2], pa[2], m1[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int x = x0 + 16 * hh + 4 * w.g + r;
                        const float pv = (x < L) ? fast_exp2(fmaf(p[hh][r], sc, -lse) * LOG2E) : 0.f;
                        const float dsv = pv * (dp[hh][r] - dr);
                        const float av = at[hh][r] * sc;
                        p[hh][r] = pv;
                        ds[hh][r] = dsv;
                        pa[hh][r] = pv * av;
                        m1[hh][r] = fmaf(dsv, av, pv * bm[hh][r]);
                        e_acc += pa[hh][r];
                        t_acc += m1[hh][r];
                    }
                }
                pb[c] = make_seqb<T>(p[0], p[1]);
                dsb[c] = make_seqb<T>(ds[0], ds[1]);
                pab[c] = make_seqb<T>(pa[0], pa[1]);
                m1b[c] = make_seqb<T>(m1[0], m1[1]);
            }
            const float E = xsum4(e_acc);
            const float Tm = xsum4(t_acc);
            f32x4 hq[LY::NT], hdo[LY::NT];
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) hq[t] = hdo[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int x0 = c * CH;
                float m1f[8], dsf[8], pf[8], paf[8], d2[8], pe[8];
                unpack_seqb<T>(m1b[c], m1f);
                unpack_seqb<T>(dsb[c], dsf);
                unpack_seqb<T>(pb[c], pf);
                unpack_seqb<T>(pab[c], paf);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    d2[e] = m1f[e] - E * dsf[e] - Tm * pf[e];
                    pe[e] = paf[e] - E * pf[e];
                }
                const SeqB<T> d2b = pack_seqb<T>(d2);
                const SeqB<T> peb = pack_seqb<T>(pe);
#pragma unroll
                for (int t = 0; t < LY::NT; ++t) {
                    hq[t] = mma_seq<T>(hq[t], seqa_tr<T, DP>(Kr, x0, t, w.l16, w.g), d2b);
                    hq[t] = mma_seq<T>(hq[t], seqa_tr<T, DP>(gKr, x0, t, w.l16, w.g), dsb[c]);
                    hdo[t] = mma_seq<T>(hdo[t], seqa_tr<T, DP>(Vr, x0, t, w.l16, w.g), peb);
                    hdo[t] = mma_seq<T>(hdo[t], seqa_tr<T, DP>(gVr, x0, t, w.l16, w.g), pb[c]);
                }
            }
            if (own < L) {
                const int64_t r = ((int64_t)bh * L + own) * DP;
                store_rows<T, DP>(a.out0, r, hq, sc, DP, w.g);
                store_rows<T, DP>(a.out3, r, hdo, 1.f, DP, w.g);
            }
            if (w.g == 0) {
                const bool ok = own < L;
                st[own] = ok ? lse : INFINITY;
                st[STAT_MAX + own] = ok ? dr : 0.f;
                st[2 * STAT_MAX + own] = ok ? E : 0.f;
                st[3 * STAT_MAX + own] = ok ? Tm : 0.f;
            }
        }
    }
    __syncthreads();  // statistics published; the row pass no longer reads K, gK, V, gV

    // ---- col pass: own = keys
    OwnFrag<T, DP> kf, gkf, vf, gvf;
    if (active) {
        own_from_lds<T, DP>(kf, Kr, own, w.g);
        own_from_lds<T, DP>(gkf, gKr, own, w.g);
        own_from_lds<T, DP>(vf, Vr, own, w.g);
        own_from_lds<T, DP>(gvf, gVr, own, w.g);
    }
    __syncthreads();  // every wave holds its key rows before Q, gQ, dO overwrite the regions
    async_rows<T, DP>(Qr, Qg, a.q.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(gQr, gQg, a.gq.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(Or, Og, a.dO.sl, L, Lp, w.wave, nw, w.lane);
    async_wait();
    __syncthreads();
    if (!active) return;
    f32x4 hk[LY::NT], hv[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) hk[t] = hv[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int x0 = 0; x0 < L; x0 += CH) {
        f32x4 p[2], dp[2], at[2], bm[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            p[hh] = dp[hh] = at[hh] = bm[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int r0 = x0 + 16 * hh;
            mma_d_sw<T, DP>(p[hh], Qr, r0, kf, w.l16, w.g);
            mma_d_sw<T, DP>(at[hh], Qr, r0, gkf, w.l16, w.g);
            mma_d_sw<T, DP>(at[hh], gQr, r0, kf, w.l16, w.g);
            mma_d_sw<T, DP>(dp[hh], Or, r0, vf, w.l16, w.g);
            mma_d_sw<T, DP>(bm[hh], Or, r0, gvf, w.l16, w.g);
        }
        f32x4 ds[2], ds2[2], pa[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int so = x0 + 16 * hh + 4 * w.g;
            const f32x4 ls = *reinterpret_cast<const f32x4*>(st + so);
            const f32x4 rs = *reinterpret_cast<const f32x4*>(st + STAT_MAX + so);
            const f32x4 es = *reinterpret_cast<const f32x4*>(st + 2 * STAT_MAX + so);
            const f32x4 ts = *reinterpret_cast<const f32x4*>(st + 3 * STAT_MAX + so);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pv = fast_exp2(fmaf(p[hh][r], sc, -ls[r]) * LOG2E);
                const float dsv = pv * (dp[hh][r] - rs[r]);
                const float av = at[hh][r] * sc;
                ds[hh][r] = dsv;
                const float m1 = fmaf(dsv, av, pv * bm[hh][r]);
                ds2[hh][r] = m1 - es[r] * dsv - ts[r] * pv;
                pa[hh][r] = pv * (av - es[r]);
            }
        }
        const SeqB<T> dsb = make_seqb<T>(ds[0], ds[1]);
        const SeqB<T> ds2b = make_seqb<T>(ds2[0], ds2[1]);
        const SeqB<T> pab = make_seqb<T>(pa[0], pa[1]);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) {
            hk[t] = mma_seq<T>(hk[t], seqa_tr<T, DP>(Qr, x0, t, w.l16, w.g), ds2b);
            hk[t] = mma_seq<T>(hk[t], seqa_tr<T, DP>(gQr, x0, t, w.l16, w.g), dsb);
            hv[t] = mma_seq<T>(hv[t], seqa_tr<T, DP>(Or, x0, t, w.l16, w.g), pab);
        }
    }
    if (own < L) {
        const int64_t r = ((int64_t)bh * L + own) * DP;
        store_rows<T, DP>(a.out1, r, hk, sc, DP, w.g);
        store_rows<T, DP>(a.out2, r, hv, 1.f, DP, w.g);
    }
}
