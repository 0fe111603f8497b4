// Long-sequence kernels for 16-bit inputs (L > 128, D a supported width): a workgroup owns NWC * 16 rows of one
// (b, h) slice and streams the other side through LDS in stages of LSTAGE rows.
// Included inside namespace ebr by ebr_attn.hip, after attn_resident.hpp (uses its LDS layout and operand readers).
//
// Each workgroup has NWC compute waves (16 own rows each, kept in registers as MFMA B operands) and one loader wave.
// The loader moves each stage global -> LDS (buffer_load ... lds; rows past L read as 0) into one of two stage
// buffers while the compute waves work on the other, so compute waves never have such a load outstanding and their
// LDS transpose reads are never held back by one. One barrier per stage hands a buffer over:
//   loader:  issue(0); for i: { wait; barrier i; issue(i + 1) into the buffer stage i - 1 used }
//   compute: for i: { barrier i; compute stage i }
// Stage rows sit in the swizzled natural layout of the resident kernels; d-contractions read them as A operands,
// seq-contractions read them transposed (ds_read_b64_tr_b16), so no transposed copy is ever written.
// In the backward kernels, the A operands of a group of MFMAs are read from LDS together and a scheduling barrier
// keeps those reads ahead of the MFMAs: left to itself, at these kernels' register use, the compiler issued each read
// just before its MFMA and waited for it there (bwd 0.52 -> 0.48 ms, bwd_bwd 1.15 -> 1.09 ms at the Maze shape). The
// forward keeps the compiler's order: the extra registers cost it a wave per SIMD and 6%.

constexpr int LSTAGE = 64;  // other-side rows per stage: two 32-row MFMA k-chunks
// Online softmax of the long forward: the exponentials of a stage are taken against the current reference point m
// first, and accepted when every row's sum of them stays at most stage_sum_max (so each P is at most that, inside
// the range of the MFMA operand type: 2^32 for bf16, 2^15 for fp16, whose largest value is 65504); otherwise m moves
// to the row maximum and the stage is redone.
template <typename T> constexpr float stage_sum_max() { return std::is_same_v<T, _Float16> ? 32768.f : 4294967296.f; }

template <typename T, int DP, int NWC> struct LongCfg {
    static constexpr int SB = LSTAGE * Sw<DP>::ROWB;  // one tensor's stage (bytes)
    static constexpr int ROWS = 16 * NWC;             // own rows per workgroup
    static constexpr int THREADS = 64 * (NWC + 1);
};

// Loader: rows [r0, r0 + LSTAGE) of one slice tensor into a stage region; rows past L read as 0.
template <typename T, int DP>
__device__ __forceinline__ void async_stage(unsigned char* region, const T* slice, int64_t srow, int L, int r0,
                                            int lane) {
    async_rows<T, DP>(region, slice + (int64_t)r0 * srow, srow, L - r0, LSTAGE, 0, 1, lane);
}

// The loader wave's loop over nst stages of ntens tensors each; ``issue(i, buf)`` starts stage i's loads into ``buf``
// and ``after(i, buf)`` runs once they have landed (before the barrier that hands the buffer over).
template <int STAGE_BYTES, class Issue, class After>
__device__ __forceinline__ void loader_loop(unsigned char* smem, int nst, Issue&& issue, After&& after) {
    issue(0, smem);
    for (int i = 0; i < nst; ++i) {
        async_wait();
        after(i, smem + (i & 1) * STAGE_BYTES);
        lds_barrier();
        if (i + 1 < nst) issue(i + 1, smem + ((i + 1) & 1) * STAGE_BYTES);
    }
}

// Stage order of the long kernels. When L is not a multiple of the stage depth, the short last stage (nv rows below
// L) is taken first, as stage 0, 16 rows at a time as far as L: its 16-row tiles wholly past L are neither multiplied
// nor read, and the seq-contractions take the k = 16 MFMA (the 30 x 30 grids, L = 900, end in a stage of 4 rows). The
// full stages follow in order and need no masking. Taken after the loop instead, the tail's code raised the loop's
// register count (the bwd_bwd col kernel from 128 to 154 VGPRs, one workgroup per CU fewer).
struct StageOrder {
    int nfull, rows;
    bool tail;
    __device__ __forceinline__ StageOrder(int L, int rows_) : nfull(L / rows_), rows(rows_), tail(L % rows_ != 0) {}
    __device__ __forceinline__ int row(int i) const { return (tail ? (i == 0 ? nfull : i - 1) : i) * rows; }
};

// =====================================================================================================================
// Forward: online softmax over the stages (reference point m in log2 units, running sum l, accumulator rescaled by
// exp2(m_old - m_new) when m moves).
// =====================================================================================================================

template <typename T, int DP, int NWC> __global__ __launch_bounds__(64 * (NWC + 1)) void k_fwd_long(Args a) {
    using LY = Lay<T, DP>;
    using C = LongCfg<T, DP, NWC>;
    constexpr int STB = 2 * C::SB;  // K, V
    __shared__ __align__(1024) unsigned char smem[2 * STB];
    const WaveIds w = wave_ids();
    int bh, blk;
    decode_block(a, bh, blk);
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    const int nst = (L + LSTAGE - 1) / LSTAGE;
    const StageOrder so(L, LSTAGE);

    if (w.wave == NWC) {
        const T* Kg = slice<T>(a.k, b, h);
        const T* Vg = slice<T>(a.v, b, h);
        loader_loop<STB>(
            smem, nst,
            [&](int i, unsigned char* buf) {
                async_stage<T, DP>(buf, Kg, a.k.sl, L, so.row(i), w.lane);
                async_stage<T, DP>(buf + C::SB, Vg, a.v.sl, L, so.row(i), w.lane);
            },
            [](int, unsigned char*) {});
        return;
    }

    const int row0 = blk * C::ROWS + w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;  // wave-uniform; inactive waves still take every barrier
    OwnFrag<T, DP> qf;
    load_own<T, DP>(qf, slice<T>(a.q, b, h), a.q.sl, own, L, DP, w.g);
    const LaneOff<T, DP> lo(w.l16, w.g);
    const float sc2 = a.scale * LOG2E;  // scores in log2 units
    f32x4 acc[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // m: the row's reference point (log2 units); l: the row's sum of P, in every lane of the row. Row sums come from
    // an MFMA with an all-ones A operand, as the products of the rounded P that also enter P V, so no lane sums.
    float m = -INFINITY, l = 0.f;
    SeqA<T> ones;
    {
        typename ET<T>::v8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (T)1.f;
        ones.v = __builtin_bit_cast(u32x4, o);
    }
    // Moves m to the row maximum of scaled scores mx (log2 units, -inf past L; every stage and tile holds a key below
    // L, so it is finite) where that exceeds m, rescaling l and acc.
    auto raise_m = [&](float mx) {
        const float mn = fmaxf(m, xmax4(mx));
        const float alpha = fast_exp2(m - mn);  // 0 while m = -inf (l and acc are still 0)
        m = mn;
        l *= alpha;
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) acc[t] *= alpha;
    };
    // A full stage of keys from Kr, Vr (all below L). The common case issues no maximum at all: exponentials against
    // m, the row sums by MFMA, one vote. The maximum is taken only when a row's sum exceeds stage_sum_max (or is not
    // finite, as in a first stage with m = -inf).
    auto stage = [&](const unsigned char* Kr, const unsigned char* Vr) {
        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
            mma_d_sw<T, DP>(s[kt], Kr, 16 * kt, qf, lo);
        }
        SeqB<T> pb[2];
        f32x4 ls;
        auto exps = [&]() {
            ls = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                f32x4 p0, p1;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p0[r] = fast_exp2(fmaf(s[2 * c][r], sc2, -m));
                    p1[r] = fast_exp2(fmaf(s[2 * c + 1][r], sc2, -m));
                }
                pb[c] = make_seqb<T>(p0, p1);
                ls = mma_seq<T>(ls, ones, pb[c]);
            }
        };
        exps();
        if (__any(!(ls[0] <= stage_sum_max<T>()))) {
            float mx = s[0][0] * sc2;  // scaled first: the scale may be negative
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = (kt == 0 ? 1 : 0); r < 4; ++r) mx = fmax_nn(mx, s[kt][r] * sc2);
            raise_m(mx);
            exps();
        }
        l += ls[0];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) acc[t] = mma_seq<T>(acc[t], seqa_tr<T, DP>(Vr, 32 * c, t, lo), pb[c]);
    };
    // One 16-key tile of the short stage (the first one taken), keys x0 .. x0 + 15 of Kr, Vr, those at nv and past
    // masked (k = 16 MFMA). It takes the maximum: m is still -inf at its first tile.
    auto tile16 = [&](const unsigned char* Kr, const unsigned char* Vr, int x0, int nv) {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
        mma_d_sw<T, DP>(s, Kr, x0, qf, lo);
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = x0 + 4 * w.g + r < nv ? s[r] * sc2 : -INFINITY;
        raise_m(fmax_nn(fmax_nn(s[0], s[1]), fmax_nn(s[2], s[3])));
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = fast_exp2(s[r] - m);
        const u32x2 pb = pack4<T>(s);
        l += ET<T>::mma16(u32x2{ones.v[0], ones.v[1]}, pb, f32x4{0.f, 0.f, 0.f, 0.f})[0];
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) acc[t] = ET<T>::mma16(seqa_tr16<T, DP>(Vr, x0, t, lo), pb, acc[t]);
    };
    if (so.tail) {
        lds_barrier();  // stage 0, the short one, in its buffer
        if (active) {
            const int nv = L - so.nfull * LSTAGE;
#pragma nounroll
            for (int x0 = 0; x0 < nv; x0 += 16) tile16(smem, smem + C::SB, x0, nv);
        }
    }
    for (int i = so.tail ? 1 : 0; i < nst; ++i) {
        lds_barrier();  // stage i in its buffer
        if (!active) continue;
        const unsigned char* Kr = smem + (i & 1) * STB;
        stage(Kr, Kr + C::SB);
    }
    if (!active) return;
    if (own < L) {
        const int64_t r = (int64_t)bh * L + own;
        store_rows<T, DP>(a.out0, r * DP, acc, 1.f / l, DP, w.g);
        if (w.g == 0) a.lse_out[r] = m * (1.f / LOG2E) + logf(l);
    }
}

// Loader helper: the statistics of a stage's LSTAGE rows [r0, r0 + LSTAGE) from fp32 [B, H, L] arrays, one row per
// loader lane: lse * log2 e (+inf past L, so P = 0 there) and up to three further row statistics (0 past L).
template <int NX> struct StageStats {
    float lse, x[NX > 0 ? NX : 1];
    __device__ __forceinline__ void load(const Args& a, int bh, int r0, int lane) {
        const int L = a.L;
        const int row = r0 + lane;
        const int64_t i = (int64_t)bh * L + (row < L ? row : L - 1);  // unconditional loads
        lse = a.lse[i];
#pragma unroll
        for (int k = 0; k < NX; ++k) x[k] = a.stats[k * a.bhl + i];
    }
    __device__ __forceinline__ void put(float* st, int r0, int L, int lane) const {
        const bool in = r0 + lane < L;
        st[lane] = in ? lse * LOG2E : INFINITY;
#pragma unroll
        for (int k = 0; k < NX; ++k) st[(k + 1) * LSTAGE + lane] = in ? x[k] : 0.f;
    }
};

// =====================================================================================================================
// Backward, row kernel: own = queries; dQ = s dS K over the K, V stages. Publishes Dr = rowsum(dO o O) of its rows
// to a.stats for the col kernel.
// =====================================================================================================================

template <typename T, int DP, int NWC> __global__ __launch_bounds__(64 * (NWC + 1)) void k_bwd_long_row(Args a) {
    using LY = Lay<T, DP>;
    using C = LongCfg<T, DP, NWC>;
    constexpr int STB = 2 * C::SB;  // K, V
    __shared__ __align__(1024) unsigned char smem[2 * STB];
    const WaveIds w = wave_ids();
    int bh, blk;
    decode_block(a, bh, blk);
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    const int nst = (L + LSTAGE - 1) / LSTAGE;
    const StageOrder so(L, LSTAGE);

    if (w.wave == NWC) {
        const T* Kg = slice<T>(a.k, b, h);
        const T* Vg = slice<T>(a.v, b, h);
        loader_loop<STB>(
            smem, nst,
            [&](int i, unsigned char* buf) {
                async_stage<T, DP>(buf, Kg, a.k.sl, L, so.row(i), w.lane);
                async_stage<T, DP>(buf + C::SB, Vg, a.v.sl, L, so.row(i), w.lane);
            },
            [](int, unsigned char*) {});
        return;
    }

    const int row0 = blk * C::ROWS + w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    OwnFrag<T, DP> qf, df, of;
    load_own<T, DP>(qf, slice<T>(a.q, b, h), a.q.sl, own, L, DP, w.g);
    load_own<T, DP>(df, slice<T>(a.dO, b, h), a.dO.sl, own, L, DP, w.g);
    load_own<T, DP>(of, reinterpret_cast<const T*>(a.o) + (int64_t)bh * L * DP, DP, own, L, DP, w.g);
    const float lraw = a.lse[(int64_t)bh * L + (own < L ? own : L - 1)];  // unconditional load
    const float lse2 = lraw * LOG2E;
    const float dr = xsum4(frag_dot<T, DP>(df, of));
    if (active && w.g == 0 && own < L) a.stats[(int64_t)bh * L + own] = dr;
    const LaneOff<T, DP> lo(w.l16, w.g);
    const float sc2 = a.scale * LOG2E;
    f32x4 acc[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // A full stage of keys from Kr, Vr (all below L).
    auto stage = [&](const unsigned char* Kr, const unsigned char* Vr) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            f32x4 p[2], dp[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                p[hh] = dp[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
                u32x4 ka[LY::NC], va[LY::NC];
#pragma unroll
                for (int q = 0; q < LY::NC; ++q) {
                    const int o = (32 * c + 16 * hh) * Sw<DP>::ROWB + lo.a[q];
                    ka[q] = *reinterpret_cast<const u32x4*>(Kr + o);
                    va[q] = *reinterpret_cast<const u32x4*>(Vr + o);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < LY::NC; ++q) {
                    p[hh] = ET<T>::mma(ka[q], qf.v[q], p[hh]);
                    dp[hh] = ET<T>::mma(va[q], df.v[q], dp[hh]);
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pv = fast_exp2(fmaf(p[hh][r], sc2, -lse2));
                    p[hh][r] = pv * (dp[hh][r] - dr);  // dS
                }
            const SeqB<T> dsb = make_seqb<T>(p[0], p[1]);
            SeqA<T> kt[LY::NT];
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) kt[t] = seqa_tr<T, DP>(Kr, 32 * c, t, lo);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) acc[t] = mma_seq<T>(acc[t], kt[t], dsb);
        }
    };
    // One 16-key tile of the short stage, keys x0 .. x0 + 15 of Kr, Vr, those at nv and past masked (k = 16 MFMA).
    auto tile16 = [&](const unsigned char* Kr, const unsigned char* Vr, int x0, int nv) {
        f32x4 p = {0.f, 0.f, 0.f, 0.f}, dp = p;
        mma_d_sw<T, DP>(p, Kr, x0, qf, lo);
        mma_d_sw<T, DP>(dp, Vr, x0, df, lo);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pv = x0 + 4 * w.g + r < nv ? fast_exp2(fmaf(p[r], sc2, -lse2)) : 0.f;
            p[r] = pv * (dp[r] - dr);  // dS
        }
        const u32x2 dsb = pack4<T>(p);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) acc[t] = ET<T>::mma16(seqa_tr16<T, DP>(Kr, x0, t, lo), dsb, acc[t]);
    };
    if (so.tail) {
        lds_barrier();  // stage 0, the short one, in its buffer
        if (active) {
            const int nv = L - so.nfull * LSTAGE;
#pragma nounroll
            for (int x0 = 0; x0 < nv; x0 += 16) tile16(smem, smem + C::SB, x0, nv);
        }
    }
    for (int i = so.tail ? 1 : 0; i < nst; ++i) {
        lds_barrier();  // stage i in its buffer
        if (!active) continue;
        const unsigned char* Kr = smem + (i & 1) * STB;
        stage(Kr, Kr + C::SB);
    }
    if (active && own < L) store_rows<T, DP>(a.out0, ((int64_t)bh * L + own) * DP, acc, a.scale, DP, w.g);
}

// =====================================================================================================================
// Backward, col kernel: own = keys; dV = P^T dO and dK = s dS^T Q over the Q, dO stages, with the stages' lse and Dr.
// =====================================================================================================================

template <typename T, int DP, int NWC> __global__ __launch_bounds__(64 * (NWC + 1)) void k_bwd_long_col(Args a) {
    using LY = Lay<T, DP>;
    using C = LongCfg<T, DP, NWC>;
    constexpr int STB = 2 * C::SB + 2 * LSTAGE * 4;  // Q, dO, [lse * log2 e | Dr]
    __shared__ __align__(1024) unsigned char smem[2 * STB];
    const WaveIds w = wave_ids();
    int bh, blk;
    decode_block(a, bh, blk);
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    const int nst = (L + LSTAGE - 1) / LSTAGE;
    const StageOrder so(L, LSTAGE);

    if (w.wave == NWC) {
        const T* Qg = slice<T>(a.q, b, h);
        const T* Og = slice<T>(a.dO, b, h);
        StageStats<1> stt;
        loader_loop<STB>(
            smem, nst,
            [&](int i, unsigned char* buf) {
                async_stage<T, DP>(buf, Qg, a.q.sl, L, so.row(i), w.lane);
                async_stage<T, DP>(buf + C::SB, Og, a.dO.sl, L, so.row(i), w.lane);
                stt.load(a, bh, so.row(i), w.lane);
            },
            [&](int i, unsigned char* buf) {
                stt.put(reinterpret_cast<float*>(buf + 2 * C::SB), so.row(i), L, w.lane);
            });
        return;
    }

    const int row0 = blk * C::ROWS + w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    OwnFrag<T, DP> kf, vf;
    load_own<T, DP>(kf, slice<T>(a.k, b, h), a.k.sl, own, L, DP, w.g);
    load_own<T, DP>(vf, slice<T>(a.v, b, h), a.v.sl, own, L, DP, w.g);
    const LaneOff<T, DP> lo(w.l16, w.g);
    const float sc2 = a.scale * LOG2E;
    f32x4 ak[LY::NT], av[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) ak[t] = av[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // A full stage of query rows from Qr, Or (dO) with their statistics st (all rows below L).
    auto stage = [&](const unsigned char* Qr, const unsigned char* Or, const float* st) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            f32x4 p[2], dp[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                p[hh] = dp[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
                u32x4 qa[LY::NC], oa[LY::NC];
#pragma unroll
                for (int q = 0; q < LY::NC; ++q) {
                    const int o = (32 * c + 16 * hh) * Sw<DP>::ROWB + lo.a[q];
                    qa[q] = *reinterpret_cast<const u32x4*>(Qr + o);
                    oa[q] = *reinterpret_cast<const u32x4*>(Or + o);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < LY::NC; ++q) {
                    p[hh] = ET<T>::mma(qa[q], kf.v[q], p[hh]);
                    dp[hh] = ET<T>::mma(oa[q], vf.v[q], dp[hh]);
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int x = 32 * c + 16 * hh + 4 * w.g;
                const f32x4 l2 = *reinterpret_cast<const f32x4*>(st + x);
                const f32x4 d2 = *reinterpret_cast<const f32x4*>(st + LSTAGE + x);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p[hh][r] = fast_exp2(fmaf(p[hh][r], sc2, -l2[r]));
                    dp[hh][r] = p[hh][r] * (dp[hh][r] - d2[r]);  // dS
                }
            }
            const SeqB<T> pb = make_seqb<T>(p[0], p[1]);
            const SeqB<T> dsb = make_seqb<T>(dp[0], dp[1]);
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) {
                const SeqA<T> ot = seqa_tr<T, DP>(Or, 32 * c, t, lo);
                const SeqA<T> qt = seqa_tr<T, DP>(Qr, 32 * c, t, lo);
                __builtin_amdgcn_sched_barrier(0);
                av[t] = mma_seq<T>(av[t], ot, pb);
                ak[t] = mma_seq<T>(ak[t], qt, dsb);
            }
        }
    };
    // One 16-row tile of the short stage, rows x0 .. x0 + 15 (k = 16 MFMA); rows past L carry lse = +inf: P = 0.
    auto tile16 = [&](const unsigned char* Qr, const unsigned char* Or, const float* st, int x0) {
        f32x4 p = {0.f, 0.f, 0.f, 0.f}, dp = p;
        mma_d_sw<T, DP>(p, Qr, x0, kf, lo);
        mma_d_sw<T, DP>(dp, Or, x0, vf, lo);
        const f32x4 l2 = *reinterpret_cast<const f32x4*>(st + x0 + 4 * w.g);
        const f32x4 d2 = *reinterpret_cast<const f32x4*>(st + LSTAGE + x0 + 4 * w.g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = fast_exp2(fmaf(p[r], sc2, -l2[r]));
            dp[r] = p[r] * (dp[r] - d2[r]);  // dS
        }
        const u32x2 pb = pack4<T>(p);
        const u32x2 dsb = pack4<T>(dp);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) {
            av[t] = ET<T>::mma16(seqa_tr16<T, DP>(Or, x0, t, lo), pb, av[t]);
            ak[t] = ET<T>::mma16(seqa_tr16<T, DP>(Qr, x0, t, lo), dsb, ak[t]);
        }
    };
    if (so.tail) {
        lds_barrier();  // stage 0, the short one, in its buffer
        if (active) {
            const int nv = L - so.nfull * LSTAGE;
#pragma nounroll
            for (int x0 = 0; x0 < nv; x0 += 16)
                tile16(smem, smem + C::SB, reinterpret_cast<const float*>(smem + 2 * C::SB), x0);
        }
    }
    for (int i = so.tail ? 1 : 0; i < nst; ++i) {
        lds_barrier();  // stage i in its buffer
        if (!active) continue;
        const unsigned char* Qr = smem + (i & 1) * STB;
        stage(Qr, Qr + C::SB, reinterpret_cast<const float*>(Qr + 2 * C::SB));
    }
    if (active && own < L) {
        const int64_t r = ((int64_t)bh * L + own) * DP;
        store_rows<T, DP>(a.out1, r, ak, a.scale, DP, w.g);
        store_rows<T, DP>(a.out2, r, av, 1.f, DP, w.g);
    }
}

// =====================================================================================================================
// Backward of the backward, row kernel: own = queries, over the K, gK, V, gV stages. E and T are complete only at the
// end of the row, so the D-wide sums are kept apart (the reference's streaming form):
//   X = sum (M1 K + dS gK), U = sum dS K, Z = sum P K, W = sum (PA V + P gV),
//   hQ = s (X - E U - T Z),   hdO = W - E O   (with M1 = dS o A + P o Bm, PA = P o A).
// Publishes Dr, E, T of its rows to a.stats ([3, B, H, L]) for the col kernel.
// =====================================================================================================================

template <typename T, int DP, int NWC, int STG>
__global__ __launch_bounds__(64 * (NWC + 1)) void k_bb_long_row(Args a) {
    using LY = Lay<T, DP>;
    using C = LongCfg<T, DP, NWC>;
    constexpr int SB = STG * Sw<DP>::ROWB;  // one tensor's stage
    constexpr int STB = 4 * SB;              // K, gK, V, gV
    __shared__ __align__(1024) unsigned char smem[2 * STB];
    const WaveIds w = wave_ids();
    int bh, blk;
    decode_block(a, bh, blk);
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    const int nst = (L + STG - 1) / STG;
    const StageOrder so(L, STG);

    if (w.wave == NWC) {
        const T* Kg = slice<T>(a.k, b, h);
        const T* gKg = slice<T>(a.gk, b, h);
        const T* Vg = slice<T>(a.v, b, h);
        const T* gVg = slice<T>(a.gv, b, h);
        loader_loop<STB>(
            smem, nst,
            [&](int i, unsigned char* buf) {
                const int r0 = so.row(i);
                async_rows<T, DP>(buf, Kg + (int64_t)r0 * a.k.sl, a.k.sl, L - r0, STG, 0, 1, w.lane);
                async_rows<T, DP>(buf + SB, gKg + (int64_t)r0 * a.gk.sl, a.gk.sl, L - r0, STG, 0, 1, w.lane);
                async_rows<T, DP>(buf + 2 * SB, Vg + (int64_t)r0 * a.v.sl, a.v.sl, L - r0, STG, 0, 1, w.lane);
                async_rows<T, DP>(buf + 3 * SB, gVg + (int64_t)r0 * a.gv.sl, a.gv.sl, L - r0, STG, 0, 1, w.lane);
            },
            [](int, unsigned char*) {});
        return;
    }

    const int row0 = blk * C::ROWS + w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    OwnFrag<T, DP> qf, gqf, df;
    float dr;
    {
        OwnFrag<T, DP> of;
        load_own<T, DP>(qf, slice<T>(a.q, b, h), a.q.sl, own, L, DP, w.g);
        load_own<T, DP>(gqf, slice<T>(a.gq, b, h), a.gq.sl, own, L, DP, w.g);
        load_own<T, DP>(df, slice<T>(a.dO, b, h), a.dO.sl, own, L, DP, w.g);
        load_own<T, DP>(of, reinterpret_cast<const T*>(a.o) + (int64_t)bh * L * DP, DP, own, L, DP, w.g);
        dr = xsum4(frag_dot<T, DP>(df, of));
    }
    const float lse2 = a.lse[(int64_t)bh * L + (own < L ? own : L - 1)] * LOG2E;  // unconditional load
    const LaneOff<T, DP> lo(w.l16, w.g);
    const float sc = a.scale;
    const float sc2 = sc * LOG2E;
    f32x4 X[LY::NT], U[LY::NT], Z[LY::NT], W[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) X[t] = U[t] = Z[t] = W[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float e_acc = 0.f, t_acc = 0.f;
    // One 16-key tile's products and statistics: p, at, dp, bm hold S, A, dP, Bm on entry (accumulator layout) and
    // P, PA, dS, M1 on return, with E and T accumulated. ``live`` masks keys past L (short stage only).
    auto elementwise = [&](f32x4& p, f32x4& at, f32x4& dp, f32x4& bm, auto live) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pv = live(r) ? fast_exp2(fmaf(p[r], sc2, -lse2)) : 0.f;
            const float dsv = pv * (dp[r] - dr);
            const float av = at[r] * sc;
            const float pa = pv * av;
            const float m1 = fmaf(dsv, av, pv * bm[r]);
            e_acc += pa;
            t_acc += m1;
            p[r] = pv;
            dp[r] = dsv;
            at[r] = pa;
            bm[r] = m1;
        }
    };
    // A full stage of keys from the K, gK, V, gV regions at Kr (all below L).
    auto stage = [&](const unsigned char* Kr) {
        const unsigned char* gKr = Kr + SB;
        const unsigned char* Vr = Kr + 2 * SB;
        const unsigned char* gVr = Kr + 3 * SB;
#pragma unroll
        for (int c = 0; c < STG / CH; ++c) {
            f32x4 p[2], at[2], dp[2], bm[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                p[hh] = at[hh] = dp[hh] = bm[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
                const int r0 = 32 * c + 16 * hh;
                {
                    u32x4 ka[LY::NC], gka[LY::NC];
#pragma unroll
                    for (int q = 0; q < LY::NC; ++q) {
                        const int o = r0 * Sw<DP>::ROWB + lo.a[q];
                        ka[q] = *reinterpret_cast<const u32x4*>(Kr + o);
                        gka[q] = *reinterpret_cast<const u32x4*>(gKr + o);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < LY::NC; ++q) {
                        p[hh] = ET<T>::mma(ka[q], qf.v[q], p[hh]);
                        at[hh] = ET<T>::mma(ka[q], gqf.v[q], at[hh]);
                        at[hh] = ET<T>::mma(gka[q], qf.v[q], at[hh]);
                    }
                }
                {
                    u32x4 va[LY::NC], gva[LY::NC];
#pragma unroll
                    for (int q = 0; q < LY::NC; ++q) {
                        const int o = r0 * Sw<DP>::ROWB + lo.a[q];
                        va[q] = *reinterpret_cast<const u32x4*>(Vr + o);
                        gva[q] = *reinterpret_cast<const u32x4*>(gVr + o);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < LY::NC; ++q) {
                        dp[hh] = ET<T>::mma(va[q], df.v[q], dp[hh]);
                        bm[hh] = ET<T>::mma(gva[q], df.v[q], bm[hh]);
                    }
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) elementwise(p[hh], at[hh], dp[hh], bm[hh], [](int) { return true; });
            const SeqB<T> pb = make_seqb<T>(p[0], p[1]);
            const SeqB<T> dsb = make_seqb<T>(dp[0], dp[1]);
            const SeqB<T> pab = make_seqb<T>(at[0], at[1]);
            const SeqB<T> m1b = make_seqb<T>(bm[0], bm[1]);
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) {
                const SeqA<T> kt = seqa_tr<T, DP>(Kr, 32 * c, t, lo);
                const SeqA<T> gkt = seqa_tr<T, DP>(gKr, 32 * c, t, lo);
                const SeqA<T> vt = seqa_tr<T, DP>(Vr, 32 * c, t, lo);
                const SeqA<T> gvt = seqa_tr<T, DP>(gVr, 32 * c, t, lo);
                __builtin_amdgcn_sched_barrier(0);
                X[t] = mma_seq<T>(X[t], kt, m1b);
                X[t] = mma_seq<T>(X[t], gkt, dsb);
                U[t] = mma_seq<T>(U[t], kt, dsb);
                Z[t] = mma_seq<T>(Z[t], kt, pb);
                W[t] = mma_seq<T>(W[t], vt, pab);
                W[t] = mma_seq<T>(W[t], gvt, pb);
            }
        }
    };
    // One 16-key tile of the short stage, keys x0 .. x0 + 15, those at nv and past masked (k = 16 MFMA).
    auto tile16 = [&](const unsigned char* Kr, int x0, int nv) {
        const unsigned char* gKr = Kr + SB;
        const unsigned char* Vr = Kr + 2 * SB;
        const unsigned char* gVr = Kr + 3 * SB;
        f32x4 p = {0.f, 0.f, 0.f, 0.f}, at = p, dp = p, bm = p;
        mma_d_sw<T, DP>(p, Kr, x0, qf, lo);
        mma_d_sw<T, DP>(at, Kr, x0, gqf, lo);
        mma_d_sw<T, DP>(at, gKr, x0, qf, lo);
        mma_d_sw<T, DP>(dp, Vr, x0, df, lo);
        mma_d_sw<T, DP>(bm, gVr, x0, df, lo);
        elementwise(p, at, dp, bm, [&](int r) { return x0 + 4 * w.g + r < nv; });
        const u32x2 pb = pack4<T>(p);
        const u32x2 dsb = pack4<T>(dp);
        const u32x2 pab = pack4<T>(at);
        const u32x2 m1b = pack4<T>(bm);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) {
            const u32x2 kt = seqa_tr16<T, DP>(Kr, x0, t, lo);
            X[t] = ET<T>::mma16(kt, m1b, X[t]);
            X[t] = ET<T>::mma16(seqa_tr16<T, DP>(gKr, x0, t, lo), dsb, X[t]);
            U[t] = ET<T>::mma16(kt, dsb, U[t]);
            Z[t] = ET<T>::mma16(kt, pb, Z[t]);
            W[t] = ET<T>::mma16(seqa_tr16<T, DP>(Vr, x0, t, lo), pab, W[t]);
            W[t] = ET<T>::mma16(seqa_tr16<T, DP>(gVr, x0, t, lo), pb, W[t]);
        }
    };
    if (so.tail) {
        lds_barrier();  // stage 0, the short one, in its buffer
        if (active) {
            const int nv = L - so.nfull * STG;
#pragma nounroll
            for (int x0 = 0; x0 < nv; x0 += 16) tile16(smem, x0, nv);
        }
    }
    for (int i = so.tail ? 1 : 0; i < nst; ++i) {
        lds_barrier();  // stage i in its buffer
        if (!active) continue;
        stage(smem + (i & 1) * STB);
    }
    if (!active) return;
    const float E = xsum4(e_acc);
    const float Tm = xsum4(t_acc);
    if (own < L) {
        const int64_t r = (int64_t)bh * L + own;
        if (w.g == 0) {
            a.stats[r] = dr;
            a.stats[a.bhl + r] = E;
            a.stats[2 * a.bhl + r] = Tm;
        }
        const T* orow = reinterpret_cast<const T*>(a.o) + r * DP;
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) {
            X[t] = X[t] - E * U[t] - Tm * Z[t];
            W[t] = W[t] - E * load4<T>(orow + 16 * t + 4 * w.g);  // O in the accumulator's lane layout
        }
        store_rows<T, DP>(a.out0, r * DP, X, sc, DP, w.g);
        store_rows<T, DP>(a.out3, r * DP, W, 1.f, DP, w.g);
    }
}

// =====================================================================================================================
// Backward of the backward, col kernel: own = keys, over the Q, gQ, dO stages with the stages' lse, Dr, E, T:
//   dS2 = dS o A + P o Bm - E dS - T P,  Pa = P o A - E P,  hK = s (dS2^T Q + dS^T gQ),  hV = Pa^T dO.
// =====================================================================================================================

template <typename T, int DP, int NWC> __global__ __launch_bounds__(64 * (NWC + 1)) void k_bb_long_col(Args a) {
    using LY = Lay<T, DP>;
    using C = LongCfg<T, DP, NWC>;
    constexpr int STB = 3 * C::SB + 4 * LSTAGE * 4;  // Q, gQ, dO, [lse * log2 e | Dr | E | T]
    __shared__ __align__(1024) unsigned char smem[2 * STB];
    const WaveIds w = wave_ids();
    int bh, blk;
    decode_block(a, bh, blk);
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    const int nst = (L + LSTAGE - 1) / LSTAGE;
    const StageOrder so(L, LSTAGE);

    if (w.wave == NWC) {
        const T* Qg = slice<T>(a.q, b, h);
        const T* gQg = slice<T>(a.gq, b, h);
        const T* Og = slice<T>(a.dO, b, h);
        StageStats<3> stt;
        loader_loop<STB>(
            smem, nst,
            [&](int i, unsigned char* buf) {
                const int r0 = so.row(i);
                async_stage<T, DP>(buf, Qg, a.q.sl, L, r0, w.lane);
                async_stage<T, DP>(buf + C::SB, gQg, a.gq.sl, L, r0, w.lane);
                async_stage<T, DP>(buf + 2 * C::SB, Og, a.dO.sl, L, r0, w.lane);
                stt.load(a, bh, r0, w.lane);
            },
            [&](int i, unsigned char* buf) {
                stt.put(reinterpret_cast<float*>(buf + 3 * C::SB), so.row(i), L, w.lane);
            });
        return;
    }

    const int row0 = blk * C::ROWS + w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    OwnFrag<T, DP> kf, gkf, vf, gvf;
    load_own<T, DP>(kf, slice<T>(a.k, b, h), a.k.sl, own, L, DP, w.g);
    load_own<T, DP>(gkf, slice<T>(a.gk, b, h), a.gk.sl, own, L, DP, w.g);
    load_own<T, DP>(vf, slice<T>(a.v, b, h), a.v.sl, own, L, DP, w.g);
    load_own<T, DP>(gvf, slice<T>(a.gv, b, h), a.gv.sl, own, L, DP, w.g);
    const LaneOff<T, DP> lo(w.l16, w.g);
    const float sc = a.scale;
    const float sc2 = sc * LOG2E;
    f32x4 hk[LY::NT], hv[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) hk[t] = hv[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // One 16-row tile's dS2, dS and Pa from its products (accumulator layout: p, at, dp, bm hold S, A, dP, Bm on
    // entry; dS2, Pa, dS on return in p, at, dp) and the statistics of its rows at st + x.
    // With E and T known, dS2 = dS (A - E) + P (Bm - T) and Pa = P (A - E): the centred forms of
    // dS o A + P o Bm - E dS - T P and P o A - E P, two VALU operations fewer per element.
    auto elementwise = [&](f32x4& p, f32x4& at, f32x4& dp, const f32x4& bm, const float* st, int x) {
        const f32x4 l2 = *reinterpret_cast<const f32x4*>(st + x);
        const f32x4 d2 = *reinterpret_cast<const f32x4*>(st + LSTAGE + x);
        const f32x4 e2 = *reinterpret_cast<const f32x4*>(st + 2 * LSTAGE + x);
        const f32x4 t2 = *reinterpret_cast<const f32x4*>(st + 3 * LSTAGE + x);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pv = fast_exp2(fmaf(p[r], sc2, -l2[r]));  // lse = +inf past L: P = 0
            const float dsv = pv * (dp[r] - d2[r]);
            const float ae = fmaf(at[r], sc, -e2[r]);
            p[r] = fmaf(dsv, ae, pv * (bm[r] - t2[r]));  // dS2
            dp[r] = dsv;
            at[r] = pv * ae;  // Pa
        }
    };
    // One 16-row tile of the short stage, rows x0 .. x0 + 15 (k = 16 MFMA).
    auto tile16 = [&](const unsigned char* Qr, const float* st, int x0) {
        const unsigned char* gQr = Qr + C::SB;
        const unsigned char* Or = Qr + 2 * C::SB;
        f32x4 p = {0.f, 0.f, 0.f, 0.f}, at = p, dp = p, bm = p;
        mma_d_sw<T, DP>(p, Qr, x0, kf, lo);
        mma_d_sw<T, DP>(at, gQr, x0, kf, lo);
        mma_d_sw<T, DP>(at, Qr, x0, gkf, lo);
        mma_d_sw<T, DP>(dp, Or, x0, vf, lo);
        mma_d_sw<T, DP>(bm, Or, x0, gvf, lo);
        elementwise(p, at, dp, bm, st, x0 + 4 * w.g);
        const u32x2 d2b = pack4<T>(p);
        const u32x2 dsb = pack4<T>(dp);
        const u32x2 peb = pack4<T>(at);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) {
            hk[t] = ET<T>::mma16(seqa_tr16<T, DP>(Qr, x0, t, lo), d2b, hk[t]);
            hk[t] = ET<T>::mma16(seqa_tr16<T, DP>(gQr, x0, t, lo), dsb, hk[t]);
            hv[t] = ET<T>::mma16(seqa_tr16<T, DP>(Or, x0, t, lo), peb, hv[t]);
        }
    };
    if (so.tail) {
        lds_barrier();  // stage 0, the short one, in its buffer
        if (active) {
            const int nv = L - so.nfull * LSTAGE;
#pragma nounroll
            for (int x0 = 0; x0 < nv; x0 += 16) tile16(smem, reinterpret_cast<const float*>(smem + 3 * C::SB), x0);
        }
    }
    for (int i = so.tail ? 1 : 0; i < nst; ++i) {
        lds_barrier();  // stage i in its buffer
        if (!active) continue;
        const unsigned char* Qr = smem + (i & 1) * STB;
        const unsigned char* gQr = Qr + C::SB;
        const unsigned char* Or = Qr + 2 * C::SB;  // dO
        const float* st = reinterpret_cast<const float*>(Qr + 3 * C::SB);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            f32x4 p[2], at[2], dp[2], bm[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                p[hh] = at[hh] = dp[hh] = bm[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
                const int x0 = 32 * c + 16 * hh;
                {
                    u32x4 qa[LY::NC], gqa[LY::NC];
#pragma unroll
                    for (int q = 0; q < LY::NC; ++q) {
                        const int o = x0 * Sw<DP>::ROWB + lo.a[q];
                        qa[q] = *reinterpret_cast<const u32x4*>(Qr + o);
                        gqa[q] = *reinterpret_cast<const u32x4*>(gQr + o);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < LY::NC; ++q) {
                        p[hh] = ET<T>::mma(qa[q], kf.v[q], p[hh]);
                        at[hh] = ET<T>::mma(gqa[q], kf.v[q], at[hh]);
                        at[hh] = ET<T>::mma(qa[q], gkf.v[q], at[hh]);
                    }
                }
                {
                    u32x4 oa[LY::NC];
#pragma unroll
                    for (int q = 0; q < LY::NC; ++q) oa[q] = *reinterpret_cast<const u32x4*>(Or + x0 * Sw<DP>::ROWB + lo.a[q]);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < LY::NC; ++q) {
                        dp[hh] = ET<T>::mma(oa[q], vf.v[q], dp[hh]);
                        bm[hh] = ET<T>::mma(oa[q], gvf.v[q], bm[hh]);
                    }
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) elementwise(p[hh], at[hh], dp[hh], bm[hh], st, 32 * c + 16 * hh + 4 * w.g);
            const SeqB<T> d2b = make_seqb<T>(p[0], p[1]);
            const SeqB<T> dsb = make_seqb<T>(dp[0], dp[1]);
            const SeqB<T> peb = make_seqb<T>(at[0], at[1]);
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) {
                const SeqA<T> qt = seqa_tr<T, DP>(Qr, 32 * c, t, lo);
                const SeqA<T> gqt = seqa_tr<T, DP>(gQr, 32 * c, t, lo);
                const SeqA<T> ot = seqa_tr<T, DP>(Or, 32 * c, t, lo);
                __builtin_amdgcn_sched_barrier(0);
                hk[t] = mma_seq<T>(hk[t], qt, d2b);
                hk[t] = mma_seq<T>(hk[t], gqt, dsb);
                hv[t] = mma_seq<T>(hv[t], ot, peb);
            }
        }
    }
    if (active && own < L) {
        const int64_t r = ((int64_t)bh * L + own) * DP;
        store_rows<T, DP>(a.out1, r, hk, sc, DP, w.g);
        store_rows<T, DP>(a.out2, r, hv, 1.f, DP, w.g);
    }
}
