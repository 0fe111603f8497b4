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
    // Depends on x mod 16 only, so every 16-row tile (and every 32-row chunk) has the same per-lane pattern.
    static __device__ __forceinline__ int swz(int x) {
        if constexpr (DP == 32) {
            return (x >> 2) & 3;
        } else if constexpr (DP == 64) {
            // bits 1 and 2 of x swapped: with 4 or more waves per CU, the A-operand reads of 16 rows x 2 chunk
            // positions then meet no bank conflict (measured with SQ_LDS_BANK_CONFLICT; the earlier
            // (x & 7) ^ (x >> 3 & 1) cost a quarter of the read cycles), and the transposed reads stay conflict-free
            return (x & 1) | ((x & 4) >> 1) | ((x & 2) << 1);
        } else {
            return x & 15;
        }
    }
    static __device__ __forceinline__ int off(int x, int c) { return x * ROWB + 16 * (c ^ swz(x)); }
};

// Per-lane byte offsets inside a 16-row tile (a) and a 32-row chunk (tr), fixed for the whole kernel.
template <typename T, int DP> struct LaneOff {
    int a[Lay<T, DP>::NC];   // A-operand / own-row read of chunk 4 c + g in row l16
    int tr[Lay<T, DP>::NT];  // transpose read of d tile t: row 4 g + (l16 >> 2), columns 16 t + 4 (l16 & 3)
    __device__ __forceinline__ LaneOff(int l16, int g) {
#pragma unroll
        for (int c = 0; c < Lay<T, DP>::NC; ++c) a[c] = Sw<DP>::off(l16, 4 * c + g);
        const int k = l16 >> 2, j = l16 & 3;
#pragma unroll
        for (int t = 0; t < Lay<T, DP>::NT; ++t) {
            const int d = 16 * t + 4 * j;
            tr[t] = Sw<DP>::off(4 * g + k, d >> 3) + (d & 7) * 2;
        }
    }
};

// Row stores through LDS. A seq-contraction accumulator holds, in lane (row l16, group g), columns 16 t + 4 g .. + 3 of
// the wave's 16 rows: stored directly, each instruction writes 32 bytes into each of 16 rows, and partial-row writes
// move about half the bytes per second of whole-row writes (measured: 3.5 against 6.5 TB/s for a pure write). So the
// wave writes its rounded rows into a private 16-row LDS area (16-byte chunks XOR-swizzled as in the regions) and reads
// them back as whole rows, 16 bytes per lane, for the global stores.
template <typename T, int DP> struct RowStage16 {
    static constexpr int BYTES = 16 * Sw<DP>::ROWB;  // one wave's area
};

// Lanes exchange data through the area, which the next tensor reuses right after: wave barriers keep every write
// before the reads and every read before the next writes (without them the compiler may let lanes that store nothing
// skip their read and write the next tensor's values before the other lanes have read these; it did for D = 32).

// ``pk[t]`` = columns 16 t + 4 g .. + 3 of row l16, rounded and packed (pack4). Rows row0 .. row0 + 15 of ``out``
// (contiguous, DP elements per row) are written where row0 + r < L.
template <typename T, int DP>
__device__ __forceinline__ void store_rows_staged(void* out, int64_t row0_off, int nvalid, const u32x2 (&pk)[DP / 16],
                                                  unsigned char* stage, int lane) {
    using S = Sw<DP>;
    const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int t = 0; t < DP / 16; ++t) {
        const int c = 2 * t + (g >> 1);  // 16-byte chunk of columns 16 t + 4 g
        *reinterpret_cast<u32x2*>(stage + l16 * S::ROWB + 16 * (c ^ S::swz(l16)) + 8 * (g & 1)) = pk[t];
    }
    __builtin_amdgcn_wave_barrier();
    constexpr int NI = 16 / S::RPI;
    u32x4 v[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int r = i * S::RPI + lane / S::NCK, c = lane % S::NCK;
        v[i] = *reinterpret_cast<const u32x4*>(stage + r * S::ROWB + 16 * (c ^ S::swz(r)));
    }
    __builtin_amdgcn_wave_barrier();
    T* o = reinterpret_cast<T*>(out) + row0_off;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int r = i * S::RPI + lane / S::NCK, c = lane % S::NCK;
        if (r < nvalid) *reinterpret_cast<u32x4*>(o + r * DP + 8 * c) = v[i];
    }
}

// The same from fp32 accumulators, each scaled by ``mul`` before rounding.
template <typename T, int DP>
__device__ __forceinline__ void store_acc_staged(void* out, int64_t row0_off, int nvalid, const f32x4 (&acc)[DP / 16],
                                                 float mul, unsigned char* stage, int lane) {
    u32x2 pk[DP / 16];
#pragma unroll
    for (int t = 0; t < DP / 16; ++t) pk[t] = pack4<T>(acc[t] * mul);
    store_rows_staged<T, DP>(out, row0_off, nvalid, pk, stage, lane);
}

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

// Own-side B fragment from a swizzled region: the 16 rows starting at ``row0`` (a multiple of 16), lane row l16.
template <typename T, int DP>
__device__ __forceinline__ void own_from_lds(OwnFrag<T, DP>& f, const unsigned char* region, int row0,
                                             const LaneOff<T, DP>& lo) {
    const unsigned char* base = region + row0 * Sw<DP>::ROWB;
#pragma unroll
    for (int c = 0; c < Lay<T, DP>::NC; ++c) f.v[c] = *reinterpret_cast<const u32x4*>(base + lo.a[c]);
}

// acc[m = x][n = own] += sum_d X[x][d] Own[own][d] for the 16 rows starting at ``row0`` (multiple of 16).
template <typename T, int DP>
__device__ __forceinline__ void mma_d_sw(f32x4& acc, const unsigned char* region, int row0, const OwnFrag<T, DP>& f,
                                         const LaneOff<T, DP>& lo) {
    const unsigned char* base = region + row0 * Sw<DP>::ROWB;
#pragma unroll
    for (int c = 0; c < Lay<T, DP>::NC; ++c) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(base + lo.a[c]);
        acc = ET<T>::mma(a, f.v[c], acc);
    }
}

// Seq-contraction A operand of d tile t for the 16 rows starting at x0, read transposed, for the k = 16 MFMA.
template <typename T, int DP>
__device__ __forceinline__ u32x2 seqa_tr16(const unsigned char* region, int x0, int t, const LaneOff<T, DP>& lo) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EBR_LDS s16x4*)(region + x0 * Sw<DP>::ROWB + lo.tr[t]));
    return __builtin_bit_cast(u32x2, v);
}

// Seq-contraction A operand of d tile t for the 32 rows starting at x0 (multiple of 32), read transposed.
template <typename T, int DP>
__device__ __forceinline__ SeqA<T> seqa_tr(const unsigned char* region, int x0, int t, const LaneOff<T, DP>& lo) {
    const unsigned char* base = region + x0 * Sw<DP>::ROWB + lo.tr[t];
    const s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EBR_LDS s16x4*)base);
    const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EBR_LDS s16x4*)(base + 16 * Sw<DP>::ROWB));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo4), h2 = __builtin_bit_cast(u32x2, hi4);
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

template <int C, int NCH, class F> __device__ __forceinline__ void static_for(F&& f) {
    if constexpr (C < NCH) {
        f(std::integral_constant<int, C>{});
        static_for<C + 1, NCH>(f);
    }
}

// P tile of a row pass (own = queries, exponent scale folded: sc2 = scale * log2 e, lse2 = lse * log2 e); keys past
// L are masked, which only the last chunk (LAST) can contain.
template <bool LAST>
__device__ __forceinline__ float row_p(float qk, float sc2, float lse2, int x, int L) {
    const float pv = fast_exp2(fmaf(qk, sc2, -lse2));
    if constexpr (LAST) return (x < L) ? pv : 0.f;
    return pv;
}

// =====================================================================================================================
// Forward: exact two-sweep softmax over the resident keys (the row maximum first, then exp, sum and P V).
// =====================================================================================================================

template <typename T, int DP, int NCH> __global__ __launch_bounds__(512) void k_fwd_res(Args a) {
    using LY = Lay<T, DP>;
    constexpr int Lp = NCH * CH;
    constexpr int RB = Lp * Sw<DP>::ROWB;
    // K, V. Once every wave has its scores, the K region holds the waves' row-store areas (the active waves' 16 rows
    // each, at most Lp rows), so the stores cost no LDS of their own.
    static_assert(2 * NCH * RowStage16<T, DP>::BYTES <= RB, "row-store areas in the K region");
    __shared__ __align__(1024) unsigned char smem[2 * RB];
    const WaveIds w = wave_ids();
    const int nw = w.nthr >> 6;
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    unsigned char* Kr = smem;
    unsigned char* Vr = smem + RB;
    async_rows<T, DP>(Kr, slice<T>(a.k, b, h), a.k.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(Vr, slice<T>(a.v, b, h), a.v.sl, L, Lp, w.wave, nw, w.lane);
    const int row0 = w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    OwnFrag<T, DP> qf;
    load_own<T, DP>(qf, slice<T>(a.q, b, h), a.q.sl, own, L, DP, w.g);
    const LaneOff<T, DP> lo(w.l16, w.g);
    async_wait();
    lds_barrier();
    if (!active) return;
    const float sc2 = a.scale * LOG2E;  // scores in log2 units
    f32x4 s[2 * NCH];
    float mx = -INFINITY;
    static_for<0, NCH>([&](auto cc) {
        constexpr int C = decltype(cc)::value;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            mma_d_sw<T, DP>(v, Kr, C * CH + 16 * hh, qf, lo);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                v[r] *= sc2;
                if constexpr (C == NCH - 1) {
                    if (C * CH + 16 * hh + 4 * w.g + r >= L) v[r] = -INFINITY;
                }
                mx = fmax_nn(mx, v[r]);
            }
            s[2 * C + hh] = v;
        }
    });
    const float m = xmax4(mx);
    lds_barrier();  // every active wave done with K (inactive ones have left)
    float lsum = 0.f;
    f32x4 acc[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    static_for<0, NCH>([&](auto cc) {
        constexpr int C = decltype(cc)::value;
        f32x4 p0 = s[2 * C], p1 = s[2 * C + 1];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p0[r] = fast_exp2(p0[r] - m);
            p1[r] = fast_exp2(p1[r] - m);
            lsum += p0[r] + p1[r];
        }
        const SeqB<T> pb = make_seqb<T>(p0, p1);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) acc[t] = mma_seq<T>(acc[t], seqa_tr<T, DP>(Vr, C * CH, t, lo), pb);
    });
    lsum = xsum4(lsum);
    store_acc_staged<T, DP>(a.out0, ((int64_t)bh * L + row0) * DP, L - row0, acc, 1.f / lsum,
                            Kr + w.wave * RowStage16<T, DP>::BYTES, w.lane);
    if (own < L && w.g == 0) a.lse_out[(int64_t)bh * L + own] = m * (1.f / LOG2E) + logf(lsum);
}

// =====================================================================================================================
// Backward: row pass (dQ) then col pass (dK, dV) on one slice.
// =====================================================================================================================

template <typename T, int DP, int NCH> struct BwdRes {
    static constexpr int RB = NCH * CH * Sw<DP>::ROWB;  // one tensor
    static constexpr bool SEP = 4 * RB <= 64 * 1024;     // K, V, Q, dO all resident at once
    static constexpr int SMEM = (SEP ? 4 : 2) * RB;
};

// At most 102 VGPRs (5 waves per SIMD), so that as many workgroups share a CU as its LDS holds: at L = 81, three of
// 6 waves and 50 KB each; the unconstrained build took 118 VGPRs and fit two.
template <typename T, int DP, int NCH>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(DP <= 64 && NCH <= 3 ? 5 : 1, 8))) void k_bwd_res(Args a) {
    using LY = Lay<T, DP>;
    using R = BwdRes<T, DP, NCH>;
    constexpr int Lp = NCH * CH;
    __shared__ __align__(1024) unsigned char smem[R::SMEM];
    __shared__ __align__(16) float st[2 * STAT_MAX];  // lse * log2 e, Dr
    const WaveIds w = wave_ids();
    const int nw = w.nthr >> 6;
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    unsigned char* Kr = smem;
    unsigned char* Vr = smem + R::RB;
    unsigned char* Qr = R::SEP ? smem + 2 * R::RB : smem;
    unsigned char* Or = R::SEP ? smem + 3 * R::RB : smem + R::RB;  // dO
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
    const float sc2 = sc * LOG2E;
    const int row0 = w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    const LaneOff<T, DP> lo(w.l16, w.g);

    // ---- row pass: own = queries
    {
        OwnFrag<T, DP> qf, df, of;
        load_own<T, DP>(qf, Qg, a.q.sl, own, L, DP, w.g);
        load_own<T, DP>(df, Og, a.dO.sl, own, L, DP, w.g);
        load_own<T, DP>(of, reinterpret_cast<const T*>(a.o) + (int64_t)bh * L * DP, DP, own, L, DP, w.g);
        const float lraw = a.lse[(int64_t)bh * L + (own < L ? own : L - 1)];  // unconditional load
        const float lse2 = (own < L) ? lraw * LOG2E : 0.f;
        const float dr = xsum4(frag_dot<T, DP>(df, of));
        async_wait();
        lds_barrier();  // regions loaded, statistics defaults written
        if (active) {
            if (w.g == 0) {
                st[own] = (own < L) ? lse2 : INFINITY;
                st[STAT_MAX + own] = (own < L) ? dr : 0.f;
            }
            f32x4 acc[LY::NT];
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                constexpr bool LAST = C == NCH - 1;
                const int x0 = C * CH;
                f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = p0, d1 = p0;
                mma_d_sw<T, DP>(p0, Kr, x0, qf, lo);
                mma_d_sw<T, DP>(p1, Kr, x0 + 16, qf, lo);
                mma_d_sw<T, DP>(d0, Vr, x0, df, lo);
                mma_d_sw<T, DP>(d1, Vr, x0 + 16, df, lo);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int x = x0 + 4 * w.g + r;
                    p0[r] = row_p<LAST>(p0[r], sc2, lse2, x, L);
                    p1[r] = row_p<LAST>(p1[r], sc2, lse2, x + 16, L);
                    d0[r] = p0[r] * (d0[r] - dr);
                    d1[r] = p1[r] * (d1[r] - dr);
                }
                const SeqB<T> dsb = make_seqb<T>(d0, d1);
#pragma unroll
                for (int t = 0; t < LY::NT; ++t) acc[t] = mma_seq<T>(acc[t], seqa_tr<T, DP>(Kr, x0, t, lo), dsb);
            });
            if (own < L) store_rows<T, DP>(a.out0, ((int64_t)bh * L + own) * DP, acc, sc, DP, w.g);
        }
    }
    lds_barrier();  // statistics published; K, V no longer read by the row pass

    // ---- col pass: own = keys
    OwnFrag<T, DP> kf, vf;
    if (active) {
        own_from_lds<T, DP>(kf, Kr, row0, lo);
        own_from_lds<T, DP>(vf, Vr, row0, lo);
    }
    if constexpr (!R::SEP) {
        lds_barrier();  // every wave holds its K, V rows before Q, dO overwrite them
        async_rows<T, DP>(Qr, Qg, a.q.sl, L, Lp, w.wave, nw, w.lane);
        async_rows<T, DP>(Or, Og, a.dO.sl, L, Lp, w.wave, nw, w.lane);
        async_wait();
        lds_barrier();
    }
    if (!active) return;
    f32x4 ak[LY::NT], av[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) ak[t] = av[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    static_for<0, NCH>([&](auto cc) {
        constexpr int C = decltype(cc)::value;
        const int x0 = C * CH;
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(st + x0 + 4 * w.g);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(st + x0 + 16 + 4 * w.g);
        const f32x4 r0 = *reinterpret_cast<const f32x4*>(st + STAT_MAX + x0 + 4 * w.g);
        const f32x4 r1 = *reinterpret_cast<const f32x4*>(st + STAT_MAX + x0 + 16 + 4 * w.g);
        f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = p0, d1 = p0;
        mma_d_sw<T, DP>(p0, Qr, x0, kf, lo);
        mma_d_sw<T, DP>(p1, Qr, x0 + 16, kf, lo);
        mma_d_sw<T, DP>(d0, Or, x0, vf, lo);
        mma_d_sw<T, DP>(d1, Or, x0 + 16, vf, lo);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p0[r] = fast_exp2(fmaf(p0[r], sc2, -l0[r]));  // lse = +inf on padded query rows -> P = 0
            p1[r] = fast_exp2(fmaf(p1[r], sc2, -l1[r]));
            d0[r] = p0[r] * (d0[r] - r0[r]);
            d1[r] = p1[r] * (d1[r] - r1[r]);
        }
        const SeqB<T> pb = make_seqb<T>(p0, p1);
        const SeqB<T> dsb = make_seqb<T>(d0, d1);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) {
            av[t] = mma_seq<T>(av[t], seqa_tr<T, DP>(Or, x0, t, lo), pb);
            ak[t] = mma_seq<T>(ak[t], seqa_tr<T, DP>(Qr, x0, t, lo), dsb);
        }
    });
    if (own < L) {
        const int64_t r = ((int64_t)bh * L + own) * DP;
        store_rows<T, DP>(a.out1, r, ak, sc, DP, w.g);
        store_rows<T, DP>(a.out2, r, av, 1.f, DP, w.g);
    }
}

// =====================================================================================================================
// Backward, persistent with a loader wave (16-bit inputs, D <= 64, L <= 96): two LDS buffers of K, V, Q, dO and lse.
// The workgroup (one per CU) takes slices s, s + G, ... (G = gridDim.x); while its compute waves (one per 16 rows)
// work on slice s in one buffer, the loader wave fills the other with slice s + G by global -> LDS loads. Compute
// waves never have such a load outstanding, so their LDS transpose reads are never held back by one.
// The row pass writes its P and dS tiles (rounded to the input type) as [query][key] rows; the col pass then is two
// plain GEMMs from the tiles, dV = P^T dO and dK = s dS^T Q: 5 GEMM units for the backward, no recomputation.
// The loader also scales lse and reduces rowsum(dO o O) of the next slice, so the compute waves issue no global loads.
//   compute waves                     loader wave
//   row pass (s): dQ, tiles           loads of slice n = s + G into the other buffer, its O rows into registers
//   --- barrier X: tiles complete
//   col pass (s): dK, dV              wait for the loads; lse (n) and rowsum(dO o O) (n) into the other buffer
//   --- barrier Y: buffer of s and the tiles free, buffer of n complete
// =====================================================================================================================

// Dot product of two 8-element 16-bit vectors in fp32.
template <typename T> __device__ __forceinline__ float dot8(u32x4 a, u32x4 b) {
    using V8 = typename ET<T>::v8;
    const V8 x = __builtin_bit_cast(V8, a), y = __builtin_bit_cast(V8, b);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (float)x[e] * (float)y[e];
    return s;
}

template <typename T, int DP, int NCH> struct BwdPipe {
    static constexpr int LP = NCH * CH;
    static constexpr int RB = LP * Sw<DP>::ROWB;  // one natural tensor region
    static constexpr int TP = LP * 2 + 32;        // tile row pitch (bytes), padded off the 256-byte bank period
    static constexpr int TB = LP * TP;            // one tile
    static constexpr int NWC = 2 * NCH;           // compute waves
    static constexpr int BUF = 4 * RB;            // K, V, Q, dO
    // Where the P and dS tiles fit beside the two buffers (D = 64: up to three 32-row chunks; D = 128: one) the col
    // pass reads them (5 GEMM units); otherwise it recomputes P and dS from the buffer (7 GEMM units, loads still
    // overlapped with the previous slice's work).
    static constexpr int STORES = NWC * RowStage16<T, DP>::BYTES;
    static constexpr bool TILES = 2 * BUF + 2 * TB + 4 * LP * 4 + STORES <= 160 * 1024;
    static constexpr int STG = 2 * BUF + (TILES ? 2 * TB : 0) + 4 * LP * 4;  // byte offset of the store areas
    // two buffers | P, dS tiles | lse * log2 e (two) | rowsum(dO o O) (two) | a row-store area per compute wave
    static constexpr int SMEM = STG + STORES;
    static constexpr int THREADS = 64 * (NWC + 1);
    static constexpr bool FITS = SMEM <= 160 * 1024;
};

// Byte offset of keys key0 .. key0 + 3 (key0 a multiple of 4) of tile row ``row``. The 8-byte group of four keys
// moves to group (key0 / 4) ^ 2 in rows with bit 3 set: under the pitch (an odd multiple of 32 bytes past a multiple
// of 256) rows r and r + 8 start on the same bank, so a store's half-wave of 16 rows at two groups each hit every bank
// twice; with the swap it hits each once (bwd_bwd at config 1: 162.6 -> 158.2 us). The transposed reads take 8 rows
// and 4 groups per half-wave, conflict-free either way.
__device__ __forceinline__ int tile_off(int row, int pitch, int key0) {
    return row * pitch + ((((key0 >> 2) ^ ((row >> 2) & 2))) << 3);
}

// 8-byte tile write: row ``row`` (query), keys key0 .. key0 + 3 (4 packed 16-bit values).
__device__ __forceinline__ void tile_store8(unsigned char* tile, int pitch, int row, int key0, u32x2 v) {
    *reinterpret_cast<u32x2*>(tile + tile_off(row, pitch, key0)) = v;
}

// B operand of a col pass from a [query][key] tile: lane (key = kb + l16, group g), k-slot 4 h + k holds
// tile[x0 + 16 h + 4 g + k][kb + l16].
template <typename T>
__device__ __forceinline__ SeqB<T> tile_seqb(const unsigned char* tile, int pitch, int x0, int kb, int l16, int g) {
    const int k = l16 >> 2, j = l16 & 3;
    const unsigned char* p = tile + tile_off(x0 + 4 * g + k, pitch, kb + 4 * j);  // row + 16 below: same swap
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EBR_LDS s16x4*)p);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EBR_LDS s16x4*)(p + 16 * pitch));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
    SeqB<T> b;
    b.v = u32x4{l2[0], l2[1], h2[0], h2[1]};
    return b;
}

// Zero the tile rows of a wave whose 16 rows are all past L.
template <int NCH>
__device__ __forceinline__ void zero_tile_rows(unsigned char* t0, unsigned char* t1, unsigned char* t2, int pitch,
                                               int own, int g) {
    const u32x2 z = {0u, 0u};
#pragma unroll
    for (int C = 0; C < NCH; ++C) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int key0 = C * CH + 16 * hh + 4 * g;
            tile_store8(t0, pitch, own, key0, z);
            tile_store8(t1, pitch, own, key0, z);
            if (t2) tile_store8(t2, pitch, own, key0, z);
        }
    }
}

template <typename T, int DP, int NCH> __global__ __launch_bounds__(64 * (2 * NCH + 1)) void k_bwd_pipe(Args a) {
    using LY = Lay<T, DP>;
    using R = BwdPipe<T, DP, NCH>;
    constexpr int Lp = R::LP;
    __shared__ __align__(1024) unsigned char smem[R::SMEM];
    const WaveIds w = wave_ids();
    const int L = a.L;
    const int nbh = a.B * a.H;
    unsigned char* TPr = smem + 2 * R::BUF;  // P (when R::TILES)
    unsigned char* TSr = TPr + R::TB;        // dS (when R::TILES)
    float* lse_buf = reinterpret_cast<float*>(smem + 2 * R::BUF + (R::TILES ? 2 * R::TB : 0));  // [2][LP]
    float* dr_buf = lse_buf + 2 * Lp;                              // [2][LP]
    int s = blockIdx.x;

    if (w.wave == R::NWC) {
        // ---- loader wave: lane t handles rows t and t + 64 for lse and rowsum(dO o O)
        constexpr int NCK = Sw<DP>::NCK;
        constexpr bool TWO = Lp > 64;  // a second row per lane
        const int t0 = w.lane, t1 = w.lane + 64;
        float lv0 = 0.f, lv1 = 0.f;
        u32x4 o0[NCK], o1[TWO ? NCK : 1];  // O rows t0, t1 (rows past L: row L - 1, finite; rowsum written as 0)
        auto issue = [&](int sl, int bsel) {
            const int b = sl / a.H, h = sl - b * a.H;
            unsigned char* base = smem + bsel * R::BUF;
            async_rows<T, DP>(base, slice<T>(a.k, b, h), a.k.sl, L, Lp, 0, 1, w.lane);
            async_rows<T, DP>(base + R::RB, slice<T>(a.v, b, h), a.v.sl, L, Lp, 0, 1, w.lane);
            async_rows<T, DP>(base + 2 * R::RB, slice<T>(a.q, b, h), a.q.sl, L, Lp, 0, 1, w.lane);
            async_rows<T, DP>(base + 3 * R::RB, slice<T>(a.dO, b, h), a.dO.sl, L, Lp, 0, 1, w.lane);
            lv0 = a.lse[(int64_t)sl * L + (t0 < L ? t0 : L - 1)];  // unconditional loads
            const T* ob = reinterpret_cast<const T*>(a.o) + (int64_t)sl * L * DP;
            const T* p0 = ob + (int64_t)(t0 < L ? t0 : L - 1) * DP;
#pragma unroll
            for (int c = 0; c < NCK; ++c) o0[c] = *reinterpret_cast<const u32x4*>(p0 + 8 * c);
            if constexpr (TWO) {
                lv1 = a.lse[(int64_t)sl * L + (t1 < L ? t1 : L - 1)];
                const T* p1 = ob + (int64_t)(t1 < L ? t1 : L - 1) * DP;
#pragma unroll
                for (int c = 0; c < NCK; ++c) o1[c] = *reinterpret_cast<const u32x4*>(p1 + 8 * c);
            }
        };
        auto rowsum = [&](const unsigned char* dor, int t, const u32x4(&o)[NCK]) {
            float d = 0.f;
#pragma unroll
            for (int c = 0; c < NCK; ++c) d += dot8<T>(*reinterpret_cast<const u32x4*>(dor + Sw<DP>::off(t, c)), o[c]);
            return t < L ? d : 0.f;
        };
        auto finish = [&](int bsel) {
            async_wait();
            float* l2 = lse_buf + bsel * Lp;
            float* d2 = dr_buf + bsel * Lp;
            const unsigned char* dor = smem + bsel * R::BUF + 3 * R::RB;
            if (t0 < Lp) {
                l2[t0] = t0 < L ? lv0 * LOG2E : INFINITY;  // padded query rows: P = 0
                d2[t0] = rowsum(dor, t0, o0);
            }
            if constexpr (TWO) {
                if (t1 < Lp) {
                    l2[t1] = t1 < L ? lv1 * LOG2E : INFINITY;
                    d2[t1] = rowsum(dor, t1, o1);
                }
            }
        };
        issue(s, 0);
        finish(0);
        lds_barrier();
        for (int it = 0;; ++it) {
            const int n = s + (int)gridDim.x;
            const bool more = n < nbh;  // uniform over the workgroup
            const int nb = (it & 1) ^ 1;
            if (more) issue(n, nb);
            lds_barrier();  // X
            if (!more) break;
            finish(nb);
            lds_barrier();  // Y
            s = n;
        }
        return;
    }

    // ---- compute waves
    const float sc = a.scale;
    const float sc2 = sc * LOG2E;
    const int row0 = w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    const LaneOff<T, DP> lo(w.l16, w.g);
    unsigned char* stage = smem + R::STG + w.wave * RowStage16<T, DP>::BYTES;
    lds_barrier();  // the first slice is in buffer 0
    for (int it = 0;; ++it) {
        const int n = s + (int)gridDim.x;
        const bool more = n < nbh;
        const int bsel = it & 1;
        unsigned char* Kr = smem + bsel * R::BUF;
        unsigned char* Vr = Kr + R::RB;
        unsigned char* Qr = Kr + 2 * R::RB;
        unsigned char* Or = Kr + 3 * R::RB;  // dO
        const float* l2 = lse_buf + bsel * Lp;

        // ---- row pass: own = queries; dQ and the P, dS tiles
        if (active) {
            OwnFrag<T, DP> qf, df;
            own_from_lds<T, DP>(qf, Qr, row0, lo);  // rows past L are 0 in the regions
            own_from_lds<T, DP>(df, Or, row0, lo);
            const float lse2 = l2[own];
            const float dr = dr_buf[bsel * Lp + own];
            f32x4 acc[LY::NT];
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                constexpr bool LAST = C == NCH - 1;
                const int x0 = C * CH;
                // the dP accumulators start at -Dr, so dS = P (dP - Dr) takes one multiply per element
                f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = {-dr, -dr, -dr, -dr}, d1 = d0;
                mma_d_sw<T, DP>(p0, Kr, x0, qf, lo);
                mma_d_sw<T, DP>(p1, Kr, x0 + 16, qf, lo);
                mma_d_sw<T, DP>(d0, Vr, x0, df, lo);
                mma_d_sw<T, DP>(d1, Vr, x0 + 16, df, lo);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int x = x0 + 4 * w.g + r;
                    p0[r] = row_p<LAST>(p0[r], sc2, lse2, x, L);  // lse = +inf on padded query rows -> P = 0
                    p1[r] = row_p<LAST>(p1[r], sc2, lse2, x + 16, L);
                    d0[r] = p0[r] * d0[r];
                    d1[r] = p1[r] * d1[r];
                }
                const SeqB<T> dsb = make_seqb<T>(d0, d1);
                if constexpr (R::TILES) {
                    const SeqB<T> pb = make_seqb<T>(p0, p1);
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int key0 = x0 + 16 * hh + 4 * w.g;
                        tile_store8(TPr, R::TP, own, key0, u32x2{pb.v[2 * hh], pb.v[2 * hh + 1]});
                        tile_store8(TSr, R::TP, own, key0, u32x2{dsb.v[2 * hh], dsb.v[2 * hh + 1]});
                    }
                }
#pragma unroll
                for (int t = 0; t < LY::NT; ++t) acc[t] = mma_seq<T>(acc[t], seqa_tr<T, DP>(Kr, x0, t, lo), dsb);
            });
            store_acc_staged<T, DP>(a.out0, ((int64_t)s * L + row0) * DP, L - row0, acc, sc, stage, w.lane);
        } else if constexpr (R::TILES) {
            zero_tile_rows<NCH>(TPr, TSr, nullptr, R::TP, own, w.g);
        }
        lds_barrier();  // X: tiles complete

        // ---- col pass: own = keys; dV = P^T dO, dK = s dS^T Q from the tiles, or with P and dS recomputed
        if (active) {
            f32x4 ak[LY::NT], av[LY::NT];
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) ak[t] = av[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            OwnFrag<T, DP> kf, vf;
            if constexpr (!R::TILES) {
                own_from_lds<T, DP>(kf, Kr, row0, lo);
                own_from_lds<T, DP>(vf, Vr, row0, lo);
            }
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                const int x0 = C * CH;
                SeqB<T> pb, dsb;
                if constexpr (R::TILES) {
                    pb = tile_seqb<T>(TPr, R::TP, x0, row0, w.l16, w.g);
                    dsb = tile_seqb<T>(TSr, R::TP, x0, row0, w.l16, w.g);
                } else {
                    const float* dr2 = dr_buf + bsel * Lp;
                    const f32x4 l0 = *reinterpret_cast<const f32x4*>(l2 + x0 + 4 * w.g);
                    const f32x4 l1 = *reinterpret_cast<const f32x4*>(l2 + x0 + 16 + 4 * w.g);
                    const f32x4 r0 = *reinterpret_cast<const f32x4*>(dr2 + x0 + 4 * w.g);
                    const f32x4 r1 = *reinterpret_cast<const f32x4*>(dr2 + x0 + 16 + 4 * w.g);
                    f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = -r0, d1 = -r1;
                    mma_d_sw<T, DP>(p0, Qr, x0, kf, lo);
                    mma_d_sw<T, DP>(p1, Qr, x0 + 16, kf, lo);
                    mma_d_sw<T, DP>(d0, Or, x0, vf, lo);
                    mma_d_sw<T, DP>(d1, Or, x0 + 16, vf, lo);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        p0[r] = fast_exp2(fmaf(p0[r], sc2, -l0[r]));  // lse = +inf on padded query rows -> P = 0
                        p1[r] = fast_exp2(fmaf(p1[r], sc2, -l1[r]));
                        d0[r] = p0[r] * d0[r];
                        d1[r] = p1[r] * d1[r];
                    }
                    pb = make_seqb<T>(p0, p1);
                    dsb = make_seqb<T>(d0, d1);
                }
#pragma unroll
                for (int t = 0; t < LY::NT; ++t) {
                    av[t] = mma_seq<T>(av[t], seqa_tr<T, DP>(Or, x0, t, lo), pb);
                    ak[t] = mma_seq<T>(ak[t], seqa_tr<T, DP>(Qr, x0, t, lo), dsb);
                }
            });
            const int64_t r = ((int64_t)s * L + row0) * DP;
            store_acc_staged<T, DP>(a.out1, r, L - row0, ak, sc, stage, w.lane);
            store_acc_staged<T, DP>(a.out2, r, L - row0, av, 1.f, stage, w.lane);
        }
        if (!more) break;
        lds_barrier();  // Y: this buffer and the tiles free, the other buffer holds slice n
        s = n;
    }
}

// =====================================================================================================================
// Backward, persistent with a loader wave for shapes whose two full buffers do not fit the LDS (D = 128, 65 <= L <= 112):
// one K, V region (X) and one Q, dO region (Y), each filled one pass ahead of its use.
//   compute waves                                  loader wave
//   row pass (s): dQ from X; own K, V rows -> regs  loads Y <- Q, dO of slice s
//   --- barrier A: X free, Y holds s
//   col pass (s): dK, dV from Y (P, dS recomputed);  loads X <- K, V of slice n = s + G
//                 own Q, dO, O rows of n -> regs
//   --- barrier B: Y free, X holds n
// The row pass takes its own Q, dO rows (and O, for Dr = rowsum(dO o O)) from global memory, loaded during the
// previous col pass: that is the one input read twice (the second read, Y's, a few microseconds later). 7 GEMM units
// as in k_bwd_res, with the loads of the next slice overlapped with this one's work.
// =====================================================================================================================

constexpr int bwd_pp_waves(int nch) { return 2 * nch > 7 ? 7 : 2 * nch; }  // compute waves (16 rows each)

template <typename T, int DP, int NCH> struct BwdPP {
    static constexpr int LP = NCH * CH;
    static constexpr int RB = LP * Sw<DP>::ROWB;
    static constexpr int NWC = bwd_pp_waves(NCH);           // L <= 16 NWC
    static constexpr int ST = 4 * RB;                       // lse * log2 e [LP] | Dr [LP]
    static constexpr int STG = ST + 2 * LP * 4;             // a row-store area per compute wave
    static constexpr int SMEM = STG + NWC * RowStage16<T, DP>::BYTES;
    static constexpr int THREADS = 64 * (NWC + 1);
    static constexpr bool FITS = SMEM <= 160 * 1024;
};

// HALF (L <= 32 NCH - 16): the last chunk holds one 16-row tile; rows past it are neither loaded nor read.
template <typename T, int DP, int NCH, bool HALF>
__global__ __launch_bounds__(64 * (bwd_pp_waves(NCH) + 1)) void k_bwd_pp(Args a) {
    using LY = Lay<T, DP>;
    using R = BwdPP<T, DP, NCH>;
    constexpr int Lp = R::LP;
    constexpr int LR = Lp - (HALF ? 16 : 0);  // rows loaded into the regions
    __shared__ __align__(1024) unsigned char smem[R::SMEM];
    unsigned char* Kr = smem;
    unsigned char* Vr = smem + R::RB;
    unsigned char* Qr = smem + 2 * R::RB;
    unsigned char* Or = smem + 3 * R::RB;  // dO
    float* l2s = reinterpret_cast<float*>(smem + R::ST);
    float* drs = l2s + Lp;
    const WaveIds w = wave_ids();
    const int L = a.L;
    const int nbh = a.B * a.H;
    int s = blockIdx.x;
    if (s >= nbh) return;  // uniform over the workgroup

    if (w.wave == R::NWC) {
        // ---- loader wave; statistics rows of no active wave (past L rounded up to 16): P = 0 and Dr = 0 there
        for (int x = (L + 15) / 16 * 16 + w.lane; x < Lp; x += 64) {
            l2s[x] = INFINITY;
            drs[x] = 0.f;
        }
        auto region2 = [&](unsigned char* r0, const Strided& t0, unsigned char* r1, const Strided& t1, int sl) {
            const int b = sl / a.H, h = sl - b * a.H;
            async_rows<T, DP>(r0, slice<T>(t0, b, h), t0.sl, L, LR, 0, 1, w.lane);
            async_rows<T, DP>(r1, slice<T>(t1, b, h), t1.sl, L, LR, 0, 1, w.lane);
        };
        region2(Kr, a.k, Vr, a.v, s);
        async_wait();
        lds_barrier();  // X holds the first slice
        for (;;) {
            region2(Qr, a.q, Or, a.dO, s);
            async_wait();
            lds_barrier();  // A
            const int n = s + (int)gridDim.x;
            const bool more = n < nbh;
            if (more) region2(Kr, a.k, Vr, a.v, n);
            async_wait();
            lds_barrier();  // B
            if (!more) break;
            s = n;
        }
        return;
    }

    // ---- compute waves
    const float sc = a.scale;
    const float sc2 = sc * LOG2E;
    const int row0 = w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;  // wave-uniform; inactive waves still take every barrier
    const LaneOff<T, DP> lo(w.l16, w.g);
    unsigned char* stage = smem + R::STG + w.wave * RowStage16<T, DP>::BYTES;
    // Own Q, dO, O rows and lse of the slice the next row pass works on, loaded from global memory at the start of
    // the col pass before it and first used after the barrier that ends that pass, so that nothing waits for them
    // in between. The loads read row min(own, L - 1); rows past L are zeroed at their use.
    OwnFrag<T, DP> qf, df, of;
    float lraw = 0.f;
    const int orow = own < L ? own : L - 1;
    auto own_raw = [&](const T* base, int64_t srow, OwnFrag<T, DP>& f) {
        const T* p = base + (int64_t)orow * srow + w.g * LY::VEC;
#pragma unroll
        for (int c = 0; c < LY::NC; ++c) f.v[c] = *reinterpret_cast<const u32x4*>(p + c * LY::CW);
    };
    auto own_rows = [&](const Strided& t, int sl, OwnFrag<T, DP>& f) {
        const int b = sl / a.H, h = sl - b * a.H;
        own_raw(slice<T>(t, b, h), t.sl, f);
    };
    auto own_o = [&](int sl, OwnFrag<T, DP>& f) {
        own_raw(reinterpret_cast<const T*>(a.o) + (int64_t)sl * L * DP, DP, f);
    };
    auto own_lse = [&](int sl) { return a.lse[(int64_t)sl * L + orow]; };
    auto zero_past_l = [&](OwnFrag<T, DP>& f) {
#pragma unroll
        for (int c = 0; c < LY::NC; ++c) f.v[c] = own < L ? f.v[c] : u32x4{0u, 0u, 0u, 0u};
    };
    if (active) {
        own_rows(a.q, s, qf);
        own_rows(a.dO, s, df);
        own_o(s, of);
        lraw = own_lse(s);
    }
    lds_barrier();  // X holds the first slice
    for (;;) {
        const int n = s + (int)gridDim.x;
        const bool more = n < nbh;
        OwnFrag<T, DP> kf, vf, qn, dn, on;
        float lrn;  // set with qn, dn, on where ``more``; read only then

        // ---- row pass: own = queries; dQ
        if (active) {
            const float dr = own < L ? xsum4(frag_dot<T, DP>(df, of)) : 0.f;
            zero_past_l(qf);
            zero_past_l(df);
            const float lse2 = (own < L) ? lraw * LOG2E : 0.f;
            if (w.g == 0) {
                l2s[own] = (own < L) ? lse2 : INFINITY;  // padded query rows: P = 0
                drs[own] = (own < L) ? dr : 0.f;
            }
            f32x4 acc[LY::NT];
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                constexpr bool LAST = C == NCH - 1;
                const int x0 = C * CH;
                f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = p0, d1 = p0;
                constexpr bool H16 = HALF && LAST;  // keys past LR: no products, P masked to 0 below
                mma_d_sw<T, DP>(p0, Kr, x0, qf, lo);
                if (!H16) mma_d_sw<T, DP>(p1, Kr, x0 + 16, qf, lo);
                mma_d_sw<T, DP>(d0, Vr, x0, df, lo);
                if (!H16) mma_d_sw<T, DP>(d1, Vr, x0 + 16, df, lo);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int x = x0 + 4 * w.g + r;
                    p0[r] = row_p<LAST>(p0[r], sc2, lse2, x, L);
                    p1[r] = row_p<LAST>(p1[r], sc2, lse2, x + 16, L);
                    d0[r] = p0[r] * (d0[r] - dr);
                    d1[r] = p1[r] * (d1[r] - dr);
                }
                if constexpr (H16) {
                    const u32x2 dsb = pack4<T>(d0);
#pragma unroll
                    for (int t = 0; t < LY::NT; ++t) acc[t] = ET<T>::mma16(seqa_tr16<T, DP>(Kr, x0, t, lo), dsb, acc[t]);
                } else {
                    const SeqB<T> dsb = make_seqb<T>(d0, d1);
#pragma unroll
                    for (int t = 0; t < LY::NT; ++t) acc[t] = mma_seq<T>(acc[t], seqa_tr<T, DP>(Kr, x0, t, lo), dsb);
                }
            });
            own_from_lds<T, DP>(kf, Kr, row0, lo);
            own_from_lds<T, DP>(vf, Vr, row0, lo);
            store_acc_staged<T, DP>(a.out0, ((int64_t)s * L + row0) * DP, L - row0, acc, sc, stage, w.lane);
        }
        lds_barrier();  // A: statistics published, X free, Y holds slice s

        // ---- col pass: own = keys; dK = s dS^T Q, dV = P^T dO with P and dS recomputed. P and dS of every chunk are
        // kept as packed MFMA operands and the products run one half of the d tiles at a time, so that only half
        // of dK and dV is accumulated in fp32 at once.
        if (active) {
            if (more) {  // the next slice's own rows, landing during this pass
                own_rows(a.q, n, qn);
                own_rows(a.dO, n, dn);
                own_o(n, on);
                lrn = own_lse(n);
            }
            SeqB<T> pbs[NCH], dsbs[NCH];
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                constexpr bool H16 = HALF && C == NCH - 1;  // query rows past LR: P and dS stay 0
                const int x0 = C * CH;
                const f32x4 l0 = *reinterpret_cast<const f32x4*>(l2s + x0 + 4 * w.g);
                const f32x4 r0 = *reinterpret_cast<const f32x4*>(drs + x0 + 4 * w.g);
                f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = p0, d1 = p0;
                mma_d_sw<T, DP>(p0, Qr, x0, kf, lo);
                mma_d_sw<T, DP>(d0, Or, x0, vf, lo);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p0[r] = fast_exp2(fmaf(p0[r], sc2, -l0[r]));  // lse = +inf on padded query rows -> P = 0
                    d0[r] = p0[r] * (d0[r] - r0[r]);
                }
                if constexpr (!H16) {
                    const f32x4 l1 = *reinterpret_cast<const f32x4*>(l2s + x0 + 16 + 4 * w.g);
                    const f32x4 r1 = *reinterpret_cast<const f32x4*>(drs + x0 + 16 + 4 * w.g);
                    mma_d_sw<T, DP>(p1, Qr, x0 + 16, kf, lo);
                    mma_d_sw<T, DP>(d1, Or, x0 + 16, vf, lo);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        p1[r] = fast_exp2(fmaf(p1[r], sc2, -l1[r]));
                        d1[r] = p1[r] * (d1[r] - r1[r]);
                    }
                }
                pbs[C] = make_seqb<T>(p0, p1);  // at H16 only the first half (words 0, 1) is read
                dsbs[C] = make_seqb<T>(d0, d1);
            });
            constexpr int NH = LY::NT / 2;
            u32x2 pk_k[LY::NT], pk_v[LY::NT];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                f32x4 ak[NH], av[NH];
#pragma unroll
                for (int t = 0; t < NH; ++t) ak[t] = av[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                static_for<0, NCH>([&](auto cc) {
                    constexpr int C = decltype(cc)::value;
                    const int x0 = C * CH;
#pragma unroll
                    for (int t = 0; t < NH; ++t) {
                        if constexpr (HALF && C == NCH - 1) {
                            const u32x2 pb2 = {pbs[C].v[0], pbs[C].v[1]}, ds2 = {dsbs[C].v[0], dsbs[C].v[1]};
                            av[t] = ET<T>::mma16(seqa_tr16<T, DP>(Or, x0, half * NH + t, lo), pb2, av[t]);
                            ak[t] = ET<T>::mma16(seqa_tr16<T, DP>(Qr, x0, half * NH + t, lo), ds2, ak[t]);
                        } else {
                            av[t] = mma_seq<T>(av[t], seqa_tr<T, DP>(Or, x0, half * NH + t, lo), pbs[C]);
                            ak[t] = mma_seq<T>(ak[t], seqa_tr<T, DP>(Qr, x0, half * NH + t, lo), dsbs[C]);
                        }
                    }
                });
#pragma unroll
                for (int t = 0; t < NH; ++t) {
                    pk_k[half * NH + t] = pack4<T>(ak[t] * sc);
                    pk_v[half * NH + t] = pack4<T>(av[t]);
                }
            }
            const int64_t r = ((int64_t)s * L + row0) * DP;
            store_rows_staged<T, DP>(a.out1, r, L - row0, pk_k, stage, w.lane);
            store_rows_staged<T, DP>(a.out2, r, L - row0, pk_v, stage, w.lane);
        }
        lds_barrier();  // B: Y free, X holds slice n
        if (!more) break;
        s = n;
        qf = qn;
        df = dn;
        of = on;
        lraw = lrn;
    }
}

// =====================================================================================================================
// Backward of the backward: register-resident row pass, then the col pass.
// Row pass, phase 1: the wave's 16 query rows x all keys of P, dS, M1 = dS A + P Bm and PA = P A, kept as packed
// 16-bit MFMA operands, and the exact E = rowsum(PA), T = rowsum(M1). Phase 2: dS2 = M1 - E dS - T P and
// Pa = PA - E P, then hQ = s (dS2 K + dS gK) and hdO = Pa V + P gV directly (9 GEMM units on the row side).
// =====================================================================================================================

template <typename T, int DP, int NCH> struct BbRes {
    static constexpr int RB = NCH * CH * Sw<DP>::ROWB;
    static constexpr int SMEM = 4 * RB;  // K, gK, V, gV; later Q, gQ, dO in the same space
};

// HALF: the slice has at most 32 NCH - 16 rows, so the last chunk holds one 16-row tile: rows past it are neither
// loaded nor read (its d-contractions use one tile, its seq-contractions the k = 16 MFMA), 12.5% fewer score
// products at NCH = 4.
template <typename T, int DP, int NCH, bool HALF> __global__ __launch_bounds__(512) void k_bb_res(Args a) {
    using LY = Lay<T, DP>;
    using R = BbRes<T, DP, NCH>;
    constexpr int Lp = NCH * CH - (HALF ? 16 : 0);  // rows loaded and read
    auto live = [](int C, int hh) { return !(HALF && C == NCH - 1 && hh == 1); };  // tile hh of chunk C below Lp
    __shared__ __align__(1024) unsigned char smem[R::SMEM];
    __shared__ __align__(16) float st[4 * STAT_MAX];  // lse * log2 e, Dr, E, T
    const WaveIds w = wave_ids();
    const int nw = w.nthr >> 6;
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L;
    unsigned char* Kr = smem;
    unsigned char* gKr = smem + R::RB;
    unsigned char* Vr = smem + 2 * R::RB;
    unsigned char* gVr = smem + 3 * R::RB;
    unsigned char* Qr = smem;
    unsigned char* gQr = smem + R::RB;
    unsigned char* Or = smem + 2 * R::RB;  // dO
    const T* Qg = slice<T>(a.q, b, h);
    const T* gQg = slice<T>(a.gq, b, h);
    const T* Og = slice<T>(a.dO, b, h);
    async_rows<T, DP>(Kr, slice<T>(a.k, b, h), a.k.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(gKr, slice<T>(a.gk, b, h), a.gk.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(Vr, slice<T>(a.v, b, h), a.v.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(gVr, slice<T>(a.gv, b, h), a.gv.sl, L, Lp, w.wave, nw, w.lane);
    StatArrays<4>{st}.defaults(w.tid, w.nthr);
    const float sc = a.scale;
    const float sc2 = sc * LOG2E;
    const int row0 = w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    const LaneOff<T, DP> lo(w.l16, w.g);

    // ---- row pass: own = queries
    {
        OwnFrag<T, DP> qf, gqf, df, of;
        load_own<T, DP>(qf, Qg, a.q.sl, own, L, DP, w.g);
        load_own<T, DP>(gqf, gQg, a.gq.sl, own, L, DP, w.g);
        load_own<T, DP>(df, Og, a.dO.sl, own, L, DP, w.g);
        load_own<T, DP>(of, reinterpret_cast<const T*>(a.o) + (int64_t)bh * L * DP, DP, own, L, DP, w.g);
        const float lraw = a.lse[(int64_t)bh * L + (own < L ? own : L - 1)];  // unconditional load
        const float lse2 = (own < L) ? lraw * LOG2E : 0.f;
        const float dr = xsum4(frag_dot<T, DP>(df, of));
        async_wait();
        lds_barrier();
        if (active) {
            SeqB<T> m1b[NCH], dsb[NCH], pb[NCH], pab[NCH];
            float e_acc = 0.f, t_acc = 0.f;
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                constexpr bool LAST = C == NCH - 1;
                const int x0 = C * CH;
                f32x4 p[2], dp[2], at[2], bm[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    p[hh] = dp[hh] = at[hh] = bm[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
                    if (!live(C, hh)) continue;  // keys past Lp: their P is masked to 0 below
                    const int r0 = x0 + 16 * hh;
                    mma_d_sw<T, DP>(p[hh], Kr, r0, qf, lo);
                    mma_d_sw<T, DP>(at[hh], Kr, r0, gqf, lo);
                    mma_d_sw<T, DP>(at[hh], gKr, r0, qf, lo);
                    mma_d_sw<T, DP>(dp[hh], Vr, r0, df, lo);
                    mma_d_sw<T, DP>(bm[hh], gVr, r0, df, lo);
                }
                f32x4 ds[2], pa[2], m1[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float pv = row_p<LAST>(p[hh][r], sc2, lse2, x0 + 16 * hh + 4 * w.g + r, L);
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
                pb[C] = make_seqb<T>(p[0], p[1]);
                dsb[C] = make_seqb<T>(ds[0], ds[1]);
                pab[C] = make_seqb<T>(pa[0], pa[1]);
                m1b[C] = make_seqb<T>(m1[0], m1[1]);
            });
            const float E = xsum4(e_acc);
            const float Tm = xsum4(t_acc);
            f32x4 hq[LY::NT], hdo[LY::NT];
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) hq[t] = hdo[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                const int x0 = C * CH;
                float m1f[8], dsf[8], pf[8], paf[8], d2[8], pe[8];
                unpack_seqb<T>(m1b[C], m1f);
                unpack_seqb<T>(dsb[C], dsf);
                unpack_seqb<T>(pb[C], pf);
                unpack_seqb<T>(pab[C], paf);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    d2[e] = m1f[e] - E * dsf[e] - Tm * pf[e];
                    pe[e] = paf[e] - E * pf[e];
                }
                const SeqB<T> d2b = pack_seqb<T>(d2);
                const SeqB<T> peb = pack_seqb<T>(pe);
#pragma unroll
                for (int t = 0; t < LY::NT; ++t) {
                    if constexpr (HALF && C == NCH - 1) {
                        auto lo2 = [](const SeqB<T>& x) { return u32x2{x.v[0], x.v[1]}; };
                        hq[t] = ET<T>::mma16(seqa_tr16<T, DP>(Kr, x0, t, lo), lo2(d2b), hq[t]);
                        hq[t] = ET<T>::mma16(seqa_tr16<T, DP>(gKr, x0, t, lo), lo2(dsb[C]), hq[t]);
                        hdo[t] = ET<T>::mma16(seqa_tr16<T, DP>(Vr, x0, t, lo), lo2(peb), hdo[t]);
                        hdo[t] = ET<T>::mma16(seqa_tr16<T, DP>(gVr, x0, t, lo), lo2(pb[C]), hdo[t]);
                    } else {
                        hq[t] = mma_seq<T>(hq[t], seqa_tr<T, DP>(Kr, x0, t, lo), d2b);
                        hq[t] = mma_seq<T>(hq[t], seqa_tr<T, DP>(gKr, x0, t, lo), dsb[C]);
                        hdo[t] = mma_seq<T>(hdo[t], seqa_tr<T, DP>(Vr, x0, t, lo), peb);
                        hdo[t] = mma_seq<T>(hdo[t], seqa_tr<T, DP>(gVr, x0, t, lo), pb[C]);
                    }
                }
            });
            if (own < L) {
                const int64_t r = ((int64_t)bh * L + own) * DP;
                store_rows<T, DP>(a.out0, r, hq, sc, DP, w.g);
                store_rows<T, DP>(a.out3, r, hdo, 1.f, DP, w.g);
            }
            if (w.g == 0) {
                const bool ok = own < L;
                st[own] = ok ? lse2 : INFINITY;
                st[STAT_MAX + own] = ok ? dr : 0.f;
                st[2 * STAT_MAX + own] = ok ? E : 0.f;
                st[3 * STAT_MAX + own] = ok ? Tm : 0.f;
            }
        }
    }
    lds_barrier();  // statistics published; the row pass no longer reads K, gK, V, gV

    // ---- col pass: own = keys
    OwnFrag<T, DP> kf, gkf, vf, gvf;
    if (active) {
        own_from_lds<T, DP>(kf, Kr, row0, lo);
        own_from_lds<T, DP>(gkf, gKr, row0, lo);
        own_from_lds<T, DP>(vf, Vr, row0, lo);
        own_from_lds<T, DP>(gvf, gVr, row0, lo);
    }
    lds_barrier();  // every wave holds its key rows before Q, gQ, dO overwrite the regions
    async_rows<T, DP>(Qr, Qg, a.q.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(gQr, gQg, a.gq.sl, L, Lp, w.wave, nw, w.lane);
    async_rows<T, DP>(Or, Og, a.dO.sl, L, Lp, w.wave, nw, w.lane);
    async_wait();
    lds_barrier();
    if (!active) return;
    f32x4 hk[LY::NT], hv[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) hk[t] = hv[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    static_for<0, NCH>([&](auto cc) {
        constexpr int C = decltype(cc)::value;
        const int x0 = C * CH;
        f32x4 p[2], dp[2], at[2], bm[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            p[hh] = dp[hh] = at[hh] = bm[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (!live(C, hh)) continue;  // query rows past Lp: their tile values are never read
            const int r0 = x0 + 16 * hh;
            mma_d_sw<T, DP>(p[hh], Qr, r0, kf, lo);
            mma_d_sw<T, DP>(at[hh], Qr, r0, gkf, lo);
            mma_d_sw<T, DP>(at[hh], gQr, r0, kf, lo);
            mma_d_sw<T, DP>(dp[hh], Or, r0, vf, lo);
            mma_d_sw<T, DP>(bm[hh], Or, r0, gvf, lo);
        }
        f32x4 ds[2], ds2[2], pa[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            ds[hh] = ds2[hh] = pa[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (!live(C, hh)) continue;
            const int so = x0 + 16 * hh + 4 * w.g;
            const f32x4 ls = *reinterpret_cast<const f32x4*>(st + so);
            const f32x4 rs = *reinterpret_cast<const f32x4*>(st + STAT_MAX + so);
            const f32x4 es = *reinterpret_cast<const f32x4*>(st + 2 * STAT_MAX + so);
            const f32x4 ts = *reinterpret_cast<const f32x4*>(st + 3 * STAT_MAX + so);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pv = fast_exp2(fmaf(p[hh][r], sc2, -ls[r]));
                const float dsv = pv * (dp[hh][r] - rs[r]);
                const float av = at[hh][r] * sc;
                ds[hh][r] = dsv;
                const float m1 = fmaf(dsv, av, pv * bm[hh][r]);
                ds2[hh][r] = m1 - es[r] * dsv - ts[r] * pv;
                pa[hh][r] = pv * (av - es[r]);
            }
        }
        if constexpr (HALF && C == NCH - 1) {
            const u32x2 dsb = pack4<T>(ds[0]), ds2b = pack4<T>(ds2[0]), pab = pack4<T>(pa[0]);
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) {
                hk[t] = ET<T>::mma16(seqa_tr16<T, DP>(Qr, x0, t, lo), ds2b, hk[t]);
                hk[t] = ET<T>::mma16(seqa_tr16<T, DP>(gQr, x0, t, lo), dsb, hk[t]);
                hv[t] = ET<T>::mma16(seqa_tr16<T, DP>(Or, x0, t, lo), pab, hv[t]);
            }
        } else {
            const SeqB<T> dsb = make_seqb<T>(ds[0], ds[1]);
            const SeqB<T> ds2b = make_seqb<T>(ds2[0], ds2[1]);
            const SeqB<T> pab = make_seqb<T>(pa[0], pa[1]);
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) {
                hk[t] = mma_seq<T>(hk[t], seqa_tr<T, DP>(Qr, x0, t, lo), ds2b);
                hk[t] = mma_seq<T>(hk[t], seqa_tr<T, DP>(gQr, x0, t, lo), dsb);
                hv[t] = mma_seq<T>(hv[t], seqa_tr<T, DP>(Or, x0, t, lo), pab);
            }
        }
    });
    if (own < L) {
        const int64_t r = ((int64_t)bh * L + own) * DP;
        store_rows<T, DP>(a.out1, r, hk, sc, DP, w.g);
        store_rows<T, DP>(a.out2, r, hv, 1.f, DP, w.g);
    }
}

// =====================================================================================================================
// Backward of the backward with the L x L tiles shared through LDS (16-bit inputs, D <= 64, L <= 96).
// The row pass (as in k_bb_res) also writes its dS2, dS and Pa tiles, rounded to the input type, into LDS as
// [query][key] rows. The col pass then needs neither the scores nor any elementwise work: with A = Q, gQ, dO read
// transposed from their natural rows and B = the tiles read transposed (lane = key, k-slots = queries),
//   hK = s (dS2^T Q + dS^T gQ),  hV = Pa^T dO
// are 3 GEMM units: 12 for the whole backward of the backward, the minimum. One compute wave per 16 rows covers every
// tile row (padded rows are written as 0).
//
// Persistent: the workgroup (one per CU: the regions fill its LDS) takes slices s, s + G, s + 2 G, ... (G =
// gridDim.x). The compute waves issue no global stores: a store instruction stalls its wave while the memory system
// is busy (all CUs store and load at once), and those stalls sat on the slice's critical path (at config 1 the kernel
// ran 35 us faster with its output stores left out). They hand their rounded output rows to the NWL loader waves
// through LDS instead, in the natural swizzled row layout of the regions: hQ, hdO into the K, gK regions right after
// barrier A (the row pass no longer reads them), hK, hV into the tile area right after barrier B (the col pass no
// longer reads it), each hand-off published by an LDS counter that every compute wave bumps once per slice. The
// loader waves read the rows into registers and store them to HBM as whole rows; they also hold the next slice's K,
// gK, V, gV in registers and write them into their regions once the hQ, hdO rows there are read. Each compute wave
// fetches its own 16 rows of the next slice's Q, gQ, dO, O and their lse into registers at the end of its row pass,
// writes its Q, gQ, dO rows into their regions once the col pass is done with them, and takes its row pass operands,
// rowsum(dO o O) and lse straight from those registers, so no wave waits for another's row statistics. Global loads
// go through registers (structured buffer loads in the loaders) because an LDS transpose read right after an
// outstanding global -> LDS load makes the compiler wait for that load. Per slice s with next slice n = s + G:
//   compute waves                                   loader waves
//   row pass (s); fetch own rows (n)                load K, gK, V, gV of n into registers; store hK, hV of s - G
//   --- barrier A: tiles complete, K, gK, V, gV (s) no longer read
//   hQ, hdO rows (s) -> K, gK regions; count        wait for the count; read them; write K, gK, V, gV (n)
//   col pass (s)
//   --- barrier B: tiles and Q, gQ, dO (s) no longer read; K, gK, V, gV (n) in place
//   hK, hV rows (s) -> tile area; count             store hQ, hdO (s); wait for the count; read them; count
//   own rows of Q, gQ, dO (n) -> regions; row pass (n), its first tile write after the loaders' count
// Every counter wait is bounded (SPIN_MAX polls), so no wave can wait forever.
// =====================================================================================================================

template <typename T, int DP, int NCH> struct BbShare {
    static constexpr int LP = NCH * CH;
    static constexpr int RB = LP * Sw<DP>::ROWB;  // one natural tensor region
    static constexpr int TP = LP * 2 + 32;        // tile row pitch (bytes), padded off the 256-byte bank period
    static constexpr int TB = LP * TP;            // one tile
    static constexpr int NWC = 2 * NCH;           // compute waves (16 rows each)
    static constexpr int NB = LP / Sw<DP>::RPI;   // 1 KB blocks per tensor
    // loader waves: each holds NB / NWL of the 1 KB blocks of each of K, gK, V, gV (16 NB / NWL VGPRs) and of two
    // output tensors (8 NB / NWL VGPRs) in registers
    static constexpr int NWL = 24 * NB / 2 > 192 ? 4 : 2;
    static_assert(NWC + NWL <= 8, "launch bound of 512 threads");
    static constexpr int NPER = NB / NWL;         // blocks per loader wave and tensor
    static_assert(NPER * NWL == NB, "the loader waves split every tensor's 1 KB blocks evenly");
    static constexpr int TILES = 7 * RB;          // byte offset of the tile area: dS2, dS, Pa
    // the tile area also parks hK and hV (two natural regions) between barrier B and the loaders' reads
    static constexpr int PARK = 3 * TB > 2 * RB ? 3 * TB : 2 * RB;
    static constexpr int CNT = TILES + PARK;      // three LDS counters
    // K, gK, V, gV | Q, gQ, dO | dS2, dS, Pa (hK, hV parked) | counters
    static constexpr int SMEM = CNT + 16;
    static constexpr int THREADS = 64 * (NWC + NWL);
};

// Structured buffer load (address = base + index * stride + offset; the stride, in bytes, sits in the descriptor).
__device__ u32x4 ebr_struct_load_b128(__amdgpu_buffer_rsrc_t rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v4i32");

constexpr int64_t STRUCT_STRIDE_MAX = 16383;  // the descriptor's 14-bit stride field (bytes)

// A loader wave's share of the 1 KB blocks of rows [0, LP) of one slice tensor: block q = wave + i * nw holds rows
// q * RPI .. q * RPI + RPI - 1; lane l carries row x = q * RPI + l / NCK, chunk position l % NCK (global chunk
// (l % NCK) ^ swz(x)), LDS offset 1024 q + 16 l. These lane values are the same for every tensor of the slice.
template <int DP, int NPER> struct StageLanes {
    int x[NPER], coff[NPER];
    __device__ __forceinline__ StageLanes(int wave, int nw, int lane) {
        using S = Sw<DP>;
#pragma unroll
        for (int i = 0; i < NPER; ++i) {
            x[i] = (wave + i * nw) * S::RPI + lane / S::NCK;
            coff[i] = 16 * ((lane % S::NCK) ^ S::swz(x[i]));
        }
    }
};

// Register staging of one tensor's share. fetch() issues the loads (row index clamped to L - 1, so every access is
// inside the slice); put() writes them to a swizzled region, rows past L as 0. take() reads a region's rows back and
// store() writes them to a contiguous [L, DP] output slice, whole rows, rows past L skipped.
template <typename T, int DP, int NPER> struct RowStage {
    u32x4 v[NPER];
    __device__ __forceinline__ void fetch(const T* slice, int64_t srow, int L, const StageLanes<DP, NPER>& sl) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            (void*)slice, (short)(srow * (int64_t)sizeof(T)), 0x7fffffff, (int)BUF_RSRC_WORD3);
#pragma unroll
        for (int i = 0; i < NPER; ++i) v[i] = ebr_struct_load_b128(r, sl.x[i] < L ? sl.x[i] : L - 1, sl.coff[i], 0, 0);
    }
    __device__ __forceinline__ void put(unsigned char* region, int L, const StageLanes<DP, NPER>& sl, int wave, int nw,
                                        int lane) const {
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < NPER; ++i)
            *reinterpret_cast<u32x4*>(region + (wave + i * nw) * 1024 + 16 * lane) = sl.x[i] < L ? v[i] : z;
    }
    __device__ __forceinline__ void take(const unsigned char* region, int wave, int nw, int lane) {
#pragma unroll
        for (int i = 0; i < NPER; ++i)
            v[i] = *reinterpret_cast<const u32x4*>(region + (wave + i * nw) * 1024 + 16 * lane);
    }
    __device__ __forceinline__ void store(void* out, int64_t slice_off, int L, const StageLanes<DP, NPER>& sl) const {
        T* o = reinterpret_cast<T*>(out) + slice_off;
#pragma unroll
        for (int i = 0; i < NPER; ++i)
            if (sl.x[i] < L) *reinterpret_cast<u32x4*>(o + (int64_t)sl.x[i] * DP + sl.coff[i] / 2) = v[i];
    }
};

// LDS counters of the output hand-offs (monotonic; each compute or loader wave adds 1 per slice).
constexpr int SPIN_MAX = 1 << 20;  // polls before a wait gives up (never reached when every wave runs)

__device__ __forceinline__ void count_up(unsigned int* c, int lane) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // this wave's LDS writes before the count
    if (lane == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void wait_count(unsigned int* c, unsigned int target) {
    for (int i = 0; i < SPIN_MAX; ++i) {
        const unsigned int v =
            __builtin_amdgcn_readfirstlane(__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (v >= target) break;
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");  // the counted writes before this wave's reads
}

// The loader waves' registers: the K, gK, V, gV rows of one slice, and two output tensors' rows in transit.
template <typename T, int DP, int NCH> struct BbLoader {
    using R = BbShare<T, DP, NCH>;
    using RS = RowStage<T, DP, R::NPER>;
    StageLanes<DP, R::NPER> sl;
    RS k, gk, v, gv, o0, o1;
    int lw, lane;
    __device__ __forceinline__ BbLoader(int lw_, int lane_) : sl(lw_, R::NWL, lane_), lw(lw_), lane(lane_) {}
    __device__ __forceinline__ void fetch(const Args& a, int s) {
        const int L = a.L;
        const int b = s / a.H, h = s - b * a.H;
        k.fetch(slice<T>(a.k, b, h), a.k.sl, L, sl);
        gk.fetch(slice<T>(a.gk, b, h), a.gk.sl, L, sl);
        v.fetch(slice<T>(a.v, b, h), a.v.sl, L, sl);
        gv.fetch(slice<T>(a.gv, b, h), a.gv.sl, L, sl);
    }
    __device__ __forceinline__ void put_k4(unsigned char* smem, int L) const {
        k.put(smem, L, sl, lw, R::NWL, lane);
        gk.put(smem + R::RB, L, sl, lw, R::NWL, lane);
        v.put(smem + 2 * R::RB, L, sl, lw, R::NWL, lane);
        gv.put(smem + 3 * R::RB, L, sl, lw, R::NWL, lane);
    }
    // two parked output tensors (rows in the region layout, R::RB bytes each, back to back) into registers
    __device__ __forceinline__ void take(const unsigned char* park) {
        o0.take(park, lw, R::NWL, lane);
        o1.take(park + R::RB, lw, R::NWL, lane);
    }
    __device__ __forceinline__ void store(void* out0, void* out1, int s, int L) const {
        const int64_t off = (int64_t)s * L * DP;
        o0.store(out0, off, L, sl);
        o1.store(out1, off, L, sl);
    }
};

// A compute wave's own rows of one slice: Q, gQ, dO and O in the own-fragment layout (lane (row l16, group g) holds
// d = c * CW + g * VEC ..), and the row's lse. fetch() loads them raw from row min(own, L - 1), so every access is
// inside the slice and no select waits on a load; clear() zeroes the rows past L where they are consumed.
template <typename T, int DP> struct OwnRows {
    OwnFrag<T, DP> q, gq, dO, o;
    float lse;
    static __device__ __forceinline__ void raw(OwnFrag<T, DP>& f, const T* base, int64_t srow, int r, int g) {
        using LY = Lay<T, DP>;
        const T* p = base + (int64_t)r * srow + g * LY::VEC;
#pragma unroll
        for (int c = 0; c < LY::NC; ++c) f.v[c] = *reinterpret_cast<const u32x4*>(p + c * LY::CW);
    }
    __device__ __forceinline__ void fetch(const Args& a, int s, int own, int g) {
        const int L = a.L;
        const int b = s / a.H, h = s - b * a.H;
        const int r = own < L ? own : L - 1;
        raw(q, slice<T>(a.q, b, h), a.q.sl, r, g);
        raw(gq, slice<T>(a.gq, b, h), a.gq.sl, r, g);
        raw(dO, slice<T>(a.dO, b, h), a.dO.sl, r, g);
        raw(o, reinterpret_cast<const T*>(a.o) + (int64_t)s * L * DP, DP, r, g);
        lse = a.lse[(int64_t)s * L + r];
    }
    __device__ __forceinline__ void clear(bool live) {
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int c = 0; c < Lay<T, DP>::NC; ++c) {
            q.v[c] = live ? q.v[c] : z;
            gq.v[c] = live ? gq.v[c] : z;
            dO.v[c] = live ? dO.v[c] : z;
            o.v[c] = live ? o.v[c] : z;
        }
        lse = live ? lse : INFINITY;  // padded query rows: P = 0
    }
    // rows row0 .. row0 + 15 of the Q, gQ, dO regions
    __device__ __forceinline__ void put(unsigned char* Qr, unsigned char* gQr, unsigned char* Or, int row0,
                                        const LaneOff<T, DP>& lo) const {
        const int base = row0 * Sw<DP>::ROWB;
#pragma unroll
        for (int c = 0; c < Lay<T, DP>::NC; ++c) {
            *reinterpret_cast<u32x4*>(Qr + base + lo.a[c]) = q.v[c];
            *reinterpret_cast<u32x4*>(gQr + base + lo.a[c]) = gq.v[c];
            *reinterpret_cast<u32x4*>(Or + base + lo.a[c]) = dO.v[c];
        }
    }
};

// A seq-contraction accumulator's 16 rows (lane (row l16, group g) holds columns 16 t + 4 g .. + 3), scaled by mul
// and rounded, into rows row0 .. row0 + 15 of a region in the swizzled natural layout.
template <typename T, int DP>
__device__ __forceinline__ void park_rows(unsigned char* region, int row0, const f32x4 (&acc)[DP / 16], float mul,
                                          int l16, int g) {
    using S = Sw<DP>;
    unsigned char* p = region + (row0 + l16) * S::ROWB + 8 * (g & 1);
#pragma unroll
    for (int t = 0; t < DP / 16; ++t) {
        const int c = 2 * t + (g >> 1);  // 16-byte chunk of columns 16 t + 4 g
        *reinterpret_cast<u32x2*>(p + 16 * (c ^ S::swz(l16))) = pack4<T>(acc[t] * mul);
    }
}

template <typename T, int DP, int NCH> __global__ __launch_bounds__(512) void k_bb_share(Args a) {
    using LY = Lay<T, DP>;
    using R = BbShare<T, DP, NCH>;
    __shared__ __align__(1024) unsigned char smem[R::SMEM];
    const WaveIds w = wave_ids();
    const int L = a.L;
    const int nbh = a.B * a.H;
    unsigned char* Kr = smem;
    unsigned char* gKr = smem + R::RB;
    unsigned char* Vr = smem + 2 * R::RB;
    unsigned char* gVr = smem + 3 * R::RB;
    unsigned char* Qr = smem + 4 * R::RB;
    unsigned char* gQr = smem + 5 * R::RB;
    unsigned char* Or = smem + 6 * R::RB;    // dO
    unsigned char* T2 = smem + R::TILES;     // dS2
    unsigned char* T1 = T2 + R::TB;          // dS
    unsigned char* Ta = T2 + 2 * R::TB;      // Pa
    unsigned char* park = T2;                // hK, hV between barrier B and the loaders' reads
    unsigned int* cnt = reinterpret_cast<unsigned int*>(smem + R::CNT);  // hQ/hdO parked, hK/hV parked, hK/hV read
    int s = blockIdx.x;
    if (w.tid < 3) cnt[w.tid] = 0u;  // before the first barrier

    if (w.wave >= R::NWC) {
        // ---- loader waves
        BbLoader<T, DP, NCH> ld(w.wave - R::NWC, w.lane);
        ld.fetch(a, s);
        ld.put_k4(smem, L);
        lds_barrier();
        unsigned int it = 0;
        int prev = -1;  // slice whose hK, hV rows sit in the registers, not yet stored
        while (true) {
            const int n = s + (int)gridDim.x;
            const bool more = n < nbh;  // uniform over the workgroup
            if (more) ld.fetch(a, n);
            if (prev >= 0) ld.store(a.out1, a.out2, prev, L);
            lds_barrier();  // A
            wait_count(cnt, R::NWC * (it + 1));
            ld.take(Kr);  // hQ, hdO of s from the K, gK regions
            if (more) ld.put_k4(smem, L);
            lds_barrier();  // B
            ld.store(a.out0, a.out3, s, L);  // after B: the segment before it gates the next row pass
            wait_count(cnt + 1, R::NWC * (it + 1));
            ld.take(park);  // hK, hV of s
            count_up(cnt + 2, w.lane);
            prev = s;
            if (!more) break;
            s = n;
            ++it;
        }
        ld.store(a.out1, a.out2, prev, L);
        return;
    }

    // ---- compute waves
    const float sc = a.scale;
    const float sc2 = sc * LOG2E;
    const int row0 = w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    const bool live = own < L;
    const LaneOff<T, DP> lo(w.l16, w.g);
    OwnRows<T, DP> nx;  // this wave's rows of the slice the next row pass takes
    nx.fetch(a, s, own, w.g);
    nx.clear(live);
    nx.put(Qr, gQr, Or, row0, lo);
    lds_barrier();  // the first slice is in LDS
    unsigned int it = 0;
    while (true) {
        const int n = s + (int)gridDim.x;
        const bool more = n < nbh;

        // ---- row pass: own = queries, plus the tile writes. P, dS, PA and M1 stay in fp32 registers between the
        // phases; only MFMA operands and tiles are rounded to the input type.
        f32x4 hq[LY::NT], hdo[LY::NT];
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) hq[t] = hdo[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (active) {
            const OwnFrag<T, DP> qf = nx.q, gqf = nx.gq, df = nx.dO;  // rows past L are 0
            const float lse2 = nx.lse * LOG2E;                       // +inf past L
            const float dr = xsum4(frag_dot<T, DP>(nx.dO, nx.o));     // rowsum(dO o O)
            float pf[NCH][8], dsf[NCH][8], paf[NCH][8], m1f[NCH][8];
            float e_acc = 0.f, t_acc = 0.f;
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                constexpr bool LAST = C == NCH - 1;
                const int x0 = C * CH;
                f32x4 p[2], dp[2], at[2], bm[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    p[hh] = at[hh] = bm[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
                    dp[hh] = f32x4{-dr, -dr, -dr, -dr};  // dP - Dr, one multiply from dS
                    const int r0 = x0 + 16 * hh;
                    mma_d_sw<T, DP>(p[hh], Kr, r0, qf, lo);
                    mma_d_sw<T, DP>(at[hh], Kr, r0, gqf, lo);
                    mma_d_sw<T, DP>(at[hh], gKr, r0, qf, lo);
                    mma_d_sw<T, DP>(dp[hh], Vr, r0, df, lo);
                    mma_d_sw<T, DP>(bm[hh], gVr, r0, df, lo);
                }
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int e = 4 * hh + r;
                        const float pv = row_p<LAST>(p[hh][r], sc2, lse2, x0 + 16 * hh + 4 * w.g + r, L);
                        const float dsv = pv * dp[hh][r];
                        const float av = at[hh][r] * sc;
                        pf[C][e] = pv;
                        dsf[C][e] = dsv;
                        paf[C][e] = pv * av;
                        m1f[C][e] = fmaf(dsv, av, pv * bm[hh][r]);
                        e_acc += paf[C][e];
                        t_acc += m1f[C][e];
                    }
                }
            });
            const float E = xsum4(e_acc);
            const float Tm = xsum4(t_acc);
            wait_count(cnt + 2, R::NWL * it);  // the loaders have read the previous slice's hK, hV from the tiles
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                const int x0 = C * CH;
                float d2[8], pe[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    d2[e] = m1f[C][e] - E * dsf[C][e] - Tm * pf[C][e];
                    pe[e] = paf[C][e] - E * pf[C][e];
                }
                const SeqB<T> d2b = pack_seqb<T>(d2);
                const SeqB<T> dsb = pack_seqb<T>(dsf[C]);
                const SeqB<T> peb = pack_seqb<T>(pe);
                const SeqB<T> pb = pack_seqb<T>(pf[C]);
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int key0 = x0 + 16 * hh + 4 * w.g;
                    tile_store8(T2, R::TP, own, key0, u32x2{d2b.v[2 * hh], d2b.v[2 * hh + 1]});
                    tile_store8(T1, R::TP, own, key0, u32x2{dsb.v[2 * hh], dsb.v[2 * hh + 1]});
                    tile_store8(Ta, R::TP, own, key0, u32x2{peb.v[2 * hh], peb.v[2 * hh + 1]});
                }
#pragma unroll
                for (int t = 0; t < LY::NT; ++t) {
                    hq[t] = mma_seq<T>(hq[t], seqa_tr<T, DP>(Kr, x0, t, lo), d2b);
                    hq[t] = mma_seq<T>(hq[t], seqa_tr<T, DP>(gKr, x0, t, lo), dsb);
                    hdo[t] = mma_seq<T>(hdo[t], seqa_tr<T, DP>(Vr, x0, t, lo), peb);
                    hdo[t] = mma_seq<T>(hdo[t], seqa_tr<T, DP>(gVr, x0, t, lo), pb);
                }
            });
        } else {
            wait_count(cnt + 2, R::NWL * it);
            zero_tile_rows<NCH>(T2, T1, Ta, R::TP, own, w.g);
        }
        // this wave's rows of the next slice (or this one again after the last: the load stays unconditional); they
        // have the col pass and two barriers to land
        nx.fetch(a, more ? n : s, own, w.g);
        lds_barrier();  // A
        if (active) {
            park_rows<T, DP>(Kr, row0, hq, sc, w.l16, w.g);
            park_rows<T, DP>(gKr, row0, hdo, 1.f, w.l16, w.g);
        }
        count_up(cnt, w.lane);

        // ---- col pass: own = keys; hK, hV from the tiles
        f32x4 hk[LY::NT], hv[LY::NT];
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) hk[t] = hv[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (active) {
            static_for<0, NCH>([&](auto cc) {
                constexpr int C = decltype(cc)::value;
                const int x0 = C * CH;
                const SeqB<T> b2 = tile_seqb<T>(T2, R::TP, x0, row0, w.l16, w.g);
                const SeqB<T> b1 = tile_seqb<T>(T1, R::TP, x0, row0, w.l16, w.g);
                const SeqB<T> ba = tile_seqb<T>(Ta, R::TP, x0, row0, w.l16, w.g);
#pragma unroll
                for (int t = 0; t < LY::NT; ++t) {
                    hk[t] = mma_seq<T>(hk[t], seqa_tr<T, DP>(Qr, x0, t, lo), b2);
                    hk[t] = mma_seq<T>(hk[t], seqa_tr<T, DP>(gQr, x0, t, lo), b1);
                    hv[t] = mma_seq<T>(hv[t], seqa_tr<T, DP>(Or, x0, t, lo), ba);
                }
            });
        }
        lds_barrier();  // B
        if (active) {
            park_rows<T, DP>(park, row0, hk, sc, w.l16, w.g);
            park_rows<T, DP>(park + R::RB, row0, hv, 1.f, w.l16, w.g);
        }
        count_up(cnt + 1, w.lane);
        if (!more) break;
        // this wave's Q, gQ, dO rows of the next slice into their regions: the next col pass reads them after
        // barrier A, the next row pass takes them from the registers
        nx.clear(live);
        nx.put(Qr, gQr, Or, row0, lo);
        s = n;
        ++it;
    }
}
