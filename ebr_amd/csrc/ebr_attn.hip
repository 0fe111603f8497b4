// gfx950 kernels of the fused second-order attention path and their C ABI (include/ebr_attn.h).
//
// Algorithm (per (b, h) slice, s = scale):
//   S = s Q K^T, lse = rowlogsumexp(S), P = exp(S - lse), O = P V                              (forward)
//   dP = dO V^T, Dr = rowsum(dO * O), dS = P (dP - Dr), dQ = s dS K, dK = s dS^T Q, dV = P^T dO  (backward)
//   A = s (gQ K^T + Q gK^T), Bm = dO gV^T, E = rowsum(P A), T = rowsum(dS A + P Bm),
//   dS2 = dS A + P Bm - E dS - T P, Pa = P A - E P,
//   hQ = s (dS2 K + dS gK), hK = s (dS2^T Q + dS^T gQ), hV = Pa^T dO, hdO = Pa V + P gV          (backward of backward)
// following reference models/fused_attn/reference.py:32-91 (dense form) and the streaming row form of
// models/fused_attn/triton_kernels.py:347-445 (hQ = s (X - E U - T Z), hdO = W - E O).
//
// Two passes over a slice, each a grid of 64-lane waves that own 16 rows and stream the other side in 32-row
// LDS chunks (attn_tiles.hpp):
//   row pass  own = queries: forward; dQ (+ Dr); hQ, hdO (+ Dr, E, T)
//   col pass  own = keys:    dK, dV; hK, hV (reads lse, Dr, E, T of the query rows)
// For L <= 128 one workgroup holds every row of a slice (one wave per 16 rows) and runs the row pass and then the
// col pass, passing the row statistics through LDS: one launch, each input read once. Longer slices run the passes
// as two launches that exchange the statistics through a caller-provided fp32 scratch.
//
// Precision (reference models/fused_attn/triton_kernels.py:15-17, 48-56, 84-90, 689-693): fp32 accumulation; for
// 16-bit inputs the L x L tiles (P, dS, dS2, ...) are rounded to the input type before they enter an MFMA; exp is
// exp2 of a small difference times log2(e); P = exp2(fma(qk, s, -lse) * log2(e)).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <type_traits>
#include <utility>

#include "../../include/ebr_attn.h"
#include "attn_tiles.hpp"

namespace ebr {

struct Strided {
    const void* p;
    int64_t sb, sh, sl;
};

struct Args {
    int B, H, L, D;
    float scale;
    int nblk;       // own-row blocks per (b, h)
    int xcd_remap;  // 1: keep the blocks of one (b, h) on one XCD
    Strided q, k, v, dO, gq, gk, gv;
    const void* o;      // contiguous [B, H, L, D]
    const float* lse;   // contiguous [B, H, L] (fp64 kernels read it as double)
    void* out0;
    void* out1;
    void* out2;
    void* out3;
    float* lse_out;     // (fp64 kernels write it as double)
    float* stats;       // [3][B * H * L] fp32: Dr, E, T (two-launch shapes only)
    int64_t bhl;        // B * H * L
    int plan;           // EBR_PLAN_*: AUTO (0) for the library's own choice of kernels
};

template <typename T> __device__ __forceinline__ const T* slice(const Strided& t, int b, int h) {
    return reinterpret_cast<const T*>(t.p) + (int64_t)b * t.sb + (int64_t)h * t.sh;
}

// Workgroup -> (bh, own block). Workgroups are dispatched round-robin over the 8 XCDs; with xcd_remap the blocks of
// one (b, h), which read the same other-side rows, land on the same XCD and share its L2.
__device__ __forceinline__ void decode_block(const Args& a, int& bh, int& blk) {
    int i = blockIdx.x;
    const int total = gridDim.x;
    if (a.xcd_remap && (total & 7) == 0) {
        const int per = total >> 3;
        i = (i & 7) * per + (i >> 3);
    }
    bh = i / a.nblk;
    blk = i - bh * a.nblk;
}

struct WaveIds {
    int tid, nthr, wave, lane, l16, g;
};

__device__ __forceinline__ WaveIds wave_ids() {
    WaveIds w;
    w.tid = threadIdx.x;
    w.nthr = blockDim.x;
    w.wave = w.tid >> 6;
    w.lane = w.tid & 63;
    w.l16 = w.lane & 15;
    w.g = w.lane >> 4;
    return w;
}

// Writes rows of a transposed seq-contraction accumulator: lane (own, g) of tile t holds d = 16 t + 4 g + r.
template <typename T, int DP>
__device__ __forceinline__ void store_rows(void* out, int64_t row_off, const f32x4 (&acc)[DP / 16], float mul, int D,
                                           int g) {
    T* p = reinterpret_cast<T*>(out) + row_off;
#pragma unroll
    for (int t = 0; t < DP / 16; ++t) {
        const int d = 16 * t + 4 * g;
        if (d < D) store4<T>(p + d, acc[t] * mul);
    }
}

// =====================================================================================================================
// Forward (row pass): online softmax over 32-key chunks.
// =====================================================================================================================

// Wider rows than DP = 128 run 256-thread workgroups (one wave per SIMD, every register for the wave).
template <typename T, int DP> __global__ __launch_bounds__(DP > 128 ? 256 : 512) void k_fwd(Args a) {
    using LY = Lay<T, DP>;
    __shared__ __align__(16) unsigned char smem[LY::NATB + (LY::NATSEQ ? LY::NATB : LY::TRB)];
    T* Kn = reinterpret_cast<T*>(smem);
    T* Vt = reinterpret_cast<T*>(smem + LY::NATB);
    const WaveIds w = wave_ids();
    const int W = w.nthr >> 6;
    int bh, blk;
    decode_block(a, bh, blk);
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L, D = a.D;
    const int row0 = blk * 16 * W + w.wave * 16;
    const int own = row0 + w.l16;
    const bool active = row0 < L;
    const Src<T, 2> src = {{slice<T>(a.k, b, h), slice<T>(a.v, b, h)}, {a.k.sl, a.v.sl}};
    T* const nat[2] = {Kn, nullptr};
    T* const tr[2] = {nullptr, Vt};
    Stage<T, DP, 2> stg;
    stg.load(src, 0, L, D, w.tid, w.nthr);

    OwnFrag<T, DP> qf;
    load_own<T, DP>(qf, slice<T>(a.q, b, h), a.q.sl, own, L, D, w.g);
    float m = -INFINITY, lsum = 0.f;
    f32x4 acc[LY::NT];
#pragma unroll
    for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float sc = a.scale;

    for (int x0 = 0; x0 < L; x0 += CH) {
        lds_barrier();
        stg.store(nat, tr, w.tid, w.nthr);
        lds_barrier();
        if (x0 + CH < L) stg.load(src, x0 + CH, L, D, w.tid, w.nthr);
        if (!active) continue;
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
        mma_d<T, DP>(s0, Kn, qf, w.l16, w.g);
        mma_d<T, DP>(s1, Kn + 16 * LY::PN, qf, w.l16, w.g);
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
        for (int t = 0; t < LY::NT; ++t) {
            const SeqA<T> va = read_seqa<T, DP>(Vt, t, w.l16, w.g);
            acc[t] = mma_seq<T>(acc[t] * alpha, va, pb);
        }
        m = mnew;
    }
    if (!active) return;
    lsum = xsum4(lsum);
    if (own < L) {
        const int64_t r = (int64_t)bh * L + own;
        store_rows<T, DP>(a.out0, r * D, acc, 1.f / lsum, D, w.g);
        if (w.g == 0) a.lse_out[r] = m + logf(lsum);
    }
}

// =====================================================================================================================
// Backward
// =====================================================================================================================

// LDS layout of one chunk stage: NN natural tiles followed by NTR transposed tiles.
template <typename T, int DP> __device__ __forceinline__ T* nat_tile(unsigned char* smem, int i) {
    return reinterpret_cast<T*>(smem + i * Lay<T, DP>::NATB);
}
// Transposed tile i; under NATSEQ the natural tile of the same tensor (tensor i of a stage has natural tile i).
template <typename T, int DP> __device__ __forceinline__ T* tr_tile(unsigned char* smem, int nn, int i) {
    if constexpr (Lay<T, DP>::NATSEQ) return nat_tile<T, DP>(smem, i);
    return reinterpret_cast<T*>(smem + nn * Lay<T, DP>::NATB + i * Lay<T, DP>::TRB);
}

// Row pass (own = 16 query rows per wave): dQ = s sum_j dS[i][j] K[j]. Other side per chunk: K (natural, transposed),
// V (natural). Publishes lse and Dr of its rows: FUSED -> LDS st ([lse | Dr], STAT_MAX each), else Dr -> a.stats.
template <typename T, int DP, bool FUSED> struct BwdRow {
    using LY = Lay<T, DP>;
    static constexpr int NN = 2, NTR = 1, SMEM = NN * LY::NATB + NTR * LY::TRB;
    OwnFrag<T, DP> qf, df;
    f32x4 acc[LY::NT];
    float dr, lse;
    int own, bh;
    bool active;

    __device__ __forceinline__ Src<T, 2> src(const Args& a, int b, int h) const {
        return {{slice<T>(a.k, b, h), slice<T>(a.v, b, h)}, {a.k.sl, a.v.sl}};
    }
    __device__ __forceinline__ void lds(unsigned char* smem, T* (&nat)[2], T* (&tr)[2]) const {
        nat[0] = nat_tile<T, DP>(smem, 0);
        nat[1] = nat_tile<T, DP>(smem, 1);
        tr[0] = tr_tile<T, DP>(smem, NN, 0);
        tr[1] = nullptr;
    }
    __device__ __forceinline__ void init(const Args& a, int bh_, int own_base, const WaveIds& w, float* st) {
        bh = bh_;
        const int b = bh / a.H, h = bh - b * a.H;
        const int L = a.L, D = a.D;
        const int row0 = own_base + w.wave * 16;
        own = row0 + w.l16;
        active = row0 < L;
        OwnFrag<T, DP> of;
        load_own<T, DP>(qf, slice<T>(a.q, b, h), a.q.sl, own, L, D, w.g);
        load_own<T, DP>(df, slice<T>(a.dO, b, h), a.dO.sl, own, L, D, w.g);
        load_own<T, DP>(of, reinterpret_cast<const T*>(a.o) + (int64_t)bh * L * D, D, own, L, D, w.g);
        const float lraw = a.lse[(int64_t)bh * L + (own < L ? own : L - 1)];  // unconditional load
        lse = (own < L) ? lraw : 0.f;
        dr = xsum4(frag_dot<T, DP>(df, of));
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (w.g == 0 && active) {
            if constexpr (FUSED) {
                st[own] = (own < L) ? lse : INFINITY;
                st[STAT_MAX + own] = (own < L) ? dr : 0.f;
            } else {
                if (own < L) a.stats[(int64_t)bh * L + own] = dr;
            }
        }
    }
    __device__ __forceinline__ void chunk(const Args& a, int x0, unsigned char* smem, const WaveIds& w) {
        if (!active) return;
        const T* Kn = nat_tile<T, DP>(smem, 0);
        const T* Vn = nat_tile<T, DP>(smem, 1);
        const T* Kt = tr_tile<T, DP>(smem, NN, 0);
        const int L = a.L;
        const float sc = a.scale;
        f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = p0, d1 = p0;
        mma_d<T, DP>(p0, Kn, qf, w.l16, w.g);
        mma_d<T, DP>(p1, Kn + 16 * LY::PN, qf, w.l16, w.g);
        mma_d<T, DP>(d0, Vn, df, w.l16, w.g);
        mma_d<T, DP>(d1, Vn + 16 * LY::PN, df, w.l16, w.g);
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
        for (int t = 0; t < LY::NT; ++t) acc[t] = mma_seq<T>(acc[t], read_seqa<T, DP>(Kt, t, w.l16, w.g), dsb);
    }
    __device__ __forceinline__ void finish(const Args& a, const WaveIds& w) {
        if (active && own < a.L) store_rows<T, DP>(a.out0, ((int64_t)bh * a.L + own) * a.D, acc, a.scale, a.D, w.g);
    }
};

// Col pass (own = 16 key rows per wave): dK = s sum_i dS[i][j] Q[i], dV = sum_i P[i][j] dO[i]. Other side per chunk:
// Q and dO (natural and transposed); row statistics lse, Dr from ``st`` with row stride ``ss``.
template <typename T, int DP> struct BwdCol {
    using LY = Lay<T, DP>;
    static constexpr int NN = 2, NTR = 2, SMEM = NN * LY::NATB + NTR * LY::TRB;
    OwnFrag<T, DP> kf, vf;
    f32x4 ak[LY::NT], av[LY::NT];
    int own, bh;
    bool active;

    __device__ __forceinline__ Src<T, 2> src(const Args& a, int b, int h) const {
        return {{slice<T>(a.q, b, h), slice<T>(a.dO, b, h)}, {a.q.sl, a.dO.sl}};
    }
    __device__ __forceinline__ void lds(unsigned char* smem, T* (&nat)[2], T* (&tr)[2]) const {
        nat[0] = nat_tile<T, DP>(smem, 0);
        nat[1] = nat_tile<T, DP>(smem, 1);
        tr[0] = tr_tile<T, DP>(smem, NN, 0);
        tr[1] = tr_tile<T, DP>(smem, NN, 1);
    }
    __device__ __forceinline__ void init(const Args& a, int bh_, int own_base, const WaveIds& w) {
        bh = bh_;
        const int b = bh / a.H, h = bh - b * a.H;
        const int row0 = own_base + w.wave * 16;
        own = row0 + w.l16;
        active = row0 < a.L;
        load_own<T, DP>(kf, slice<T>(a.k, b, h), a.k.sl, own, a.L, a.D, w.g);
        load_own<T, DP>(vf, slice<T>(a.v, b, h), a.v.sl, own, a.L, a.D, w.g);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) ak[t] = av[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __device__ __forceinline__ void chunk(const Args& a, unsigned char* smem, const float* st, int ss,
                                          const WaveIds& w) {
        if (!active) return;
        const T* Qn = nat_tile<T, DP>(smem, 0);
        const T* On = nat_tile<T, DP>(smem, 1);
        const T* Qt = tr_tile<T, DP>(smem, NN, 0);
        const T* Ot = tr_tile<T, DP>(smem, NN, 1);
        const float sc = a.scale;
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(st + 4 * w.g);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(st + 16 + 4 * w.g);
        const f32x4 r0 = *reinterpret_cast<const f32x4*>(st + ss + 4 * w.g);
        const f32x4 r1 = *reinterpret_cast<const f32x4*>(st + ss + 16 + 4 * w.g);
        f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, d0 = p0, d1 = p0;
        mma_d<T, DP>(p0, Qn, kf, w.l16, w.g);
        mma_d<T, DP>(p1, Qn + 16 * LY::PN, kf, w.l16, w.g);
        mma_d<T, DP>(d0, On, vf, w.l16, w.g);
        mma_d<T, DP>(d1, On + 16 * LY::PN, vf, w.l16, w.g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p0[r] = fast_exp2(fmaf(p0[r], sc, -l0[r]) * LOG2E);  // lse = +inf on padded rows -> P = 0
            p1[r] = fast_exp2(fmaf(p1[r], sc, -l1[r]) * LOG2E);
            d0[r] = p0[r] * (d0[r] - r0[r]);
            d1[r] = p1[r] * (d1[r] - r1[r]);
        }
        const SeqB<T> pb = make_seqb<T>(p0, p1);
        const SeqB<T> dsb = make_seqb<T>(d0, d1);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) {
            av[t] = mma_seq<T>(av[t], read_seqa<T, DP>(Ot, t, w.l16, w.g), pb);
            ak[t] = mma_seq<T>(ak[t], read_seqa<T, DP>(Qt, t, w.l16, w.g), dsb);
        }
    }
    __device__ __forceinline__ void finish(const Args& a, const WaveIds& w) {
        if (active && own < a.L) {
            const int64_t r = ((int64_t)bh * a.L + own) * a.D;
            store_rows<T, DP>(a.out1, r, ak, a.scale, a.D, w.g);
            store_rows<T, DP>(a.out2, r, av, 1.f, a.D, w.g);
        }
    }
};

// =====================================================================================================================
// Backward of the backward
// =====================================================================================================================

// Row pass (own = 16 query rows per wave), streaming form (E and T are known only at the end of the row):
//   X = sum_j (dS A + P Bm) K + dS gK,  U = dS K,  Z = P K,  W = (P A) V + P gV,
//   hQ = s (X - E U - T Z),  hdO = W - E O.
// Other side per chunk: K, gK, V, gV (natural and transposed). Publishes lse, Dr, E, T of its rows:
// FUSED -> LDS st ([lse | Dr | E | T], STAT_MAX each), else Dr, E, T -> a.stats.
template <typename T, int DP, bool FUSED> struct BbRow {
    using LY = Lay<T, DP>;
    static constexpr int NN = 4, NTR = 4, SMEM = NN * LY::NATB + NTR * LY::TRB;
    OwnFrag<T, DP> qf, gqf, df;
    f32x4 X[LY::NT], U[LY::NT], Z[LY::NT], Wv[LY::NT];
    float dr, lse, e_acc, t_acc;
    int own, bh;
    bool active;

    __device__ __forceinline__ Src<T, 4> src(const Args& a, int b, int h) const {
        return {{slice<T>(a.k, b, h), slice<T>(a.gk, b, h), slice<T>(a.v, b, h), slice<T>(a.gv, b, h)},
                {a.k.sl, a.gk.sl, a.v.sl, a.gv.sl}};
    }
    __device__ __forceinline__ void lds(unsigned char* smem, T* (&nat)[4], T* (&tr)[4]) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            nat[i] = nat_tile<T, DP>(smem, i);
            tr[i] = tr_tile<T, DP>(smem, NN, i);
        }
    }
    __device__ __forceinline__ void init(const Args& a, int bh_, int own_base, const WaveIds& w) {
        bh = bh_;
        const int b = bh / a.H, h = bh - b * a.H;
        const int L = a.L, D = a.D;
        const int row0 = own_base + w.wave * 16;
        own = row0 + w.l16;
        active = row0 < L;
        OwnFrag<T, DP> of;
        load_own<T, DP>(qf, slice<T>(a.q, b, h), a.q.sl, own, L, D, w.g);
        load_own<T, DP>(gqf, slice<T>(a.gq, b, h), a.gq.sl, own, L, D, w.g);
        load_own<T, DP>(df, slice<T>(a.dO, b, h), a.dO.sl, own, L, D, w.g);
        load_own<T, DP>(of, reinterpret_cast<const T*>(a.o) + (int64_t)bh * L * D, D, own, L, D, w.g);
        const float lraw = a.lse[(int64_t)bh * L + (own < L ? own : L - 1)];  // unconditional load
        lse = (own < L) ? lraw : 0.f;
        dr = xsum4(frag_dot<T, DP>(df, of));
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) X[t] = U[t] = Z[t] = Wv[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        e_acc = t_acc = 0.f;
    }
    __device__ __forceinline__ void chunk(const Args& a, int x0, unsigned char* smem, const WaveIds& w) {
        if (!active) return;
        const T* Kn = nat_tile<T, DP>(smem, 0);
        const T* gKn = nat_tile<T, DP>(smem, 1);
        const T* Vn = nat_tile<T, DP>(smem, 2);
        const T* gVn = nat_tile<T, DP>(smem, 3);
        const T* Kt = tr_tile<T, DP>(smem, NN, 0);
        const T* gKt = tr_tile<T, DP>(smem, NN, 1);
        const T* Vt = tr_tile<T, DP>(smem, NN, 2);
        const T* gVt = tr_tile<T, DP>(smem, NN, 3);
        const int L = a.L;
        const float sc = a.scale;
        f32x4 p[2], dp[2], at[2], bm[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            p[hh] = dp[hh] = at[hh] = bm[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int off = hh * 16 * LY::PN;
            mma_d<T, DP>(p[hh], Kn + off, qf, w.l16, w.g);
            mma_d<T, DP>(at[hh], Kn + off, gqf, w.l16, w.g);
            mma_d<T, DP>(at[hh], gKn + off, qf, w.l16, w.g);
            mma_d<T, DP>(dp[hh], Vn + off, df, w.l16, w.g);
            mma_d<T, DP>(bm[hh], gVn + off, df, w.l16, w.g);
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
        const SeqB<T> pb = make_seqb<T>(p[0], p[1]);
        const SeqB<T> dsb = make_seqb<T>(ds[0], ds[1]);
        const SeqB<T> pab = make_seqb<T>(pa[0], pa[1]);
        const SeqB<T> m1b = make_seqb<T>(m1[0], m1[1]);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) {
            const SeqA<T> ka = read_seqa<T, DP>(Kt, t, w.l16, w.g);
            X[t] = mma_seq<T>(X[t], ka, m1b);
            U[t] = mma_seq<T>(U[t], ka, dsb);
            Z[t] = mma_seq<T>(Z[t], ka, pb);
            X[t] = mma_seq<T>(X[t], read_seqa<T, DP>(gKt, t, w.l16, w.g), dsb);
            Wv[t] = mma_seq<T>(Wv[t], read_seqa<T, DP>(Vt, t, w.l16, w.g), pab);
            Wv[t] = mma_seq<T>(Wv[t], read_seqa<T, DP>(gVt, t, w.l16, w.g), pb);
        }
    }
    __device__ __forceinline__ void finish(const Args& a, const WaveIds& w, float* st) {
        const float E = xsum4(e_acc);
        const float Tm = xsum4(t_acc);
        const int L = a.L, D = a.D;
        if (active && own < L) {
            const int64_t r = ((int64_t)bh * L + own) * D;
            const T* O = reinterpret_cast<const T*>(a.o) + r;
#pragma unroll
            for (int t = 0; t < LY::NT; ++t) {
                const int d = 16 * t + 4 * w.g;
                if (d < D) {
                    const f32x4 hq = (X[t] - E * U[t] - Tm * Z[t]) * a.scale;
                    const f32x4 hdo = Wv[t] - E * load4<T>(O + d);
                    store4<T>(reinterpret_cast<T*>(a.out0) + r + d, hq);
                    store4<T>(reinterpret_cast<T*>(a.out3) + r + d, hdo);
                }
            }
        }
        if (w.g == 0 && active) {
            if constexpr (FUSED) {
                const bool ok = own < L;
                st[own] = ok ? lse : INFINITY;
                st[STAT_MAX + own] = ok ? dr : 0.f;
                st[2 * STAT_MAX + own] = ok ? E : 0.f;
                st[3 * STAT_MAX + own] = ok ? Tm : 0.f;
            } else if (own < L) {
                const int64_t r = (int64_t)bh * L + own;
                a.stats[r] = dr;
                a.stats[a.bhl + r] = E;
                a.stats[2 * a.bhl + r] = Tm;
            }
        }
    }
};

// Col pass (own = 16 key rows per wave): hK = s sum_i (dS2[i][j] Q[i] + dS[i][j] gQ[i]), hV = sum_i Pa[i][j] dO[i].
// Other side per chunk: Q, gQ, dO (natural and transposed); row statistics lse, Dr, E, T from ``st`` (stride ``ss``).
template <typename T, int DP> struct BbCol {
    using LY = Lay<T, DP>;
    static constexpr int NN = 3, NTR = 3, SMEM = NN * LY::NATB + NTR * LY::TRB;
    OwnFrag<T, DP> kf, gkf, vf, gvf;
    f32x4 hk[LY::NT], hv[LY::NT];
    int own, bh;
    bool active;

    __device__ __forceinline__ Src<T, 3> src(const Args& a, int b, int h) const {
        return {{slice<T>(a.q, b, h), slice<T>(a.gq, b, h), slice<T>(a.dO, b, h)}, {a.q.sl, a.gq.sl, a.dO.sl}};
    }
    __device__ __forceinline__ void lds(unsigned char* smem, T* (&nat)[3], T* (&tr)[3]) const {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            nat[i] = nat_tile<T, DP>(smem, i);
            tr[i] = tr_tile<T, DP>(smem, NN, i);
        }
    }
    __device__ __forceinline__ void init(const Args& a, int bh_, int own_base, const WaveIds& w) {
        bh = bh_;
        const int b = bh / a.H, h = bh - b * a.H;
        const int row0 = own_base + w.wave * 16;
        own = row0 + w.l16;
        active = row0 < a.L;
        load_own<T, DP>(kf, slice<T>(a.k, b, h), a.k.sl, own, a.L, a.D, w.g);
        load_own<T, DP>(gkf, slice<T>(a.gk, b, h), a.gk.sl, own, a.L, a.D, w.g);
        load_own<T, DP>(vf, slice<T>(a.v, b, h), a.v.sl, own, a.L, a.D, w.g);
        load_own<T, DP>(gvf, slice<T>(a.gv, b, h), a.gv.sl, own, a.L, a.D, w.g);
#pragma unroll
        for (int t = 0; t < LY::NT; ++t) hk[t] = hv[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __device__ __forceinline__ void chunk(const Args& a, unsigned char* smem, const float* st, int ss,
                                          const WaveIds& w) {
        if (!active) return;
        const T* Qn = nat_tile<T, DP>(smem, 0);
        const T* gQn = nat_tile<T, DP>(smem, 1);
        const T* On = nat_tile<T, DP>(smem, 2);
        const T* Qt = tr_tile<T, DP>(smem, NN, 0);
        const T* gQt = tr_tile<T, DP>(smem, NN, 1);
        const T* Ot = tr_tile<T, DP>(smem, NN, 2);
        const float sc = a.scale;
        f32x4 p[2], dp[2], at[2], bm[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            p[hh] = dp[hh] = at[hh] = bm[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int off = hh * 16 * LY::PN;
            mma_d<T, DP>(p[hh], Qn + off, kf, w.l16, w.g);
            mma_d<T, DP>(at[hh], Qn + off, gkf, w.l16, w.g);
            mma_d<T, DP>(at[hh], gQn + off, kf, w.l16, w.g);
            mma_d<T, DP>(dp[hh], On + off, vf, w.l16, w.g);
            mma_d<T, DP>(bm[hh], On + off, gvf, w.l16, w.g);
        }
        f32x4 ds[2], ds2[2], pa[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int so = 16 * hh + 4 * w.g;
            const f32x4 ls = *reinterpret_cast<const f32x4*>(st + so);
            const f32x4 rs = *reinterpret_cast<const f32x4*>(st + ss + so);
            const f32x4 es = *reinterpret_cast<const f32x4*>(st + 2 * ss + so);
            const f32x4 ts = *reinterpret_cast<const f32x4*>(st + 3 * ss + so);
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
            hk[t] = mma_seq<T>(hk[t], read_seqa<T, DP>(Qt, t, w.l16, w.g), ds2b);
            hk[t] = mma_seq<T>(hk[t], read_seqa<T, DP>(gQt, t, w.l16, w.g), dsb);
            hv[t] = mma_seq<T>(hv[t], read_seqa<T, DP>(Ot, t, w.l16, w.g), pab);
        }
    }
    __device__ __forceinline__ void finish(const Args& a, const WaveIds& w) {
        if (active && own < a.L) {
            const int64_t r = ((int64_t)bh * a.L + own) * a.D;
            store_rows<T, DP>(a.out1, r, hk, a.scale, a.D, w.g);
            store_rows<T, DP>(a.out2, r, hv, 1.f, a.D, w.g);
        }
    }
};

// =====================================================================================================================
// Pass drivers. Each chunk: barrier, write the staged registers to LDS, barrier, issue the next chunk's loads (they
// stay in flight during this chunk's MFMA work), compute. The one-workgroup kernels prefetch the col pass's first
// chunk during the row pass's last chunk.
// =====================================================================================================================

template <int NS> struct NoStats {};

template <typename T, int DP, class Row, class Col, int NCOL, int NSTAT>
__device__ __forceinline__ void fused_two_pass(const Args& a, unsigned char* smem, float* st) {
    const WaveIds w = wave_ids();
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L, D = a.D;
    for (int i = w.tid; i < STAT_MAX; i += w.nthr) {
        st[i] = INFINITY;
#pragma unroll
        for (int s = 1; s <= NSTAT; ++s) st[s * STAT_MAX + i] = 0.f;
    }
    Row row;
    const auto rsrc = row.src(a, b, h);
    constexpr int NROW = sizeof(rsrc.p) / sizeof(rsrc.p[0]);
    T* rn[NROW];
    T* rt[NROW];
    row.lds(smem, rn, rt);
    Stage<T, DP, NROW> rst;
    Stage<T, DP, NCOL> cst;
    Col col;
    const auto csrc = col.src(a, b, h);
    T* cn[NCOL];
    T* ct[NCOL];
    col.lds(smem, cn, ct);

    rst.load(rsrc, 0, L, D, w.tid, w.nthr);
    lds_barrier();  // statistics defaults visible before the row pass publishes
    if constexpr (NSTAT == 1) {
        row.init(a, bh, 0, w, st);
    } else {
        row.init(a, bh, 0, w);
    }
    for (int x0 = 0; x0 < L; x0 += CH) {
        lds_barrier();
        rst.store(rn, rt, w.tid, w.nthr);
        lds_barrier();
        if (x0 + CH < L)
            rst.load(rsrc, x0 + CH, L, D, w.tid, w.nthr);
        else
            cst.load(csrc, 0, L, D, w.tid, w.nthr);
        row.chunk(a, x0, smem, w);
    }
    if constexpr (NSTAT == 1) {
        row.finish(a, w);
    } else {
        row.finish(a, w, st);
    }
    col.init(a, bh, 0, w);
    for (int x0 = 0; x0 < L; x0 += CH) {
        lds_barrier();
        cst.store(cn, ct, w.tid, w.nthr);
        lds_barrier();
        if (x0 + CH < L) cst.load(csrc, x0 + CH, L, D, w.tid, w.nthr);
        col.chunk(a, smem, st + x0, STAT_MAX, w);
    }
    col.finish(a, w);
}

template <typename T, int DP> struct FusedSmem {
    static constexpr int BWD = BwdRow<T, DP, true>::SMEM > BwdCol<T, DP>::SMEM ? BwdRow<T, DP, true>::SMEM
                                                                                  : BwdCol<T, DP>::SMEM;
    static constexpr int BB = BbRow<T, DP, true>::SMEM > BbCol<T, DP>::SMEM ? BbRow<T, DP, true>::SMEM
                                                                             : BbCol<T, DP>::SMEM;
};

template <typename T, int DP> __global__ __launch_bounds__(512) void k_bwd_fused(Args a) {
    __shared__ __align__(16) unsigned char smem[FusedSmem<T, DP>::BWD];
    __shared__ __align__(16) float st[2 * STAT_MAX];
    fused_two_pass<T, DP, BwdRow<T, DP, true>, BwdCol<T, DP>, 2, 1>(a, smem, st);
}

template <typename T, int DP> __global__ __launch_bounds__(512) void k_bb_fused(Args a) {
    __shared__ __align__(16) unsigned char smem[FusedSmem<T, DP>::BB];
    __shared__ __align__(16) float st[4 * STAT_MAX];
    fused_two_pass<T, DP, BbRow<T, DP, true>, BbCol<T, DP>, 3, 3>(a, smem, st);
}

#include "attn_resident.hpp"
#include "attn_long.hpp"

// Two-launch row kernel: own rows [blk * 16 W, (blk + 1) * 16 W) of one (b, h); statistics go to a.stats.
template <typename T, int DP, class Row, int NROW, bool BB>
__device__ __forceinline__ void stream_row(const Args& a, unsigned char* smem) {
    const WaveIds w = wave_ids();
    int bh, blk;
    decode_block(a, bh, blk);
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L, D = a.D;
    Row row;
    const auto src = row.src(a, b, h);
    T* rn[NROW];
    T* rt[NROW];
    row.lds(smem, rn, rt);
    Stage<T, DP, NROW> rst;
    rst.load(src, 0, L, D, w.tid, w.nthr);
    if constexpr (BB) {
        row.init(a, bh, blk * (w.nthr >> 2), w);
    } else {
        row.init(a, bh, blk * (w.nthr >> 2), w, nullptr);
    }
    for (int x0 = 0; x0 < L; x0 += CH) {
        lds_barrier();
        rst.store(rn, rt, w.tid, w.nthr);
        lds_barrier();
        if (x0 + CH < L) rst.load(src, x0 + CH, L, D, w.tid, w.nthr);
        row.chunk(a, x0, smem, w);
    }
    if constexpr (BB) {
        row.finish(a, w, nullptr);
    } else {
        row.finish(a, w);
    }
}

// Two-launch col kernel: own rows [blk * 16 W, (blk + 1) * 16 W) of one (b, h); statistics staged from a.lse/a.stats.
template <typename T, int DP, class Col, int NCOL, int NSTAT>
__device__ __forceinline__ void stream_col(const Args& a, unsigned char* smem) {
    const WaveIds w = wave_ids();
    int bh, blk;
    decode_block(a, bh, blk);
    const int b = bh / a.H, h = bh - b * a.H;
    const int L = a.L, D = a.D;
    Col col;
    const auto src = col.src(a, b, h);
    T* cn[NCOL];
    T* ct[NCOL];
    col.lds(smem, cn, ct);
    float* stc = reinterpret_cast<float*>(smem + Col::SMEM);
    Stage<T, DP, NCOL> cst;
    StatStage<NSTAT> sst;
    const int64_t rb = (int64_t)bh * L;
    cst.load(src, 0, L, D, w.tid, w.nthr);
    sst.load(a.lse, a.stats, a.bhl, rb, 0, L, w.tid);
    col.init(a, bh, blk * (w.nthr >> 2), w);
    for (int x0 = 0; x0 < L; x0 += CH) {
        lds_barrier();
        cst.store(cn, ct, w.tid, w.nthr);
        sst.store(stc, w.tid);
        lds_barrier();
        if (x0 + CH < L) {
            cst.load(src, x0 + CH, L, D, w.tid, w.nthr);
            sst.load(a.lse, a.stats, a.bhl, rb, x0 + CH, L, w.tid);
        }
        col.chunk(a, smem, stc, CH, w);
    }
    col.finish(a, w);
}

template <typename T, int DP> __global__ __launch_bounds__(256) void k_bwd_row(Args a) {
    __shared__ __align__(16) unsigned char smem[BwdRow<T, DP, false>::SMEM];
    stream_row<T, DP, BwdRow<T, DP, false>, 2, false>(a, smem);
}

template <typename T, int DP> __global__ __launch_bounds__(256) void k_bwd_col(Args a) {
    __shared__ __align__(16) unsigned char smem[BwdCol<T, DP>::SMEM + 2 * CH * 4];
    stream_col<T, DP, BwdCol<T, DP>, 2, 1>(a, smem);
}

template <typename T, int DP> __global__ __launch_bounds__(256) void k_bb_row(Args a) {
    __shared__ __align__(16) unsigned char smem[BbRow<T, DP, false>::SMEM];
    stream_row<T, DP, BbRow<T, DP, false>, 4, true>(a, smem);
}

template <typename T, int DP> __global__ __launch_bounds__(256) void k_bb_col(Args a) {
    __shared__ __align__(16) unsigned char smem[BbCol<T, DP>::SMEM + 4 * CH * 4];
    stream_col<T, DP, BbCol<T, DP>, 3, 3>(a, smem);
}

// =====================================================================================================================
// Host side: argument checks, plan, launch.
// =====================================================================================================================

constexpr int STREAM_WAVES = 4;  // waves (x16 own rows) per workgroup of the two-launch kernels

static bool fused_shape(int L) { return L <= STAT_MAX; }

// One wave per 16 rows, at least MIN_THREADS threads (the chunk staging assumes it).
static int fused_threads(int L) {
    const int t = 64 * ((L + 15) / 16);
    return t < MIN_THREADS ? MIN_THREADS : t;
}

static int elem_size(int dtype) { return dtype == EBR_DTYPE_F64 ? 8 : (dtype == EBR_DTYPE_F32 ? 4 : 2); }

// The resident one-workgroup kernels (16-bit inputs): D must be a full chunk width and every slice's byte range
// (rows 0 .. L-1 of each strided input) must be addressable with 32-bit buffer offsets.
static bool strided_fits(const Strided& t, int L, int D, int es) {
    return ((int64_t)(L - 1) * t.sl + D) * es < ((int64_t)1 << 31);
}
static bool resident_shape(const Args& a, int dp, int es, bool grads) {
    if (es != 2 || a.D != dp || a.L > STAT_MAX) return false;
    bool ok = strided_fits(a.q, a.L, a.D, es) && strided_fits(a.k, a.L, a.D, es) && strided_fits(a.v, a.L, a.D, es);
    if (grads) {
        ok = ok && strided_fits(a.dO, a.L, a.D, es) && strided_fits(a.gq, a.L, a.D, es) &&
             strided_fits(a.gk, a.L, a.D, es) && strided_fits(a.gv, a.L, a.D, es);
    }
    return ok;
}

// k_bb_share loads rows with structured buffer loads, whose descriptor holds the row stride in 14 bits.
static bool struct_strides_fit(const Args& a) {
    const Strided* t[7] = {&a.q, &a.k, &a.v, &a.dO, &a.gq, &a.gk, &a.gv};
    for (const Strided* x : t)
        if (x->sl * 2 > STRUCT_STRIDE_MAX) return false;
    return true;
}

static int check_shape(int dtype, int B, int H, int L, int D) {
    if (dtype != EBR_DTYPE_F32 && dtype != EBR_DTYPE_BF16 && dtype != EBR_DTYPE_F16 && dtype != EBR_DTYPE_F64)
        return EBR_ERR_DTYPE;
    if (B < 1 || H < 1 || L < 1 || D < 1 || D > (dtype == EBR_DTYPE_F64 ? DMAX_F64 : DMAX_WIDE)) return EBR_ERR_SHAPE;
    const int vec = dtype == EBR_DTYPE_F64 ? 1 : (dtype == EBR_DTYPE_F32 ? 4 : 8);
    if (D % vec) return EBR_ERR_SHAPE;
    if ((int64_t)B * H * L >= ((int64_t)1 << 31)) return EBR_ERR_SHAPE;
    return EBR_OK;
}

// A forced plan must name a family; fp64 has one (its exact kernels) and takes EBR_PLAN_AUTO only.
static int check_plan(int dtype, int plan) {
    if (plan < EBR_PLAN_AUTO || plan > EBR_PLAN_LONG) return EBR_ERR_PLAN;
    if (dtype == EBR_DTYPE_F64 && plan != EBR_PLAN_AUTO) return EBR_ERR_PLAN;
    return EBR_OK;
}

// Row starts must be 16-byte aligned, except for fp64 (element-wise kernels): 8-byte aligned elements.
static int row_align(int es) { return es == 8 ? 8 : 16; }

static int check_ptr(const void* p, int es, bool need) {
    if (!p) return need ? EBR_ERR_NULL : EBR_OK;
    return ((uintptr_t)p % row_align(es)) ? EBR_ERR_ALIGN : EBR_OK;
}

static int check_strided(const void* p, const int64_t* s, int es) {
    int rc = check_ptr(p, es, true);
    if (rc) return rc;
    if (!s) return EBR_ERR_NULL;
    for (int i = 0; i < 3; ++i)
        if (s[i] < 0 || ((s[i] * es) % row_align(es))) return EBR_ERR_ALIGN;
    return EBR_OK;
}

static Strided mk(const void* p, const int64_t* s) {
    Strided t;
    t.p = p;
    t.sb = s ? s[0] : 0;
    t.sh = s ? s[1] : 0;
    t.sl = s ? s[2] : 0;
    return t;
}

static int launch_rc() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? EBR_OK : EBR_ERR_HIP_BASE + (int)e;
}

// Grid of a persistent kernel: as many workgroups as the current device holds at once (at most ``work``). Queried on
// every call (device attribute and the kernel's occupancy, host-side lookups that enqueue nothing), so the library
// keeps no state between calls. One workgroup per work item when the runtime cannot tell: the kernels are correct at
// any grid.
static int persistent_grid(const void* kernel, int threads, int64_t work) {
    int dev = 0, ncu = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess || ncu < 1 || per < 1) {
        (void)hipGetLastError();
        return (int)work;
    }
    const int64_t slots = (int64_t)ncu * per;
    return (int)(work < slots ? work : slots);
}

#include "attn_f64.hpp"

template <template <typename, int> class F, typename... Rest>
static int dispatch(int dtype, int D, Rest&&... rest) {
    if (dtype == EBR_DTYPE_F32) {
        if (D <= 16) return F<float, 16>::run(rest...);
        if (D <= 32) return F<float, 32>::run(rest...);
        if (D <= 64) return F<float, 64>::run(rest...);
        if (D <= 128) return F<float, 128>::run(rest...);
        return F<float, DMAX_WIDE>::run(rest...);
    }
    if (dtype == EBR_DTYPE_BF16) {
        if (D <= 32) return F<__bf16, 32>::run(rest...);
        if (D <= 64) return F<__bf16, 64>::run(rest...);
        if (D <= 128) return F<__bf16, 128>::run(rest...);
        return F<__bf16, DMAX_WIDE>::run(rest...);
    }
    if (D <= 32) return F<_Float16, 32>::run(rest...);
    if (D <= 64) return F<_Float16, 64>::run(rest...);
    if (D <= 128) return F<_Float16, 128>::run(rest...);
    return F<_Float16, DMAX_WIDE>::run(rest...);
}

// The long-sequence kernels (16-bit inputs, L > 128): D a full chunk width, 32-bit buffer offsets per slice.
// Compute waves (x16 own rows) per workgroup of the long kernels: 7 when the grid still holds at least four
// workgroups per CU (more rows per workgroup share each staged K/V tile: the Maze shape runs 15% faster than with 4,
// measured), else 4 (more, smaller workgroups for small batches).
constexpr int LONG_WAVES = 4;
constexpr int LONG_WAVES_WIDE = 7;
static bool long_wide(int64_t bh, int L) {
    const int64_t rows = 16 * LONG_WAVES_WIDE;
    return bh * ((L + rows - 1) / rows) >= 1024;
}
// k_bb_long_row's stage depth: 128 rows for the wide workgroup, the one workgroup a CU holds at its register use
// (two 64 KB stage buffers; half the barriers and stage hand-overs of 64-row stages: Maze bwd_bwd 1.016 -> 1.001 ms,
// measured), 64 for the 4-wave workgroups of small grids, two of which share a CU's LDS (32 rows with three
// workgroups per CU was slower).
constexpr int BB_ROW_STAGE = 64;
constexpr int BB_ROW_STAGE_WIDE = 128;
// k_bb_long_row needs about 150 VGPRs, so a SIMD holds 3 of its waves and a CU one 8-wave workgroup: 10 compute waves
// (+ the loader) fill the CU with one workgroup of 160 rows instead (Maze bwd_bwd 1.26 -> 1.18 ms, measured). The
// other long kernels keep 7: their wider variants measured slower (bwd with 9: 0.51 -> 0.70 ms; fwd with 6 or 13).
constexpr int BB_ROW_WAVES_WIDE = 10;
static bool long_shape(const Args& a, int dp, bool grads) {
    if (a.L <= STAT_MAX || a.D != dp) return false;
    const int es = 2;
    bool ok = strided_fits(a.q, a.L, a.D, es) && strided_fits(a.k, a.L, a.D, es) && strided_fits(a.v, a.L, a.D, es);
    if (grads) {
        ok = ok && strided_fits(a.dO, a.L, a.D, es) && strided_fits(a.gq, a.L, a.D, es) &&
             strided_fits(a.gk, a.L, a.D, es) && strided_fits(a.gv, a.L, a.D, es);
    }
    return ok;
}

static void plan_long(Args& a, int64_t bh, int rows) {
    a.nblk = (a.L + rows - 1) / rows;
    a.xcd_remap = 1;
    (void)bh;
}

static void plan_stream(Args& a, int64_t bh, int& grid, int& threads) {
    a.nblk = (a.L + 16 * STREAM_WAVES - 1) / (16 * STREAM_WAVES);
    a.xcd_remap = 1;
    grid = (int)(bh * a.nblk);
    threads = 64 * STREAM_WAVES;
}

// Whether a launcher may take kernel family f under the call's plan (EBR_PLAN_AUTO takes the first that applies).
static bool plan_allows(const Args& a, int f) { return a.plan == EBR_PLAN_AUTO || a.plan == f; }

template <typename T, int DP> struct FwdLaunch {
    static int run(Args a, hipStream_t s) {
        const int64_t bh = (int64_t)a.B * a.H;
        if constexpr (!ET<T>::F32 && DP <= 128) {
            if (plan_allows(a, EBR_PLAN_RESIDENT) && resident_shape(a, DP, 2, false)) {
                a.nblk = 1;
                const dim3 grid((int)bh), block(fused_threads(a.L));
                switch ((a.L + CH - 1) / CH) {
                    case 1: hipLaunchKernelGGL((k_fwd_res<T, DP, 1>), grid, block, 0, s, a); break;
                    case 2: hipLaunchKernelGGL((k_fwd_res<T, DP, 2>), grid, block, 0, s, a); break;
                    case 3: hipLaunchKernelGGL((k_fwd_res<T, DP, 3>), grid, block, 0, s, a); break;
                    default: hipLaunchKernelGGL((k_fwd_res<T, DP, 4>), grid, block, 0, s, a); break;
                }
                return launch_rc();
            }
        }
        if constexpr (!ET<T>::F32 && DP <= 128) {
            if (plan_allows(a, EBR_PLAN_LONG) && long_shape(a, DP, false)) {  // streamed stages, a loader wave
                auto run = [&](auto nw) {
                    constexpr int NW = decltype(nw)::value;
                    using C = LongCfg<T, DP, NW>;
                    plan_long(a, bh, C::ROWS);
                    hipLaunchKernelGGL((k_fwd_long<T, DP, NW>), dim3((int)(bh * a.nblk)), dim3(C::THREADS), 0, s, a);
                    return launch_rc();
                };
                return long_wide(bh, a.L) ? run(std::integral_constant<int, LONG_WAVES_WIDE>{})
                                          : run(std::integral_constant<int, LONG_WAVES>{});
            }
        }
        if (!plan_allows(a, EBR_PLAN_GENERIC)) return EBR_ERR_PLAN;
        int grid, threads;
        if (DP <= 128 && fused_shape(a.L)) {
            a.nblk = 1;
            a.xcd_remap = 0;
            grid = (int)bh;
            threads = fused_threads(a.L);
        } else {
            plan_stream(a, bh, grid, threads);
        }
        hipLaunchKernelGGL((k_fwd<T, DP>), dim3(grid), dim3(threads), 0, s, a);
        return launch_rc();
    }
};

template <typename T, int DP> struct BwdLaunch {
    static int run(Args a, hipStream_t s) {
        const int64_t bh = (int64_t)a.B * a.H;
        if constexpr (!ET<T>::F32 && DP <= 128) {
            a.gq = a.gk = a.gv = a.dO;  // only q, k, v, dO are read
            if ((plan_allows(a, EBR_PLAN_PERSISTENT) || a.plan == EBR_PLAN_RESIDENT) &&
                resident_shape(a, DP, 2, true)) {
                a.nblk = 1;
                const int nch = (a.L + CH - 1) / CH;
                // persistent, double-buffered with a loader wave (k_bwd_pipe), wherever two buffers of K, V, Q, dO
                // fit the LDS: D <= 64 up to four chunks, D = 128 up to two (the P and dS tiles where they fit too);
                // D = 128 with three chunks, or four up to L = 112, runs k_bwd_pp
                auto pipe = [&](auto nchc) {
                    constexpr int N = decltype(nchc)::value;
                    static_assert(BwdPipe<T, DP, N>::FITS, "two buffers fit the LDS");
                    const int thr = BwdPipe<T, DP, N>::THREADS;
                    const dim3 pg(persistent_grid(reinterpret_cast<const void*>(k_bwd_pipe<T, DP, N>), thr, bh));
                    hipLaunchKernelGGL((k_bwd_pipe<T, DP, N>), pg, dim3(thr), 0, s, a);
                    return launch_rc();
                };
                if (a.plan == EBR_PLAN_RESIDENT) {
                    // one (b, h) per workgroup, P and dS recomputed in the col pass (k_bwd_res)
                } else if constexpr (DP <= 64) {
                    switch (nch) {
                        case 1: return pipe(std::integral_constant<int, 1>{});
                        case 2: return pipe(std::integral_constant<int, 2>{});
                        case 3: return pipe(std::integral_constant<int, 3>{});
                        default: return pipe(std::integral_constant<int, 4>{});
                    }
                } else {
                    if (nch == 1) return pipe(std::integral_constant<int, 1>{});
                    if (nch == 2) return pipe(std::integral_constant<int, 2>{});
                    // one K, V and one Q, dO region, each loaded a pass ahead (k_bwd_pp), up to 7 compute waves
                    auto pp = [&](auto nchc, auto halfc) {
                        constexpr int N = decltype(nchc)::value;
                        constexpr bool HALF = decltype(halfc)::value;
                        static_assert(BwdPP<T, DP, N>::FITS, "the two regions and the store areas fit the LDS");
                        const int thr = BwdPP<T, DP, N>::THREADS;
                        const dim3 pg(
                            persistent_grid(reinterpret_cast<const void*>(k_bwd_pp<T, DP, N, HALF>), thr, bh));
                        hipLaunchKernelGGL((k_bwd_pp<T, DP, N, HALF>), pg, dim3(thr), 0, s, a);
                        return launch_rc();
                    };
                    using yes = std::true_type;
                    using no = std::false_type;
                    if (nch == 3) {
                        return a.L <= 3 * CH - 16 ? pp(std::integral_constant<int, 3>{}, yes{})
                                                  : pp(std::integral_constant<int, 3>{}, no{});
                    }
                    // four chunks: 7 compute waves, L <= 112, so the last chunk always holds one 16-row tile
                    static_assert(16 * BwdPP<T, DP, 4>::NWC == 4 * CH - 16, "HALF at four chunks");
                    if (a.L <= 16 * BwdPP<T, DP, 4>::NWC) return pp(std::integral_constant<int, 4>{}, yes{});
                }
                if (a.plan == EBR_PLAN_PERSISTENT) return EBR_ERR_PLAN;  // D = 128, L > 112
                const dim3 grid((int)bh), block(fused_threads(a.L));
                switch (nch) {
                    case 1: hipLaunchKernelGGL((k_bwd_res<T, DP, 1>), grid, block, 0, s, a); break;
                    case 2: hipLaunchKernelGGL((k_bwd_res<T, DP, 2>), grid, block, 0, s, a); break;
                    case 3: hipLaunchKernelGGL((k_bwd_res<T, DP, 3>), grid, block, 0, s, a); break;
                    default: hipLaunchKernelGGL((k_bwd_res<T, DP, 4>), grid, block, 0, s, a); break;
                }
                return launch_rc();
            }
        }
        if constexpr (!ET<T>::F32 && DP <= 128) {
            if (plan_allows(a, EBR_PLAN_LONG) && long_shape(a, DP, true)) {  // k_bwd_long_row, k_bwd_long_col
                auto run = [&](auto nw) {
                    constexpr int NW = decltype(nw)::value;
                    using C = LongCfg<T, DP, NW>;
                    if (!a.stats) return (int)EBR_ERR_SCRATCH;  // the row kernel publishes its statistics there
                    plan_long(a, bh, C::ROWS);
                    const dim3 grid((int)(bh * a.nblk)), block(C::THREADS);
                    hipLaunchKernelGGL((k_bwd_long_row<T, DP, NW>), grid, block, 0, s, a);
                    const int rc = launch_rc();
                    if (rc) return rc;
                    hipLaunchKernelGGL((k_bwd_long_col<T, DP, NW>), grid, block, 0, s, a);
                    return launch_rc();
                };
                return long_wide(bh, a.L) ? run(std::integral_constant<int, LONG_WAVES_WIDE>{})
                                          : run(std::integral_constant<int, LONG_WAVES>{});
            }
        }
        if (!plan_allows(a, EBR_PLAN_GENERIC)) return EBR_ERR_PLAN;
        if constexpr (DP <= 128) {  // wider rows take the two launches at any L (512-thread workgroups would spill)
            if (fused_shape(a.L)) {
                a.nblk = 1;
                a.xcd_remap = 0;
                hipLaunchKernelGGL((k_bwd_fused<T, DP>), dim3((int)bh), dim3(fused_threads(a.L)), 0, s, a);
                return launch_rc();
            }
        }
        int grid, threads;
        if (!a.stats) return (int)EBR_ERR_SCRATCH;  // the row kernel publishes its statistics there
        plan_stream(a, bh, grid, threads);
        hipLaunchKernelGGL((k_bwd_row<T, DP>), dim3(grid), dim3(threads), 0, s, a);
        int rc = launch_rc();
        if (rc) return rc;
        hipLaunchKernelGGL((k_bwd_col<T, DP>), dim3(grid), dim3(threads), 0, s, a);
        return launch_rc();
    }
};

template <typename T, int DP> struct BbLaunch {
    static int run(Args a, hipStream_t s) {
        const int64_t bh = (int64_t)a.B * a.H;
        if constexpr (DP > 128) {  // wider rows: the two streamed launches at any L
            if (!plan_allows(a, EBR_PLAN_GENERIC)) return EBR_ERR_PLAN;
            int grid, threads;
            if (!a.stats) return (int)EBR_ERR_SCRATCH;  // the row kernel publishes its statistics there
            plan_stream(a, bh, grid, threads);
            hipLaunchKernelGGL((k_bb_row<T, DP>), dim3(grid), dim3(threads), 0, s, a);
            const int rc = launch_rc();
            if (rc) return rc;
            hipLaunchKernelGGL((k_bb_col<T, DP>), dim3(grid), dim3(threads), 0, s, a);
            return launch_rc();
        } else if (fused_shape(a.L)) {
            a.nblk = 1;
            a.xcd_remap = 0;
            const dim3 grid((int)bh), block(fused_threads(a.L));
            if (a.plan == EBR_PLAN_LONG) return EBR_ERR_PLAN;
            if (a.plan == EBR_PLAN_GENERIC || !resident_shape(a, DP, (int)sizeof(T), true)) {
                if (!plan_allows(a, EBR_PLAN_GENERIC)) return EBR_ERR_PLAN;
                hipLaunchKernelGGL((k_bb_fused<T, DP>), grid, block, 0, s, a);
            } else if constexpr (!ET<T>::F32) {
                const int nch = (a.L + CH - 1) / CH;
                // tiles shared through LDS, persistent with loader waves (k_bb_share), where its regions fit the LDS:
                // D <= 64 up to three chunks, D = 128 up to two
                auto share = [&](auto nchc) {
                    constexpr int N = decltype(nchc)::value;
                    static_assert(BbShare<T, DP, N>::SMEM <= 160 * 1024, "the regions fit the LDS");
                    const int thr = BbShare<T, DP, N>::THREADS;
                    const dim3 pg(persistent_grid(reinterpret_cast<const void*>(k_bb_share<T, DP, N>), thr, bh));
                    hipLaunchKernelGGL((k_bb_share<T, DP, N>), pg, dim3(thr), 0, s, a);
                    return launch_rc();
                };
                if (a.plan != EBR_PLAN_RESIDENT && struct_strides_fit(a)) {
                    if (nch == 1) return share(std::integral_constant<int, 1>{});
                    if (nch == 2) return share(std::integral_constant<int, 2>{});
                    if constexpr (DP <= 64) {
                        if (nch == 3) return share(std::integral_constant<int, 3>{});
                    }
                }
                if (a.plan == EBR_PLAN_PERSISTENT) return EBR_ERR_PLAN;  // regions past the LDS, or long strides
                const bool half = a.L <= nch * CH - 16;  // the last chunk holds one 16-row tile
                switch (nch) {
                    case 1: hipLaunchKernelGGL((k_bb_res<T, DP, 1, false>), grid, block, 0, s, a); break;
                    case 2: hipLaunchKernelGGL((k_bb_res<T, DP, 2, false>), grid, block, 0, s, a); break;
                    case 3:
                        if (half) hipLaunchKernelGGL((k_bb_res<T, DP, 3, true>), grid, block, 0, s, a);
                        else hipLaunchKernelGGL((k_bb_res<T, DP, 3, false>), grid, block, 0, s, a);
                        break;
                    default:
                        if (half) hipLaunchKernelGGL((k_bb_res<T, DP, 4, true>), grid, block, 0, s, a);
                        else hipLaunchKernelGGL((k_bb_res<T, DP, 4, false>), grid, block, 0, s, a);
                        break;
                }
            }
            return launch_rc();
        }
        if constexpr (!ET<T>::F32 && DP <= 128) {
            if (plan_allows(a, EBR_PLAN_LONG) && long_shape(a, DP, true)) {  // k_bb_long_row, k_bb_long_col
                auto run = [&](auto nw) {
                    constexpr int NW = decltype(nw)::value;
                    // D = 128: the row kernel keeps the col kernel's waves and 64-row stages (two 128-row stages of
                    // four 256-byte-row tensors would take 256 KB of LDS)
                    constexpr bool WIDE = NW == LONG_WAVES_WIDE && DP <= 64;
                    constexpr int NWR = WIDE ? BB_ROW_WAVES_WIDE : NW;
                    constexpr int STG = WIDE ? BB_ROW_STAGE_WIDE : BB_ROW_STAGE;
                    {  // the row kernel has a row blocking of its own; the col kernel reads only its statistics
                        Args ar = a;
                        using CR = LongCfg<T, DP, NWR>;
                        if (!a.stats) return (int)EBR_ERR_SCRATCH;  // the row kernel publishes its statistics there
                        plan_long(ar, bh, CR::ROWS);
                        hipLaunchKernelGGL((k_bb_long_row<T, DP, NWR, STG>), dim3((int)(bh * ar.nblk)),
                                           dim3(CR::THREADS), 0, s, ar);
                    }
                    const int rc = launch_rc();
                    if (rc) return rc;
                    using C = LongCfg<T, DP, NW>;
                    plan_long(a, bh, C::ROWS);
                    const dim3 grid((int)(bh * a.nblk)), block(C::THREADS);
                    hipLaunchKernelGGL((k_bb_long_col<T, DP, NW>), grid, block, 0, s, a);
                    return launch_rc();
                };
                return long_wide(bh, a.L) ? run(std::integral_constant<int, LONG_WAVES_WIDE>{})
                                          : run(std::integral_constant<int, LONG_WAVES>{});
            }
        }
        if (!plan_allows(a, EBR_PLAN_GENERIC)) return EBR_ERR_PLAN;
        int grid, threads;
        if (!a.stats) return (int)EBR_ERR_SCRATCH;  // the row kernel publishes its statistics there
        plan_stream(a, bh, grid, threads);
        hipLaunchKernelGGL((k_bb_row<T, DP>), dim3(grid), dim3(threads), 0, s, a);
        int rc = launch_rc();
        if (rc) return rc;
        hipLaunchKernelGGL((k_bb_col<T, DP>), dim3(grid), dim3(threads), 0, s, a);
        return launch_rc();
    }
};

static Args base_args(int B, int H, int L, int D, float scale) {
    Args a = {};
    a.B = B;
    a.H = H;
    a.L = L;
    a.D = D;
    a.scale = scale;
    a.bhl = (int64_t)B * H * L;
    return a;
}

}  // namespace ebr

using namespace ebr;

extern "C" {

int ebr_attn_abi_version(void) { return EBR_ATTN_ABI_VERSION; }

const char* ebr_attn_arch(void) { return "gfx950"; }

const char* ebr_attn_error_string(int code) {
    switch (code) {
        case EBR_OK: return "ok";
        case EBR_ERR_DTYPE: return "unsupported dtype (expected fp32, bf16, fp16 or fp64)";
        case EBR_ERR_SHAPE:
            return "unsupported shape (need B, H, L >= 1, B*H*L < 2^31, D <= 256 and a multiple of 8 for 16-bit "
                   "or 4 for fp32, any D <= 256 for fp64)";
        case EBR_ERR_ALIGN:
            return "row start not 16-byte aligned (8-byte for fp64) (base pointer or a B/H/L stride)";
        case EBR_ERR_NULL: return "required pointer is NULL";
        case EBR_ERR_SCRATCH: return "scratch buffer required for this shape but NULL";
        case EBR_ERR_PLAN: return "the forced plan (EBR_PLAN_*) does not run this dtype, shape or stride pattern";
        case EBR_ERR_NOALLOC_SIZE:
            return "shape needs more row-statistics scratch than the no-allocation entry point holds "
                   "(EBR_NOALLOC_SCRATCH_BYTES)";
        default: break;
    }
    if (code >= EBR_ERR_HIP_BASE) return hipGetErrorString((hipError_t)(code - EBR_ERR_HIP_BASE));
    return "unknown error code";
}

int64_t ebr_attn_scratch_bytes(int op, int B, int H, int L, int D) {  // fp64 calls need none
    if (B < 1 || H < 1 || L < 1) return 0;
    if (fused_shape(L) && D <= 128) return 0;  // one workgroup per (b, h): no statistics leave it
    const int64_t bhl = (int64_t)B * H * L;
    if (op == EBR_OP_BWD) return bhl * 4;
    if (op == EBR_OP_BWD_BWD) return 3 * bhl * 4;
    return 0;
}

int ebr_attn_fwd(int dtype, int B, int H, int L, int D, float scale, const void* q, const int64_t q_str[3],
                 const void* k, const int64_t k_str[3], const void* v, const int64_t v_str[3], void* o, void* lse,
                 void* stream) {
    return ebr_attn_fwd_plan(dtype, B, H, L, D, scale, q, q_str, k, k_str, v, v_str, o, lse, stream, EBR_PLAN_AUTO);
}

int ebr_attn_fwd_plan(int dtype, int B, int H, int L, int D, float scale, const void* q, const int64_t q_str[3],
                      const void* k, const int64_t k_str[3], const void* v, const int64_t v_str[3], void* o,
                      void* lse, void* stream, int plan) {
    int rc = check_shape(dtype, B, H, L, D);
    if (!rc) rc = check_plan(dtype, plan);
    if (rc) return rc;
    const int es = elem_size(dtype);
    if ((rc = check_strided(q, q_str, es)) || (rc = check_strided(k, k_str, es)) ||
        (rc = check_strided(v, v_str, es)) || (rc = check_ptr(o, es, true)) || (rc = check_ptr(lse, 4, true)))
        return rc;
    Args a = base_args(B, H, L, D, scale);
    a.q = mk(q, q_str);
    a.k = mk(k, k_str);
    a.v = mk(v, v_str);
    a.out0 = o;
    a.lse_out = static_cast<float*>(lse);
    a.plan = plan;
    if (dtype == EBR_DTYPE_F64) return f64_fwd(a, (hipStream_t)stream);
    return dispatch<FwdLaunch>(dtype, D, a, (hipStream_t)stream);
}

int ebr_attn_bwd(int dtype, int B, int H, int L, int D, float scale, const void* q, const int64_t q_str[3],
                 const void* k, const int64_t k_str[3], const void* v, const int64_t v_str[3], const void* o,
                 const void* lse, const void* dO, const int64_t dO_str[3], void* dq, void* dk, void* dv,
                 float* scratch, void* stream) {
    return ebr_attn_bwd_plan(dtype, B, H, L, D, scale, q, q_str, k, k_str, v, v_str, o, lse, dO, dO_str, dq, dk, dv,
                             scratch, stream, EBR_PLAN_AUTO);
}

int ebr_attn_bwd_plan(int dtype, int B, int H, int L, int D, float scale, const void* q, const int64_t q_str[3],
                      const void* k, const int64_t k_str[3], const void* v, const int64_t v_str[3], const void* o,
                      const void* lse, const void* dO, const int64_t dO_str[3], void* dq, void* dk, void* dv,
                      float* scratch, void* stream, int plan) {
    int rc = check_shape(dtype, B, H, L, D);
    if (!rc) rc = check_plan(dtype, plan);
    if (rc) return rc;
    const int es = elem_size(dtype);
    if ((rc = check_strided(q, q_str, es)) || (rc = check_strided(k, k_str, es)) ||
        (rc = check_strided(v, v_str, es)) || (rc = check_strided(dO, dO_str, es)) ||
        (rc = check_ptr(o, es, true)) || (rc = check_ptr(lse, 4, true)) || (rc = check_ptr(dq, es, true)) ||
        (rc = check_ptr(dk, es, true)) || (rc = check_ptr(dv, es, true)))
        return rc;
    if (dtype != EBR_DTYPE_F64 && ebr_attn_scratch_bytes(EBR_OP_BWD, B, H, L, D) > 0 && !scratch)
        return EBR_ERR_SCRATCH;
    Args a = base_args(B, H, L, D, scale);
    a.q = mk(q, q_str);
    a.k = mk(k, k_str);
    a.v = mk(v, v_str);
    a.dO = mk(dO, dO_str);
    a.o = o;
    a.lse = static_cast<const float*>(lse);
    a.out0 = dq;
    a.out1 = dk;
    a.out2 = dv;
    a.stats = scratch;
    a.plan = plan;
    if (dtype == EBR_DTYPE_F64) return f64_bwd(a, (hipStream_t)stream);
    return dispatch<BwdLaunch>(dtype, D, a, (hipStream_t)stream);
}

int ebr_attn_bwd_bwd(int dtype, int B, int H, int L, int D, float scale, const void* q, const int64_t q_str[3],
                     const void* k, const int64_t k_str[3], const void* v, const int64_t v_str[3], const void* o,
                     const void* lse, const void* dO, const int64_t dO_str[3], const void* gq,
                     const int64_t gq_str[3], const void* gk, const int64_t gk_str[3], const void* gv,
                     const int64_t gv_str[3], void* hq, void* hk, void* hv, void* hdo, float* scratch,
                     void* stream) {
    return ebr_attn_bwd_bwd_plan(dtype, B, H, L, D, scale, q, q_str, k, k_str, v, v_str, o, lse, dO, dO_str, gq,
                                 gq_str, gk, gk_str, gv, gv_str, hq, hk, hv, hdo, scratch, stream, EBR_PLAN_AUTO);
}

int ebr_attn_bwd_bwd_plan(int dtype, int B, int H, int L, int D, float scale, const void* q,
                          const int64_t q_str[3], const void* k, const int64_t k_str[3], const void* v,
                          const int64_t v_str[3], const void* o, const void* lse, const void* dO,
                          const int64_t dO_str[3], const void* gq, const int64_t gq_str[3], const void* gk,
                          const int64_t gk_str[3], const void* gv, const int64_t gv_str[3], void* hq, void* hk,
                          void* hv, void* hdo, float* scratch, void* stream, int plan) {
    int rc = check_shape(dtype, B, H, L, D);
    if (!rc) rc = check_plan(dtype, plan);
    if (rc) return rc;
    const int es = elem_size(dtype);
    if ((rc = check_strided(q, q_str, es)) || (rc = check_strided(k, k_str, es)) ||
        (rc = check_strided(v, v_str, es)) || (rc = check_strided(dO, dO_str, es)) ||
        (rc = check_strided(gq, gq_str, es)) || (rc = check_strided(gk, gk_str, es)) ||
        (rc = check_strided(gv, gv_str, es)) || (rc = check_ptr(o, es, true)) || (rc = check_ptr(lse, 4, true)) ||
        (rc = check_ptr(hq, es, true)) || (rc = check_ptr(hk, es, true)) || (rc = check_ptr(hv, es, true)) ||
        (rc = check_ptr(hdo, es, true)))
        return rc;
    if (dtype != EBR_DTYPE_F64 && ebr_attn_scratch_bytes(EBR_OP_BWD_BWD, B, H, L, D) > 0 && !scratch)
        return EBR_ERR_SCRATCH;
    Args a = base_args(B, H, L, D, scale);
    a.q = mk(q, q_str);
    a.k = mk(k, k_str);
    a.v = mk(v, v_str);
    a.dO = mk(dO, dO_str);
    a.gq = mk(gq, gq_str);
    a.gk = mk(gk, gk_str);
    a.gv = mk(gv, gv_str);
    a.o = o;
    a.lse = static_cast<const float*>(lse);
    a.out0 = hq;
    a.out1 = hk;
    a.out2 = hv;
    a.out3 = hdo;
    a.stats = scratch;
    a.plan = plan;
    if (dtype == EBR_DTYPE_F64) return f64_bwd_bwd(a, (hipStream_t)stream);
    return dispatch<BbLaunch>(dtype, D, a, (hipStream_t)stream);
}

}  // extern "C"
