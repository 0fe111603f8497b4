// MFMA fragments, LDS chunk staging and lane reductions for the gfx950 attention kernels.
//
// Every contraction in the attention path is written as one of two shapes, both on the 16x16 MFMA tile
// (v_mfma_f32_16x16x32_{bf16,f16} for 16-bit inputs, v_mfma_f32_16x16x4_f32 for fp32):
//
//   d-contraction   C[m = x][n = own]  = sum_d X[x][d] * Own[own][d]
//                   A = rows of the "other side" tensor X from LDS in natural [x][d] layout,
//                   B = the wave's own 16 rows, kept in registers for the whole pass.
//   seq-contraction C[m = d][n = own] += sum_x Xt[d][x] * P[x][own]
//                   A = the other side tensor transposed ([d][x] layout in LDS),
//                   B = an L x L tile straight out of a d-contraction accumulator.
//
// A 16x16 accumulator holds, in lane l, column n = l % 16 and rows m = 4 * (l / 16) + r (r = 0..3). Read as an
// MFMA B operand, that is "column n = l % 16, k-slots in lane group l / 16" - exactly the B layout - so the L x L
// tiles never leave registers between the two contractions. For 16-bit inputs a 32-wide k chunk is two such tiles:
// lane group g holds rows x = 16 h + 4 g + r of tiles h = 0, 1 in k-slots s = 4 h + r. The transposed LDS copy
// stores column x at position 8 g + 4 h + r so that the matching A operand is one 16-byte LDS read. Which k-slot a
// value occupies inside the MFMA does not matter for the result: A and B use the same slot for the same x.
//
// Chunks of the other side are CH = 32 rows. Rows at or beyond L are zero-filled; the kernels mask what zeros do not
// neutralise (scores of padded keys).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ebr {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;

constexpr int CH = 32;                      // other-side rows per LDS chunk
constexpr float LOG2E = 1.4426950408889634f;
constexpr int STAT_MAX = 128;               // longest L handled by the one-workgroup-per-(b,h) kernels
constexpr int DMAX_WIDE = 256;              // widest head dim, 16-bit and fp32 (above 128: the streamed kernels)
constexpr int DMAX_F64 = 256;               // widest head dim of the fp64 kernels

template <typename T> struct ET;

template <> struct ET<__bf16> {
    static constexpr bool F32 = false;
    static constexpr int VEC = 8;           // elements per 16-byte vector
    static constexpr int PADN = 8;          // natural layout row padding (elements)
    static constexpr int PADT = 8;          // transposed layout row padding (elements)
    using v8 = bf16x8;
    using v4 = bf16x4;
    static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0,
                                                       0);
    }
    // k = 16 (v_mfma_f32_16x16x16_bf16): lane (row or column l16, group g) holds k = 4 g .. 4 g + 3
    static __device__ __forceinline__ f32x4 mma16(u32x2 a, u32x2 b, f32x4 c) {
        typedef __attribute__((ext_vector_type(4))) short s4;
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0,
                                                         0);
    }
};

template <> struct ET<_Float16> {
    static constexpr bool F32 = false;
    static constexpr int VEC = 8;
    static constexpr int PADN = 8;
    static constexpr int PADT = 8;
    using v8 = f16x8;
    using v4 = f16x4;
    static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0,
                                                      0);
    }
    static __device__ __forceinline__ f32x4 mma16(u32x2 a, u32x2 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4, a), __builtin_bit_cast(v4, b), c, 0, 0, 0);
    }
};

template <> struct ET<float> {
    static constexpr bool F32 = true;
    static constexpr int VEC = 4;
    static constexpr int PADN = 4;
    static constexpr int PADT = 4;
};

// Layout constants of one (T, DP) instantiation. DP is the head dimension padded to the d-chunk width.
template <typename T, int DP> struct Lay {
    static constexpr int VEC = ET<T>::VEC;
    static constexpr int CW = 4 * VEC;                   // d covered by one MFMA k step: 32 (16-bit) / 16 (fp32)
    static constexpr int NC = DP / CW;                   // 16-byte vectors per lane for a full row of D
    static constexpr int NT = DP / 16;                   // output d tiles of a seq-contraction
    static constexpr int PN = DP + ET<T>::PADN;          // natural row pitch (elements)
    static constexpr int PT = CH + ET<T>::PADT;          // transposed row pitch (elements)
    static constexpr int NATB = CH * PN * (int)sizeof(T);  // bytes of one natural chunk
    // fp32 above DP = 128: a transposed copy of each chunk does not fit beside the natural one (the backward of the
    // backward stages four tensors), so seq-contractions read their A operand from the natural rows, one element per
    // k slot, and a tensor wanted in both layouts is staged once.
    static constexpr bool NATSEQ = ET<T>::F32 && DP > 128;
    static constexpr int TRB = NATSEQ ? 0 : DP * PT * (int)sizeof(T);  // bytes of one transposed chunk
    static_assert(DP % CW == 0, "DP must be a multiple of the d-chunk width");
    static_assert(NATB % 16 == 0 && TRB % 16 == 0, "LDS regions must stay 16-byte aligned");
};

// Column of chunk-local row x in the transposed LDS layout (see the header comment).
template <typename T> __device__ __forceinline__ int tr_col(int x) {
    if constexpr (ET<T>::F32) {
        return x;
    } else {
        return ((x & 15) >> 2) * 8 + (x >> 4) * 4 + (x & 3);
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// Lane reductions over the four 16-lane groups (lanes l, l^16, l^32, l^48 hold the same own row).
// ---------------------------------------------------------------------------------------------------------------------

// gfx950's v_permlane16_swap / v_permlane32_swap exchange 16-lane rows between two registers without LDS. Called
// with the same register twice, every lane ends up holding its own value in one result and the value of lane
// l ^ 16 (l ^ 32) in the other, so one swap and one VALU op reduce over a lane pair. The same pairs and order as a
// shuffle-xor reduction: the sums are bit-identical to it.
__device__ __forceinline__ void xpair16(float v, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

__device__ __forceinline__ void xpair32(float v, float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

// max(a, b) for values that are never NaN (scores, -inf for masked keys): med3(a, b, +inf) selects v_max3_f32
// chains without the NaN-quieting copies that fmaxf adds to MFMA results.
__device__ __forceinline__ float fmax_nn(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, INFINITY); }

__device__ __forceinline__ float xsum4(float v) {
    float a, b;
    xpair16(v, a, b);
    xpair32(a + b, a, b);
    return a + b;
}

__device__ __forceinline__ float xmax4(float v) {
    float a, b;
    xpair16(v, a, b);
    xpair32(fmax_nn(a, b), a, b);
    return fmax_nn(a, b);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS operations (lgkmcnt(0)), not for its global
// loads, so loads issued before it stay in flight (``__syncthreads`` would wait for every memory operation).
// Completion of global -> LDS loads is waited for explicitly with ``vm_wait`` before such a barrier.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt(63), expcnt(7): not waited
    __builtin_amdgcn_s_barrier();
}

// Wait until at most N of this wave's vector-memory operations are outstanding (N < 16).
template <int N> __device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 16, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0x0f70 | N);
}

// ---------------------------------------------------------------------------------------------------------------------
// Own-side B fragments: lane (row = own, group g) holds d = c * CW + g * VEC + [0, VEC) for c < NC.
// ---------------------------------------------------------------------------------------------------------------------

template <typename T, int DP> struct OwnFrag {
    u32x4 v[Lay<T, DP>::NC];
};

template <typename T, int DP>
__device__ __forceinline__ void load_own(OwnFrag<T, DP>& f, const T* base, int64_t srow, int row, int L, int D,
                                         int g) {
    using LY = Lay<T, DP>;
    // Unconditional loads from a clamped (always valid) address, then a select: no branch, so the loads of several
    // fragments stay in flight together.
    const T* p = base + (int64_t)(row < L ? row : L - 1) * srow;
#pragma unroll
    for (int c = 0; c < LY::NC; ++c) {
        const int d0 = c * LY::CW + g * LY::VEC;
        const u32x4 z = {0u, 0u, 0u, 0u};
        const u32x4 v = *reinterpret_cast<const u32x4*>(p + (d0 < D ? d0 : D - LY::VEC));
        f.v[c] = (row < L && d0 < D) ? v : z;
    }
}

// sum_d a[d] * b[d] over this lane's slots, in fp32.
template <typename T, int DP>
__device__ __forceinline__ float frag_dot(const OwnFrag<T, DP>& a, const OwnFrag<T, DP>& b) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < Lay<T, DP>::NC; ++c) {
        if constexpr (ET<T>::F32) {
            const f32x4 x = __builtin_bit_cast(f32x4, a.v[c]);
            const f32x4 y = __builtin_bit_cast(f32x4, b.v[c]);
            s += x[0] * y[0] + x[1] * y[1] + x[2] * y[2] + x[3] * y[3];
        } else {
            using V8 = typename ET<T>::v8;
            const V8 x = __builtin_bit_cast(V8, a.v[c]);
            const V8 y = __builtin_bit_cast(V8, b.v[c]);
#pragma unroll
            for (int e = 0; e < 8; ++e) s += (float)x[e] * (float)y[e];
        }
    }
    return s;
}

// ---------------------------------------------------------------------------------------------------------------------
// d-contraction: acc[m = x][n = own] += sum_d Xn[x][d] * Own[own][d] for the 16 rows starting at Xn_tile.
// ---------------------------------------------------------------------------------------------------------------------

template <typename T, int DP>
__device__ __forceinline__ void mma_d(f32x4& acc, const T* Xn_tile, const OwnFrag<T, DP>& f, int l16, int g) {
    using LY = Lay<T, DP>;
    const T* p = Xn_tile + l16 * LY::PN + g * LY::VEC;
#pragma unroll
    for (int c = 0; c < LY::NC; ++c) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(p + c * LY::CW);
        if constexpr (ET<T>::F32) {
            const f32x4 af = __builtin_bit_cast(f32x4, a);
            const f32x4 bf = __builtin_bit_cast(f32x4, f.v[c]);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[e], bf[e], acc, 0, 0, 0);
        } else {
            acc = ET<T>::mma(a, f.v[c], acc);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// seq-contraction over one 32-row chunk: acc[t][m = d][n = own] += sum_x Xt[d][x] * P[x][own].
// SeqB is the B operand built from the two accumulator tiles p0 (rows 0..15) and p1 (rows 16..31).
// ---------------------------------------------------------------------------------------------------------------------

template <typename T> struct SeqB {
    u32x4 v;  // 8 values in k-slot order s = 4 h + r
};
template <> struct SeqB<float> {
    f32x4 h0, h1;
};

template <typename T> __device__ __forceinline__ SeqB<T> make_seqb(f32x4 p0, f32x4 p1) {
    SeqB<T> b;
    if constexpr (ET<T>::F32) {
        b.h0 = p0;
        b.h1 = p1;
    } else {
        using V8 = typename ET<T>::v8;
        V8 r;
        r[0] = (T)p0[0];
        r[1] = (T)p0[1];
        r[2] = (T)p0[2];
        r[3] = (T)p0[3];
        r[4] = (T)p1[0];
        r[5] = (T)p1[1];
        r[6] = (T)p1[2];
        r[7] = (T)p1[3];
        b.v = __builtin_bit_cast(u32x4, r);
    }
    return b;
}

// The 8 values of a 16-bit SeqB as fp32 (slot order s = 4 h + r) and back.
template <typename T> __device__ __forceinline__ void unpack_seqb(const SeqB<T>& b, float (&f)[8]) {
    using V8 = typename ET<T>::v8;
    const V8 v = __builtin_bit_cast(V8, b.v);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (float)v[e];
}

template <typename T> __device__ __forceinline__ SeqB<T> pack_seqb(const float (&f)[8]) {
    using V8 = typename ET<T>::v8;
    V8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (T)f[e];
    SeqB<T> b;
    b.v = __builtin_bit_cast(u32x4, v);
    return b;
}

template <typename T> struct SeqA {
    u32x4 v;
};
template <> struct SeqA<float> {
    f32x4 h0, h1;
};

// A operand of d tile t: lane (d = 16 t + l16, group g). Under NATSEQ, Xt holds the chunk's natural rows.
template <typename T, int DP> __device__ __forceinline__ SeqA<T> read_seqa(const T* Xt, int t, int l16, int g) {
    using LY = Lay<T, DP>;
    SeqA<T> a;
    if constexpr (LY::NATSEQ) {
        const T* q = Xt + 16 * t + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            a.h0[r] = q[(4 * g + r) * LY::PN];
            a.h1[r] = q[(16 + 4 * g + r) * LY::PN];
        }
        return a;
    }
    const T* p = Xt + (16 * t + l16) * LY::PT;
    if constexpr (ET<T>::F32) {
        a.h0 = *reinterpret_cast<const f32x4*>(p + 4 * g);
        a.h1 = *reinterpret_cast<const f32x4*>(p + 16 + 4 * g);
    } else {
        a.v = *reinterpret_cast<const u32x4*>(p + 8 * g);
    }
    return a;
}

template <typename T> __device__ __forceinline__ f32x4 mma_seq(f32x4 acc, const SeqA<T>& a, const SeqB<T>& b) {
    if constexpr (ET<T>::F32) {
#pragma unroll
        for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.h0[r], b.h0[r], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.h1[r], b.h1[r], acc, 0, 0, 0);
        return acc;
    } else {
        return ET<T>::mma(a.v, b.v, acc);
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// Register-staged chunk loads: every thread issues the global loads of its share of N tensors' chunk at once
// (``load``), keeps them in flight while the previous chunk is computed, then writes them to LDS, natural and/or
// transposed (``store``). Workgroups have at least MIN_THREADS threads, which fixes the per-thread share.
// ---------------------------------------------------------------------------------------------------------------------

constexpr int MIN_THREADS = 256;

template <typename T, int N> struct Src {
    const T* p[N];
    int64_t srow[N];
};

template <typename T, int DP, int N> struct Stage {
    using LY = Lay<T, DP>;
    static constexpr int VPR = DP / LY::VEC;  // 16-byte vectors per row
    static constexpr int TOTAL = CH * VPR;    // vectors per tensor chunk
    static constexpr int ITEMS = (TOTAL + MIN_THREADS - 1) / MIN_THREADS;
    u32x4 r[N][ITEMS];

    __device__ __forceinline__ void load(const Src<T, N>& s, int x0, int L, int D, int tid, int nthr) {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            const int it = tid + i * nthr;
            const int x = it % CH;  // consecutive lanes take consecutive rows (conflict-free transposed writes)
            const int c = it / CH;
            const int row = x0 + x;
            const int d0 = c * LY::VEC;
            const bool ok = it < TOTAL && row < L && d0 < D;
            const int64_t rr = row < L ? row : L - 1;  // clamped: the load is unconditional (no branch)
            const int dd = (it < TOTAL && d0 < D) ? d0 : D - LY::VEC;
#pragma unroll
            for (int t = 0; t < N; ++t) {
                const u32x4 z = {0u, 0u, 0u, 0u};
                const u32x4 v = *reinterpret_cast<const u32x4*>(s.p[t] + rr * s.srow[t] + dd);
                r[t][i] = ok ? v : z;
            }
        }
    }

    // Xn[t] / Xt[t] may be null (that layout is not wanted for tensor t). Under NATSEQ, Xt[t] takes natural rows too
    // and may alias Xn[t].
    __device__ __forceinline__ void store(T* const (&Xn)[N], T* const (&Xt)[N], int tid, int nthr) const {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            const int it = tid + i * nthr;
            if (it >= TOTAL) continue;
            const int x = it % CH;
            const int c = it / CH;
            const int d0 = c * LY::VEC;
            const int col = tr_col<T>(x);
#pragma unroll
            for (int t = 0; t < N; ++t) {
                if (Xn[t]) *reinterpret_cast<u32x4*>(Xn[t] + x * LY::PN + d0) = r[t][i];
                if constexpr (LY::NATSEQ) {
                    if (Xt[t] && Xt[t] != Xn[t]) *reinterpret_cast<u32x4*>(Xt[t] + x * LY::PN + d0) = r[t][i];
                } else if (Xt[t]) {
                    T* p = Xt[t] + d0 * LY::PT + col;
                    if constexpr (ET<T>::F32) {
                        const f32x4 e = __builtin_bit_cast(f32x4, r[t][i]);
#pragma unroll
                        for (int j = 0; j < 4; ++j) p[j * LY::PT] = e[j];
                    } else {
                        using V8 = typename ET<T>::v8;
                        const V8 e = __builtin_bit_cast(V8, r[t][i]);
#pragma unroll
                        for (int j = 0; j < 8; ++j) p[j * LY::PT] = e[j];
                    }
                }
            }
        }
    }
};

// Row statistics of one query chunk for a two-launch col pass: lse (+inf past L) and up to 3 scratch rows.
template <int NS> struct StatStage {
    float r[NS + 1];
    __device__ __forceinline__ void load(const float* lse, const float* stats, int64_t bhl, int64_t row_base, int x0,
                                         int L, int tid) {
        const int x = x0 + tid;
        const bool ok = tid < CH && x < L;
        const int64_t xc = row_base + (ok ? x : L - 1);  // clamped: unconditional loads, then selects
        const float l0 = lse[xc];
        r[0] = ok ? l0 : INFINITY;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float v = stats[s * bhl + xc];
            r[s + 1] = ok ? v : 0.f;
        }
    }
    __device__ __forceinline__ void store(float* st, int tid) const {
        if (tid < CH) {
#pragma unroll
            for (int s = 0; s <= NS; ++s) st[s * CH + tid] = r[s];
        }
    }
};

// ---------------------------------------------------------------------------------------------------------------------
// Row stores of seq-contraction outputs: lane (own, g) of tile t holds d = 16 t + 4 g + r.
// ---------------------------------------------------------------------------------------------------------------------

template <typename T> __device__ __forceinline__ void store4(T* p, f32x4 v) {
    if constexpr (ET<T>::F32) {
        *reinterpret_cast<f32x4*>(p) = v;
    } else {
        using V4 = typename ET<T>::v4;
        V4 r;
        r[0] = (T)v[0];
        r[1] = (T)v[1];
        r[2] = (T)v[2];
        r[3] = (T)v[3];
        *reinterpret_cast<u32x2*>(p) = __builtin_bit_cast(u32x2, r);
    }
}

// Four values rounded to a 16-bit type, packed as store4 writes them.
template <typename T> __device__ __forceinline__ u32x2 pack4(f32x4 v) {
    using V4 = typename ET<T>::v4;
    V4 r;
    r[0] = (T)v[0];
    r[1] = (T)v[1];
    r[2] = (T)v[2];
    r[3] = (T)v[3];
    return __builtin_bit_cast(u32x2, r);
}

template <typename T> __device__ __forceinline__ f32x4 load4(const T* p) {
    if constexpr (ET<T>::F32) {
        return *reinterpret_cast<const f32x4*>(p);
    } else {
        using V4 = typename ET<T>::v4;
        const V4 r = __builtin_bit_cast(V4, *reinterpret_cast<const u32x2*>(p));
        return f32x4{(float)r[0], (float)r[1], (float)r[2], (float)r[3]};
    }
}

}  // namespace ebr
