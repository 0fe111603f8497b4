/* C ABI of the MI355X (gfx950) fused second-order attention library, libebr_attn.so.
 *
 * Non-causal softmax attention on [B, H, L, D] tensors: the forward, its backward and the backward of the
 * backward. Each entry replaces one op of the reference's fused path and takes the same arguments in the same
 * meaning; only the calling convention is C (plain pointers, sizes and strides, no framework types).
 *
 * Conventions shared by every entry point:
 *   - dtype: EBR_DTYPE_F32, EBR_DTYPE_BF16, EBR_DTYPE_F16 or EBR_DTYPE_F64; all tensor arguments of one call share
 *     it, except lse and the scratch: lse is fp32 (fp64 for EBR_DTYPE_F64, as the reference keeps fp64 for fp64
 *     inputs, reference.py:14-16), the scratch fp32.
 *   - Strided inputs pass their element strides for the B, H and L dimensions as int64_t[3]; the D dimension is
 *     unit-stride. A stride may be 0 (an expanded row, e.g. an all-zero cotangent). Every row start must be 16-byte
 *     aligned: base pointer 16-byte aligned and each stride a multiple of 16 bytes (fp64: 8 bytes, i.e. any
 *     element-aligned view).
 *   - o, lse and every output are contiguous [B, H, L, D] (lse: [B, H, L], natural log).
 *   - scale is the softmax scale (D ** -0.5 by default), already rounded to fp32.
 *   - stream is a hipStream_t (NULL = the null stream). Kernels are enqueued on it; nothing synchronises.
 *   - The caller owns every buffer; the library allocates nothing and keeps no pointer after returning.
 *   - Return value: 0 on success, otherwise an EBR_ERR_* code or EBR_ERR_HIP_BASE + hipError_t;
 *     ebr_attn_error_string() describes it. Argument checks run before anything is enqueued.
 *   - Supported shapes: B, H, L >= 1; D <= 256 and a multiple of 8 (16-bit) or 4 (fp32); any D <= 256 for fp64.
 *     D above 128 runs the two streamed launches (EBR_PLAN_GENERIC) at every L.
 *   - fp64 runs exact fp64 vector-ALU kernels (the reference's fp64 path serves gradcheck shapes) and needs no
 *     scratch.
 */
#ifndef EBR_ATTN_H
#define EBR_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EBR_ATTN_ABI_VERSION 3

enum {
    EBR_DTYPE_F32 = 0,
    EBR_DTYPE_BF16 = 1,
    EBR_DTYPE_F16 = 2,
    EBR_DTYPE_F64 = 3,
};

enum {
    EBR_OK = 0,
    EBR_ERR_DTYPE = 1,       /* dtype code not supported (the reference raises TypeError) */
    EBR_ERR_SHAPE = 2,       /* B, H, L or D outside the supported range (the reference raises ValueError) */
    EBR_ERR_ALIGN = 3,       /* a pointer or stride breaks the 16-byte row alignment rule */
    EBR_ERR_NULL = 4,        /* a required pointer is NULL */
    EBR_ERR_SCRATCH = 5,     /* scratch is NULL but this shape needs one (see ebr_attn_scratch_bytes) */
    EBR_ERR_NOALLOC_SIZE = 6, /* the shape needs more scratch than EBR_NOALLOC_SCRATCH_BYTES (no-allocation entry) */
    EBR_ERR_PLAN = 7,        /* the forced plan does not run this dtype, shape or stride pattern (*_plan entries) */
    EBR_ERR_HIP_BASE = 1000, /* EBR_ERR_HIP_BASE + hipError_t of a failed launch */
};

enum {
    EBR_OP_FWD = 0,
    EBR_OP_BWD = 1,
    EBR_OP_BWD_BWD = 2,
};

/* Forward: o = softmax(scale * q k^T) v and lse = row logsumexp of scale * q k^T.
 * Replaces ebr_fused::attn_fwd(q, k, v, scale) -> (o, lse)
 *   (reference models/fused_attn/ops.py:65-77; Triton launcher models/fused_attn/triton_kernels.py:696-728). */
int ebr_attn_fwd(int dtype, int B, int H, int L, int D, float scale,
                 const void* q, const int64_t q_str[3],
                 const void* k, const int64_t k_str[3],
                 const void* v, const int64_t v_str[3],
                 void* o, void* lse, void* stream);

/* Backward: (dq, dk, dv) = gradient of <dO, o> with respect to (q, k, v); rowsum(dO * o) uses the stored o.
 * Replaces ebr_fused::attn_bwd(q, k, v, o, lse, do, scale) -> (dq, dk, dv)
 *   (reference models/fused_attn/ops.py:80-95; Triton launcher models/fused_attn/triton_kernels.py:731-839).
 * scratch: fp32, ebr_attn_scratch_bytes(EBR_OP_BWD, ...) bytes; may be NULL when that size is 0. */
int ebr_attn_bwd(int dtype, int B, int H, int L, int D, float scale,
                 const void* q, const int64_t q_str[3],
                 const void* k, const int64_t k_str[3],
                 const void* v, const int64_t v_str[3],
                 const void* o, const void* lse,
                 const void* dO, const int64_t dO_str[3],
                 void* dq, void* dk, void* dv, float* scratch, void* stream);

/* Backward of the backward: (hq, hk, hv, hdo) = derivative of <gq, dq> + <gk, dk> + <gv, dv> with respect to
 * (q, k, v, dO). The reference op also takes dq, which it does not read; this entry omits it.
 * Replaces ebr_fused::attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, scale) -> (hq, hk, hv, hdo)
 *   (reference models/fused_attn/ops.py:98-121; Triton launcher models/fused_attn/triton_kernels.py:842-968).
 * scratch: fp32, ebr_attn_scratch_bytes(EBR_OP_BWD_BWD, ...) bytes; may be NULL when that size is 0. */
int ebr_attn_bwd_bwd(int dtype, int B, int H, int L, int D, float scale,
                     const void* q, const int64_t q_str[3],
                     const void* k, const int64_t k_str[3],
                     const void* v, const int64_t v_str[3],
                     const void* o, const void* lse,
                     const void* dO, const int64_t dO_str[3],
                     const void* gq, const int64_t gq_str[3],
                     const void* gk, const int64_t gk_str[3],
                     const void* gv, const int64_t gv_str[3],
                     void* hq, void* hk, void* hv, void* hdo, float* scratch, void* stream);

/* Kernel families the *_plan entry points can force: the reference's launch-plan override (PLAN_OVERRIDE, a module
 * dictionary read by the Triton launchers, models/fused_attn/triton_kernels.py:610-615, 673-676) as a per-call
 * argument, since the library keeps no state. EBR_PLAN_AUTO is the library's own choice, the one the entry points
 * without a plan argument always make. A family that does not run the call's dtype, shape or strides returns
 * EBR_ERR_PLAN before anything is enqueued; fp64 takes EBR_PLAN_AUTO only. */
enum {
    EBR_PLAN_AUTO = 0,
    EBR_PLAN_GENERIC = 1,    /* fp32, bf16, fp16: one (b, h) per workgroup up to L = 128 (D <= 128), else two launches */
    EBR_PLAN_RESIDENT = 2,   /* bf16 / fp16, L <= 128, D of 32, 64 or 128: one (b, h) per workgroup, operands in LDS */
    EBR_PLAN_PERSISTENT = 3, /* bf16 / fp16, L <= 128, D <= 128 (bwd, bwd_bwd): persistent workgroups, loader waves */
    EBR_PLAN_LONG = 4,       /* bf16 / fp16, L > 128, D of 32, 64 or 128: 64-row stages streamed by a loader wave */
};

/* ebr_attn_fwd, ebr_attn_bwd and ebr_attn_bwd_bwd with the kernel family forced by plan (EBR_PLAN_*); same
 * arguments otherwise. The reference sets its plans through PLAN_OVERRIDE (triton_kernels.py:612-615, 673-676). */
int ebr_attn_fwd_plan(int dtype, int B, int H, int L, int D, float scale,
                      const void* q, const int64_t q_str[3],
                      const void* k, const int64_t k_str[3],
                      const void* v, const int64_t v_str[3],
                      void* o, void* lse, void* stream, int plan);
int ebr_attn_bwd_plan(int dtype, int B, int H, int L, int D, float scale,
                      const void* q, const int64_t q_str[3],
                      const void* k, const int64_t k_str[3],
                      const void* v, const int64_t v_str[3],
                      const void* o, const void* lse,
                      const void* dO, const int64_t dO_str[3],
                      void* dq, void* dk, void* dv, float* scratch, void* stream, int plan);
int ebr_attn_bwd_bwd_plan(int dtype, int B, int H, int L, int D, float scale,
                          const void* q, const int64_t q_str[3],
                          const void* k, const int64_t k_str[3],
                          const void* v, const int64_t v_str[3],
                          const void* o, const void* lse,
                          const void* dO, const int64_t dO_str[3],
                          const void* gq, const int64_t gq_str[3],
                          const void* gk, const int64_t gk_str[3],
                          const void* gv, const int64_t gv_str[3],
                          void* hq, void* hk, void* hv, void* hdo, float* scratch, void* stream, int plan);

/* Bytes of the library's own device scratch array behind ebr_attn_bwd_bwd_noalloc (one copy per GPU). */
#define EBR_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)

/* ebr_attn_bwd_bwd without the scratch argument, for callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc. It has no counterpart in the reference (whose
 * launchers allocate their statistics buffers, models/fused_attn/triton_kernels.py:910-912). Same arguments, kernels
 * and results as ebr_attn_bwd_bwd; the fp32 row statistics that shapes with L > 128 (or D > 128) exchange between their two
 * launches ([3, B, H, L], ebr_attn_scratch_bytes) live in a device array of the library, EBR_NOALLOC_SCRATCH_BYTES
 * per GPU, held until the process ends. Shapes that need more return EBR_ERR_NOALLOC_SIZE before anything is
 * enqueued. It calls no allocating routine. Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (concurrent streams or threads) race and must be serialised by the caller. */
int ebr_attn_bwd_bwd_noalloc(int dtype, int B, int H, int L, int D, float scale,
                             const void* q, const int64_t q_str[3],
                             const void* k, const int64_t k_str[3],
                             const void* v, const int64_t v_str[3],
                             const void* o, const void* lse,
                             const void* dO, const int64_t dO_str[3],
                             const void* gq, const int64_t gq_str[3],
                             const void* gk, const int64_t gk_str[3],
                             const void* gv, const int64_t gv_str[3],
                             void* hq, void* hk, void* hv, void* hdo, void* stream);

/* Bytes of fp32 scratch an op needs for this shape (0 when the shape runs in one workgroup per (b, h)).
 * No reference counterpart: the Triton launchers allocate their row-statistics buffers themselves
 *   (models/fused_attn/triton_kernels.py:679-686, 910-912); here the caller does. */
int64_t ebr_attn_scratch_bytes(int op, int B, int H, int L, int D);

/* Text for a return code. No reference counterpart (Python exceptions carry the message there). */
const char* ebr_attn_error_string(int code);

/* EBR_ATTN_ABI_VERSION of the loaded library. No reference counterpart. */
int ebr_attn_abi_version(void);

/* Offload architecture the library was built for, e.g. "gfx950". No reference counterpart. */
const char* ebr_attn_arch(void);

#ifdef __cplusplus
}
#endif

#endif /* EBR_ATTN_H */
