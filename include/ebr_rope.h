/* C ABI of the fused 2D-RoPE split and merge in libebr_attn.so (gfx950).
 *
 * The split turns one qkv projection [B, N, 3*H*D] into the rotated q, k and plain v the attention reads, each a
 * contiguous [B, H, N, D]; the merge is its exact adjoint (the backward of the split, and the split is the backward of
 * the merge). With cos, sin the fp32 [N, D] tables (the rotate_half sign folded into sin) and quarter_swap the
 * permutation (a, b, c, d) -> (b, a, d, c) of the four quarters of D:
 *   split:  q = round(round(x_q * cos + quarter_swap(x_q) * sin) * t)   (the "* t" step only when qscale != NULL)
 *           k = round(x_k * cos + quarter_swap(x_k) * sin),  v = x_v
 *   merge:  g_q = round(g * cos + quarter_swap(g * sin)) with g = round(dq * t) when qscale != NULL, else dq
 *           g_k = round(dk * cos + quarter_swap(dk * sin)),  g_v = dv
 * Arithmetic is fp32; round() is the rounding to the tensor dtype (identity for fp32). t = qscale[h] is a per-head
 * temperature (fp32 [H]).
 *
 * Conventions are those of ebr_attn.h (dtype codes, error codes, streams, ownership). D must be a multiple of 4 and
 * at most 256; every tensor's last dimension is unit-stride. Element strides are int64_t.
 */
#ifndef EBR_ROPE_H
#define EBR_ROPE_H

#include <stdint.h>

#include "ebr_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces the reference's rope_split (models/fused_attn/rope_split_triton.py:124-160; semantics of ref_split,
 * models/fused_attn/rope_split.py:32-50; op ebr_fused::rope_split, rope_split.py:74-79).
 * qkv: [B, N, 3*H*D] with element strides qkv_sb (B) and qkv_sn (N); q, k, v: contiguous [B, H, N, D] outputs. */
int ebr_rope_split(int dtype, int B, int N, int H, int D, const void* qkv, int64_t qkv_sb, int64_t qkv_sn,
                   const float* cos, const float* sin, const float* qscale, void* q, void* k, void* v,
                   void* stream);

/* Replaces the reference's rope_merge (models/fused_attn/rope_split_triton.py:163-195; semantics of ref_merge,
 * models/fused_attn/rope_split.py:53-66; op ebr_fused::rope_merge, rope_split.py:89-94).
 * dq, dk, dv: [B, H, N, D] with element strides [3] for B, H, N; g: contiguous [B, N, 3*H*D] output. */
int ebr_rope_merge(int dtype, int B, int H, int N, int D, const void* dq, const int64_t dq_str[3], const void* dk,
                   const int64_t dk_str[3], const void* dv, const int64_t dv_str[3], const float* cos,
                   const float* sin, const float* qscale, void* g, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EBR_ROPE_H */
