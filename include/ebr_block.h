/* C ABI of the energy network's fused pointwise blocks in libebr_attn.so (gfx950): rms_norm over the last dimension
 * and the SwiGLU activation, each with its backward and the backward of that backward, as the graded latent descent
 * differentiates the energy twice.
 *
 * Tensors are contiguous rows of one dtype (EBR_DTYPE_F32, _BF16, _F16 or _F64). Arithmetic is fp32 (fp64 for fp64);
 * outputs are rounded once to the dtype. Conventions otherwise as in ebr_attn.h (error codes, streams, ownership).
 */
#ifndef EBR_BLOCK_H
#define EBR_BLOCK_H

#include <stdint.h>

#include "ebr_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* y = x / sqrt(mean(x^2) + eps) per row of C elements, statistics in fp32.
 * Replaces the reference's rms_norm (models/layers.py:37-42) in the energy blocks (models/attention.py:264-266). */
int ebr_block_rmsnorm(int dtype, int64_t rows, int C, float eps, const void* x, void* y, void* stream);

/* dx of y = rms_norm(x) given dy. */
int ebr_block_rmsnorm_bwd(int dtype, int64_t rows, int C, float eps, const void* x, const void* dy, void* dx,
                          void* stream);

/* Gradients of <c, dx> with respect to x (gx) and dy (gdy), dx being ebr_block_rmsnorm_bwd's output. */
int ebr_block_rmsnorm_bwd2(int dtype, int64_t rows, int C, float eps, const void* x, const void* dy, const void* c,
                           void* gx, void* gdy, void* stream);

/* y = silu(gate) * up for rows of gu = [gate | up] (2 I elements each), y rows of I.
 * Replaces the reference's SwiGLU activation (models/layers.py:74-84: gate_up_proj(x).chunk(2), silu(gate) * up). */
int ebr_block_swiglu(int dtype, int64_t rows, int I, const void* gu, void* y, void* stream);

/* dgu = [dgate | dup] of y given dy. */
int ebr_block_swiglu_bwd(int dtype, int64_t rows, int I, const void* gu, const void* dy, void* dgu, void* stream);

/* Gradients of <c, dgu> with respect to gu (ggu, rows of 2 I) and dy (gdy, rows of I). */
int ebr_block_swiglu_bwd2(int dtype, int64_t rows, int I, const void* gu, const void* dy, const void* c, void* ggu,
                          void* gdy, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EBR_BLOCK_H */
