/* C ABI of the fused latent-descent wrapper in libebr_attn.so (gfx950): the pointwise work around every descent
 * microstep z -> sphere(rms_norm(z) + noise - alpha * dE/dz).
 *
 * Tensors are contiguous. z, noise, v, g and outputs share the dtype (EBR_DTYPE_F32, _BF16 or _F16); sigma and alpha
 * are fp32 per-row arrays [B]; rms is fp32 [B]; active is a byte per row [B] (non-zero = the row moves) or NULL (all
 * rows move). Arithmetic is fp32; every intermediate the eager formula keeps in the tensor dtype is rounded to it.
 * sigma and alpha are used as given: a caller whose per-row values are tensors of the data dtype passes them rounded
 * to it (as the eager formula's .to(dtype) does), a Python scalar is passed at fp32 (as torch's opmath uses it).
 * Conventions otherwise as in ebr_attn.h (error codes, streams, ownership).
 */
#ifndef EBR_DESCENT_H
#define EBR_DESCENT_H

#include <stdint.h>

#include "ebr_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* v = rms_norm(z) (+ noise) (* sigma[b]) over the last dim of z [B, L, C]: noise NULL -> v = rms_norm(z); sigma NULL
 * -> v = rms_norm(z) + noise; else v = rms_norm(z) + round(noise * sigma[b]).
 * Replaces the reference's _noisy_point / _noisy_point_replayed (models/energy.py:226-232, rms_norm
 * models/layers.py:37-42). */
int ebr_descent_noisy_point(int dtype, int B, int L, int C, float eps, const void* z, const void* noise,
                            const float* sigma, void* v, void* stream);

/* dz of v = rms_norm(z) + ... given dv (noise and sigma carry no gradient). */
int ebr_descent_noisy_point_bwd(int dtype, int B, int L, int C, float eps, const void* z, const void* dv, void* dz,
                                void* stream);

/* out = where(active[b], sphere(v - round(alpha[b] * g)), z) per row b of [B, N] (N = L * C), with
 * sphere(u) = u / max(sqrt(mean(u^2)), eps) over the whole row; rms[b] receives that denominator (1 for rows that do
 * not move). z may be NULL when active is NULL.
 * Replaces the reference's _step_and_project (models/energy.py:235-241, sphere :219-222). */
int ebr_descent_step_project(int dtype, int B, int64_t N, float eps, const void* v, const void* g,
                             const float* alpha, const void* z, const uint8_t* active, void* out, float* rms,
                             void* stream);

/* Gradients of the step given dout: active rows get dv = du, dg = round(-du * alpha[b]), dz = 0 with du the sphere's
 * backward; rows that do not move get dz = dout, dv = dg = 0. rms is the forward's. dz may be NULL when active is NULL
 * (it would be all zero). */
int ebr_descent_step_project_bwd(int dtype, int B, int64_t N, float eps, const void* v, const void* g,
                                 const float* alpha, const uint8_t* active, const float* rms, const void* dout,
                                 void* dv, void* dg, void* dz, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EBR_DESCENT_H */
