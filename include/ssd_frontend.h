/*
 * ssd_frontend.h — C ABI of the block front-end kernels that produce the SSD
 * scan's inputs on MI355X (gfx950): the trapezoidal coefficients and the
 * data-dependent rotary embedding of B and C.
 *
 * Plain C: raw device pointers, sizes, a hipStream_t passed as void*; no
 * allocation, no host synchronisation; stateless and re-entrant. These
 * replace the device work of
 *   fused_trapezoidal / FusedTrapezoidal   r2/dhammic-ai/src/kernels/trapezoidal.py:89-331
 *       (forward kernel :89-122, backward kernel :125-210, autograd :214-317)
 *                                          -> ssd_trapezoidal_fwd / ssd_trapezoidal_bwd
 *   fused_rope / FusedRoPE                 r2/dhammic-ai/src/kernels/rope.py:1-321
 *       (math :4-10, shapes :12-15, forward / backward :243-306)
 *                                          -> ssd_rope_fwd / ssd_rope_bwd
 * The third front-end piece, the in-projection and its split
 * (r2/dhammic-ai/src/kernels/inproj_split.py:142-175), is one library GEMM
 * whose outputs are zero-copy column views; it needs no kernel of its own.
 *
 * Layouts are row-major and contiguous. Arithmetic is fp32 in registers
 * whatever the storage dtype (enum ssd_dtype of ssd_mi355x.h: 0 fp32, 1 bf16).
 * Status codes are those of ssd_mi355x.h (0 ok, negative on failure).
 */
#ifndef SSD_FRONTEND_H
#define SSD_FRONTEND_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Trapezoidal coefficients (trapezoidal.py:3-13), per row r < rows and head h < nheads:
 *   s = dt_raw + dt_bias[h];  dt = softplus(s);  lam = sigmoid(lam_raw);  A = -exp(A_log[h])
 *   dA = dt A;  beta = (1 - lam) dt exp(dA);  gamma = lam dt
 * dt_raw, lam_raw, dt, dA, beta, gamma: (rows, nheads) in `dtype`; dt_bias, A_log: (nheads,)
 * in `dtype` (the reference casts both to the input dtype before the kernel, :236-237). */
int ssd_trapezoidal_fwd(int32_t dtype, int64_t rows, int64_t nheads, const void* dt_raw, const void* lam_raw,
                        const void* dt_bias, const void* A_log, void* dt, void* dA, void* beta, void* gamma,
                        void* stream);

/* fp32 workspace bytes of ssd_trapezoidal_bwd (per-block partial sums of the two head gradients). */
size_t ssd_trapezoidal_bwd_workspace(int64_t rows, int64_t nheads);

/* Backward (trapezoidal.py:28-52): d_dt_raw, d_lam_raw (rows, nheads) in `dtype`; d_dt_bias,
 * d_A_log (nheads,) fp32, reduced over rows in a fixed order. Any incoming gradient pointer may be
 * NULL (a zero gradient). */
int ssd_trapezoidal_bwd(int32_t dtype, int64_t rows, int64_t nheads, const void* dt_raw, const void* lam_raw,
                        const void* dt_bias, const void* A_log, const void* g_dt, const void* g_dA,
                        const void* g_beta, const void* g_gamma, void* d_dt_raw, void* d_lam_raw, float* d_dt_bias,
                        float* d_A_log, void* workspace, size_t workspace_bytes, void* stream);

/* Rotary embedding with data-dependent angles (rope.py:4-10): for each pair k of the last axis,
 *   out[2k] = cos(a_k) x[2k] - sin(a_k) x[2k+1],   out[2k+1] = sin(a_k) x[2k] + cos(a_k) x[2k+1].
 * x, out: (batch, seqlen, nheads, 2 half_dim) in `dtype`; angles (batch, seqlen, per_head ? nheads : 1,
 * half_dim) in `angle_dtype`. */
int ssd_rope_fwd(int32_t dtype, int32_t angle_dtype, int64_t batch, int64_t seqlen, int64_t nheads,
                 int64_t half_dim, int32_t per_head, const void* x, const void* angles, void* out, void* stream);

/* Backward (rope.py:263-303): dx in `dtype` (the inverse rotation of dy); dangles in `angle_dtype`,
 * summed over heads when the angles are shared (per_head == 0), computed in fp32. */
int ssd_rope_bwd(int32_t dtype, int32_t angle_dtype, int64_t batch, int64_t seqlen, int64_t nheads,
                 int64_t half_dim, int32_t per_head, const void* x, const void* angles, const void* dy, void* dx,
                 void* dangles, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SSD_FRONTEND_H */
