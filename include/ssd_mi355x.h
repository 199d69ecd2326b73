/*
 * ssd_mi355x.h — C ABI of the MI355X (gfx950) fused chunked SSD scan.
 *
 * Plain C: raw device pointers, sizes and a hipStream_t passed as void*.
 * No torch types, no allocation inside any entry point (the caller passes
 * the workspace), no host synchronisation. Every entry point is stateless
 * and re-entrant.
 *
 * The reference has no native FFI for this path: its Python autograd op
 * launches Triton kernels and torch.einsum directly. These entry points
 * replace the device work behind
 *   fused_ssd_scan / FusedSSDScan.forward  r2/dhammic-ai/src/kernels/ssd_scan.py:539-583, :440-465
 *       (body: _ssd_forward_impl :330-421)                   -> ssd_fwd
 *   FusedSSDScan.backward                  ssd_scan.py:467-533 -> ssd_bwd
 *   the cache tensors the op returns       ssd_scan.py:380-382 (L), :402-406 (decay_chunk),
 *                                          :364-368 (A_cumsum)  -> ssd_materialize_L,
 *                                          ssd_decay_chunk, ssd_fwd(A_cumsum_out)
 * and the composition around it in the caller
 *   Mamba3Block._forward_impl              r2/dhammic-ai/src/mamba_base_engine.py:152-191
 *       (zero-pad :154-165, + D*x :187, norm(y)*silu(z) :191)  -> ssd_fwd / ssd_bwd flags
 *
 * Layouts (all row-major, contiguous):
 *   x, y, dy, dx, z, dz       (batch, seqlen, nheads, headdim)        dtype
 *   B, C, dB, dC              (batch, seqlen, ngroups, dstate)        dtype
 *   dt, ddt                   (batch, seqlen, nheads)                 fp32
 *   A, dA  a_mode PER_HEAD    (nheads,)                               fp32
 *          a_mode PER_TOKEN   (batch, seqlen, nheads)                 dtype  (log-decay a = A, no dt)
 *          a_mode CUMSUM      (batch, nheads, nchunks, chunk)         dtype  (the reference's A_cumsum);
 *                             dA is then (batch, seqlen, nheads) in dtype, see dA_skip
 *   D, dD                     (nheads,)                               fp32
 *   norm_weight, dnorm_weight (nheads*headdim,)                       fp32
 *   init, final, dinit, dfinal(nseq, nheads, headdim, dstate)         state_dtype
 *   cu_seqlens                (nseq+1,) int32, device memory; requires batch == 1
 *   A_cumsum_out              (batch, nheads, nchunks, chunk)         dtype
 * With cu_seqlens, nseq sequences are packed along seqlen; without it nseq == batch.
 *
 * Semantics: per sequence, the reference's chunked SSD on X = dt*x, a = dt*A
 * (or a = A per token), head h reading group h/(nheads/ngroups) of B and C,
 * every decay exponent clamped to [-20, 20] with strict gradient masks, then
 * y += D*x and, with z, y = rmsnorm(y over nheads*headdim)*w*silu(z).
 * Chunks start at every sequence start; a sequence whose length is not a
 * multiple of `chunk` ends in a partial chunk (the reference's zero right-pad).
 */
#ifndef SSD_MI355X_H
#define SSD_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum ssd_status {
  SSD_OK = 0,
  SSD_ERR_INVALID = -1,      /* bad shape, pointer or flag combination        */
  SSD_ERR_UNSUPPORTED = -2,  /* valid for the reference, outside kernel limits */
  SSD_ERR_WORKSPACE = -3,    /* workspace pointer missing or too small        */
  SSD_ERR_HIP = -4,          /* a HIP launch reported an error                */
  SSD_ERR_TOO_LARGE = -5     /* ssd_fwd_noalloc: workspace beyond its scratch */
};

enum ssd_dtype { SSD_DTYPE_F32 = 0, SSD_DTYPE_BF16 = 1 };

enum ssd_a_mode {
  SSD_A_PER_HEAD = 0,   /* a = dt * A[h]                        (extended API) */
  SSD_A_PER_TOKEN = 1,  /* a = A[b, t, h], dt absent            (reference API) */
  SSD_A_CUMSUM = 2      /* a's in-chunk inclusive cumsum given (reference cache path,
                           ssd_scan.py:364-366); dA needs dA_skip below          */
};

/* Terms of the log-decay gradient left out, one bit per place the reference
 * op takes its decay from a cache instead of from A (ssd_scan.py:364-406; a
 * cached tensor receives no gradient, :533):
 *   INTRA   the intra-chunk decay L            (L cached,           :370-382)
 *   CUMSUM  the state-build and output decays  (A_cumsum cached,    :364-368, :389-391, :414)
 *   CHUNK   the inter-chunk decay_chunk        (decay_chunk or A_cumsum cached, :399-406)
 * a_mode CUMSUM requires CUMSUM and CHUNK; its dA (per token) then holds the
 * INTRA term when that bit is clear, and is not written when it is set. */
enum ssd_dA_skip {
  SSD_DA_SKIP_INTRA = 1,
  SSD_DA_SKIP_CUMSUM = 2,
  SSD_DA_SKIP_CHUNK = 4
};

/* Trapezoidal two-SSD mode (ssd_desc_t.trapz), the caller's pair of SSD calls
 * in r2/dhammic-ai/src/mamba_base_engine.py:167-191:
 *   y = SSD(gamma*x, a, B, C) + SSD(beta*x_prev, a, B_prev, C)  [+ D*x] [gated norm]
 * with x_prev[t] = x[t-1], B_prev[t] = B[t-1] (zero at each sequence's first
 * token), a = A per token (a_mode PER_TOKEN) and gamma, beta (b, seqlen, h) in
 * dtype (trapezoidal.py:7-13). Computed as ONE scan: with
 * rho[t] = beta[t+1] exp(-a[t+1]) (0 at a sequence's last token) the pair equals
 * SSD((gamma + rho)*x, a, B, C) - rho[t] (C[t].B[t]) x[t] exactly (the state then
 * carries the beta input of the next token one step early); the kernels run that
 * scan strictly causal with the diagonal as a per-token D, D + gamma[t] (C[t].B[t]).
 * The rounding is that of one SSD call while rho is of the order of gamma, which
 * the trapezoidal coefficients give (beta exp(-a) = (1 - lam) dt). The reference's
 * second call reuses the first call's cache, so the beta path gives no decay
 * gradient (ssd_scan.py:533): DROP_BETA_DA reproduces that, EXACT_DA returns
 * the gradient of the pair through both paths. dA is then (b, seqlen, h) in
 * dtype, and ssd_bwd_args_t.dgamma / dbeta receive the other two gradients.
 * Requires a_mode PER_TOKEN, has_dt == 0, has_init == 0, want_A_cumsum == 0,
 * dA_skip == 0; the ssd_*_args_t gamma and beta pointers. */
enum ssd_trapz {
  SSD_TRAPZ_OFF = 0,
  SSD_TRAPZ_DROP_BETA_DA = 1,   /* the reference's gradients (beta path: no dA)  */
  SSD_TRAPZ_EXACT_DA = 2        /* dA through both paths                         */
};

/* Kernel limits: chunk <= 256, headdim <= 128, dstate <= 128. */
#define SSD_MAX_CHUNK 256
#define SSD_MAX_HEADDIM 128
#define SSD_MAX_DSTATE 128

typedef struct ssd_desc {
  int64_t batch, seqlen, nheads, headdim, ngroups, dstate, chunk;
  int64_t nseq;          /* sequences when varlen != 0 (batch must be 1); else ignored */
  int32_t dtype;         /* enum ssd_dtype of x, B, C, z, y and per-token A          */
  int32_t state_dtype;   /* enum ssd_dtype of init / final / dinit / dfinal          */
  int32_t a_mode;        /* enum ssd_a_mode                                          */
  int32_t has_dt, has_D, has_z, has_init, has_dfinal, varlen;
  int32_t want_final;    /* ssd_fwd writes final_state                               */
  int32_t want_A_cumsum; /* ssd_fwd writes A_cumsum_out (needs varlen == 0)          */
  float norm_eps;        /* gated RMSNorm epsilon (has_z)                            */
  int32_t dA_skip;       /* enum ssd_dA_skip bits; 0: the full gradient              */
  int32_t trapz;         /* enum ssd_trapz                                           */
} ssd_desc_t;

/* Kernel launches of ssd_fwd / ssd_bwd, in launch order. For profiling, a
 * caller may pass `events`: an array of 2*SSD_NUM_PHASES hipEvent_t handles
 * (created by the caller); events[2*k] is recorded on the stream right before
 * the launch(es) of phase k and events[2*k+1] right after. Phases that do not
 * run for a descriptor are not recorded. NULL disables recording.
 * SSD_PH_CHUNK_TABLE is recorded for packed sequences only (a fixed-length
 * batch's table is written by the SSD_PH_CUMSUM launch).
 * SSD_PH_NORM_DW is no longer recorded: the norm weight's gradient is reduced in
 * the backward's last launch, timed as SSD_PH_BWD_REDUCE_HEADS. */
enum ssd_phase {
  SSD_PH_CHUNK_TABLE = 0, SSD_PH_CUMSUM = 1, SSD_PH_FWD_STATE = 2, SSD_PH_FWD_PASS = 3,
  SSD_PH_FWD_SCAN = 4, SSD_PH_NORM_FWD = 5,
  SSD_PH_NORM_BWD = 6, SSD_PH_NORM_DW = 7, SSD_PH_BWD_STATE = 8, SSD_PH_BWD_PASS = 9,
  SSD_PH_BWD_COL = 10, SSD_PH_BWD_ROW = 11, SSD_PH_BWD_FINISH = 12, SSD_PH_BWD_REDUCE_BC = 13,
  SSD_PH_BWD_REDUCE_HEADS = 14,
  /* trapz: the coefficient kernel (and, DROP_BETA_DA, the gamma-path state pass)
   * of the forward; the gamma-path backward (DROP_BETA_DA) and the per-token
   * gradient kernels of the backward */
  SSD_PH_TRAPZ_PREP = 15, SSD_PH_TRAPZ_GAMMA = 16, SSD_PH_TRAPZ_POST = 17,
  SSD_NUM_PHASES = 18
};

typedef struct ssd_fwd_args {
  const void* x; const float* dt; const void* A; const void* B; const void* C;
  const float* D; const void* z; const float* norm_weight; const void* init;
  const int32_t* cu_seqlens;
  void* y; void* final_state; void* A_cumsum_out;
  void* const* events;   /* optional, see enum ssd_phase */
  const void* gamma; const void* beta;   /* trapz: (batch, seqlen, nheads) dtype */
} ssd_fwd_args_t;

typedef struct ssd_bwd_args {
  const void* x; const float* dt; const void* A; const void* B; const void* C;
  const float* D; const void* z; const float* norm_weight; const void* init;
  const int32_t* cu_seqlens;
  const void* dy; const void* dfinal;
  void* dx; float* ddt; void* dA; void* dB; void* dC; float* dD; void* dz;
  float* dnorm_weight; void* dinit;
  void* const* events;   /* optional, see enum ssd_phase */
  const void* gamma; const void* beta;   /* trapz: as in ssd_fwd_args_t           */
  void* dgamma; void* dbeta;             /* trapz: (batch, seqlen, nheads) dtype  */
} ssd_bwd_args_t;

enum ssd_workspace_kind {
  SSD_WS_SAVED = 0,     /* written by ssd_fwd, read by ssd_bwd: keep it between them */
  SSD_WS_FWD_SCRATCH = 1,
  SSD_WS_BWD_SCRATCH = 2
};

/* Host-only: checks the descriptor against the layouts and limits above. */
int ssd_validate(const ssd_desc_t* desc);

/* Host-only: bytes of workspace of the given kind (0 if the descriptor is invalid). */
size_t ssd_workspace_bytes(const ssd_desc_t* desc, int kind);

/* Forward: y (and final_state, A_cumsum_out when asked); fills `saved`. */
int ssd_fwd(const ssd_desc_t* desc, const ssd_fwd_args_t* args,
            void* saved, size_t saved_bytes, void* scratch, size_t scratch_bytes,
            void* stream);

/* Forward without any allocation: as ssd_fwd, with both forward workspaces in a
 * file-scope device array of SSD_NOALLOC_SCRATCH_BYTES per GPU (allocated with
 * the library's code object and held until the process ends). No counterpart in
 * the reference: it is for callers that cannot allocate (HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc). Forward only (nothing is kept
 * for ssd_bwd). Returns SSD_ERR_TOO_LARGE when ssd_workspace_bytes(SAVED),
 * rounded up to 256 bytes, plus ssd_workspace_bytes(FWD_SCRATCH) exceeds the
 * scratch. Every call on one GPU shares that GPU's array: calls that overlap on
 * one GPU (other streams, other threads) race; the forward writes every part of
 * the array it reads, so nothing is cleared between calls. */
#define SSD_NOALLOC_SCRATCH_BYTES (64u << 20)
int ssd_fwd_noalloc(const ssd_desc_t* desc, const ssd_fwd_args_t* args, void* stream);

/* Backward: all requested gradients (a NULL output pointer skips that output,
 * except dx, dB, dC which are required). `saved` must be the buffer the
 * matching ssd_fwd filled, unchanged. */
int ssd_bwd(const ssd_desc_t* desc, const ssd_bwd_args_t* args,
            const void* saved, size_t saved_bytes, void* scratch, size_t scratch_bytes,
            void* stream);

/* Reference cache tensors, from the per-token log-decay a (b, seqlen, h) in desc->dtype:
 *   L           (b, h, nchunks, chunk, chunk) = exp(clamp(segsum(a)))  with the -1e4 fill
 *   decay_chunk (b, h, nchunks+1, nchunks+1) = exp(clamp(segsum(pad(A_cumsum[..., -1]))))
 * from A_cumsum (b, h, nchunks, chunk). Both need varlen == 0 and seqlen % chunk == 0. */
int ssd_materialize_L(const ssd_desc_t* desc, const void* a, void* L, void* stream);
int ssd_decay_chunk(const ssd_desc_t* desc, const void* A_cumsum, void* decay_chunk, void* stream);

const char* ssd_status_string(int status);

/* ABI version of this header (bumped on any layout change). */
int ssd_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SSD_MI355X_H */
