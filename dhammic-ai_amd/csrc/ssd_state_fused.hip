// Chunk states and the inter-chunk recurrence in one pass (bf16 inputs).
//
// Forward (ssd_scan.py:387-410): per sequence and head, walking the chunks in
// order,
//   hin[c] = run;  run = exp(clamp(total_c)) * run + st_c,
//   st_c[p][n] = sum_s x[s][p] * exp(clamp(cs_last - cs_s)) * dt_s * B[s][n]
// and final = run. Backward (the reverse recurrence for the gradient leaving
// each chunk, the adjoint of the above plus the Y_off term :412-415):
//   dst[c] = run;  dtot_c = sum run * exp(clamp(total_c)) * hin[c] * pass(total_c);
//   run = exp(clamp(total_c)) * run + dh_c,
//   dh_c[p][n] = sum_l dy[l][p] * exp(clamp(cs_l)) * C[l][n]
// and dinit = run. The running state stays in the MFMA accumulator registers;
// nothing but hin / dst (bf16) and the final / initial state is written.
//
// One block per (32-wide n tile, head, sequence) with one wave per 32-wide p
// tile (64 * Ppad / 32 threads); wave w owns the 32 x 32 state tile (p tile w,
// the block's n tile). Blocks of one (head, sequence) are numbered onto one XCD
// (same block index mod 8) so their shared x / dy rows are read from HBM once.
// Tokens are staged 64 at a time (x or dy rows, B or C columns scaled per
// token) and both MFMA operands are read with ds_read_b64_tr_b16 (the
// contraction is over tokens, the tiles' row index; the tiles use the
// transpose-read pitch). Global loads run three 64-token steps ahead through a
// ring of three register stages.
#include "ssd_launch.h"
#include "ssd_tile.h"

template <int PT>
struct StateStage {
  static constexpr int NTHR = 64 * PT;
  TileStage<64, 32 * PT, NTHR> u;  // x or dy rows, all Ppad columns
  TileStage<64, 32, NTHR> v;       // B or C rows, the block's 32 columns
};

template <int PT>
__device__ __forceinline__ void state_load(StateStage<PT>& st, const bf16* U, const bf16* V, int64_t urow,
                                           int64_t vrow, int64_t row0, int t0, int len, int P, int nw,
                                           int64_t ucol, int64_t vcol) {
  const int nrows = min(64, len - t0);
  tstage_load_v(st.u, U + (row0 + t0) * urow + ucol, urow, nrows, P);
  tstage_load_v(st.v, V + (row0 + t0) * vrow + vcol, vrow, nrows, nw);
}

// Stores the staged rows; V rows are scaled by coef[r] (fp32) before rounding.
template <int PT>
__device__ __forceinline__ void state_store(const StateStage<PT>& st, bf16* tu, bf16* tv, const float* coef) {
  constexpr int NTHR = StateStage<PT>::NTHR;
  tstage_store<64, 32 * PT, NTHR, tpitch_tr<32 * PT>()>(st.u, tu);
#pragma unroll
  for (int q = 0; q < TileStage<64, 32, NTHR>::PER; ++q) {
    const int id = threadIdx.x + q * NTHR;
    if (TileStage<64, 32, NTHR>::NVEC % NTHR == 0 || id < TileStage<64, 32, NTHR>::NVEC) {
      const int r = id / 4, k = (id % 4) * 8;
      const float sc = coef[r];
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)((float)st.v.v[q][e] * sc);
      *reinterpret_cast<bf16x8*>(tv + toff<32, tpitch_tr<32>()>(r, k)) = o;
    }
  }
}

// Scalars of one 64-token step: its chunk's row range and total log-decay, and
// the per-token inputs of the coefficients (threads < 64: token t0 + tid).
struct StepCoef {
  float cs_tok, dt_tok, tot;
  int row0, len;
};

template <int PT, bool FWD>
__global__ void __launch_bounds__(64 * PT) __attribute__((amdgpu_waves_per_eu(2, 2))) k_state_fused(SsdDims d, const ChunkInfo* __restrict__ chunks,
                                                         const int32_t* __restrict__ seq_chunk0,
                                                         const float* __restrict__ cs, const float* __restrict__ dt,
                                                         const bf16* __restrict__ U, const bf16* __restrict__ V,
                                                         bf16* __restrict__ hst, const bf16* __restrict__ hin_in,
                                                         const void* __restrict__ s_in, void* __restrict__ s_out,
                                                         int state_bf16, float* __restrict__ dtot_part) {
  constexpr int PP = 32 * PT;
  constexpr int UPI = tpitch_tr<PP>(), VPI = tpitch_tr<32>();
  __shared__ __align__(16) bf16 tu[2][tsize<64, PP, UPI>()];
  __shared__ __align__(16) bf16 tv[2][tsize<64, 32, VPI>()];
  __shared__ float coef[2][64];
  __shared__ float red[4];
  // per-wave 32 x 32 bf16 tile between the accumulator layout and whole 64-byte row
  // pieces of HBM: the state written at a chunk start, and (backward) h_in at its end
  constexpr int TP = 40;  // row pitch (elements)
  __shared__ __align__(16) bf16 s_tile[PT][32 * TP];
  // block -> (n tile, unit = (head, sequence)); the n tiles of a unit share an XCD
  const int NTn = d.Npad / 32;
  const int x8 = blockIdx.x & 7, rr = blockIdx.x >> 3;
  const int nt = rr % NTn;
  const int unit = (rr / NTn) * 8 + x8;
  if (unit >= d.H * d.nseq) return;
  const int h = unit % d.H, sq = unit / d.H;
  const int g = h / d.hpg;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t urow = (int64_t)d.H * d.P, vrow = (int64_t)d.G * d.N;
  const int64_t ucol = (int64_t)h * d.P, vcol = (int64_t)g * d.N + 32 * nt;
  const int nw = min(32, d.N - 32 * nt);  // valid columns of the block's n tile
  const int n = 32 * nt + (lane & 31);
  const int prow0 = 32 * w;

  // running state: rows p = 32 w + acc_row(v), column n
  floatx16 run;
  zero(run);
  if (s_in) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int p = prow0 + acc_row(v, lane);
      if (p < d.P && n < d.N) {
        const int64_t o = (((int64_t)sq * d.H + h) * d.P + p) * d.N + n;
        run[v] = state_bf16 ? (float)reinterpret_cast<const bf16*>(s_in)[o] : reinterpret_cast<const float*>(s_in)[o];
      }
    }
  }
  const int c0 = seq_chunk0[sq], c1 = seq_chunk0[sq + 1];
  const int nch = c1 - c0;
  auto chunk_of = [&](int k) { return FWD ? c0 + k : c1 - 1 - k; };

  // load cursor (kl, tl): the next step whose inputs are fetched
  int kl = 0, tl = 0;
  auto load_next = [&](StateStage<PT>& st, StepCoef& cf) {
    if (kl >= nch) return;
    const int c = chunk_of(kl);
    const ChunkInfo ci = chunks[c];
    state_load<PT>(st, U, V, urow, vrow, ci.row0, tl, ci.len, d.P, nw, ucol, vcol);
    cf.row0 = ci.row0;
    cf.len = ci.len;
    cf.tot = cs[((int64_t)c * d.H + h) * d.Qpad + d.Qpad - 1];
    cf.cs_tok = 0.0f;
    cf.dt_tok = 1.0f;
    if (threadIdx.x < 64) {
      const int l = tl + threadIdx.x;
      cf.cs_tok = cs[((int64_t)c * d.H + h) * d.Qpad + min(l, d.Qpad - 1)];
      if (FWD && d.has_dt && l < ci.len) cf.dt_tok = dt[(int64_t)(ci.row0 + l) * d.H + h];
    }
    tl += 64;
    if (tl >= ci.len) {
      ++kl;
      tl = 0;
    }
  };

  // compute cursor (k, t0)
  int k = 0, t0 = 0, buf = 0;
  floatx16 acc;
  zero(acc);
  bf16x8 hin_v[2];  // this lane's two 8-element row pieces of h_in (rows (lane + 64 q) / 4)
  // one 64-token step on the inputs in (st, cf); refills them with the step three ahead
  auto step = [&](StateStage<PT>& st, StepCoef& cf) {
    const int c = chunk_of(k);
    const int clen = cf.len;
    const float tot = cf.tot;
    const int64_t soff = ((int64_t)c * d.H + h) * d.Ppad * d.Npad;
    if (t0 == 0) {
      // state entering (forward) / gradient leaving (backward) chunk c: accumulator layout
      // -> this wave's LDS tile -> 16-byte row pieces (16 rows x 64 bytes per store)
      bf16* tw = s_tile[w];
#pragma unroll
      for (int v = 0; v < 16; ++v) tw[acc_row(v, lane) * TP + (lane & 31)] = (bf16)run[v];
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int id = lane + 64 * q, r = id >> 2, c8 = (id & 3) * 8;
        const int64_t o = soff + (int64_t)(prow0 + r) * d.Npad + 32 * nt + c8;
        *reinterpret_cast<bf16x8*>(hst + o) = *reinterpret_cast<const bf16x8*>(tw + r * TP + c8);
        if (!FWD) hin_v[q] = *reinterpret_cast<const bf16x8*>(hin_in + o);  // consumed at the end of the chunk
      }
      __builtin_amdgcn_wave_barrier();
    }
    if (threadIdx.x < 64) {
      const int l = t0 + threadIdx.x;
      float v = 0.0f;
      if (l < clen) v = FWD ? exp_clamp(tot - cf.cs_tok) * cf.dt_tok : exp_clamp(cf.cs_tok);
      coef[buf][threadIdx.x] = v;
    }
    __syncthreads();  // coef visible; this buffer's previous readers are done
    state_store<PT>(st, tu[buf], tv[buf], coef[buf]);
    __syncthreads();
    load_next(st, cf);  // st / cf are free now: refill with the step three ahead
#pragma unroll
    for (int kk = 0; kk < 64; kk += 16)
      mfma(acc, ttr_std<PP, UPI>(tu[buf], kk, prow0, lane), ttr_std<32, VPI>(tv[buf], kk, 0, lane));
    buf ^= 1;
    t0 += 64;
    if (t0 >= clen) {
      // end of chunk c
      const float dec = exp_clamp(tot);
      if (!FWD) {
        bf16* th = s_tile[w];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int id = lane + 64 * q, r = id >> 2, c8 = (id & 3) * 8;
          *reinterpret_cast<bf16x8*>(th + r * TP + c8) = hin_v[q];
        }
        __builtin_amdgcn_wave_barrier();
        float contrib = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; ++v) contrib += run[v] * (float)th[acc_row(v, lane) * TP + (lane & 31)];
        __builtin_amdgcn_wave_barrier();
        contrib *= dec * clamp_pass(tot);
        for (int o = 32; o > 0; o >>= 1) contrib += __shfl_xor(contrib, o, 64);
        if (lane == 0) red[w] = contrib;
        __syncthreads();
        if (threadIdx.x == 0) {
          float sum = 0.0f;
          for (int q = 0; q < PT; ++q) sum += red[q];
          dtot_part[((int64_t)c * d.H + h) * NTn + nt] = sum;
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) run[v] = dec * run[v] + acc[v];
      zero(acc);
      ++k;
      t0 = 0;
    }
  };

  StateStage<PT> st0, st1, st2;
  StepCoef cf0, cf1, cf2;
  load_next(st0, cf0);
  load_next(st1, cf1);
  load_next(st2, cf2);
  while (k < nch) {
    step(st0, cf0);
    if (k >= nch) break;
    step(st1, cf1);
    if (k >= nch) break;
    step(st2, cf2);
  }
  // final state (forward) / gradient of the initial state (backward)
  if (s_out) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int p = prow0 + acc_row(v, lane);
      if (p < d.P && n < d.N) {
        const int64_t o = (((int64_t)sq * d.H + h) * d.P + p) * d.N + n;
        if (state_bf16) reinterpret_cast<bf16*>(s_out)[o] = (bf16)run[v];
        else reinterpret_cast<float*>(s_out)[o] = run[v];
      }
    }
  }
}

bool state_fused_supported(int dtype, const SsdDims& d) {
  return dtype == 1 && d.P % 8 == 0 && d.N % 8 == 0 && d.vec_x && d.vec_bc;
}

int state_fused_slices(const SsdDims& d) { return d.Npad / 32; }

template <bool FWD>
static hipError_t state_fused_t(const SsdDims& d, const SsdBufs& b, const void* U, const void* V, const float* dt,
                                bf16* hst, const bf16* hin_in, const void* s_in, void* s_out, int state_bf16,
                                hipStream_t s) {
  const int units = d.H * d.nseq;
  const dim3 grid((units + 7) / 8 * 8 * (d.Npad / 32));
  const bf16* u = reinterpret_cast<const bf16*>(U);
  const bf16* v = reinterpret_cast<const bf16*>(V);
  switch (d.Ppad / 32) {
    case 1:
      hipLaunchKernelGGL((k_state_fused<1, FWD>), grid, dim3(64), 0, s, d, b.chunks, b.seq_chunk0, b.cs, dt, u, v,
                         hst, hin_in, s_in, s_out, state_bf16, b.dtot_part);
      break;
    case 2:
      hipLaunchKernelGGL((k_state_fused<2, FWD>), grid, dim3(128), 0, s, d, b.chunks, b.seq_chunk0, b.cs, dt, u, v,
                         hst, hin_in, s_in, s_out, state_bf16, b.dtot_part);
      break;
    default:
      hipLaunchKernelGGL((k_state_fused<4, FWD>), grid, dim3(256), 0, s, d, b.chunks, b.seq_chunk0, b.cs, dt, u, v,
                         hst, hin_in, s_in, s_out, state_bf16, b.dtot_part);
  }
  return hipGetLastError();
}
hipError_t launch_state_fwd_fused(const SsdDims& d, const SsdBufs& b, const void* x, const void* B, const float* dt,
                                  const void* init, void* final_state, int state_dtype, hipStream_t s) {
  return state_fused_t<true>(d, b, x, B, dt, reinterpret_cast<bf16*>(b.hin), nullptr, init, final_state,
                             state_dtype == 1, s);
}

hipError_t launch_state_bwd_fused(const SsdDims& d, const SsdBufs& b, const void* dy, const void* C,
                                  const void* dfinal, void* dinit, int state_dtype, hipStream_t s) {
  return state_fused_t<false>(d, b, dy, C, nullptr, b.dst16, reinterpret_cast<const bf16*>(b.hin), dfinal, dinit,
                              state_dtype == 1, s);
}
