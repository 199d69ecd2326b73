// Forward chunk scan: Y = (C B^T * L) X + exp(cs) C h_in^T (+ D x).
#include "ssd_launch.h"

// ---------------------------------------------------------------------------
// One block per (row block rb of 64 tokens, head h, chunk c); 4 waves, each
// owning a 32-row half and a 32-column group of every 64-wide tile.
//   Y_off (ssd_scan.py:412-415): acc = C_rb h_in^T over K = N (h_in read from
//       global, [p][n] layout = k-contiguous), then rows scaled by exp(cs_l).
//   Y_diag (:370-385): for each column block j <= rb,
//       S = C_rb B_j^T (K = N), M = S * exp(clamp(cs_l - cs_s)) * dt_s on the
//       causal part (exact zero above the diagonal), acc += M x_j (K = 64).
//   The reference's acausal e^-20 entries (the clamped -1e4 fill, :111-116)
//   are not reproduced: they change Y by at most e^-20 * sum|terms|.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) k_chunk_scan_fwd(SsdDims d, const ChunkInfo* __restrict__ chunks,
                                                        const float* __restrict__ cs, const T* __restrict__ hin,
                                                        const T* __restrict__ x, const float* __restrict__ dt,
                                                        const T* __restrict__ Bm, const T* __restrict__ Cm,
                                                        const float* __restrict__ Dv, T* __restrict__ y) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int rb = blockIdx.x, h = blockIdx.y, c = blockIdx.z;
  const ChunkInfo ci = chunks[c];
  if (rb * SSD_BLK >= ci.len) return;
  const int g = h / d.hpg;
  const int NP = lds_pitch<T>(d.Npad), BP = lds_pitch<T>(SSD_BLK);
  float* s_cs = reinterpret_cast<float*>(smem);            // [Qpad]
  float* s_dt = s_cs + d.Qpad;                               // [Qpad]
  T* Ci = reinterpret_cast<T*>(s_dt + d.Qpad);               // [64][NP]
  T* Bj = Ci + SSD_BLK * NP;                                 // [64][NP]
  T* xT = Bj + SSD_BLK * NP;                                 // [Ppad][BP]
  T* Mt = xT + d.Ppad * BP;                                  // [64][BP]

  const float* csc = cs + ((int64_t)c * d.H + h) * d.Qpad;
  for (int l = threadIdx.x; l < d.Qpad; l += blockDim.x) {
    s_cs[l] = csc[l];
    s_dt[l] = (d.has_dt && l < ci.len) ? dt[(int64_t)(ci.row0 + l) * d.H + h] : 1.0f;
  }
  const int64_t brow = (int64_t)d.G * d.N, xrow = (int64_t)d.H * d.P;
  const int r0 = rb * SSD_BLK;
  for (int idx = threadIdx.x; idx < SSD_BLK * d.Npad; idx += blockDim.x) {
    const int l = idx / d.Npad, n = idx % d.Npad;
    float v = 0.0f;
    if (r0 + l < ci.len && n < d.N) v = to_f(Cm[(int64_t)(ci.row0 + r0 + l) * brow + (int64_t)g * d.N + n]);
    Ci[l * NP + n] = from_f<T>(v);
  }
  __syncthreads();

  const int lane = lane_id();
  const int w = threadIdx.x >> 6, wr = w & 1, wc = w >> 1;
  floatx16 acc[2];
  zero(acc[0]);
  zero(acc[1]);
  // Y_off
  const T* hrow = hin + ((int64_t)c * d.H + h) * d.Ppad * d.Npad;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int p0 = wc * 32 + 64 * t;
    if (p0 < d.Ppad) mma_tile<T>(acc[t], Ci + wr * 32 * NP, NP, hrow + (int64_t)p0 * d.Npad, d.Npad, d.Npad);
  }
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const float sc = exp_clamp(s_cs[r0 + wr * 32 + acc_row(v, lane)]);
    acc[0][v] *= sc;
    acc[1][v] *= sc;
  }
  // Y_diag
  for (int j = 0; j <= rb; ++j) {
    const int s0 = j * SSD_BLK;
    __syncthreads();
    for (int idx = threadIdx.x; idx < SSD_BLK * d.Npad; idx += blockDim.x) {
      const int l = idx / d.Npad, n = idx % d.Npad;
      float v = 0.0f;
      if (s0 + l < ci.len && n < d.N) v = to_f(Bm[(int64_t)(ci.row0 + s0 + l) * brow + (int64_t)g * d.N + n]);
      Bj[l * NP + n] = from_f<T>(v);
    }
    for (int idx = threadIdx.x; idx < SSD_BLK * d.Ppad; idx += blockDim.x) {
      const int l = idx / d.Ppad, p = idx % d.Ppad;
      float v = 0.0f;
      if (s0 + l < ci.len && p < d.P) v = to_f(x[(int64_t)(ci.row0 + s0 + l) * xrow + (int64_t)h * d.P + p]);
      xT[p * BP + l] = from_f<T>(v);
    }
    __syncthreads();
    floatx16 sacc;
    zero(sacc);
    mma_tile<T>(sacc, Ci + wr * 32 * NP, NP, Bj + wc * 32 * NP, NP, d.Npad);
    const int sl = wc * 32 + (lane & 31);
    const int s = s0 + sl;
    const float cs_s = s_cs[s], dt_s = s_dt[s];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int ll = wr * 32 + acc_row(v, lane);
      const int l = r0 + ll;
      float m = 0.0f;
      if (s <= l && l < ci.len) m = sacc[v] * exp_clamp(s_cs[l] - cs_s) * dt_s;
      Mt[ll * BP + sl] = from_f<T>(m);
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int p0 = wc * 32 + 64 * t;
      if (p0 < d.Ppad) mma_tile<T>(acc[t], Mt + wr * 32 * BP, BP, xT + p0 * BP, BP, SSD_BLK);
    }
  }
  // epilogue: + D x, store
  const float Dh = d.has_D ? Dv[h] : 0.0f;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int p = wc * 32 + 64 * t + (lane & 31);
    if (p >= d.P) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int l = r0 + wr * 32 + acc_row(v, lane);
      if (l >= ci.len) continue;
      const int64_t o = (int64_t)(ci.row0 + l) * xrow + (int64_t)h * d.P + p;
      float yv = acc[t][v];
      if (d.has_D) yv += Dh * to_f(x[o]);
      y[o] = from_f<T>(yv);
    }
  }
}

size_t lds_chunk_scan_fwd(int dtype, const SsdDims& d) {
  const size_t es = dtype == 1 ? 2 : 4;
  const int NP = d.Npad + 16 / (int)es, BP = SSD_BLK + 16 / (int)es;
  return 2 * sizeof(float) * d.Qpad + es * ((size_t)2 * SSD_BLK * NP + (size_t)d.Ppad * BP + (size_t)SSD_BLK * BP);
}

hipError_t launch_chunk_scan_fwd(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, void* y,
                                 hipStream_t s) {
  dim3 grid(d.Qpad / SSD_BLK, d.H, d.max_chunks);
  const size_t lds = lds_chunk_scan_fwd(dtype, d);
  if (dtype == 1) ensure_lds(k_chunk_scan_fwd<bf16>, lds);
  else ensure_lds(k_chunk_scan_fwd<float>, lds);
  if (dtype == 1)
    hipLaunchKernelGGL(k_chunk_scan_fwd<bf16>, grid, dim3(256), lds, s, d, b.chunks, b.cs,
                       reinterpret_cast<const bf16*>(b.hin), reinterpret_cast<const bf16*>(in.x), in.dt,
                       reinterpret_cast<const bf16*>(in.B), reinterpret_cast<const bf16*>(in.C), in.D,
                       reinterpret_cast<bf16*>(y));
  else
    hipLaunchKernelGGL(k_chunk_scan_fwd<float>, grid, dim3(256), lds, s, d, b.chunks, b.cs,
                       reinterpret_cast<const float*>(b.hin), reinterpret_cast<const float*>(in.x), in.dt,
                       reinterpret_cast<const float*>(in.B), reinterpret_cast<const float*>(in.C), in.D,
                       reinterpret_cast<float*>(y));
  return hipGetLastError();
}
