// Backward of the chunked SSD scan (the gradient that FusedSSDScan.backward,
// r2/dhammic-ai/src/kernels/ssd_scan.py:467-533, obtains by re-running the
// forward under autograd), written out per chunk. Notation per (chunk, head),
// rows l (outputs) and columns s (inputs) of the chunk:
//   S = C B^T, L[l,s] = exp(clamp(cs_l - cs_s)) (s <= l), M = S*L, X = dt*x
//   dM[l,s] = dY_l . X_s, dS = dM*L, G = dM*M*pass(cs_l - cs_s)
//   w_s = exp(clamp(cs_last - cs_s)), dst = gradient of the state leaving the chunk
//   h = state entering the chunk
// gives
//   dX_s = sum_l M[l,s] dY_l + w_s B_s dst^T         dx = dt dX + D dY
//   dB_s = sum_l dS[l,s] C_l + w_s X_s dst            (summed over the heads of a group)
//   dC_l = sum_s dS[l,s] B_s + exp(cs_l) dY_l h       (summed over the heads of a group)
//   dcs_l = sum_s G[l,s] - sum_l' G[l',l] + pass(cs_l) C_l.(exp(cs_l) dY_l h)
//           - pass_w(s=l) X_l.(w_l B_l dst^T) + [l = last](sum of the latter + dtotal)
//   da = reverse cumsum of dcs within the chunk; ddt = x.dX + A da; dA = sum dt da.
// Column-side work (dX, dB, column sums of G) and row-side work (dC, row sums
// of G) run in two kernels so each keeps one set of accumulators; each
// recomputes S and dM for its block pairs.
#include "ssd_launch.h"

namespace {

template <typename T>
struct BwdCommon {
  const ChunkInfo* chunks;
  const float* cs;
  const T* hin;
  const float* dst;
  const T* x;
  const float* dt;
  const T* Bm;
  const T* Cm;
  const float* Dv;
  const T* dy;
};

// Stage rows [r0, r0+64) of a (rows, heads*width) tensor (head column offset
// col0) into LDS, k-contiguous: dst[r][k] (pitch P), zero outside [0, len) x [0, width).
template <typename T>
__device__ __forceinline__ void stage_rows(T* __restrict__ out, int pitch, const T* __restrict__ src,
                                           int64_t row_stride, int64_t col0, int row0, int r0, int len,
                                           int width, int wpad) {
  for (int idx = threadIdx.x; idx < SSD_BLK * wpad; idx += blockDim.x) {
    const int r = idx / wpad, k = idx % wpad;
    float v = 0.0f;
    if (r0 + r < len && k < width) v = to_f(src[(int64_t)(row0 + r0 + r) * row_stride + col0 + k]);
    out[r * pitch + k] = from_f<T>(v);
  }
}

// Same rows, transposed: out[k][r] (pitch P).
template <typename T>
__device__ __forceinline__ void stage_rows_t(T* __restrict__ out, int pitch, const T* __restrict__ src,
                                             int64_t row_stride, int64_t col0, int row0, int r0, int len,
                                             int width, int wpad) {
  for (int idx = threadIdx.x; idx < SSD_BLK * wpad; idx += blockDim.x) {
    const int r = idx / wpad, k = idx % wpad;
    float v = 0.0f;
    if (r0 + r < len && k < width) v = to_f(src[(int64_t)(row0 + r0 + r) * row_stride + col0 + k]);
    out[k * pitch + r] = from_f<T>(v);
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Column side: block (j, group*slices, chunk) owns columns s in block j and the
// heads of one slice of group g. Per head: dX_j (written as dx), column sums
// of G, the E term, x.dX per row and the D partial; across the slice's heads
// it accumulates dB_j.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) k_bwd_col(SsdDims d, SsdBufs bf, BwdCommon<T> in, T* __restrict__ dx,
                                                 T* __restrict__ dB) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int j = blockIdx.x, c = blockIdx.z;
  const int g = blockIdx.y / bf.nslices, slc = blockIdx.y % bf.nslices;
  const ChunkInfo ci = in.chunks[c];
  const int s0 = j * SSD_BLK;
  if (s0 >= ci.len) return;
  const int h_lo = g * d.hpg + slc * bf.hslice;
  const int h_hi = min(h_lo + bf.hslice, (g + 1) * d.hpg);
  const int NP = lds_pitch<T>(d.Npad), PP = lds_pitch<T>(d.Ppad), BP = lds_pitch<T>(SSD_BLK);
  float* s_cs = reinterpret_cast<float*>(smem);
  float* s_dt = s_cs + d.Qpad;
  float* red = s_dt + d.Qpad;                       // [4][64]
  T* Bj = reinterpret_cast<T*>(red + 4 * SSD_BLK);  // [64][NP]
  T* xj = Bj + SSD_BLK * NP;                        // [64][PP]
  T* regA = xj + SSD_BLK * PP;
  T* Ci = regA;                                     // [64][NP]
  T* dYi = Ci + SSD_BLK * NP;                       // [64][PP]
  T* dYiT = dYi + SSD_BLK * PP;                     // [Ppad][BP]
  T* CiT = dYiT + d.Ppad * BP;                      // [Npad][BP]
  T* MT = CiT + d.Npad * BP;                        // [64][BP]
  T* dST = MT + SSD_BLK * BP;                       // [64][BP]
  T* dstT = regA;                                   // [Npad][PP] (after the i loop)
  T* dstN = dstT + d.Npad * PP;                     // [Ppad][NP]

  const int lane = lane_id();
  const int w = threadIdx.x >> 6, wr = w & 1, wc = w >> 1;
  const int64_t brow = (int64_t)d.G * d.N, xrow = (int64_t)d.H * d.P;
  stage_rows<T>(Bj, NP, in.Bm, brow, (int64_t)g * d.N, ci.row0, s0, ci.len, d.N, d.Npad);

  floatx16 accB[2];
  zero(accB[0]);
  zero(accB[1]);
  const int nblk_len = (ci.len + SSD_BLK - 1) / SSD_BLK;
  const int sl = wc * 32 + (lane & 31);  // this lane's column in the S tile
  const int s = s0 + sl;

  for (int h = h_lo; h < h_hi; ++h) {
    __syncthreads();
    const float* csc = in.cs + ((int64_t)c * d.H + h) * d.Qpad;
    for (int l = threadIdx.x; l < d.Qpad; l += blockDim.x) {
      s_cs[l] = csc[l];
      s_dt[l] = (d.has_dt && l < ci.len) ? in.dt[(int64_t)(ci.row0 + l) * d.H + h] : 1.0f;
    }
    stage_rows<T>(xj, PP, in.x, xrow, (int64_t)h * d.P, ci.row0, s0, ci.len, d.P, d.Ppad);
    floatx16 accX[2];
    zero(accX[0]);
    zero(accX[1]);
    float gcol = 0.0f;
    for (int i = j; i < nblk_len; ++i) {
      const int r0 = i * SSD_BLK;
      __syncthreads();
      stage_rows<T>(Ci, NP, in.Cm, brow, (int64_t)g * d.N, ci.row0, r0, ci.len, d.N, d.Npad);
      stage_rows<T>(dYi, PP, in.dy, xrow, (int64_t)h * d.P, ci.row0, r0, ci.len, d.P, d.Ppad);
      stage_rows_t<T>(dYiT, BP, in.dy, xrow, (int64_t)h * d.P, ci.row0, r0, ci.len, d.P, d.Ppad);
      stage_rows_t<T>(CiT, BP, in.Cm, brow, (int64_t)g * d.N, ci.row0, r0, ci.len, d.N, d.Npad);
      __syncthreads();
      floatx16 sacc, macc;
      zero(sacc);
      zero(macc);
      mma_tile<T>(sacc, Ci + wr * 32 * NP, NP, Bj + wc * 32 * NP, NP, d.Npad);
      mma_tile<T>(macc, dYi + wr * 32 * PP, PP, xj + wc * 32 * PP, PP, d.Ppad);
      const float cs_s = s_cs[s], dt_s = s_dt[s];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int ll = wr * 32 + acc_row(v, lane);
        const int l = r0 + ll;
        float m = 0.0f, dsv = 0.0f;
        if (s <= l && l < ci.len) {
          const float dd = s_cs[l] - cs_s;
          const float Lv = exp_clamp(dd);
          m = sacc[v] * Lv;
          const float dm = macc[v] * dt_s;
          dsv = dm * Lv;
          gcol += dm * m * clamp_pass(dd);
        }
        MT[sl * BP + ll] = from_f<T>(m);
        dST[sl * BP + ll] = from_f<T>(dsv);
      }
      __syncthreads();
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int p0 = wc * 32 + 64 * t;
        if (p0 < d.Ppad) mma_tile<T>(accX[t], MT + wr * 32 * BP, BP, dYiT + p0 * BP, BP, SSD_BLK);
        const int n0 = wc * 32 + 64 * t;
        if (n0 < d.Npad) mma_tile<T>(accB[t], dST + wr * 32 * BP, BP, CiT + n0 * BP, BP, SSD_BLK);
      }
    }
    // column sums of G: both lane halves, then the two row-half waves
    gcol += __shfl_xor(gcol, 32, 64);
    __syncthreads();
    if (lane < 32) red[wr * SSD_BLK + sl] = gcol;
    // state part: dst of this (chunk, head) staged as T, both orientations
    const float* dsrc = in.dst + ((int64_t)c * d.H + h) * d.Ppad * d.Npad;
    for (int idx = threadIdx.x; idx < d.Ppad * d.Npad; idx += blockDim.x) {
      const int p = idx / d.Npad, n = idx % d.Npad;
      const T v = from_f<T>(dsrc[idx]);
      dstN[p * NP + n] = v;
      dstT[n * PP + p] = v;
    }
    __syncthreads();
    float* colG = bf.colG + ((int64_t)c * d.H + h) * d.Qpad;
    if (threadIdx.x < SSD_BLK) colG[s0 + threadIdx.x] = red[threadIdx.x] + red[SSD_BLK + threadIdx.x];
    const float cs_last = s_cs[d.Qpad - 1];
    floatx16 tmp[2];
    float erow[16], xrowsum[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) { erow[v] = 0.0f; xrowsum[v] = 0.0f; }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      zero(tmp[t]);
      const int p0 = wc * 32 + 64 * t;
      if (p0 < d.Ppad) mma_tile<T>(tmp[t], Bj + wr * 32 * NP, NP, dstN + p0 * NP, NP, d.Npad);
    }
    float dpart = 0.0f;
    const float Dh = d.has_D ? in.Dv[h] : 0.0f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int sr = wr * 32 + acc_row(v, lane);
      const int sg = s0 + sr;
      const float ws = sg < ci.len ? exp_clamp(cs_last - s_cs[sg]) : 0.0f;
      const float dts = s_dt[sg];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int p = wc * 32 + 64 * t + (lane & 31);
        if (p >= d.Ppad) continue;
        const float xv = to_f(xj[sr * PP + p]);
        const float tx = tmp[t][v] * ws;
        erow[v] += xv * tx;
        const float dX = accX[t][v] + tx;
        xrowsum[v] += xv * dX;
        if (sg < ci.len && p < d.P) {
          const int64_t o = (int64_t)(ci.row0 + sg) * xrow + (int64_t)h * d.P + p;
          const float dyv = to_f(in.dy[o]);
          dx[o] = from_f<T>(dts * dX + Dh * dyv);
          dpart += xv * dyv;
        }
      }
      erow[v] = row_reduce32(erow[v]) * dts * clamp_pass(cs_last - s_cs[sg]);
      xrowsum[v] = row_reduce32(xrowsum[v]);
    }
    // dB state part: w_s dt_s x_s dst (K = P)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int n0 = wc * 32 + 64 * t;
      if (n0 >= d.Npad) continue;
      floatx16 tb;
      zero(tb);
      mma_tile<T>(tb, xj + wr * 32 * PP, PP, dstT + n0 * PP, PP, d.Ppad);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int sg = s0 + wr * 32 + acc_row(v, lane);
        const float ws = sg < ci.len ? exp_clamp(cs_last - s_cs[sg]) * s_dt[sg] : 0.0f;
        accB[t][v] += tb[v] * ws;
      }
    }
    // combine the two column-half waves for the row quantities, and the D partial
    for (int o = 32; o > 0; o >>= 1) dpart += __shfl_xor(dpart, o, 64);
    __syncthreads();
    if ((lane & 31) == 0) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int sr = wr * 32 + acc_row(v, lane);
        red[wc * SSD_BLK + sr] = erow[v];
        red[(2 + wc) * SSD_BLK + sr] = xrowsum[v];
      }
    }
    __syncthreads();
    if (threadIdx.x < SSD_BLK) {
      const int64_t base = ((int64_t)c * d.H + h) * d.Qpad + s0 + threadIdx.x;
      bf.eterm[base] = red[threadIdx.x] + red[SSD_BLK + threadIdx.x];
      bf.xdx[base] = red[2 * SSD_BLK + threadIdx.x] + red[3 * SSD_BLK + threadIdx.x];
    }
    // D partial: the four wave sums in a fixed order
    __syncthreads();
    if (lane == 0) red[w] = dpart;
    __syncthreads();
    if (threadIdx.x == 0)
      bf.dD_part[((int64_t)c * d.H + h) * (d.Qpad / SSD_BLK) + j] = red[0] + red[1] + red[2] + red[3];
  }
  // dB for the slice
  const bool direct = bf.nslices == 1;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int n = wc * 32 + 64 * t + (lane & 31);
    if (n >= d.N) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int sg = s0 + wr * 32 + acc_row(v, lane);
      if (sg >= ci.len) continue;
      const int64_t o = (int64_t)(ci.row0 + sg) * brow + (int64_t)g * d.N + n;
      if (direct) dB[o] = from_f<T>(accB[t][v]);
      else bf.dB_part[(int64_t)slc * d.R * brow + o] = accB[t][v];
    }
  }
}

// ---------------------------------------------------------------------------
// Row side: block (i, group*slices, chunk) owns rows l in block i. Per head:
// row sums of G and the Y_off term of dcs; across the slice's heads dC_i.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) k_bwd_row(SsdDims d, SsdBufs bf, BwdCommon<T> in, T* __restrict__ dC) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int i = blockIdx.x, c = blockIdx.z;
  const int g = blockIdx.y / bf.nslices, slc = blockIdx.y % bf.nslices;
  const ChunkInfo ci = in.chunks[c];
  const int r0 = i * SSD_BLK;
  if (r0 >= ci.len) return;
  const int h_lo = g * d.hpg + slc * bf.hslice;
  const int h_hi = min(h_lo + bf.hslice, (g + 1) * d.hpg);
  const int NP = lds_pitch<T>(d.Npad), PP = lds_pitch<T>(d.Ppad), BP = lds_pitch<T>(SSD_BLK);
  float* s_cs = reinterpret_cast<float*>(smem);
  float* s_dt = s_cs + d.Qpad;
  float* red = s_dt + d.Qpad;                       // [4][64]
  T* Ci = reinterpret_cast<T*>(red + 4 * SSD_BLK);  // [64][NP]
  T* dYi = Ci + SSD_BLK * NP;                       // [64][PP]
  T* regA = dYi + SSD_BLK * PP;
  T* Bj = regA;                                     // [64][NP]
  T* xj = Bj + SSD_BLK * NP;                        // [64][PP]
  T* BjT = xj + SSD_BLK * PP;                       // [Npad][BP]
  T* dSt = BjT + d.Npad * BP;                       // [64][BP]
  T* hT = regA;                                     // [Npad][PP] (after the j loop)

  const int lane = lane_id();
  const int w = threadIdx.x >> 6, wr = w & 1, wc = w >> 1;
  const int64_t brow = (int64_t)d.G * d.N, xrow = (int64_t)d.H * d.P;
  stage_rows<T>(Ci, NP, in.Cm, brow, (int64_t)g * d.N, ci.row0, r0, ci.len, d.N, d.Npad);
  floatx16 accC[2];
  zero(accC[0]);
  zero(accC[1]);
  const int sl = wc * 32 + (lane & 31);

  for (int h = h_lo; h < h_hi; ++h) {
    __syncthreads();
    const float* csc = in.cs + ((int64_t)c * d.H + h) * d.Qpad;
    for (int l = threadIdx.x; l < d.Qpad; l += blockDim.x) {
      s_cs[l] = csc[l];
      s_dt[l] = (d.has_dt && l < ci.len) ? in.dt[(int64_t)(ci.row0 + l) * d.H + h] : 1.0f;
    }
    stage_rows<T>(dYi, PP, in.dy, xrow, (int64_t)h * d.P, ci.row0, r0, ci.len, d.P, d.Ppad);
    float grow[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) grow[v] = 0.0f;
    for (int jb = 0; jb <= i; ++jb) {
      const int s0 = jb * SSD_BLK;
      __syncthreads();
      stage_rows<T>(Bj, NP, in.Bm, brow, (int64_t)g * d.N, ci.row0, s0, ci.len, d.N, d.Npad);
      stage_rows<T>(xj, PP, in.x, xrow, (int64_t)h * d.P, ci.row0, s0, ci.len, d.P, d.Ppad);
      stage_rows_t<T>(BjT, BP, in.Bm, brow, (int64_t)g * d.N, ci.row0, s0, ci.len, d.N, d.Npad);
      __syncthreads();
      floatx16 sacc, macc;
      zero(sacc);
      zero(macc);
      mma_tile<T>(sacc, Ci + wr * 32 * NP, NP, Bj + wc * 32 * NP, NP, d.Npad);
      mma_tile<T>(macc, dYi + wr * 32 * PP, PP, xj + wc * 32 * PP, PP, d.Ppad);
      const int s = s0 + sl;
      const float cs_s = s_cs[s], dt_s = s_dt[s];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int ll = wr * 32 + acc_row(v, lane);
        const int l = r0 + ll;
        float dsv = 0.0f, gv = 0.0f;
        if (s <= l && l < ci.len) {
          const float dd = s_cs[l] - cs_s;
          const float Lv = exp_clamp(dd);
          const float dm = macc[v] * dt_s;
          dsv = dm * Lv;
          gv = dm * sacc[v] * Lv * clamp_pass(dd);
        }
        dSt[ll * BP + sl] = from_f<T>(dsv);
        grow[v] += row_reduce32(gv);
      }
      __syncthreads();
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int n0 = wc * 32 + 64 * t;
        if (n0 < d.Npad) mma_tile<T>(accC[t], dSt + wr * 32 * BP, BP, BjT + n0 * BP, BP, SSD_BLK);
      }
    }
    // Y_off part: tmp = exp(cs_l) dY_l h (K = P); h staged transposed
    __syncthreads();
    const T* hsrc = in.hin + ((int64_t)c * d.H + h) * d.Ppad * d.Npad;
    for (int idx = threadIdx.x; idx < d.Ppad * d.Npad; idx += blockDim.x) {
      const int p = idx / d.Npad, n = idx % d.Npad;
      hT[n * PP + p] = hsrc[idx];
    }
    if ((lane & 31) == 0) {
#pragma unroll
      for (int v = 0; v < 16; ++v) red[wc * SSD_BLK + wr * 32 + acc_row(v, lane)] = grow[v];
    }
    __syncthreads();
    float offrow[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) offrow[v] = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int n0 = wc * 32 + 64 * t;
      if (n0 >= d.Npad) continue;
      floatx16 tmp;
      zero(tmp);
      mma_tile<T>(tmp, dYi + wr * 32 * PP, PP, hT + n0 * PP, PP, d.Ppad);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int ll = wr * 32 + acc_row(v, lane);
        const int l = r0 + ll;
        const float e = l < ci.len ? exp_clamp(s_cs[l]) : 0.0f;
        const float tv = tmp[v] * e;
        offrow[v] += tv * to_f(Ci[ll * NP + n0 + (lane & 31)]);
        accC[t][v] += tv;
      }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) offrow[v] = row_reduce32(offrow[v]);
    if ((lane & 31) == 0) {
#pragma unroll
      for (int v = 0; v < 16; ++v) red[(2 + wc) * SSD_BLK + wr * 32 + acc_row(v, lane)] = offrow[v];
    }
    __syncthreads();
    if (threadIdx.x < SSD_BLK) {
      const int l = r0 + threadIdx.x;
      const int64_t base = ((int64_t)c * d.H + h) * d.Qpad + l;
      bf.rowG[base] = red[threadIdx.x] + red[SSD_BLK + threadIdx.x];
      bf.dcs_off[base] = (red[2 * SSD_BLK + threadIdx.x] + red[3 * SSD_BLK + threadIdx.x]) * clamp_pass(s_cs[l]);
    }
  }
  const bool direct = bf.nslices == 1;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int n = wc * 32 + 64 * t + (lane & 31);
    if (n >= d.N) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int l = r0 + wr * 32 + acc_row(v, lane);
      if (l >= ci.len) continue;
      const int64_t o = (int64_t)(ci.row0 + l) * brow + (int64_t)g * d.N + n;
      if (direct) dC[o] = from_f<T>(accC[t][v]);
      else bf.dC_part[(int64_t)slc * d.R * brow + o] = accC[t][v];
    }
  }
}

// ---------------------------------------------------------------------------
// Finish: dcs per position, da = reverse in-chunk cumsum (the adjoint of the
// inclusive cumsum, ssd_scan.py:368), then ddt / per-token dA / dA partials.
// One wave per (chunk, head).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) k_bwd_finish(SsdDims d, SsdBufs bf, const ChunkInfo* __restrict__ chunks,
                                                    const float* __restrict__ Ah, const float* __restrict__ dt,
                                                    float* __restrict__ ddt, T* __restrict__ dA_tok) {
  const int c = blockIdx.x;
  const int h = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = lane_id();
  if (h >= d.H) return;
  const ChunkInfo ci = chunks[c];
  const int64_t ch = (int64_t)c * d.H + h;
  if (ci.len == 0) {
    if (lane == 0) bf.dA_part[ch] = 0.0f;
    return;
  }
  const int per = d.Qpad / 64;
  const int64_t base = ch * d.Qpad;
  float v[4];
  float esum = 0.0f;
  for (int e = 0; e < per; ++e) {
    const int l = lane * per + e;
    float x = 0.0f;
    if (l < ci.len) {
      x = bf.rowG[base + l] - bf.colG[base + l] + bf.dcs_off[base + l] - bf.eterm[base + l];
      esum += bf.eterm[base + l];
    }
    v[e] = x;
  }
  for (int o = 32; o > 0; o >>= 1) esum += __shfl_xor(esum, o, 64);
  float dtot = 0.0f;
  for (int k = 0; k < bf.npass_blk; ++k) dtot += bf.dtot_part[ch * bf.npass_blk + k];
  const int last = ci.len - 1;
  if (last / per == lane) v[last % per] += esum + dtot;
  // reverse inclusive scan: local suffix, then exclusive suffix of lane totals
  float run = 0.0f;
  for (int e = per - 1; e >= 0; --e) {
    run += v[e];
    v[e] = run;
  }
  float incl = run;
  for (int off = 1; off < 64; off <<= 1) {
    float o = __shfl_down(incl, off, 64);
    if (lane + off < 64) incl += o;
  }
  const float excl = incl - run;
  float dAp = 0.0f;
  for (int e = 0; e < per; ++e) {
    const int l = lane * per + e;
    if (l >= ci.len) continue;
    const float da = v[e] + excl;
    const int64_t row = ci.row0 + l;
    if (d.a_mode == 0) {
      const float dtv = d.has_dt ? dt[row * d.H + h] : 1.0f;
      if (ddt && d.has_dt) ddt[row * d.H + h] = bf.xdx[base + l] + Ah[h] * da;
      dAp += dtv * da;
    } else if (d.a_mode == 1) {
      if (dA_tok) dA_tok[row * d.H + h] = from_f<T>(da);
    }
  }
  for (int o = 32; o > 0; o >>= 1) dAp += __shfl_xor(dAp, o, 64);
  if (lane == 0) bf.dA_part[ch] = dAp;
}

size_t lds_bwd_col(int dtype, const SsdDims& d) {
  const size_t es = dtype == 1 ? 2 : 4;
  const size_t NP = d.Npad + 16 / es, PP = d.Ppad + 16 / es, BP = SSD_BLK + 16 / es;
  const size_t fixed = sizeof(float) * (2 * d.Qpad + 4 * SSD_BLK) + es * (SSD_BLK * NP + SSD_BLK * PP);
  const size_t regA = es * (SSD_BLK * NP + SSD_BLK * PP + d.Ppad * BP + d.Npad * BP + 2 * SSD_BLK * BP);
  const size_t regB = es * (d.Npad * PP + d.Ppad * NP);
  return fixed + (regA > regB ? regA : regB);
}

size_t lds_bwd_row(int dtype, const SsdDims& d) {
  const size_t es = dtype == 1 ? 2 : 4;
  const size_t NP = d.Npad + 16 / es, PP = d.Ppad + 16 / es, BP = SSD_BLK + 16 / es;
  const size_t fixed = sizeof(float) * (2 * d.Qpad + 4 * SSD_BLK) + es * (SSD_BLK * NP + SSD_BLK * PP);
  const size_t regA = es * (SSD_BLK * NP + SSD_BLK * PP + d.Npad * BP + SSD_BLK * BP);
  const size_t regB = es * (d.Npad * PP);
  return fixed + (regA > regB ? regA : regB);
}

template <typename T>
static BwdCommon<T> make_common(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy) {
  BwdCommon<T> c;
  c.chunks = b.chunks;
  c.cs = b.cs;
  c.hin = reinterpret_cast<const T*>(b.hin);
  c.dst = b.dst;
  c.x = reinterpret_cast<const T*>(in.x);
  c.dt = in.dt;
  c.Bm = reinterpret_cast<const T*>(in.B);
  c.Cm = reinterpret_cast<const T*>(in.C);
  c.Dv = in.D;
  c.dy = reinterpret_cast<const T*>(dy);
  return c;
}

hipError_t launch_bwd_col(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy,
                          void* dx, void* dB, hipStream_t s) {
  dim3 grid(d.Qpad / SSD_BLK, d.G * b.nslices, d.max_chunks);
  const size_t lds = lds_bwd_col(dtype, d);
  if (dtype == 1) ensure_lds(k_bwd_col<bf16>, lds);
  else ensure_lds(k_bwd_col<float>, lds);
  if (dtype == 1)
    hipLaunchKernelGGL(k_bwd_col<bf16>, grid, dim3(256), lds, s, d, b, make_common<bf16>(d, b, in, dy),
                       reinterpret_cast<bf16*>(dx), reinterpret_cast<bf16*>(dB));
  else
    hipLaunchKernelGGL(k_bwd_col<float>, grid, dim3(256), lds, s, d, b, make_common<float>(d, b, in, dy),
                       reinterpret_cast<float*>(dx), reinterpret_cast<float*>(dB));
  return hipGetLastError();
}

hipError_t launch_bwd_row(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy,
                          void* dC, hipStream_t s) {
  dim3 grid(d.Qpad / SSD_BLK, d.G * b.nslices, d.max_chunks);
  const size_t lds = lds_bwd_row(dtype, d);
  if (dtype == 1) ensure_lds(k_bwd_row<bf16>, lds);
  else ensure_lds(k_bwd_row<float>, lds);
  if (dtype == 1)
    hipLaunchKernelGGL(k_bwd_row<bf16>, grid, dim3(256), lds, s, d, b, make_common<bf16>(d, b, in, dy),
                       reinterpret_cast<bf16*>(dC));
  else
    hipLaunchKernelGGL(k_bwd_row<float>, grid, dim3(256), lds, s, d, b, make_common<float>(d, b, in, dy),
                       reinterpret_cast<float*>(dC));
  return hipGetLastError();
}

hipError_t launch_bwd_finish(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, float* ddt,
                             void* dA_tok, hipStream_t s) {
  dim3 grid(d.max_chunks, (d.H + 3) / 4);
  const float* Ah = d.a_mode == 0 ? reinterpret_cast<const float*>(in.A) : nullptr;
  if (dtype == 1)
    hipLaunchKernelGGL(k_bwd_finish<bf16>, grid, dim3(256), 0, s, d, b, b.chunks, Ah, in.dt, ddt,
                       reinterpret_cast<bf16*>(dA_tok));
  else
    hipLaunchKernelGGL(k_bwd_finish<float>, grid, dim3(256), 0, s, d, b, b.chunks, Ah, in.dt, ddt,
                       reinterpret_cast<float*>(dA_tok));
  return hipGetLastError();
}
