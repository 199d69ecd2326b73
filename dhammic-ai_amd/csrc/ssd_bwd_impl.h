// Backward kernel templates of the chunked SSD scan (the gradient that FusedSSDScan.backward,
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
#pragma once

#include "ssd_launch.h"

size_t lds_bwd_col(int dtype, const SsdDims& d);
size_t lds_bwd_row(int dtype, const SsdDims& d);



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



// Cross-wave reduction of partial accumulator tiles: waves (0, q) and (1, q)
// (q = w >> 1) hold partial sums of the same NTILE tiles; wave r keeps tiles
// t with t % 2 == r and receives the other wave's partial of them through
// `buf` (2 * NTILE * 4 KiB of LDS). Must be called by all 256 threads.
template <int NTILE>
__device__ __forceinline__ void reduce_pair(floatx16 (&acc)[NTILE], float* __restrict__ buf) {
  const int lane = lane_id(), w = threadIdx.x >> 6, r = w & 1, q = w >> 1;
  __syncthreads();
#pragma unroll
  for (int t = 0; t < NTILE; ++t)
    if (t % 2 != r) {
      float* o = buf + ((q * NTILE + t) * 16) * 64 + lane;
#pragma unroll
      for (int v = 0; v < 16; ++v) o[v * 64] = acc[t][v];
    }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < NTILE; ++t)
    if (t % 2 == r) {
      const float* o = buf + ((q * NTILE + t) * 16) * 64 + lane;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[t][v] += o[v * 64];
    }
}

// Stage one (chunk, head) state tile, stored [Ppad][Npad] in global memory, as T
// into LDS: natural [p][n] (pitch np, optional) and transposed [n][p] (pitch pp).
// Lanes take consecutive p so the transposed 2-byte stores hit consecutive banks.
template <typename T, typename S>
__device__ __forceinline__ void stage_state(const S* __restrict__ src, int Ppad, int Npad, T* __restrict__ nat,
                                            int np, T* __restrict__ tr, int pp) {
  const int ngrp = Npad / 4;
  for (int id = threadIdx.x; id < Ppad * ngrp; id += blockDim.x) {
    const int p = id % Ppad, n = (id / Ppad) * 4;
    const S* g = src + (int64_t)p * Npad + n;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const T v = from_f<T>(to_f(g[e]));
      if (nat) nat[p * np + n + e] = v;
      tr[(n + e) * pp + p] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Column side: block (j, group*slices, chunk) owns columns s in block j and the
// heads of one slice of group g. Units (head, row block i >= j); the C and dY
// rows of the next unit are loaded into registers while the current unit
// computes. Wave w holds the S / dM tile of rows l in half wr = w%2 and
// columns s in half wc = w/2; M = S*L and dS = dM*dt*L stay in registers and
// are the A operands of dX += M^T dY and dB += dS^T C (partial over wr,
// reduced across the wave pair at the end).
// Per head: dX_j -> dx, column sums of G, the E term, x.dX per row, the D
// partial; across the slice's heads: dB_j.
// ---------------------------------------------------------------------------
template <typename T, int PT, int NT>
__global__ void __launch_bounds__(256) k_bwd_col(SsdDims d, SsdBufs bf, BwdCommon<T> in, T* __restrict__ dx,
                                                 T* __restrict__ dB) {
  constexpr int PPAD = 32 * PT, NPAD = 32 * NT;
  constexpr int NP = lds_pitch<T>(NPAD), PP = lds_pitch<T>(PPAD), BP = lds_pitch<T>(SSD_BLK);
  extern __shared__ __align__(16) unsigned char smem[];
  const int j = blockIdx.x, c = blockIdx.z;
  const int g = blockIdx.y / bf.nslices, slc = blockIdx.y % bf.nslices;
  const ChunkInfo ci = in.chunks[c];
  const int s0 = j * SSD_BLK;
  if (s0 >= ci.len) return;
  const int h_lo = g * d.hpg + slc * bf.hslice;
  const int h_hi = min(h_lo + bf.hslice, (g + 1) * d.hpg);
  float* s_cs = reinterpret_cast<float*>(smem);
  float* s_dt = s_cs + d.Qpad;
  float* red = s_dt + d.Qpad;                       // [4][64]
  T* Bj = reinterpret_cast<T*>(red + 4 * SSD_BLK);  // [64][NP]
  T* xj = Bj + SSD_BLK * NP;                        // [64][PP]
  T* regA = xj + SSD_BLK * PP;
  T* Ci = regA;                                     // [64][NP]
  T* dYi = Ci + SSD_BLK * NP;                       // [64][PP]
  T* dYiT = dYi + SSD_BLK * PP;                     // [Ppad][BP]
  T* CiT = dYiT + PPAD * BP;                      // [Npad][BP]
  T* dstN = regA;                                   // [Ppad][NP] (head epilogue)
  T* dstT = dstN + PPAD * NP;                     // [Npad][PP]
  float* xred = reinterpret_cast<float*>(dstT + NPAD * PP);  // 2 * max(PT, NT) * 4 KiB

  const int lane = lane_id();
  const int w = threadIdx.x >> 6, wr = w & 1, wc = w >> 1;
  const int64_t brow = (int64_t)d.G * d.N, xrow = (int64_t)d.H * d.P;
  const int nblk_len = (ci.len + SSD_BLK - 1) / SSD_BLK;
  const int ni = nblk_len - j;
  const int nunits = (h_hi - h_lo) * ni;
  const int sl = wc * 32 + (lane & 31);  // this lane's column s in the S tile
  const int s = s0 + sl;

  TileRegs<T, 32 * NT> rc;
  TileRegs<T, 32 * PT> ry;
  auto load_unit = [&](int u) {
    const int h = h_lo + u / ni, r0 = (j + u % ni) * SSD_BLK;
    tile_load<T, true>(rc, in.Cm, brow, (int64_t)g * d.N, ci.row0, r0, ci.len, d.N, NPAD, d.vec_bc);
    tile_load<T, true>(ry, in.dy, xrow, (int64_t)h * d.P, ci.row0, r0, ci.len, d.P, PPAD, d.vec_x);
  };
  load_unit(0);
  stage_nat<T>(Bj, NP, in.Bm, brow, (int64_t)g * d.N, ci.row0, s0, ci.len, d.N, NPAD, d.vec_bc);

  floatx16 accB[NT], accX[PT];
#pragma unroll
  for (int t = 0; t < NT; ++t) zero(accB[t]);
  float gcol = 0.0f, cs_s = 0.0f, dt_s = 1.0f;
  for (int u = 0; u < nunits; ++u) {
    const int h = h_lo + u / ni, i = j + u % ni, r0 = i * SSD_BLK;
    if (i == j) {  // first unit of head h
      __syncthreads();
      const float* csc = in.cs + ((int64_t)c * d.H + h) * d.Qpad;
      for (int l = threadIdx.x; l < d.Qpad; l += blockDim.x) {
        s_cs[l] = csc[l];
        s_dt[l] = (d.has_dt && l < ci.len) ? in.dt[(int64_t)(ci.row0 + l) * d.H + h] : 1.0f;
      }
      stage_nat<T>(xj, PP, in.x, xrow, (int64_t)h * d.P, ci.row0, s0, ci.len, d.P, PPAD, d.vec_x);
#pragma unroll
      for (int t = 0; t < PT; ++t) zero(accX[t]);
      gcol = 0.0f;
    }
    __syncthreads();
    if (i == j) {
      cs_s = s_cs[s];
      dt_s = s_dt[s];
    }
    tile_store_nat<T, true>(rc, Ci, NP, NPAD);
    tile_store_tr<T>(rc, CiT, BP, NPAD);
    tile_store_nat<T, true>(ry, dYi, PP, PPAD);
    tile_store_tr<T>(ry, dYiT, BP, PPAD);
    __syncthreads();
    if (u + 1 < nunits) load_unit(u + 1);
    {
      floatx16 sacc, macc;
      zero(sacc);
      zero(macc);
      mma_k<T, NPAD>(sacc, Ci + wr * 32 * NP, NP, Bj + wc * 32 * NP, NP);
      mma_k<T, PPAD>(macc, dYi + wr * 32 * PP, PP, xj + wc * 32 * PP, PP);
      float csl[16];
      rows16(s_cs + r0 + wr * 32, csl);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int l = r0 + wr * 32 + acc_row(v, lane);
        const bool ok = s + (d.trapz ? 1 : 0) <= l && l < ci.len;  // trapezoidal mode: strictly causal
        const float dd = csl[v] - cs_s;
        const float Lv = ok ? exp_clamp(dd) : 0.0f;
        const float m = sacc[v] * Lv;
        const float dm = macc[v] * dt_s;
        gcol += dm * m * clamp_pass(dd);
        sacc[v] = m;        // M tile
        macc[v] = dm * Lv;  // dS tile
      }
      const AccFrags<T> mf = acc_frags<T>(sacc), sf = acc_frags<T>(macc);
#pragma unroll
      for (int t = 0; t < PT; ++t) mma_xt_f<T>(accX[t], mf, dYiT + t * 32 * BP + wr * 32, BP);
#pragma unroll
      for (int t = 0; t < NT; ++t) mma_xt_f<T>(accB[t], sf, CiT + t * 32 * BP + wr * 32, BP);
    }
    if (i != nblk_len - 1) continue;

    // ---- head epilogue ----
    gcol += __shfl_xor(gcol, 32, 64);
    reduce_pair<PT>(accX, xred);  // starts with a barrier: the unit's LDS reads are done
    if (lane < 32) red[wr * SSD_BLK + sl] = gcol;
    stage_state<T, float>(in.dst + ((int64_t)c * d.H + h) * PPAD * NPAD, PPAD, NPAD, dstN, NP, dstT, PP);
    __syncthreads();
    float* colG = bf.colG + ((int64_t)c * d.H + h) * d.Qpad;
    if (threadIdx.x < SSD_BLK) colG[s0 + threadIdx.x] = red[threadIdx.x] + red[SSD_BLK + threadIdx.x];
    __syncthreads();  // the gcol partials are read before the e / xs partials overwrite them
    const float cs_last = s_cs[d.Qpad - 1];
    float dpart = 0.0f;
    const float Dh = d.has_D ? in.Dv[h] : 0.0f;
    {
      // this wave's p tiles of the state term tmp = B_s dst^T (K = N)
      floatx16 tmp[(PT + 1) / 2];
#pragma unroll
      for (int t = 0; t < PT; ++t) {
        if (t % 2 != wr) continue;
        zero(tmp[t / 2]);
        mma_k<T, NPAD>(tmp[t / 2], Bj + wc * 32 * NP, NP, dstN + t * 32 * NP, NP);
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int sr = wc * 32 + acc_row(v, lane);
        const int sg = s0 + sr;
        const float ws = sg < ci.len ? exp_clamp(cs_last - s_cs[sg]) : 0.0f;
        const float dts = s_dt[sg];
        float e = 0.0f, xs = 0.0f;
#pragma unroll
        for (int t = 0; t < PT; ++t) {
          if (t % 2 != wr) continue;
          const int p = t * 32 + (lane & 31);
          const float xv = to_f(xj[sr * PP + p]);
          const float tx = tmp[t / 2][v] * ws;
          e += xv * tx;
          const float dX = accX[t][v] + tx;
          xs += xv * dX;
          if (sg < ci.len && p < d.P) {
            const int64_t o = (int64_t)(ci.row0 + sg) * xrow + (int64_t)h * d.P + p;
            const float dyv = to_f(in.dy[o]);
            const float Dl = d.trapz ? bf.Dtok[(int64_t)(ci.row0 + sg) * d.H + h] : Dh;
            dx[o] = from_f<T>(dts * dX + Dl * dyv);
            dpart += xv * dyv;
          }
        }
        e = row_reduce32(e) * dts * clamp_pass(cs_last - s_cs[sg]);
        xs = row_reduce32(xs);
        if ((lane & 31) == 0) {
          red[wr * SSD_BLK + sr] = e;
          red[(2 + wr) * SSD_BLK + sr] = xs;
        }
      }
    }
    // dB state part: w_s dt_s x_s dst (K = P), on this wave's share of the n tiles
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t % 2 != wr) continue;
      floatx16 tb;
      zero(tb);
      mma_k<T, PPAD>(tb, xj + wc * 32 * PP, PP, dstT + t * 32 * PP, PP);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int sg = s0 + wc * 32 + acc_row(v, lane);
        const float ws = sg < ci.len ? exp_clamp(cs_last - s_cs[sg]) * s_dt[sg] : 0.0f;
        accB[t][v] += tb[v] * ws;
      }
    }
    for (int o = 32; o > 0; o >>= 1) dpart += __shfl_xor(dpart, o, 64);
    __syncthreads();
    if (threadIdx.x < SSD_BLK) {
      const int64_t base = ((int64_t)c * d.H + h) * d.Qpad + s0 + threadIdx.x;
      bf.eterm[base] = red[threadIdx.x] + red[SSD_BLK + threadIdx.x];
      bf.xdx[base] = red[2 * SSD_BLK + threadIdx.x] + red[3 * SSD_BLK + threadIdx.x];
    }
    __syncthreads();
    if (lane == 0) red[w] = dpart;
    __syncthreads();
    if (threadIdx.x == 0)
      bf.dD_part[((int64_t)c * d.H + h) * (d.Qpad / SSD_BLK) + j] = red[0] + red[1] + red[2] + red[3];
  }
  // dB for the slice: combine the wave pair, then store this wave's tiles
  reduce_pair<NT>(accB, xred);
  const bool direct = bf.nslices == 1;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t % 2 != wr) continue;
    const int n = t * 32 + (lane & 31);
    if (n >= d.N) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int sg = s0 + wc * 32 + acc_row(v, lane);
      if (sg >= ci.len) continue;
      const int64_t o = (int64_t)(ci.row0 + sg) * brow + (int64_t)g * d.N + n;
      if (direct) dB[o] = from_f<T>(accB[t][v]);
      else bf.dB_part[(int64_t)slc * d.R * brow + o] = accB[t][v];
    }
  }
}

// ---------------------------------------------------------------------------
// Row side: block (i, group*slices, chunk) owns rows l in block i. Units
// (head, column block j <= i); the B and x rows of the next unit are loaded
// into registers while the current unit computes. Wave w holds the S^T / dM^T
// tile of rows s in half wr = w%2 and columns l in half wc = w/2, so dS^T
// stays in registers as the A operand of dC += dS B (partial over wr).
// Per head: row sums of G and the Y_off term of dcs; across heads: dC_i.
// ---------------------------------------------------------------------------
template <typename T, int PT, int NT>
__global__ void __launch_bounds__(256) k_bwd_row(SsdDims d, SsdBufs bf, BwdCommon<T> in, T* __restrict__ dC) {
  constexpr int PPAD = 32 * PT, NPAD = 32 * NT;
  constexpr int NP = lds_pitch<T>(NPAD), PP = lds_pitch<T>(PPAD), BP = lds_pitch<T>(SSD_BLK);
  extern __shared__ __align__(16) unsigned char smem[];
  const int i = blockIdx.x, c = blockIdx.z;
  const int g = blockIdx.y / bf.nslices, slc = blockIdx.y % bf.nslices;
  const ChunkInfo ci = in.chunks[c];
  const int r0 = i * SSD_BLK;
  if (r0 >= ci.len) return;
  const int h_lo = g * d.hpg + slc * bf.hslice;
  const int h_hi = min(h_lo + bf.hslice, (g + 1) * d.hpg);
  float* s_cs = reinterpret_cast<float*>(smem);
  float* s_dt = s_cs + d.Qpad;
  float* red = s_dt + d.Qpad;                       // [4][64]
  T* Ci = reinterpret_cast<T*>(red + 4 * SSD_BLK);  // [64][NP]
  T* dYi = Ci + SSD_BLK * NP;                       // [64][PP]
  T* regA = dYi + SSD_BLK * PP;
  T* Bj = regA;                                     // [64][NP]
  T* xj = Bj + SSD_BLK * NP;                        // [64][PP]
  T* BjT = xj + SSD_BLK * PP;                       // [Npad][BP]
  T* hT = regA;                                     // [Npad][PP] (head epilogue)
  float* xred = reinterpret_cast<float*>(hT + NPAD * PP);  // 2 * NT * 4 KiB

  const int lane = lane_id();
  const int w = threadIdx.x >> 6, wr = w & 1, wc = w >> 1;
  const int64_t brow = (int64_t)d.G * d.N, xrow = (int64_t)d.H * d.P;
  const int nj = i + 1;
  const int nunits = (h_hi - h_lo) * nj;
  const int lcol = wc * 32 + (lane & 31);  // this lane's l in the S^T tile
  const int l_me = r0 + lcol;
  const bool l_ok = l_me < ci.len;

  TileRegs<T, 32 * NT> rb;
  TileRegs<T, 32 * PT> rx;
  auto load_unit = [&](int u) {
    const int h = h_lo + u / nj, s0 = (u % nj) * SSD_BLK;
    tile_load<T, true>(rb, in.Bm, brow, (int64_t)g * d.N, ci.row0, s0, ci.len, d.N, NPAD, d.vec_bc);
    tile_load<T, false>(rx, in.x, xrow, (int64_t)h * d.P, ci.row0, s0, ci.len, d.P, PPAD, d.vec_x);
  };
  load_unit(0);
  stage_nat<T>(Ci, NP, in.Cm, brow, (int64_t)g * d.N, ci.row0, r0, ci.len, d.N, NPAD, d.vec_bc);
  floatx16 accC[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) zero(accC[t]);
  float grow = 0.0f, cs_l = 0.0f;

  for (int u = 0; u < nunits; ++u) {
    const int h = h_lo + u / nj, jb = u % nj, s0 = jb * SSD_BLK;
    if (jb == 0) {  // first unit of head h
      __syncthreads();
      const float* csc = in.cs + ((int64_t)c * d.H + h) * d.Qpad;
      for (int l = threadIdx.x; l < d.Qpad; l += blockDim.x) {
        s_cs[l] = csc[l];
        s_dt[l] = (d.has_dt && l < ci.len) ? in.dt[(int64_t)(ci.row0 + l) * d.H + h] : 1.0f;
      }
      stage_nat<T>(dYi, PP, in.dy, xrow, (int64_t)h * d.P, ci.row0, r0, ci.len, d.P, PPAD, d.vec_x);
      grow = 0.0f;
    }
    __syncthreads();
    if (jb == 0) cs_l = s_cs[l_me];
    tile_store_nat<T, true>(rb, Bj, NP, NPAD);
    tile_store_tr<T>(rb, BjT, BP, NPAD);
    tile_store_nat<T, false>(rx, xj, PP, PPAD);
    __syncthreads();
    if (u + 1 < nunits) load_unit(u + 1);
    {
      floatx16 st, mt;
      zero(st);
      zero(mt);
      mma_k<T, NPAD>(st, Bj + wr * 32 * NP, NP, Ci + wc * 32 * NP, NP);   // S^T[s][l]
      mma_k<T, PPAD>(mt, xj + wr * 32 * PP, PP, dYi + wc * 32 * PP, PP);  // dM'^T[s][l]
      float css[16], dts[16];
      rows16(s_cs + s0 + wr * 32, css);
      rows16(s_dt + s0 + wr * 32, dts);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int sg = s0 + wr * 32 + acc_row(v, lane);
        const bool ok = sg + (d.trapz ? 1 : 0) <= l_me && l_ok;
        const float dd = cs_l - css[v];
        const float Lv = ok ? exp_clamp(dd) : 0.0f;
        const float dsv = mt[v] * dts[v] * Lv;
        grow += dsv * st[v] * clamp_pass(dd);
        mt[v] = dsv;  // dS^T tile
      }
      const AccFrags<T> sf = acc_frags<T>(mt);
#pragma unroll
      for (int t = 0; t < NT; ++t) mma_xt_f<T>(accC[t], sf, BjT + t * 32 * BP + wr * 32, BP);
    }
    if (jb != i) continue;

    // ---- head epilogue: Y_off term tmp = exp(cs_l) dY_l h (K = P); h staged transposed ----
    grow += __shfl_xor(grow, 32, 64);
    __syncthreads();
    if (lane < 32) red[wr * SSD_BLK + lcol] = grow;
    stage_state<T, T>(in.hin + ((int64_t)c * d.H + h) * PPAD * NPAD, PPAD, NPAD, nullptr, 0, hT, PP);
    __syncthreads();
    float offrow[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) offrow[v] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t % 2 != wr) continue;
      floatx16 tmp;
      zero(tmp);
      mma_k<T, PPAD>(tmp, dYi + wc * 32 * PP, PP, hT + t * 32 * PP, PP);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int ll = wc * 32 + acc_row(v, lane);
        const int l = r0 + ll;
        const float e = l < ci.len ? exp_clamp(s_cs[l]) : 0.0f;
        const float tv = tmp[v] * e;
        offrow[v] += tv * to_f(Ci[ll * NP + t * 32 + (lane & 31)]);
        accC[t][v] += tv;
      }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) offrow[v] = row_reduce32(offrow[v]);
    if ((lane & 31) == 0) {
#pragma unroll
      for (int v = 0; v < 16; ++v) red[(2 + wr) * SSD_BLK + wc * 32 + acc_row(v, lane)] = offrow[v];
    }
    __syncthreads();
    if (threadIdx.x < SSD_BLK) {
      const int l = r0 + threadIdx.x;
      const int64_t base = ((int64_t)c * d.H + h) * d.Qpad + l;
      bf.rowG[base] = red[threadIdx.x] + red[SSD_BLK + threadIdx.x];
      bf.dcs_off[base] = (red[2 * SSD_BLK + threadIdx.x] + red[3 * SSD_BLK + threadIdx.x]) * clamp_pass(s_cs[l]);
    }
  }
  reduce_pair<NT>(accC, xred);
  const bool direct = bf.nslices == 1;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t % 2 != wr) continue;
    const int n = t * 32 + (lane & 31);
    if (n >= d.N) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int l = r0 + wc * 32 + acc_row(v, lane);
      if (l >= ci.len) continue;
      const int64_t o = (int64_t)(ci.row0 + l) * brow + (int64_t)g * d.N + n;
      if (direct) dC[o] = from_f<T>(accC[t][v]);
      else bf.dC_part[(int64_t)slc * d.R * brow + o] = accC[t][v];
    }
  }
}

template <typename T>
BwdCommon<T> make_common(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy) {
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

template <typename T, int PT, int NT>
hipError_t bwd_col_t(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy, void* dx, void* dB,
                            hipStream_t s) {
  dim3 grid(d.Qpad / SSD_BLK, d.G * b.nslices, d.max_chunks);
  const size_t lds = lds_bwd_col(sizeof(T) == 2 ? 1 : 0, d);
  ensure_lds(k_bwd_col<T, PT, NT>, lds);
  hipLaunchKernelGGL((k_bwd_col<T, PT, NT>), grid, dim3(256), lds, s, d, b, make_common<T>(d, b, in, dy),
                     reinterpret_cast<T*>(dx), reinterpret_cast<T*>(dB));
  return hipGetLastError();
}

template <typename T, int PT>
hipError_t bwd_col_n(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy, void* dx, void* dB,
                            hipStream_t s) {
  switch (d.Npad / 32) {
    case 1: return bwd_col_t<T, PT, 1>(d, b, in, dy, dx, dB, s);
    case 2: return bwd_col_t<T, PT, 2>(d, b, in, dy, dx, dB, s);
    default: return bwd_col_t<T, PT, 4>(d, b, in, dy, dx, dB, s);
  }
}

template <typename T>
hipError_t bwd_col_d(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy, void* dx, void* dB,
                            hipStream_t s) {
  switch (d.Ppad / 32) {
    case 1: return bwd_col_n<T, 1>(d, b, in, dy, dx, dB, s);
    case 2: return bwd_col_n<T, 2>(d, b, in, dy, dx, dB, s);
    default: return bwd_col_n<T, 4>(d, b, in, dy, dx, dB, s);
  }
}


template <typename T, int PT, int NT>
hipError_t bwd_row_t(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy, void* dC,
                            hipStream_t s) {
  dim3 grid(d.Qpad / SSD_BLK, d.G * b.nslices, d.max_chunks);
  const size_t lds = lds_bwd_row(sizeof(T) == 2 ? 1 : 0, d);
  ensure_lds(k_bwd_row<T, PT, NT>, lds);
  hipLaunchKernelGGL((k_bwd_row<T, PT, NT>), grid, dim3(256), lds, s, d, b, make_common<T>(d, b, in, dy),
                     reinterpret_cast<T*>(dC));
  return hipGetLastError();
}

template <typename T, int PT>
hipError_t bwd_row_n(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy, void* dC,
                            hipStream_t s) {
  switch (d.Npad / 32) {
    case 1: return bwd_row_t<T, PT, 1>(d, b, in, dy, dC, s);
    case 2: return bwd_row_t<T, PT, 2>(d, b, in, dy, dC, s);
    default: return bwd_row_t<T, PT, 4>(d, b, in, dy, dC, s);
  }
}

template <typename T>
hipError_t bwd_row_d(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy, void* dC,
                            hipStream_t s) {
  switch (d.Ppad / 32) {
    case 1: return bwd_row_n<T, 1>(d, b, in, dy, dC, s);
    case 2: return bwd_row_n<T, 2>(d, b, in, dy, dC, s);
    default: return bwd_row_n<T, 4>(d, b, in, dy, dC, s);
  }
}


