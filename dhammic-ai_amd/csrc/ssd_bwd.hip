// Backward of the chunked SSD scan: dtype dispatch of the column / row
// kernels (ssd_bwd_impl.h, instantiated in ssd_bwd_bf16.hip / ssd_bwd_f32.hip),
// the finish kernel and the LDS sizes the host checks.
#include "ssd_launch.h"

hipError_t launch_bwd_col_bf16(const SsdDims&, const SsdBufs&, const SsdIn&, const void*, void*, void*, hipStream_t);
hipError_t launch_bwd_col_f32(const SsdDims&, const SsdBufs&, const SsdIn&, const void*, void*, void*, hipStream_t);
hipError_t launch_bwd_row_bf16(const SsdDims&, const SsdBufs&, const SsdIn&, const void*, void*, hipStream_t);
hipError_t launch_bwd_row_f32(const SsdDims&, const SsdBufs&, const SsdIn&, const void*, void*, hipStream_t);

hipError_t launch_bwd_col(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy,
                          void* dx, void* dB, hipStream_t s) {
  return dtype == 1 ? launch_bwd_col_bf16(d, b, in, dy, dx, dB, s) : launch_bwd_col_f32(d, b, in, dy, dx, dB, s);
}

hipError_t launch_bwd_row(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy,
                          void* dC, hipStream_t s) {
  return dtype == 1 ? launch_bwd_row_bf16(d, b, in, dy, dC, s) : launch_bwd_row_f32(d, b, in, dy, dC, s);
}

// ---------------------------------------------------------------------------
// Finish: dcs per position, da = reverse in-chunk cumsum (the adjoint of the
// inclusive cumsum, ssd_scan.py:368), then ddt / per-token dA / dA partials.
// One wave per (chunk, head); lane L owns the PER = Qpad / 64 consecutive positions
// PER L .. PER L + PER - 1 and reads them with one load per array (with PER
// separate dword loads, the lines of the ~10 MB in flight per XCD were evicted
// between them and fetched up to four times).
// ---------------------------------------------------------------------------
template <int PER>
__device__ __forceinline__ void ld_per(const float* __restrict__ p, float (&o)[PER]) {
  if constexpr (PER == 4) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = v[e];
  } else if constexpr (PER == 2) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    o[0] = v.x;
    o[1] = v.y;
  } else {
#pragma unroll
    for (int e = 0; e < PER; ++e) o[e] = p[e];
  }
}

template <typename T, int PER>
__global__ void __launch_bounds__(256) k_bwd_finish(SsdDims d, SsdBufs bf, const ChunkInfo* __restrict__ chunks,
                                                    const float* __restrict__ Ah, const float* __restrict__ dt,
                                                    float* __restrict__ ddt, T* __restrict__ dA_tok,
                                                    float* __restrict__ da32) {
  // dt / ddt of the block's four heads are 16 contiguous bytes per position when H % 4 == 0: then
  // thread t moves position t's four values with one 16-byte access through LDS (the per-head
  // 4-byte accesses touch a line per lane, four times as many L2 requests)
  __shared__ float s_dt[4][256], s_ddt[4][256];
  const int c = blockIdx.x;
  const int w = threadIdx.x >> 6;
  const int h = blockIdx.y * 4 + w;
  const int lane = lane_id();
  if (h >= d.H) return;  // never taken when H % 4 == 0 (every wave of the block then has a head)
  const ChunkInfo ci = chunks[c];
  const int64_t ch = (int64_t)c * d.H + h;
  if (ci.len == 0) {
    if (lane == 0) bf.dA_part[ch] = 0.0f;
    return;
  }
  const bool vec_dt = d.a_mode == 0 && d.has_dt && (d.H & 3) == 0 && (reinterpret_cast<uintptr_t>(dt) & 15) == 0;
  const bool vec_ddt = vec_dt && ddt != nullptr && (reinterpret_cast<uintptr_t>(ddt) & 15) == 0;
  if (vec_dt) {
    const int tp = threadIdx.x;  // position; Qpad <= 256 = blockDim.x
    floatx4 q = {0.0f, 0.0f, 0.0f, 0.0f};
    if (tp < ci.len) q = *reinterpret_cast<const floatx4*>(dt + (ci.row0 + tp) * (int64_t)d.H + blockIdx.y * 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) s_dt[e][tp] = q[e];
    __syncthreads();
  }
  constexpr int per = PER;
  const int64_t base = ch * d.Qpad;
  const int64_t pstride = (int64_t)d.max_chunks * d.H * d.Qpad;  // between partial arrays
  const int l0 = lane * PER;
  float v[PER], t[PER];
  float esum = 0.0f;
  {
    // rowG partial k covers the rows of blocks >= k (column set k of the fused path starts at
    // column block k); the column / row path writes one partial. Rows below 64 k of partial k are
    // never written, so each position takes partial k only from its own block on: with PER = 3 a
    // lane's positions can straddle two blocks (lane 21 holds positions 63..65).
    // Terms (ssd_dA_skip): INTRA = rowG - colG (the segsum of L), CUMSUM = dcs_off (Y_off decay) and
    // -E + [last] sum E (state-build decay), CHUNK = [last] dtot (the chunk-to-chunk decay).
    const bool t_intra = !(d.dA_skip & 1), t_cs = !(d.dA_skip & 2);
    float x[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) x[e] = 0.0f;
    if (t_intra) {
      ld_per<PER>(bf.rowG + base + l0, x);
      for (int k = 1; k < bf.nrowg && k <= (l0 + PER - 1) / 64; ++k) {
        ld_per<PER>(bf.rowG + k * pstride + base + l0, t);
#pragma unroll
        for (int e = 0; e < PER; ++e) x[e] += (k <= (l0 + e) / 64) ? t[e] : 0.0f;
      }
      ld_per<PER>(bf.colG + base + l0, t);
#pragma unroll
      for (int e = 0; e < PER; ++e) x[e] -= t[e];
    }
    if (t_cs) {
      for (int k = 0; k < bf.ndcs; ++k) {
        ld_per<PER>(bf.dcs_off + k * pstride + base + l0, t);
#pragma unroll
        for (int e = 0; e < PER; ++e) x[e] += t[e];
      }
      ld_per<PER>(bf.eterm + base + l0, t);
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const bool ok = l0 + e < ci.len;
      const float et = t_cs ? t[e] : 0.0f;
      v[e] = ok ? x[e] - et : 0.0f;
      esum += ok ? et : 0.0f;
    }
  }
  for (int o = 32; o > 0; o >>= 1) esum += __shfl_xor(esum, o, 64);
  float dtot = 0.0f;
  if (!(d.dA_skip & 4))
    for (int k = 0; k < bf.npass_blk; ++k) dtot += bf.dtot_part[ch * bf.npass_blk + k];
  const int last = ci.len - 1;
#pragma unroll
  for (int e = 0; e < per; ++e)
    if (l0 + e == last) v[e] += esum + dtot;
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
  if (ddt && d.has_dt) ld_per<PER>(bf.xdx + base + l0, t);
#pragma unroll
  for (int e = 0; e < per; ++e) {
    const int l = l0 + e;
    if (l >= ci.len) continue;
    const float da = v[e] + excl;
    const int64_t row = ci.row0 + l;
    if (d.a_mode == 0) {
      const float dtv = vec_dt ? s_dt[w][l] : (d.has_dt ? dt[row * d.H + h] : 1.0f);
      if (vec_ddt) s_ddt[w][l] = t[e] + Ah[h] * da;
      else if (ddt && d.has_dt) ddt[row * d.H + h] = t[e] + Ah[h] * da;
      dAp += dtv * da;
    } else {
      // per-token decay (with dt: the trapezoidal mode's scan, where a does not depend on dt)
      if (dA_tok) dA_tok[row * d.H + h] = from_f<T>(da);
      if (da32) da32[row * d.H + h] = da;
      if (ddt && d.has_dt) ddt[row * d.H + h] = t[e];
    }
  }
  for (int o = 32; o > 0; o >>= 1) dAp += __shfl_xor(dAp, o, 64);
  if (lane == 0) bf.dA_part[ch] = dAp;
  if (vec_ddt) {
    __syncthreads();
    const int tp = threadIdx.x;
    if (tp < ci.len) {
      floatx4 q;
#pragma unroll
      for (int e = 0; e < 4; ++e) q[e] = s_ddt[e][tp];
      *reinterpret_cast<floatx4*>(ddt + (ci.row0 + tp) * (int64_t)d.H + blockIdx.y * 4) = q;
    }
  }
}

size_t lds_bwd_col(int dtype, const SsdDims& d) {
  const size_t es = dtype == 1 ? 2 : 4;
  const size_t NP = d.Npad + 16 / es, PP = d.Ppad + 16 / es, BP = SSD_BLK + 16 / es;
  const size_t tiles = (d.Ppad > d.Npad ? d.Ppad : d.Npad) / 32;
  const size_t fixed = sizeof(float) * (2 * d.Qpad + 4 * SSD_BLK) + es * (SSD_BLK * NP + SSD_BLK * PP);
  const size_t regA = es * (SSD_BLK * NP + SSD_BLK * PP + d.Ppad * BP + d.Npad * BP);
  const size_t regB = es * (d.Ppad * NP + d.Npad * PP) + 2 * tiles * 4096;
  return fixed + (regA > regB ? regA : regB);
}

size_t lds_bwd_row(int dtype, const SsdDims& d) {
  const size_t es = dtype == 1 ? 2 : 4;
  const size_t NP = d.Npad + 16 / es, PP = d.Ppad + 16 / es, BP = SSD_BLK + 16 / es;
  const size_t fixed = sizeof(float) * (2 * d.Qpad + 4 * SSD_BLK) + es * (SSD_BLK * NP + SSD_BLK * PP);
  const size_t regA = es * (SSD_BLK * NP + SSD_BLK * PP + d.Npad * BP);
  const size_t regB = es * (d.Npad * PP) + 2 * (d.Npad / 32) * 4096;
  return fixed + (regA > regB ? regA : regB);
}

template <int PER>
static void bwd_finish_launch(int dtype, dim3 grid, const SsdDims& d, const SsdBufs& b, const float* Ah,
                              const float* dt, float* ddt, void* dA_tok, float* da32, hipStream_t s) {
  if (dtype == 1)
    hipLaunchKernelGGL((k_bwd_finish<bf16, PER>), grid, dim3(256), 0, s, d, b, b.chunks, Ah, dt, ddt,
                       reinterpret_cast<bf16*>(dA_tok), da32);
  else
    hipLaunchKernelGGL((k_bwd_finish<float, PER>), grid, dim3(256), 0, s, d, b, b.chunks, Ah, dt, ddt,
                       reinterpret_cast<float*>(dA_tok), da32);
}

hipError_t launch_bwd_finish(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, float* ddt,
                             void* dA_tok, float* da32, hipStream_t s) {
  dim3 grid(d.max_chunks, (d.H + 3) / 4);
  const float* Ah = d.a_mode == 0 ? reinterpret_cast<const float*>(in.A) : nullptr;
  switch (d.Qpad / 64) {
    case 1: bwd_finish_launch<1>(dtype, grid, d, b, Ah, in.dt, ddt, dA_tok, da32, s); break;
    case 2: bwd_finish_launch<2>(dtype, grid, d, b, Ah, in.dt, ddt, dA_tok, da32, s); break;
    case 3: bwd_finish_launch<3>(dtype, grid, d, b, Ah, in.dt, ddt, dA_tok, da32, s); break;
    default: bwd_finish_launch<4>(dtype, grid, d, b, Ah, in.dt, ddt, dA_tok, da32, s);
  }
  return hipGetLastError();
}
