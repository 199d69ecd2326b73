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
      // rowG partial k covers the rows of blocks >= k (column set k of the fused
      // path starts at column block k); the column / row path writes one partial
      float rg = 0.0f;
      for (int k = 0; k < bf.nrowg && k <= l / 64; ++k)
        rg += bf.rowG[(int64_t)k * d.max_chunks * d.H * d.Qpad + base + l];
      float off = 0.0f;
      for (int k = 0; k < bf.ndcs; ++k) off += bf.dcs_off[(int64_t)k * d.max_chunks * d.H * d.Qpad + base + l];
      x = rg - bf.colG[base + l] + off - bf.eterm[base + l];
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
