// Deterministic reductions of per-block partials (fixed summation order, no
// atomics), so repeated backward calls are bitwise identical.
#include "ssd_launch.h"

// out[i] = sum_s part[s][i], s = 0..nslices-1 in order.
template <typename T>
__global__ void k_reduce_slices(int64_t nelem, int nslices, const float* __restrict__ part, T* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nelem; i += (int64_t)gridDim.x * blockDim.x) {
    float acc = 0.0f;
    for (int s = 0; s < nslices; ++s) acc += part[(int64_t)s * nelem + i];
    out[i] = from_f<T>(acc);
  }
}

hipError_t launch_reduce_slices(int dtype, int64_t nelem, int nslices, const float* part, void* out,
                                hipStream_t s) {
  int64_t blocks64 = (nelem + 255) / 256;
  if (blocks64 > 65536) blocks64 = 65536;
  if (blocks64 < 1) blocks64 = 1;
  const unsigned blocks = (unsigned)blocks64;
  if (dtype == 1)
    hipLaunchKernelGGL(k_reduce_slices<bf16>, dim3(blocks), dim3(256), 0, s, nelem, nslices, part,
                       reinterpret_cast<bf16*>(out));
  else
    hipLaunchKernelGGL(k_reduce_slices<float>, dim3(blocks), dim3(256), 0, s, nelem, nslices, part,
                       reinterpret_cast<float*>(out));
  return hipGetLastError();
}

// out[k] = sum_b part[b][k]: block of 1024 threads = 16 columns x 64 row groups
// (width / 16 blocks, so a 4096-wide row fills the chip); row group g sums rows
// g, g + 64, ... in order, then the group sums are added in a fixed tree order
// (deterministic).
__global__ void __launch_bounds__(1024) k_reduce_rows(int nblocks, int width, const float* __restrict__ part,
                                                      float* __restrict__ out) {
  __shared__ float red[64][16];
  const int col = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int k = blockIdx.x * 16 + col;
  float acc = 0.0f;
  if (k < width)
    for (int b = grp; b < nblocks; b += 64) acc += part[(int64_t)b * width + k];
  red[grp][col] = acc;
  __syncthreads();
  for (int o = 32; o > 0; o >>= 1) {
    if (grp < o) red[grp][col] += red[grp + o][col];
    __syncthreads();
  }
  if (grp == 0 && k < width) out[k] = red[0][col];
}

hipError_t launch_reduce_rows(int nblocks, int width, const float* part, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_reduce_rows, dim3((width + 15) / 16), dim3(1024), 0, s, nblocks, width, part, out);
  return hipGetLastError();
}

// The backward's last launch: blocks [0, nh) reduce the per-head dA / dD partials of head blockIdx.x
// (threads 0-255: over valid chunks, strided by 256, then a fixed tree), blocks [nh, nh + nr) the norm-weight partials of 16
// columns each (the order of k_reduce_rows). The two reductions are independent; one launch instead of
// two saves a dispatch on the backward's critical path.
__global__ void __launch_bounds__(1024) k_reduce_tail(SsdDims d, const ChunkInfo* __restrict__ chunks,
                                                     const float* __restrict__ dA_part,
                                                     const float* __restrict__ dD_part, float* __restrict__ dA,
                                                     float* __restrict__ dD, int nh, int nblocks, int width,
                                                     const float* __restrict__ part, float* __restrict__ out) {
  __shared__ float ra[256], rd[256];
  __shared__ float red[64][16];
  const int t = threadIdx.x;
  if ((int)blockIdx.x < nh) {
    const int h = blockIdx.x;
    const int nrb = d.Qpad / SSD_BLK;
    if (t < 256) {
      float a = 0.0f, dd = 0.0f;
      for (int c = t; c < d.max_chunks; c += 256) {
        const int len = chunks[c].len;
        if (len == 0) continue;
        a += dA_part[(int64_t)c * d.H + h];
        for (int j = 0; j < nrb; ++j)
          if (j * SSD_BLK < len) dd += dD_part[((int64_t)c * d.H + h) * nrb + j];
      }
      ra[t] = a;
      rd[t] = dd;
    }
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (t < o) {
        ra[t] += ra[t + o];
        rd[t] += rd[t + o];
      }
      __syncthreads();
    }
    if (t == 0) {
      if (dA) dA[h] = ra[0];
      if (dD) dD[h] = rd[0];
    }
    return;
  }
  const int col = t & 15, grp = t >> 4;
  const int k = ((int)blockIdx.x - nh) * 16 + col;
  float acc = 0.0f;
  if (k < width)
    for (int b = grp; b < nblocks; b += 64) acc += part[(int64_t)b * width + k];
  red[grp][col] = acc;
  __syncthreads();
  for (int o = 32; o > 0; o >>= 1) {
    if (grp < o) red[grp][col] += red[grp + o][col];
    __syncthreads();
  }
  if (grp == 0 && k < width) out[k] = red[0][col];
}

hipError_t launch_reduce_tail(const SsdDims& d, const SsdBufs& b, float* dA_head, float* dD, int nblocks, int width,
                              const float* part, float* out, hipStream_t s) {
  const int nh = (dA_head || dD) ? d.H : 0;
  const int nr = out ? (width + 15) / 16 : 0;
  if (nh + nr == 0) return hipSuccess;
  hipLaunchKernelGGL(k_reduce_tail, dim3(nh + nr), dim3(1024), 0, s, d, b.chunks, b.dA_part, b.dD_part, dA_head, dD,
                     nh, nblocks, width, part, out);
  return hipGetLastError();
}
