// Gated RMSNorm epilogue over the nheads*headdim channels of each token:
//   out = y * rsqrt(mean(y^2) + eps) * w * silu(z)
// (r2/dhammic-ai/src/mamba_base_engine.py:191 with FusedRMSNormModule,
// r2/dhammic-ai/src/kernels/rmsnorm.py:222-235; backward derivation as in
// rmsnorm.py:16-40 with the silu gate folded in).
#include "ssd_launch.h"

__device__ __forceinline__ float silu_f(float z) { return z / (1.0f + __expf(-z)); }

// Sum over the block (256 threads) in a fixed order.
__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

template <typename T>
__global__ void __launch_bounds__(256) k_gated_norm_fwd(int64_t R, int HP, float eps, const T* __restrict__ ypre,
                                                        const T* __restrict__ z, const float* __restrict__ w,
                                                        T* __restrict__ y, float* __restrict__ rstd) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const T* yr = ypre + r * HP;
  float ss = 0.0f;
  for (int k = threadIdx.x; k < HP; k += blockDim.x) {
    const float v = to_f(yr[k]);
    ss += v * v;
  }
  ss = block_sum(ss, red);
  const float rs = rsqrtf(ss / (float)HP + eps);
  if (threadIdx.x == 0) rstd[r] = rs;
  const T* zr = z + r * HP;
  T* outr = y + r * HP;
  for (int k = threadIdx.x; k < HP; k += blockDim.x)
    outr[k] = from_f<T>(to_f(yr[k]) * rs * w[k] * silu_f(to_f(zr[k])));
}

// Per row: g = dout*w*silu(z); dy = rs*g - y*rs^3*(g.y)/HP; dz = dout*y*rs*w*silu'(z);
// dw accumulated per block over its rows in LDS, written as one partial row.
template <typename T>
__global__ void __launch_bounds__(256) k_gated_norm_bwd(int64_t R, int HP, const T* __restrict__ ypre,
                                                        const T* __restrict__ z, const float* __restrict__ w,
                                                        const float* __restrict__ rstd, const T* __restrict__ dout,
                                                        T* __restrict__ dy, T* __restrict__ dz,
                                                        float* __restrict__ dw_part) {
  extern __shared__ float s_dw[];  // [HP]
  __shared__ float red[4];
  for (int k = threadIdx.x; k < HP; k += blockDim.x) s_dw[k] = 0.0f;
  for (int64_t r = blockIdx.x; r < R; r += gridDim.x) {
    const T* yr = ypre + r * HP;
    const T* zr = z + r * HP;
    const T* dr = dout + r * HP;
    const float rs = rstd[r];
    float dot = 0.0f;
    for (int k = threadIdx.x; k < HP; k += blockDim.x)
      dot += to_f(dr[k]) * w[k] * silu_f(to_f(zr[k])) * to_f(yr[k]);
    dot = block_sum(dot, red);
    const float coef = rs * rs * rs * dot / (float)HP;
    for (int k = threadIdx.x; k < HP; k += blockDim.x) {
      const float yv = to_f(yr[k]), zv = to_f(zr[k]), dv = to_f(dr[k]);
      const float sg = 1.0f / (1.0f + __expf(-zv));
      const float sl = zv * sg;
      const float g = dv * w[k] * sl;
      dy[r * HP + k] = from_f<T>(rs * g - yv * coef);
      dz[r * HP + k] = from_f<T>(dv * yv * rs * w[k] * sg * (1.0f + zv * (1.0f - sg)));
      s_dw[k] += dv * yv * rs * sl;
    }
  }
  __syncthreads();
  for (int k = threadIdx.x; k < HP; k += blockDim.x) dw_part[(int64_t)blockIdx.x * HP + k] = s_dw[k];
}

hipError_t launch_gated_norm_fwd(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, void* y,
                                 hipStream_t s) {
  const int HP = d.H * d.P;
  if (dtype == 1)
    hipLaunchKernelGGL(k_gated_norm_fwd<bf16>, dim3((unsigned)d.R), dim3(256), 0, s, d.R, HP, d.eps,
                       reinterpret_cast<const bf16*>(b.ypre), reinterpret_cast<const bf16*>(in.z), in.w,
                       reinterpret_cast<bf16*>(y), b.rstd);
  else
    hipLaunchKernelGGL(k_gated_norm_fwd<float>, dim3((unsigned)d.R), dim3(256), 0, s, d.R, HP, d.eps,
                       reinterpret_cast<const float*>(b.ypre), reinterpret_cast<const float*>(in.z), in.w,
                       reinterpret_cast<float*>(y), b.rstd);
  return hipGetLastError();
}

hipError_t launch_gated_norm_bwd(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in,
                                 const void* dout, void* dz, hipStream_t s) {
  const int HP = d.H * d.P;
  const size_t lds = sizeof(float) * HP;
  if (dtype == 1)
    hipLaunchKernelGGL(k_gated_norm_bwd<bf16>, dim3(b.norm_blocks), dim3(256), lds, s, d.R, HP,
                       reinterpret_cast<const bf16*>(b.ypre), reinterpret_cast<const bf16*>(in.z), in.w, b.rstd,
                       reinterpret_cast<const bf16*>(dout), reinterpret_cast<bf16*>(b.dyp),
                       reinterpret_cast<bf16*>(dz), b.dw_part);
  else
    hipLaunchKernelGGL(k_gated_norm_bwd<float>, dim3(b.norm_blocks), dim3(256), lds, s, d.R, HP,
                       reinterpret_cast<const float*>(b.ypre), reinterpret_cast<const float*>(in.z), in.w, b.rstd,
                       reinterpret_cast<const float*>(dout), reinterpret_cast<float*>(b.dyp),
                       reinterpret_cast<float*>(dz), b.dw_part);
  return hipGetLastError();
}
