// Gated RMSNorm epilogue over the nheads*headdim channels of each token:
//   out = y * rsqrt(mean(y^2) + eps) * w * silu(z)
// (r2/dhammic-ai/src/mamba_base_engine.py:191 with FusedRMSNormModule,
// r2/dhammic-ai/src/kernels/rmsnorm.py:222-235; backward derivation as in
// rmsnorm.py:16-40 with the silu gate folded in).
//
// bf16 rows of HP = nheads*headdim channels: a block of 256 threads holds a
// row in registers, thread t owning the 8-element vectors t, t + 256, ...
// (HP <= 256 * 8 * VPT); every input is read once and every output written
// once, 16 bytes per access. dw is accumulated per thread over the rows a
// block walks (each thread owns fixed channels) and the per-block partials are
// summed by k_reduce_rows.
// fp32 rows (the small-shape test path) use the scalar kernels below.
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

// ---------------------------------------------------------------------------
// bf16, vectorised: thread t owns channels 8 * (t + 256 q) .. +7, q < VPT.
// ---------------------------------------------------------------------------
template <int VPT>
__global__ void __launch_bounds__(256) k_gated_norm_fwd_v(int64_t R, int HP, float eps, const bf16* __restrict__ ypre,
                                                          const bf16* __restrict__ z, const float* __restrict__ w,
                                                          bf16* __restrict__ y, float* __restrict__ rstd) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int nv = HP / 8;
  bf16x8 yv[VPT], zv[VPT];
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int v = threadIdx.x + 256 * q;
    if (v < nv) {
      yv[q] = *reinterpret_cast<const bf16x8*>(ypre + r * HP + 8 * v);
      zv[q] = *reinterpret_cast<const bf16x8*>(z + r * HP + 8 * v);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int q = 0; q < VPT; ++q)
    if (threadIdx.x + 256 * q < nv)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)yv[q][e] * (float)yv[q][e];
  ss = block_sum(ss, red);
  const float rs = rsqrtf(ss / (float)HP + eps);
  if (threadIdx.x == 0) rstd[r] = rs;
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int v = threadIdx.x + 256 * q;
    if (v >= nv) continue;
    const floatx4 w0 = *reinterpret_cast<const floatx4*>(w + 8 * v);
    const floatx4 w1 = *reinterpret_cast<const floatx4*>(w + 8 * v + 4);
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float we = e < 4 ? w0[e] : w1[e - 4];
      o[e] = (bf16)((float)yv[q][e] * rs * we * silu_f((float)zv[q][e]));
    }
    *reinterpret_cast<bf16x8*>(y + r * HP + 8 * v) = o;
  }
}

// Per row: g = dout*w*silu(z); dy = rs*g - y*rs^3*(g.y)/HP; dz = dout*y*rs*w*silu'(z);
// dw partial per block (the block's rows), one row of HP floats per block.
template <int VPT>
__global__ void __launch_bounds__(256) k_gated_norm_bwd_v(int64_t R, int HP, const bf16* __restrict__ ypre,
                                                          const bf16* __restrict__ z, const float* __restrict__ w,
                                                          const float* __restrict__ rstd, const bf16* __restrict__ dout,
                                                          bf16* __restrict__ dy, bf16* __restrict__ dz,
                                                          float* __restrict__ dw_part) {
  __shared__ float red[4];
  const int nv = HP / 8;
  float dwa[VPT][8];
  float wv[VPT][8];
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int v = threadIdx.x + 256 * q;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dwa[q][e] = 0.0f;
      wv[q][e] = v < nv ? w[8 * v + e] : 0.0f;
    }
  }
  for (int64_t r = blockIdx.x; r < R; r += gridDim.x) {
    bf16x8 yv[VPT], zv[VPT], dv[VPT];
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      const int v = threadIdx.x + 256 * q;
      if (v < nv) {
        yv[q] = *reinterpret_cast<const bf16x8*>(ypre + r * HP + 8 * v);
        zv[q] = *reinterpret_cast<const bf16x8*>(z + r * HP + 8 * v);
        dv[q] = *reinterpret_cast<const bf16x8*>(dout + r * HP + 8 * v);
      }
    }
    const float rs = rstd[r];
    float sg[VPT][8];
    float dot = 0.0f;
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      if (threadIdx.x + 256 * q >= nv) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float zf = (float)zv[q][e];
        sg[q][e] = 1.0f / (1.0f + __expf(-zf));
        dot += (float)dv[q][e] * wv[q][e] * zf * sg[q][e] * (float)yv[q][e];
      }
    }
    dot = block_sum(dot, red);
    const float coef = rs * rs * rs * dot / (float)HP;
#pragma unroll
    for (int q = 0; q < VPT; ++q) {
      const int v = threadIdx.x + 256 * q;
      if (v >= nv) continue;
      bf16x8 oy, oz;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float yf = (float)yv[q][e], zf = (float)zv[q][e], df = (float)dv[q][e];
        const float s = sg[q][e], sl = zf * s;
        const float g = df * wv[q][e] * sl;
        oy[e] = (bf16)(rs * g - yf * coef);
        oz[e] = (bf16)(df * yf * rs * wv[q][e] * s * (1.0f + zf * (1.0f - s)));
        dwa[q][e] += df * yf * rs * sl;
      }
      *reinterpret_cast<bf16x8*>(dy + r * HP + 8 * v) = oy;
      *reinterpret_cast<bf16x8*>(dz + r * HP + 8 * v) = oz;
    }
  }
#pragma unroll
  for (int q = 0; q < VPT; ++q) {
    const int v = threadIdx.x + 256 * q;
    if (v >= nv) continue;
    floatx4 a, b;
    a[0] = dwa[q][0]; a[1] = dwa[q][1]; a[2] = dwa[q][2]; a[3] = dwa[q][3];
    b[0] = dwa[q][4]; b[1] = dwa[q][5]; b[2] = dwa[q][6]; b[3] = dwa[q][7];
    *reinterpret_cast<floatx4*>(dw_part + (int64_t)blockIdx.x * HP + 8 * v) = a;
    *reinterpret_cast<floatx4*>(dw_part + (int64_t)blockIdx.x * HP + 8 * v + 4) = b;
  }
}

// ---------------------------------------------------------------------------
// Scalar kernels (fp32 rows, or widths that are not a multiple of 8).
// ---------------------------------------------------------------------------
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

// Vectors per thread of the vectorised kernels for this row width (0: not vectorisable).
static int norm_vpt(int dtype, const SsdDims& d) {
  const int HP = d.H * d.P;
  if (dtype != 1 || HP % 8 || !d.vec_x) return 0;
  const int nv = HP / 8;
  if (nv <= 256) return 1;
  if (nv <= 512) return 2;
  if (nv <= 1024) return 4;
  if (nv <= 2048) return 8;
  return 0;
}

hipError_t launch_gated_norm_fwd(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, void* y,
                                 hipStream_t s) {
  const int HP = d.H * d.P;
  const dim3 grid((unsigned)d.R);
  const bf16* yp = reinterpret_cast<const bf16*>(b.ypre);
  const bf16* zp = reinterpret_cast<const bf16*>(in.z);
  bf16* yo = reinterpret_cast<bf16*>(y);
  switch (norm_vpt(dtype, d)) {
    case 1: hipLaunchKernelGGL(k_gated_norm_fwd_v<1>, grid, dim3(256), 0, s, d.R, HP, d.eps, yp, zp, in.w, yo, b.rstd); break;
    case 2: hipLaunchKernelGGL(k_gated_norm_fwd_v<2>, grid, dim3(256), 0, s, d.R, HP, d.eps, yp, zp, in.w, yo, b.rstd); break;
    case 4: hipLaunchKernelGGL(k_gated_norm_fwd_v<4>, grid, dim3(256), 0, s, d.R, HP, d.eps, yp, zp, in.w, yo, b.rstd); break;
    case 8: hipLaunchKernelGGL(k_gated_norm_fwd_v<8>, grid, dim3(256), 0, s, d.R, HP, d.eps, yp, zp, in.w, yo, b.rstd); break;
    default:
      if (dtype == 1)
        hipLaunchKernelGGL(k_gated_norm_fwd<bf16>, grid, dim3(256), 0, s, d.R, HP, d.eps, yp, zp, in.w, yo, b.rstd);
      else
        hipLaunchKernelGGL(k_gated_norm_fwd<float>, grid, dim3(256), 0, s, d.R, HP, d.eps,
                           reinterpret_cast<const float*>(b.ypre), reinterpret_cast<const float*>(in.z), in.w,
                           reinterpret_cast<float*>(y), b.rstd);
  }
  return hipGetLastError();
}

hipError_t launch_gated_norm_bwd(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in,
                                 const void* dout, void* dz, hipStream_t s) {
  const int HP = d.H * d.P;
  const dim3 grid(b.norm_blocks);
  const bf16* yp = reinterpret_cast<const bf16*>(b.ypre);
  const bf16* zp = reinterpret_cast<const bf16*>(in.z);
  const bf16* dp = reinterpret_cast<const bf16*>(dout);
  bf16* dyo = reinterpret_cast<bf16*>(b.dyp);
  bf16* dzo = reinterpret_cast<bf16*>(dz);
  switch (norm_vpt(dtype, d)) {
    case 1: hipLaunchKernelGGL(k_gated_norm_bwd_v<1>, grid, dim3(256), 0, s, d.R, HP, yp, zp, in.w, b.rstd, dp, dyo, dzo, b.dw_part); break;
    case 2: hipLaunchKernelGGL(k_gated_norm_bwd_v<2>, grid, dim3(256), 0, s, d.R, HP, yp, zp, in.w, b.rstd, dp, dyo, dzo, b.dw_part); break;
    case 4: hipLaunchKernelGGL(k_gated_norm_bwd_v<4>, grid, dim3(256), 0, s, d.R, HP, yp, zp, in.w, b.rstd, dp, dyo, dzo, b.dw_part); break;
    case 8: hipLaunchKernelGGL(k_gated_norm_bwd_v<8>, grid, dim3(256), 0, s, d.R, HP, yp, zp, in.w, b.rstd, dp, dyo, dzo, b.dw_part); break;
    default: {
      const size_t lds = sizeof(float) * HP;
      if (dtype == 1)
        hipLaunchKernelGGL(k_gated_norm_bwd<bf16>, grid, dim3(256), lds, s, d.R, HP, yp, zp, in.w, b.rstd, dp, dyo,
                           dzo, b.dw_part);
      else
        hipLaunchKernelGGL(k_gated_norm_bwd<float>, grid, dim3(256), lds, s, d.R, HP,
                           reinterpret_cast<const float*>(b.ypre), reinterpret_cast<const float*>(in.z), in.w,
                           b.rstd, reinterpret_cast<const float*>(dout), reinterpret_cast<float*>(b.dyp),
                           reinterpret_cast<float*>(dz), b.dw_part);
    }
  }
  return hipGetLastError();
}
