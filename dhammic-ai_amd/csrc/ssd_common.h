// Device-side building blocks shared by the SSD kernels (gfx950, wave64).
//
// MFMA tiling: one wave computes a 32x32 fp32 tile with
//   bf16: v_mfma_f32_32x32x16_bf16  (K = 16 per instruction)
//   fp32: 8 x v_mfma_f32_32x32x2_f32 (K = 16 per group of eight)
// Operand fragments: lane l supplies A[l%32][k0 + (l/32)*8 + t] and
// B[k0 + (l/32)*8 + t][l%32] for t = 0..7, i.e. eight consecutive k per lane,
// so every operand is kept k-contiguous in LDS (or global) and read as one
// 16-byte vector (bf16) or two (fp32). For fp32 the eight values of a lane are
// spread over eight K=2 instructions; A and B use the same spreading, so the
// sum over k is unchanged.
// Accumulator layout (both variants): lane l, register v holds
//   row 8*(v/4) + 4*(l/32) + v%4, column l%32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define SSD_WAVE 64
#define SSD_LO (-20.0f)
#define SSD_HI (20.0f)

// exp(clamp(v, -20, 20)): every decay exponent of the reference path
// (r2/dhammic-ai/src/kernels/ssd_scan.py:53-54, :116, :212).
__device__ __forceinline__ float exp_clamp(float v) {
  return __expf(fminf(fmaxf(v, SSD_LO), SSD_HI));
}
// Strict pass mask of the clamp backward (ssd_scan.py:192, :230).
__device__ __forceinline__ float clamp_pass(float v) {
  return (v > SSD_LO && v < SSD_HI) ? 1.0f : 0.0f;
}

template <typename T> __device__ __forceinline__ float to_f(T v);
template <> __device__ __forceinline__ float to_f<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f<bf16>(bf16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f(float v);
template <> __device__ __forceinline__ float from_f<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float v) { return (bf16)v; }

template <typename T> struct Frag;
template <> struct Frag<bf16> { bf16x8 v; };
template <> struct Frag<float> { float v[8]; };

// Eight consecutive elements at p (16-byte aligned for bf16, 32-byte for fp32 in LDS).
__device__ __forceinline__ Frag<bf16> ld_frag(const bf16* p) {
  Frag<bf16> f;
  f.v = *reinterpret_cast<const bf16x8*>(p);
  return f;
}
__device__ __forceinline__ Frag<float> ld_frag(const float* p) {
  Frag<float> f;
  floatx4 a = *reinterpret_cast<const floatx4*>(p);
  floatx4 b = *reinterpret_cast<const floatx4*>(p + 4);
  f.v[0] = a[0]; f.v[1] = a[1]; f.v[2] = a[2]; f.v[3] = a[3];
  f.v[4] = b[0]; f.v[5] = b[1]; f.v[6] = b[2]; f.v[7] = b[3];
  return f;
}

// Eight consecutive fp32 values (global, 16-byte aligned) converted to T.
template <typename T> __device__ __forceinline__ Frag<T> ld_frag_f32(const float* p);
template <> __device__ __forceinline__ Frag<float> ld_frag_f32<float>(const float* p) {
  return ld_frag(p);
}
template <> __device__ __forceinline__ Frag<bf16> ld_frag_f32<bf16>(const float* p) {
  floatx4 a = *reinterpret_cast<const floatx4*>(p);
  floatx4 b = *reinterpret_cast<const floatx4*>(p + 4);
  Frag<bf16> f;
  f.v[0] = (bf16)a[0]; f.v[1] = (bf16)a[1]; f.v[2] = (bf16)a[2]; f.v[3] = (bf16)a[3];
  f.v[4] = (bf16)b[0]; f.v[5] = (bf16)b[1]; f.v[6] = (bf16)b[2]; f.v[7] = (bf16)b[3];
  return f;
}

__device__ __forceinline__ void mma(floatx16& acc, const Frag<bf16>& a, const Frag<bf16>& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(floatx16& acc, const Frag<float>& a, const Frag<float>& b) {
#pragma unroll
  for (int t = 0; t < 8; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.v[t], b.v[t], acc, 0, 0, 0);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
// Row (0..31) of accumulator register v for this lane; the column is lane % 32.
__device__ __forceinline__ int acc_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

__device__ __forceinline__ void zero(floatx16& a) {
#pragma unroll
  for (int v = 0; v < 16; ++v) a[v] = 0.0f;
}

// acc(32x32) += A[32 x K] * B[K x 32] with A(i, k) = a[i*lda + k] and
// B(k, j) = b[j*ldb + k] (both k-contiguous), K a multiple of 16.
template <typename T>
__device__ __forceinline__ void mma_tile(floatx16& acc, const T* a, int lda, const T* b, int ldb, int K) {
  const int lane = lane_id();
  const T* ap = a + (lane & 31) * lda + (lane >> 5) * 8;
  const T* bp = b + (lane & 31) * ldb + (lane >> 5) * 8;
  for (int k0 = 0; k0 < K; k0 += 16) {
    Frag<T> fa = ld_frag(ap + k0);
    Frag<T> fb = ld_frag(bp + k0);
    mma(acc, fa, fb);
  }
}

// Sum over the 32 columns of each row: after the call every lane holds, for
// each of its 16 registers, the full row sum (lanes of one 32-lane half agree).
__device__ __forceinline__ float row_reduce32(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 8, 64);
  v += __shfl_xor(v, 16, 64);
  return v;
}

// Round x up to a multiple of m.
__host__ __device__ __forceinline__ int round_up(int x, int m) { return (x + m - 1) / m * m; }

// LDS row pitch (elements) for a k-contiguous tile of width w: +16 bytes so
// consecutive rows start in different banks.
template <typename T> __host__ __device__ constexpr int lds_pitch(int w) { return w + 16 / (int)sizeof(T); }

// One entry of the chunk table: chunk k of sequence `seq` covers rows
// [row0, row0 + len) of the packed token axis; `first` marks k == 0.
struct ChunkInfo {
  int32_t row0;
  int32_t len;
  int32_t seq;
  int32_t idx_in_seq;
};
