// bf16 LDS tiles and MFMA operand access for gfx950 (wave64).
//
// A tile is ROWS x W bf16 (W = 32, 64 or 128 elements per row), stored row
// after row with a pitch of PI elements. The default PI = W + 8 starts
// consecutive rows 16 bytes apart in the bank space, so eight consecutive rows
// read at the same column chunk (the k-contiguous operand read of
// v_mfma_f32_32x32x16_bf16) hit eight different bank groups. Tiles read only
// through ds_read_b64_tr_b16 (four consecutive rows, 32 bytes each) use
// PI = W + 16 instead: rows then start 32 bytes apart modulo 128 and the four
// rows never share a bank. Every address is a per-lane row offset plus a
// compile-time or wave-uniform part.
//
// Operand conventions of v_mfma_f32_32x32x16_bf16 (used throughout):
//   A[i][k]: lane L supplies i = L % 32, k = 8 * (L / 32) + t, t = 0..7
//   B[k][j]: lane L supplies j = L % 32, k = 8 * (L / 32) + t
//   D[i][j]: lane L, register v holds i = 8 * (v / 4) + 4 * (L / 32) + v % 4, j = L % 32
//
// ds_read_b64_tr_b16 (measured lane layout): inside each 16-lane group, lane q
// receives element q % 4 of the 8-byte loads of lanes 4e + q / 4, e = 0..3.
// So if lane q of a group loads row kb + q / 4, columns m0 + 4 * (q % 4) .. +3,
// lane q ends up holding column m0 + q of rows kb .. kb + 3: a k-contiguous
// operand read from a tile whose rows are the contraction index.
#pragma once

#include "ssd_common.h"

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int W>
__host__ __device__ constexpr int tpitch() {
  static_assert(W == 32 || W == 64 || W == 128, "tile width");
  return W + 8;
}
// Pitch of a tile read only with ds_read_b64_tr_b16.
template <int W>
__host__ __device__ constexpr int tpitch_tr() {
  static_assert(W == 32 || W == 64 || W == 128, "tile width");
  return W + 16;
}
// Elements of a ROWS x W tile.
template <int ROWS, int W, int PI = tpitch<W>()>
__host__ __device__ constexpr int tsize() { return ROWS * PI; }

// Element offset of (row r, column k) in a W-wide tile.
template <int W, int PI = tpitch<W>()>
__device__ __forceinline__ int toff(int r, int k) {
  return r * PI + k;
}

// Eight consecutive columns k .. k+7 (k % 8 == 0) of row r.
template <int W, int PI = tpitch<W>()>
__device__ __forceinline__ bf16x8 tld8(const bf16* t, int r, int k) {
  return *reinterpret_cast<const bf16x8*>(t + toff<W, PI>(r, k));
}

// Four consecutive columns k .. k+3 (k % 4 == 0) of row r.
template <int W, int PI = tpitch<W>()>
__device__ __forceinline__ bf16x4 tld4(const bf16* t, int r, int k) {
  return *reinterpret_cast<const bf16x4*>(t + toff<W, PI>(r, k));
}

// The lane id as a value the compiler cannot treat as loop-invariant: address
// arithmetic derived from it is recomputed where used instead of being hoisted
// out of long loops (and kept live in registers across them).
__device__ __forceinline__ int opaque_lane() {
  int l = threadIdx.x & 63;
  asm volatile("" : "+v"(l));
  return l;
}

// Rows kb .. kb+3 of column m0 + (L % 16) (m0 % 16 == 0, kb % 4 == 0); L = lane id.
template <int W, int PI = tpitch<W>()>
__device__ __forceinline__ bf16x4 ttr4(const bf16* t, int kb, int m0, int L) {
  const int q = L & 15;
  const bf16* p = t + toff<W, PI>(kb + (q >> 2), m0 + ((q & 3) << 2));
  const shortx4 v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) shortx4*)(p));
  return __builtin_bit_cast(bf16x4, v);
}

// Makes v opaque to the optimizer at this point. Used at the top of long loops
// on loop-invariant bf16 register tiles: otherwise their bf16 -> fp32
// conversions are hoisted out of the loop and the tile takes twice the registers.
__device__ __forceinline__ void launder(bf16x8& v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ bf16x8 cat8(bf16x4 a, bf16x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// k-contiguous operand (A[i][k] with i = mbase + lane % 32, or B[k][j] with
// j = mbase + lane % 32), k = k0 + 8 * (lane / 32) + t, read from a tile whose
// row index is k and column index is i (or j).
template <int W, int PI = tpitch<W>()>
__device__ __forceinline__ bf16x8 ttr_std(const bf16* t, int k0, int mbase, int L) {
  const int h = L >> 5;
  const int m0 = mbase + (((L >> 4) & 1) << 4);
  return cat8(ttr4<W, PI>(t, k0 + 8 * h, m0, L), ttr4<W, PI>(t, k0 + 8 * h + 4, m0, L));
}

// Operand partner of an accumulator tile reused in place (see acc_frag): for
// MFMA step kk over the 32 rows k0 .. k0+31, lane L supplies the rows
// k0 + 16 kk + 8 (t / 4) + 4 (L / 32) + t % 4, the order in which the
// accumulator registers 8 kk .. 8 kk + 7 hold them.
template <int W, int PI = tpitch<W>()>
__device__ __forceinline__ bf16x8 ttr_perm(const bf16* t, int k0, int kk, int mbase, int L) {
  const int h = L >> 5;
  const int m0 = mbase + (((L >> 4) & 1) << 4);
  return cat8(ttr4<W, PI>(t, k0 + 16 * kk + 4 * h, m0, L), ttr4<W, PI>(t, k0 + 16 * kk + 8 + 4 * h, m0, L));
}

// Registers 8 kk .. 8 kk + 7 of an accumulator tile X, as bf16: used as the B
// operand this is B[k][j] = X[row(8 kk + t)][j]; used as the A operand it is
// A[i][k] = X[row(8 kk + t)][i] (X transposed). The partner operand must list
// its k in the same row order (ttr_perm).
__device__ __forceinline__ bf16x8 acc_frag(const floatx16& x, int kk) {
  bf16x8 f;
#pragma unroll
  for (int t = 0; t < 8; ++t) f[t] = (bf16)x[8 * kk + t];
  return f;
}

__device__ __forceinline__ void mfma(floatx16& acc, const bf16x8& a, const bf16x8& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
}

// 16 x 16 x 32 product into registers 4 I .. 4 I + 3 of acc (lane L holds column L % 16,
// rows 4 (L / 16) + 0..3 of the 16 x 16 tile).
template <int I>
__device__ __forceinline__ void mfma16(floatx16& acc, const bf16x8& a, const bf16x8& b) {
  floatx4 c = __builtin_shufflevector(acc, acc, 4 * I, 4 * I + 1, 4 * I + 2, 4 * I + 3);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[4 * I + e] = c[e];
}

// ---------------------------------------------------------------------------
// Global -> LDS staging of a ROWS x W bf16 tile from a row-major tensor, with
// rows >= nrows and columns >= width zero-filled. Thread t handles 16-byte
// vectors t, t + NTHR, ... (row-major order, so a wave reads whole rows).
// `vec` (uniform): 16-byte global loads are aligned (width, row stride and
// column offset multiples of 8 elements, 16-byte aligned base).
// ---------------------------------------------------------------------------
template <int ROWS, int W, int NTHR>
struct TileStage {
  static constexpr int NVEC = ROWS * W / 8;
  static constexpr int PER = (NVEC + NTHR - 1) / NTHR;
  bf16x8 v[PER];
};

template <int ROWS, int W, int NTHR>
__device__ __forceinline__ void tstage_load(TileStage<ROWS, W, NTHR>& s, const bf16* __restrict__ g, int64_t ld,
                                            int nrows, int width, bool vec) {
  constexpr int CPR = W / 8;
#pragma unroll
  for (int q = 0; q < TileStage<ROWS, W, NTHR>::PER; ++q) {
    const int id = threadIdx.x + q * NTHR;
    if (TileStage<ROWS, W, NTHR>::NVEC % NTHR == 0 || id < TileStage<ROWS, W, NTHR>::NVEC) {
      const int r = id / CPR, k = (id % CPR) * 8;
      const bf16* p = g + (int64_t)r * ld + k;
      bf16x8 v;
      if (r < nrows && vec && k < width) {
        v = *reinterpret_cast<const bf16x8*>(p);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (r < nrows && k + e < width) ? p[e] : (bf16)0.0f;
      }
      s.v[q] = v;
    }
  }
}

template <int ROWS, int W, int NTHR, int PI = tpitch<W>()>
__device__ __forceinline__ void tstage_store(const TileStage<ROWS, W, NTHR>& s, bf16* t) {
  constexpr int CPR = W / 8;
#pragma unroll
  for (int q = 0; q < TileStage<ROWS, W, NTHR>::PER; ++q) {
    const int id = threadIdx.x + q * NTHR;
    if (TileStage<ROWS, W, NTHR>::NVEC % NTHR == 0 || id < TileStage<ROWS, W, NTHR>::NVEC) {
      const int r = id / CPR, k = (id % CPR) * 8;
      *reinterpret_cast<bf16x8*>(t + toff<W, PI>(r, k)) = s.v[q];
    }
  }
}

// ---------------------------------------------------------------------------
// Raw buffer loads: the hardware range check returns zeros for an offset at or
// beyond the resource's size, so a masked load needs no branch. Loads issued
// in straight-line code (no per-lane branch around them) keep their vmcnt
// waits exact, which lets several stages of loads stay in flight.
// ---------------------------------------------------------------------------
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#define SSD_BUF_SIZE 0x7ffffff0
// Resource over [base, base + SSD_BUF_SIZE) bytes; base must be wave-uniform (it is
// read from the first active lane, so the descriptor lives in scalar registers and the
// loads need no per-lane descriptor loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
  const uint64_t v = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  void* u = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, SSD_BUF_SIZE, 0x00020000);
}
// 16 bytes at byte offset `off`, or zeros when `ok` is false.
__device__ __forceinline__ bf16x8 buf_ld16(__amdgpu_buffer_rsrc_t r, int off, bool ok) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, ok ? off : SSD_BUF_SIZE, 0, 0);
  return __builtin_bit_cast(bf16x8, v);
}
// One fp32 at byte offset `off`, or 0 when `ok` is false.
__device__ __forceinline__ float buf_ldf(__amdgpu_buffer_rsrc_t r, int off, bool ok) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, ok ? off : SSD_BUF_SIZE, 0, 0));
}

// Vector-only variant: 16-byte loads are valid (row stride and column offset
// multiples of 8 elements, width a multiple of 8, 16-byte aligned base). Rows
// >= nrows and columns >= width read as zeros through the buffer range check
// (the tile spans less than 2 GiB from g). `g` must be wave-uniform.
template <int ROWS, int W, int NTHR>
__device__ __forceinline__ void tstage_load_v(TileStage<ROWS, W, NTHR>& s, const bf16* __restrict__ g, int64_t ld,
                                              int nrows, int width) {
  constexpr int CPR = W / 8;
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(g);
#pragma unroll
  for (int q = 0; q < TileStage<ROWS, W, NTHR>::PER; ++q) {
    const int id = threadIdx.x + q * NTHR;
    if (TileStage<ROWS, W, NTHR>::NVEC % NTHR == 0 || id < TileStage<ROWS, W, NTHR>::NVEC) {
      const int r = id / CPR, k = (id % CPR) * 8;
      s.v[q] = buf_ld16(rs, (int)(((int64_t)r * ld + k) * 2), r < nrows && k < width);
    }
  }
}

// Same, from an fp32 row-major source (converted to bf16); rows of `ld` floats,
// 16-byte aligned rows (ld % 4 == 0, W <= ld).
template <int ROWS, int W, int NTHR>
__device__ __forceinline__ void tstage_load_f32(TileStage<ROWS, W, NTHR>& s, const float* __restrict__ g,
                                                int64_t ld) {
  constexpr int CPR = W / 8;
#pragma unroll
  for (int q = 0; q < TileStage<ROWS, W, NTHR>::PER; ++q) {
    const int id = threadIdx.x + q * NTHR;
    if (TileStage<ROWS, W, NTHR>::NVEC % NTHR == 0 || id < TileStage<ROWS, W, NTHR>::NVEC) {
      const int r = id / CPR, k = (id % CPR) * 8;
      const float* p = g + (int64_t)r * ld + k;
      const floatx4 a = *reinterpret_cast<const floatx4*>(p);
      const floatx4 b = *reinterpret_cast<const floatx4*>(p + 4);
      bf16x8 v;
      v[0] = (bf16)a[0]; v[1] = (bf16)a[1]; v[2] = (bf16)a[2]; v[3] = (bf16)a[3];
      v[4] = (bf16)b[0]; v[5] = (bf16)b[1]; v[6] = (bf16)b[2]; v[7] = (bf16)b[3];
      s.v[q] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Unpadded tiles filled by buffer_load ... lds (whole 1 KB rows of lanes): the
// 16-byte granules of each row are permuted instead of padding the rows.
// ---------------------------------------------------------------------------
// Permuted granule of logical granule g in row r of a W-wide bf16 tile.
// Tiles read with ds_read_b64_tr_b16 (four rows, two granules per 16 lanes).
// Rows r and r ^ 1 sit in opposite halves of the LDS's 256-byte bank window,
// so (r & 3) alone spreads four rows of 32 lanes over all 64 banks. Bit 3 of r
// is for the 16 x 16 x 32 operand, whose 16-lane groups read rows k .. k + 3
// and k + 8 .. k + 11 in one half-wave: without it the two groups hit the same
// banks (a 32-wide read keeps bit 3 fixed over a half-wave and is unaffected).
// 128-wide rows (256 bytes) all start in the same bank window, so there the four
// rows of a read take a quarter of the row each ((r & 3) << 2), bit 3 again
// moving the second 16-lane group's rows to the other granules of their quarter.
template <int W>
__device__ __forceinline__ int swz_tr(int r, int g) {
  return W == 128 ? g ^ ((r & 3) << 2) ^ ((r >> 2) & 2) : (W >= 64 ? g ^ ((r & 3) << 1) ^ ((r >> 2) & 2) : g);
}
// Tiles read by rows (16 consecutive rows at one granule):
template <int W>
__device__ __forceinline__ int swz_nat(int r, int g) {
  return W == 128 ? g ^ (r & 15) : (W == 64 ? g ^ ((r >> 1) & 7) : g ^ ((r >> 2) & 3));
}

// k-contiguous operand with i = mbase + L % 32 from a transposed-read tile
// (row index k), as ttr_std does for padded tiles.
template <int W>
__device__ __forceinline__ bf16x4 swz_tr4(const bf16* t, int kb, int m0, int L) {
  const int q = L & 15;
  const int r = kb + (q >> 2), col = m0 + ((q & 3) << 2);
  const bf16* p = t + r * W + (swz_tr<W>(r, col >> 3) << 3) + (col & 7);
  const shortx4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) shortx4*)(p));
  return __builtin_bit_cast(bf16x4, v);
}
template <int W>
__device__ __forceinline__ bf16x8 swz_tr8(const bf16* t, int k0, int mbase, int L) {
  const int h = L >> 5;
  const int m0 = mbase + (((L >> 4) & 1) << 4);
  return cat8(swz_tr4<W>(t, k0 + 8 * h, m0, L), swz_tr4<W>(t, k0 + 8 * h + 4, m0, L));
}
// The ttr_perm operand order (rows k0 + 16 kk + 4 (L / 32) + 0..3, then + 8) from a permuted tile.
template <int W>
__device__ __forceinline__ bf16x8 swz_tr_perm(const bf16* t, int k0, int kk, int mbase, int L) {
  const int h = L >> 5;
  const int m0 = mbase + (((L >> 4) & 1) << 4);
  return cat8(swz_tr4<W>(t, k0 + 16 * kk + 4 * h, m0, L), swz_tr4<W>(t, k0 + 16 * kk + 8 + 4 * h, m0, L));
}
// The same for the 16 x 16 x 32 MFMA operand layout: i = mbase + L % 16, k = k0 + 8 (L / 16) + 0..7.
template <int W>
__device__ __forceinline__ bf16x8 swz_tr8_16(const bf16* t, int k0, int mbase, int L) {
  const int kb = k0 + 8 * (L >> 4);
  return cat8(swz_tr4<W>(t, kb, mbase, L), swz_tr4<W>(t, kb + 4, mbase, L));
}
template <int W>
__device__ __forceinline__ bf16x8 swz_nat8(const bf16* t, int r, int col) {
  return *reinterpret_cast<const bf16x8*>(t + r * W + (swz_nat<W>(r, col >> 3) << 3));
}

// vmcnt-only wait (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14, expcnt 7, lgkmcnt 15)
template <int N>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt(0xF70 | (N & 15) | ((N >> 4) << 14));
}

// Workgroup barrier for LDS written by ds_write (lgkmcnt) and by buffer_load ... lds
// whose writer has already retired it with its own vmcnt wait. Unlike
// __syncthreads() (a release fence over all memory, which the compiler implements
// as vmcnt(0): every outstanding global load, store and LDS DMA of the wave), it
// leaves the wave's later DMAs in flight across the barrier. The "memory" clobber
// keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One step of an LDS ring filled by buffer_load ... lds: issue(nxt) refills a free slot,
// body(cur) consumes the current one. Passing the two slots as distinct __restrict__
// pointers (after inlining: disjoint alias scopes on every access derived from them)
// tells the compiler that the new DMAs do not write what the body reads, so it adds
// no vmcnt wait of its own for them; the caller's explicit waits order the slots.
template <typename Issue, typename Body>
__device__ __forceinline__ void ring_step(const unsigned char* __restrict__ cur, unsigned char* __restrict__ nxt,
                                          bool refill, Issue&& issue, Body&& body) {
  if (refill) issue(nxt);
  body(cur);
}

// exp2 of a value already clamped; the decays below are all exp(clamp(d, -20, 20))
// evaluated as exp2(clamp(d * log2 e, +-20 log2 e)).
__device__ __forceinline__ float exp2_fast(float v) { return __builtin_amdgcn_exp2f(v); }
__device__ __forceinline__ float clamp_med3(float v, float lo, float hi) { return __builtin_amdgcn_fmed3f(v, lo, hi); }

#define SSD_LOG2E 1.4426950408889634f
#define SSD_T2 (20.0f * SSD_LOG2E)

// v + v of lane L ^ 32, with no LDS round trip: v_permlane32_swap of v with
// itself yields the lower half-wave's values in one result and the upper
// half's in the other, for every lane. Both lanes of a pair get the same sum.
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum of v over the wave, in every lane: DPP within each 16-lane row, then
// v_permlane16_swap / v_permlane32_swap across rows.
__device__ __forceinline__ float wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));  // row_half_mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));  // row_mirror
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return add_xor32(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

// Value of x at lane L ^ m within each 16-lane row, for the DPP controls below.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum of v over the 32 lanes of each half-wave, for 16 values at once.
// Afterwards lane L returns the sum of v[(L >> 1) & 15] over its half.
// A butterfly that halves the values at every stage, the lane's bit of the
// stage choosing the half it keeps; all of it in VALU, with no LDS round trip:
// lanes L ^ 16 by v_permlane16_swap (the odd rows of its first operand trade
// places with the even rows of its second, so one add completes a pair), then
// DPP within rows: L ^ 8 (row_ror:8), L ^ 7 (row_half_mirror, which pairs lanes
// of opposite bit 2 as L ^ 4 would and keeps the summed lane sets disjoint),
// L ^ 2 and L ^ 1 (quad_perm).
__device__ __forceinline__ float half_reduce16(float (&v)[16], int L) {
  float a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 8]), false, false);
    a[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  float c[4];
  {
    const bool b = (L >> 3) & 1;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float send = b ? a[k] : a[k + 4];
      const float keep = b ? a[k + 4] : a[k];
      c[k] = keep + dpp_f<0x128>(send);  // row_ror:8
    }
  }
  float e[2];
  {
    const bool b = (L >> 2) & 1;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float send = b ? c[k] : c[k + 2];
      const float keep = b ? c[k + 2] : c[k];
      e[k] = keep + dpp_f<0x141>(send);  // row_half_mirror
    }
  }
  float f;
  {
    const bool b = (L >> 1) & 1;
    const float send = b ? e[0] : e[1];
    const float keep = b ? e[1] : e[0];
    f = keep + dpp_f<0x4E>(send);  // quad_perm 2,3,0,1
  }
  return f + dpp_f<0xB1>(f);  // quad_perm 1,0,3,2
}
