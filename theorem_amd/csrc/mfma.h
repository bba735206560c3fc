// MFMA fragment helpers for the Gated DeltaNet chunk kernels (gfx950).
//
// All products use v_mfma_f32_16x16x32_bf16.  With g = lane / 16 and j = lane % 16
// a lane holds (see common.h):
//   A fragment  X[m = j][k = kidx(g, 0..7)]     B fragment  Y[k = kidx(g, 0..7)][n = j]
//   accumulator D[m = 4g + r][n = j], r = 0..3
// where kidx is the contraction order of the step.  Two orders are used:
//   natural  kidx(g, i) = 8g + i
//   paired   kidx(g, i) = 4g + i (i < 4),  16 + 4g + (i - 4) (i >= 4)
// The paired order is exactly what a lane holds in the accumulators of two
// vertically adjacent 16x16 tiles, so an accumulator pair becomes the next
// product's operand without any lane exchange.
//
// Operand sources:
//   * a tile whose contraction index runs along its (contiguous) columns is read
//     with one 16-byte load (natural order) or two 8-byte loads (paired order);
//   * a tile whose contraction index runs down its rows (a row-major LDS tile
//     used "transposed") is read with two ds_read_b64_tr_b16.  That instruction,
//     within each 16-lane group, gives output lane j element r = element (j % 4)
//     of the 8 bytes addressed by source lane 4r + j / 4.  Source lane s of group
//     g therefore points at row  base(g, half) + s / 4,  column  col0 + 4 (s % 4),
//     and lane j receives rows base .. base + 3 of column col0 + j.
//
// fp32 operands are represented as bf16 hi + lo (hi + lo = x to ~2^-16
// relative); a product of two fp32 operands is hi*hi + hi*lo + lo*hi.
#pragma once

#include "common.h"

namespace thm {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ bf16x4 ds_read_tr16(const bf16* lds_ptr) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr));
  return __builtin_bit_cast(bf16x4, v);
}

__device__ __forceinline__ bf16x8 concat(bf16x4 a, bf16x4 b) {
  bf16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// Fragment of a row-major LDS tile (pitch in elements) whose contraction index
// runs down the rows: rows row_h0 + 0..3 (elements 0..3) and row_h1 + 0..3
// (elements 4..7) of column col0 + lane % 16.  row_h0 / row_h1 are this lane's
// group base rows.
__device__ __forceinline__ bf16x8 frag_tr(const bf16* tile, int pitch, int row_h0, int row_h1,
                                          int col0) {
  const int s = lane_id() & 15;
  const int c = col0 + 4 * (s & 3);
  const bf16x4 a = ds_read_tr16(tile + (row_h0 + (s >> 2)) * pitch + c);
  const bf16x4 b = ds_read_tr16(tile + (row_h1 + (s >> 2)) * pitch + c);
  return concat(a, b);
}

// Natural-order base rows for contraction step `k0` (multiple of 32).
__device__ __forceinline__ int tr_row_natural(int k0, int half) {
  return k0 + 8 * (lane_id() >> 4) + 4 * half;
}
// Paired-order base rows for contraction step `k0`.
__device__ __forceinline__ int tr_row_paired(int k0, int half) {
  return k0 + 4 * (lane_id() >> 4) + 16 * half;
}

// 8 contiguous bf16 (16-byte aligned) from LDS or global memory.
__device__ __forceinline__ bf16x8 load8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
// Paired order from a row whose contraction runs along the columns: elements
// [k0 + 4g, +4) and [k0 + 16 + 4g, +4).
__device__ __forceinline__ bf16x8 load8_paired(const bf16* row, int k0) {
  const int g = lane_id() >> 4;
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(row + k0 + 4 * g);
  const bf16x4 b = *reinterpret_cast<const bf16x4*>(row + k0 + 16 + 4 * g);
  return concat(a, b);
}

__device__ __forceinline__ bf16x8 to_bf16x8(const float* v) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (bf16)v[i];
  return r;
}

__device__ __forceinline__ void split_bf16x8(const float* v, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bf16 h = (bf16)v[i];
    hi[i] = h;
    lo[i] = (bf16)(v[i] - (float)h);
  }
}

// Load 8 consecutive elements of type T (16-byte aligned for bf16, 32-byte for
// fp32) as floats; `nt` selects a non-temporal (streaming) load.
__device__ __forceinline__ void load8f(const bf16* p, float* v, bool nt = false) {
  unpack16(nt ? ldg16_nt(p) : ldg16(p), v, bf16{});
}
__device__ __forceinline__ void load8f(const float* p, float* v, bool nt = false) {
  unpack16(nt ? ldg16_nt(p) : ldg16(p), v, 0.f);
  unpack16(nt ? ldg16_nt(p + 4) : ldg16(p + 4), v + 4, 0.f);
}
// Paired order: elements [k0 + 4g, +4) and [k0 + 16 + 4g, +4).
__device__ __forceinline__ void load8f_paired(const bf16* row, int k0, float* v) {
  const int g = lane_id() >> 4;
  const u32x2 a = *reinterpret_cast<const u32x2*>(row + k0 + 4 * g);
  const u32x2 b = *reinterpret_cast<const u32x2*>(row + k0 + 16 + 4 * g);
  const uint32_t w[4] = {a[0], a[1], b[0], b[1]};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void load8f_paired(const float* row, int k0, float* v) {
  const int g = lane_id() >> 4;
  const f32x4 a = *reinterpret_cast<const f32x4*>(row + k0 + 4 * g);
  const f32x4 b = *reinterpret_cast<const f32x4*>(row + k0 + 16 + 4 * g);
  v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
  v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
}

// Store 4 consecutive outputs (16 bytes fp32 / 8 bytes bf16).  Plain stores:
// these partial-line writes rely on L2 write-combining, which streaming
// (non-temporal) stores bypass.
__device__ __forceinline__ void store4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ void store4(bf16* p, f32x4 v) {
  bf16x4 r;
  r[0] = (bf16)v[0]; r[1] = (bf16)v[1]; r[2] = (bf16)v[2]; r[3] = (bf16)v[3];
  *reinterpret_cast<bf16x4*>(p) = r;
}

// Write 4 consecutive outputs to LDS in the output dtype (the type of the
// unused tag pointer), rounded as store4 rounds them.
__device__ __forceinline__ void lds_store4(char* p, f32x4 v, const float*) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ void lds_store4(char* p, f32x4 v, const bf16*) {
  bf16x4 r;
  r[0] = (bf16)v[0]; r[1] = (bf16)v[1]; r[2] = (bf16)v[2]; r[3] = (bf16)v[3];
  *reinterpret_cast<bf16x4*>(p) = r;
}

// Write 4 (fp32 -> bf16 hi[, lo]) values to LDS.
__device__ __forceinline__ void lds_put4(bf16* hi, bf16* lo, const float* v, bool with_lo) {
  bf16x4 h, l;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = (bf16)v[i];
    l[i] = (bf16)(v[i] - (float)h[i]);
  }
  *reinterpret_cast<bf16x4*>(hi) = h;
  if (with_lo) *reinterpret_cast<bf16x4*>(lo) = l;
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

}  // namespace thm
