// Vector-memory instructions issued by hand, for pipelines whose waits are
// counted by hand (gfx950).
//
// The compiler's automatic wait insertion treats every LDS read after a
// global -> LDS DMA as dependent on it and waits for all outstanding vector
// memory operations (vmcnt(0)), which serialises a multi-stage LDS ring.  The
// kernels that use these helpers therefore issue their DMA loads and their
// global stores here, in inline assembly the compiler does not track, and
// wait with an explicit vmcnt(N): loads and stores retire in issue order on
// one counter, so once at most N operations are outstanding, every operation
// issued before the last N has completed.
//
// All operands named `base` and `lds` must be wave-uniform; `voff` is a
// per-lane 32-bit byte offset from `base`.
#pragma once

#include "common.h"

namespace thm {

typedef __attribute__((address_space(3))) void lds_void_t;

// 32-bit LDS address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(size_t)(lds_void_t*)p;
}

// A wave-uniform pointer, moved to scalar registers.  The compiler cannot
// always prove a pointer uniform (a select between kernel arguments by a
// uniform wave index, for example) and would hand the scalar operand of the
// instructions below a vector register; for a value already in scalar
// registers this folds away.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}

// global -> LDS, 16 bytes per lane: lane i's bytes [base + voff_i, +16) land at
// LDS [lds + 16 i, +16).  M0 (the LDS base register) is restored afterwards.
__device__ __forceinline__ void dma_b128(const void* base, uint32_t voff, uint32_t lds) {
  base = uniform_ptr(base);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(base), "s"(lds)
      : "memory");
}

// global -> LDS, 4 bytes per lane: lane i's bytes [base + voff_i, +4) land at
// LDS [lds + 4 i, +4).
__device__ __forceinline__ void dma_b32(const void* base, uint32_t voff, uint32_t lds) {
  base = uniform_ptr(base);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(base), "s"(lds)
      : "memory");
}

// Vector global stores of 16 / 8 bytes per lane at base + voff.  A store of
// more than 8 bytes reads its upper data registers a cycle after issue, and a
// VALU write to them must wait for that; the compiler inserts that wait for the
// stores it emits but not after inline assembly, so the wait states are part of
// the statement.
__device__ __forceinline__ void st_b128(void* base, uint32_t voff, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, %2\n\ts_nop 1" : : "v"(voff), "v"(v), "s"(base) : "memory");
}
__device__ __forceinline__ void st_b64(void* base, uint32_t voff, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, %2" : : "v"(voff), "v"(v), "s"(base) : "memory");
}

// Wait until at most N vector memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Transpose the 4x4 matrix held by each quad of lanes (lane 4m + q holds row q
// in v[0..3]): afterwards lane 4m + q holds column q, i.e. r[i] = the v[q] of
// lane 4m + i.  Two DPP butterfly steps (quad_perm xor 1, xor 2).  Every lane
// of every row and bank is written from a lane of its own quad, so the DPP's
// "old" operand is never observed: mov_dpp leaves it undefined, where
// update_dpp with old = 0 cost a v_mov of 0 into each destination.
__device__ __forceinline__ float dpp_quad_xor1(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_quad_xor2(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ f32x4 quad_transpose(f32x4 v) {
  const int q = lane_id() & 3;
  const bool q0 = q & 1, q1 = q & 2;
  const float x0 = dpp_quad_xor1(v[1]), x1 = dpp_quad_xor1(v[0]);
  const float x2 = dpp_quad_xor1(v[3]), x3 = dpp_quad_xor1(v[2]);
  f32x4 a;
  a[0] = q0 ? x0 : v[0];
  a[1] = q0 ? v[1] : x1;
  a[2] = q0 ? x2 : v[2];
  a[3] = q0 ? v[3] : x3;
  const float y0 = dpp_quad_xor2(a[2]), y1 = dpp_quad_xor2(a[3]);
  const float y2 = dpp_quad_xor2(a[0]), y3 = dpp_quad_xor2(a[1]);
  f32x4 r;
  r[0] = q1 ? y0 : a[0];
  r[1] = q1 ? y1 : a[1];
  r[2] = q1 ? a[2] : y2;
  r[3] = q1 ? a[3] : y3;
  return r;
}

// Re-layout of a 16x16 accumulator tile for row-contiguous stores.  In the
// MFMA layout lane 4m + q of each 16-lane group holds column 4m + q, rows 0..3
// (v[0..3]).  Afterwards lane 4a + b holds row a, columns 4b .. 4b + 3, so the
// four lanes of a quad cover 16 contiguous elements of one row.  A vector
// store whose consecutive lanes fall in different rows is split into more
// memory requests: a 16-row store of 16-byte lanes occupies a CU's address
// unit for ~62 cycles in the quad-transposed layout and ~18 in this one
// (measured on MI355X).  A quad transpose (DPP), then the lane transpose
// 4a + b <- 4b + a through ds_bpermute.
__device__ __forceinline__ int row_quad_src_addr() {
  const int l = lane_id();
  return ((l & ~15) + 4 * (l & 3) + ((l >> 2) & 3)) * 4;
}
__device__ __forceinline__ f32x4 acc_to_row_quads(f32x4 v) {
  const f32x4 t = quad_transpose(v);  // lane 4m + q: row q, columns 4m .. 4m + 3
  const int src = row_quad_src_addr();
  f32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(t[i])));
  return r;
}
// The same for a tile stored as bf16: the four values of a lane are packed
// first, so the lane transpose moves two dwords instead of four.
__device__ __forceinline__ u32x2 acc_to_row_quads_bf16(f32x4 v) {
  const f32x4 t = quad_transpose(v);
  bf16x4 o;
  o[0] = (bf16)t[0]; o[1] = (bf16)t[1]; o[2] = (bf16)t[2]; o[3] = (bf16)t[3];
  const u32x2 pk = __builtin_bit_cast(u32x2, o);
  const int src = row_quad_src_addr();
  u32x2 r;
  r[0] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)pk[0]);
  r[1] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)pk[1]);
  return r;
}

// Two accumulator tiles of one output row, columns 32 m + 4 grp .. + 3 (lo)
// and 32 m + 16 + 4 grp .. + 3 (hi) of this lane (grp = lane / 16), as bf16
// with 16 bytes per lane: lanes grp and grp ^ 1 (16 lanes apart) exchange one
// tile each, so lane grp holds the 8 consecutive columns
// 32 m + pair_col(grp) .. + 7, and the 4 lanes of a row cover 64 contiguous
// bytes.  (Storing lo and hi as 8-byte pieces puts 32-byte runs of 16 rows in
// one store instruction, which the memory path takes far more slowly.)
__device__ __forceinline__ constexpr int pair_col(int grp) { return 8 * (grp >> 1) + 16 * (grp & 1); }
__device__ __forceinline__ u32x4 acc_pair_to_b128(f32x4 lo, f32x4 hi) {
  const int l = lane_id();
  const bool odd = (l >> 4) & 1;
  const f32x4 send = odd ? lo : hi, keep = odd ? hi : lo;
  bf16x4 sb, kb;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sb[i] = (bf16)send[i];
    kb[i] = (bf16)keep[i];
  }
  const u32x2 sp = __builtin_bit_cast(u32x2, sb), kp = __builtin_bit_cast(u32x2, kb);
  const int src = (l ^ 16) * 4;
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)sp[0]);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)sp[1]);
  return odd ? u32x4{r0, r1, kp[0], kp[1]} : u32x4{kp[0], kp[1], r0, r1};
}

}  // namespace thm
