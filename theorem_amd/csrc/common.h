// Shared gfx950 (CDNA4) device helpers for the Theorem MI355X kernels.
//
// Conventions used by every kernel in this directory:
//   * wave64; a "lane" is threadIdx.x % 64.
//   * bf16 values are __bf16; fp32 -> bf16 conversion is round-to-nearest-even
//     (a plain cast, which gfx950 lowers to v_cvt_pk_bf16_f32).
//   * MFMA v_mfma_f32_16x16x32_bf16 operand layouts (lane l, g = l / 16):
//       A operand : row m = l % 16,  k = 8g .. 8g+7  (8 bf16)
//       B operand : col n = l % 16,  k = 8g .. 8g+7  (8 bf16)
//       C/D       : col n = l % 16,  rows 4g .. 4g+3 (4 fp32)
//     The contraction index k may be permuted freely as long as A and B use
//     the same permutation; the kernels use that to feed an accumulator tile
//     pair straight back into the next MFMA without a lane shuffle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/theorem_mi355x.h"

namespace thm {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// exp(x) through the hardware base-2 exponential (v_exp_f32).
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// Wave-uniform value of lane `src` (v_readlane).
__device__ __forceinline__ float readlane(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

// Whole-wave shift right by one lane (DPP wave_shr:1): lane l receives lane
// l-1's `v`; lane 0 receives `fill`.
__device__ __forceinline__ float wave_shr1(float v, float fill) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), 0x138, 0xf, 0xf, false));
}

// Workgroup barrier that orders LDS only.  __syncthreads() also fences global
// memory, which makes every wave wait for all of its outstanding global
// loads and stores (s_waitcnt vmcnt(0)) at each barrier; the kernels here use
// barriers only to hand LDS tiles between waves, so in-flight prefetch loads
// and output stores are left running.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wave-scope LDS hand-off between lanes of one wavefront: LDS writes of some
// lanes before it are visible to LDS reads of other lanes after it.  The wave
// executes its LDS instructions in order, so this emits no instruction; the
// fences and the wave barrier stop the compiler from moving an LDS read of
// one lane's data above another lane's write (which it may do when it can
// prove the two addresses of one lane differ).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Head index and first token row of tile `tile` of a [B, T / 64, H] tile
// grid with the head fastest.  Every entry point that uses it checks that the
// tile count is below 2^31, so 32-bit unsigned division is exact; it replaces
// the 64-bit division sequences of int64_t % and /.
struct TileCoord {
  int64_t hh, tok0;
};
__device__ __forceinline__ TileCoord tile_coord(int64_t tile, int64_t H, int64_t NT, int64_t T) {
  const uint32_t t = (uint32_t)tile, h = (uint32_t)H, nt = (uint32_t)NT;
  const uint32_t bc = t / h, b = bc / nt;
  return {(int64_t)(t - bc * h), (int64_t)b * T + (int64_t)(bc - b * nt) * 64};
}

// HIP rejects a launch of more than 2^32 - 1 work-items in total.  Every entry
// point checks its grid against this on the host (with its largest block),
// so an oversized shape returns THM_ERR_BAD_SHAPE instead of a launch error.
inline bool launch_fits(int64_t workgroups, int64_t threads) {
  return workgroups >= 0 && workgroups <= (int64_t)UINT32_MAX / threads;
}

// Compute units of the current device (queried once per device, then cached;
// 0 if the query fails).  Used to size persistent grids.
inline int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    __atomic_store_n(&cached[dev], n, __ATOMIC_RELAXED);
  }
  return n;
}

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }


// 16-byte global load of raw bits; non-temporal (streaming) 16-byte load / store.
__device__ __forceinline__ u32x4 ldg16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 ldg16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void stg16_nt(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}


// Unpack 16 bytes into floats: 4 fp32 or 8 bf16.
__device__ __forceinline__ void unpack16(u32x4 r, float* out, float /*tag*/) {
  out[0] = __uint_as_float(r[0]);
  out[1] = __uint_as_float(r[1]);
  out[2] = __uint_as_float(r[2]);
  out[3] = __uint_as_float(r[3]);
}
__device__ __forceinline__ void unpack16(u32x4 r, float* out, bf16 /*tag*/) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(r[i] << 16);
    out[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ u32x4 pack16(const float* v, float /*tag*/) {
  u32x4 r;
  r[0] = __float_as_uint(v[0]);
  r[1] = __float_as_uint(v[1]);
  r[2] = __float_as_uint(v[2]);
  r[3] = __float_as_uint(v[3]);
  return r;
}
__device__ __forceinline__ u32x4 pack16(const float* v, bf16 /*tag*/) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bf16x2 p;
    p[0] = (bf16)v[2 * i];
    p[1] = (bf16)v[2 * i + 1];
    r[i] = __builtin_bit_cast(uint32_t, p);
  }
  return r;
}

template <typename T>
struct ElemsPer16 {
  static constexpr int value = 16 / (int)sizeof(T);
};

}  // namespace thm
