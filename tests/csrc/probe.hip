// Test-only probe library: exercises single CDNA4 (gfx950) instructions whose
// lane layouts the production kernels rely on, so the tests can compare them
// against a CPU model of the layout.  Every probe runs one 64-lane wavefront
// and touches only the buffers it is handed (sizes fixed below).
//
//   probe_mfma_16x16x32_bf16 : a[64][8] bf16, b[64][8] bf16 -> c[64][4] f32
//   probe_mfma_32x32x16_bf16 : a[64][8] bf16, b[64][8] bf16 -> c[64][16] f32
//   probe_ds_read_tr16_b64   : addr[64] int32 (element offsets into a 1024-entry
//                              LDS array holding lds[i] = i) -> out[64][4] int16
//   probe_dpp_wave_shr1      : src[64] int32, old[64] int32 -> out[64] int32
//   probe_cvt_bf16           : x[n] f32 -> y[n] bf16 (n even, n <= 4096)
//   probe_quad_transpose     : x[64][4] f32 -> y[64][4] f32 (thm::quad_transpose)
//   probe_mfma_16x16x4_f32   : a[64] f32, b[64] f32 -> c[64][4] f32
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../theorem_amd/csrc/vmem.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(64) k_mfma16(const bf16x8* a, const bf16x8* b, f32x4* c) {
  const int l = threadIdx.x;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[l], b[l], acc, 0, 0, 0);
  c[l] = acc;
}

__global__ void __launch_bounds__(64) k_mfma32(const bf16x8* a, const bf16x8* b, f32x16* c) {
  const int l = threadIdx.x;
  f32x16 acc;
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[l], b[l], acc, 0, 0, 0);
  c[l] = acc;
}

__global__ void __launch_bounds__(64) k_tr16(const int* addr, short* out) {
  __shared__ __attribute__((aligned(16))) short lds[1024];
  const int l = threadIdx.x;
  for (int i = l; i < 1024; i += 64) lds[i] = (short)i;
  __syncthreads();
  int e = addr[l];
  e = (e < 0 ? 0 : (e > 1020 ? 1020 : e)) & ~3;  // keep the 8-byte read in bounds
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(lds + e));
  out[4 * l + 0] = v[0];
  out[4 * l + 1] = v[1];
  out[4 * l + 2] = v[2];
  out[4 * l + 3] = v[3];
}

__global__ void __launch_bounds__(64) k_dpp(const int* src, const int* old, int* out) {
  const int l = threadIdx.x;
  out[l] = __builtin_amdgcn_update_dpp(old[l], src[l], 0x138, 0xf, 0xf, false);
}

__global__ void k_cvt(const float* x, bf16x2* y, int npairs) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < npairs) {
    bf16x2 r;
    r[0] = (__bf16)x[2 * i];
    r[1] = (__bf16)x[2 * i + 1];
    y[i] = r;
  }
}

__global__ void __launch_bounds__(64) k_quad_transpose(const f32x4* x, f32x4* y) {
  y[threadIdx.x] = thm::quad_transpose(x[threadIdx.x]);
}

__global__ void __launch_bounds__(64) k_mfma16f32(const float* a, const float* b, f32x4* c) {
  const int l = threadIdx.x;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[l], b[l], acc, 0, 0, 0);
  c[l] = acc;
}

extern "C" {
int probe_mfma_16x16x4_f32(const void* a, const void* b, void* c, void* stream) {
  hipLaunchKernelGGL(k_mfma16f32, dim3(1), dim3(64), 0, (hipStream_t)stream, (const float*)a, (const float*)b, (f32x4*)c);
  return (int)hipGetLastError();
}
int probe_quad_transpose(const void* x, void* y, void* stream) {
  hipLaunchKernelGGL(k_quad_transpose, dim3(1), dim3(64), 0, (hipStream_t)stream, (const f32x4*)x, (f32x4*)y);
  return (int)hipGetLastError();
}
int probe_mfma_16x16x32_bf16(const void* a, const void* b, void* c, void* stream) {
  hipLaunchKernelGGL(k_mfma16, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const bf16x8*)a, (const bf16x8*)b, (f32x4*)c);
  return (int)hipGetLastError();
}
int probe_mfma_32x32x16_bf16(const void* a, const void* b, void* c, void* stream) {
  hipLaunchKernelGGL(k_mfma32, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const bf16x8*)a, (const bf16x8*)b, (f32x16*)c);
  return (int)hipGetLastError();
}
int probe_ds_read_tr16_b64(const void* addr, void* out, void* stream) {
  hipLaunchKernelGGL(k_tr16, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const int*)addr, (short*)out);
  return (int)hipGetLastError();
}
int probe_dpp_wave_shr1(const void* src, const void* old, void* out, void* stream) {
  hipLaunchKernelGGL(k_dpp, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const int*)src, (const int*)old, (int*)out);
  return (int)hipGetLastError();
}
int probe_cvt_bf16(const void* x, void* y, int n, void* stream) {
  if (n <= 0 || (n & 1) || n > 4096) return -1;
  const int np = n / 2;
  hipLaunchKernelGGL(k_cvt, dim3((np + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     (const float*)x, (bf16x2*)y, np);
  return (int)hipGetLastError();
}
}
