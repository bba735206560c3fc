// Gate preprocessing of the chunked Gated DeltaNet forward for MI355X (gfx950):
//   g[b, t, h] = sum over t' in t's 64-token chunk, t' <= t, of f(a[b, t', h])
// with f = identity or f = logsigmoid (log(sigmoid(x))).  g is the chunk-local
// cumulative log decay every chunk kernel takes; the reference builds it in
// its input generators (kernels/chunk_fwd_h/reference.py:15-47: chunk-local
// cumsum of a per-token decay) and the gated delta rule uses logsigmoid gates.
//
// HBM-bound (read a once, write g once).  One lane per (b, chunk, head): the
// lane walks the chunk's 64 tokens in order (fp32 running sum), and the H
// lanes of one (b, chunk) read and write H consecutive values per token, so
// each step of a wavefront touches contiguous memory.
#include <math.h>

#include "common.h"

namespace thm {
namespace {

constexpr int kBT = 64;

__device__ __forceinline__ float logsigmoid(float x) {
  // log(sigmoid(x)) = min(x, 0) - log1p(exp(-|x|)), exact in both tails.
  return fminf(x, 0.f) - log1pf(expf(-fabsf(x)));
}

template <typename IT, bool LOGSIG>
__global__ void __launch_bounds__(256)
chunk_local_cumsum_kernel(const IT* __restrict__ a, float* __restrict__ g, int64_t T, int64_t H,
                          int64_t NT, int64_t lanes) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= lanes) return;
  const int64_t h = idx % H;
  const int64_t bc = idx / H;  // b * NT + c
  const int64_t c = bc % NT, b = bc / NT;
  const int64_t base = (b * T + c * kBT) * H + h;
  float acc = 0.f;
#pragma unroll 8
  for (int t = 0; t < kBT; ++t) {
    const float x = to_f32(a[base + t * H]);
    acc += LOGSIG ? logsigmoid(x) : x;
    g[base + t * H] = acc;
  }
}

template <typename IT>
hipError_t launch_cumsum(const void* a, void* g, int64_t B, int64_t T, int64_t H, bool logsig,
                         hipStream_t s) {
  const int64_t NT = T / kBT;
  const int64_t lanes = B * NT * H;
  const dim3 grid((unsigned)((lanes + 255) / 256));
  if (logsig)
    hipLaunchKernelGGL((chunk_local_cumsum_kernel<IT, true>), grid, dim3(256), 0, s, (const IT*)a,
                       (float*)g, T, H, NT, lanes);
  else
    hipLaunchKernelGGL((chunk_local_cumsum_kernel<IT, false>), grid, dim3(256), 0, s, (const IT*)a,
                       (float*)g, T, H, NT, lanes);
  return hipGetLastError();
}

}  // namespace
}  // namespace thm

extern "C" int thm_chunk_local_cumsum(const void* a, void* g, int64_t B, int64_t T, int64_t H,
                                      int32_t chunk_size, int32_t a_dtype, int32_t mode,
                                      void* stream) {
  using namespace thm;
  if (chunk_size != kBT) return THM_ERR_BAD_ARGUMENT;
  if (mode != THM_GATE_IDENTITY && mode != THM_GATE_LOGSIGMOID) return THM_ERR_BAD_ARGUMENT;
  if (B < 0 || T < 0 || H <= 0 || T % kBT) return THM_ERR_BAD_SHAPE;
  if (a_dtype != THM_DTYPE_F32 && a_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if (B == 0 || T == 0) return THM_OK;
  if (!a || !g) return THM_ERR_NULL_POINTER;
  if (((uintptr_t)a % (a_dtype == THM_DTYPE_F32 ? 4 : 2)) || ((uintptr_t)g % 4)) return THM_ERR_MISALIGNED;
  if (B * (T / kBT) * H > (INT64_C(1) << 38)) return THM_ERR_BAD_SHAPE;  // grid fits 32 bits
  hipStream_t s = (hipStream_t)stream;
  const bool logsig = mode == THM_GATE_LOGSIGMOID;
  const hipError_t e = (a_dtype == THM_DTYPE_F32) ? launch_cumsum<float>(a, g, B, T, H, logsig, s)
                                                  : launch_cumsum<bf16>(a, g, B, T, H, logsig, s);
  return (int)e;
}
