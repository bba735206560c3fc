// Gate preprocessing of the chunked Gated DeltaNet forward for MI355X (gfx950):
//   g[b, t, h] = sum over t' in t's 64-token chunk, t' <= t, of f(a[b, t', h])
// with f = identity or f = logsigmoid (log(sigmoid(x))).  g is the chunk-local
// cumulative log decay every chunk kernel takes; the reference builds it in
// its input generators (kernels/chunk_fwd_h/reference.py:15-47: chunk-local
// cumsum of a per-token decay) and the gated delta rule uses logsigmoid gates.
//
// One 256-thread workgroup per (b, chunk, group of up to 16 heads):
//   1. the chunk's 64 x hn block of a is read row by row (each token's hn
//      heads are contiguous), f applied elementwise, and written to LDS;
//   2. wave w scans heads w, w + 4, ...: lane t holds token t, and a 6-step
//      wave-level inclusive scan (shuffle up by 1, 2, ..., 32) forms the
//      running sums;
//   3. the block is written back row by row.
// Every element gets its own lane (a lane per (b, chunk, head) walking 64
// tokens left one wave per CU at config 4: 26 us for 8 MB).  The sums are
// formed in scan order, not left to right: they agree with a sequential
// fp32 sum to rounding.
#include <math.h>

#include "common.h"

namespace thm {
namespace {

constexpr int kBT = 64;

__device__ __forceinline__ float logsigmoid(float x) {
  // log(sigmoid(x)) = min(x, 0) - log1p(exp(-|x|)), exact in both tails.
  return fminf(x, 0.f) - log1pf(expf(-fabsf(x)));
}

constexpr int kCsThreads = 256;
constexpr int kCsHeads = 16;           // heads per workgroup
constexpr int kCsPitch = kCsHeads + 1; // LDS row pitch (floats)

template <typename IT, bool LOGSIG>
__global__ void __launch_bounds__(kCsThreads)
chunk_local_cumsum_kernel(const IT* __restrict__ a, float* __restrict__ g, int64_t T, int64_t H,
                          int64_t NT, int64_t HG) {
  __shared__ float blk[kBT * kCsPitch];
  const int64_t id = blockIdx.x;
  const int64_t hgi = id % HG, bc = id / HG;
  const int64_t c = bc % NT, b = bc / NT;
  const int64_t h0 = hgi * kCsHeads;
  const int hn = (int)(H - h0 < kCsHeads ? H - h0 : kCsHeads);
  const int64_t base = (b * T + c * kBT) * H + h0;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kBT * kCsHeads / kCsThreads; ++i) {
    const int e = tid + i * kCsThreads;
    if (e < kBT * hn) {
      const int t = e / hn, hl = e - t * hn;
      const float x = to_f32(a[base + (int64_t)t * H + hl]);
      blk[t * kCsPitch + hl] = LOGSIG ? logsigmoid(x) : x;
    }
  }
  __syncthreads();
  const int lane = tid & 63;
  for (int hl = tid >> 6; hl < hn; hl += kCsThreads / 64) {
    float v = blk[lane * kCsPitch + hl];
#pragma unroll
    for (int d = 1; d < kBT; d <<= 1) {
      const float y = __shfl_up(v, d, 64);
      if (lane >= d) v += y;
    }
    blk[lane * kCsPitch + hl] = v;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kBT * kCsHeads / kCsThreads; ++i) {
    const int e = tid + i * kCsThreads;
    if (e < kBT * hn) {
      const int t = e / hn, hl = e - t * hn;
      g[base + (int64_t)t * H + hl] = blk[t * kCsPitch + hl];
    }
  }
}

template <typename IT>
hipError_t launch_cumsum(const void* a, void* g, int64_t B, int64_t T, int64_t H, bool logsig,
                         hipStream_t s) {
  const int64_t NT = T / kBT;
  const int64_t HG = (H + kCsHeads - 1) / kCsHeads;
  const dim3 grid((unsigned)(B * NT * HG));
  if (logsig)
    hipLaunchKernelGGL((chunk_local_cumsum_kernel<IT, true>), grid, dim3(kCsThreads), 0, s, (const IT*)a,
                       (float*)g, T, H, NT, HG);
  else
    hipLaunchKernelGGL((chunk_local_cumsum_kernel<IT, false>), grid, dim3(kCsThreads), 0, s, (const IT*)a,
                       (float*)g, T, H, NT, HG);
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
  const int64_t nbt = B * (T / kBT), hg = (H + kCsHeads - 1) / kCsHeads;  // grid = nbt x hg
  if (B > (INT64_C(1) << 40) / T || hg > (int64_t)UINT32_MAX / nbt || !launch_fits(nbt * hg, kCsThreads))
    return THM_ERR_BAD_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const bool logsig = mode == THM_GATE_LOGSIGMOID;
  const hipError_t e = (a_dtype == THM_DTYPE_F32) ? launch_cumsum<float>(a, g, B, T, H, logsig, s)
                                                  : launch_cumsum<bf16>(a, g, B, T, H, logsig, s);
  return (int)e;
}
