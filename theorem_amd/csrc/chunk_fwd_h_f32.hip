// fp32 inputs of the Gated DeltaNet state recurrence: the register-prefetch
// kernel of chunk_fwd_h_reg.h, or on small grids the role-split kernel of
// chunk_fwd_h_small.h, every (K, V) and form, called from
// thm_chunk_fwd_h (chunk_fwd_h.hip).  A unit of its own because it is compiled
// with the default code generation: forcing MFMA accumulators into VGPRs,
// which helps the bf16 kernels, made this kernel (two chunks of fp32 operands
// held in registers, AGPRs as extra storage) slower: 884 against 775 us at
// config 4.
#include "chunk_fwd_h_reg.h"
#include "chunk_fwd_h_small.h"

namespace thm {
namespace {

// Small grids (fewer workgroups of 64 columns than kHDmaMinGrid) take the
// role-split kernel of chunk_fwd_h_small.h where its stages fit in LDS (every
// shape but K = 128 in the delta form), the register kernel otherwise; both
// give bit-identical results.
template <int K, int V, bool DELTA>
hipError_t launch_f32(const void* k, const void* w, const void* vu, const void* g, const void* h0, void* h,
                      void* vnew, void* ht, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  if constexpr (pipe::SCfg<K, kHSmallNW, DELTA, 4>::kFits) {
    if (B * H * (V / kHBV) < kHDmaMinGrid)
      return launch_h_small<float, K, V, kHSmallNW, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
  }
  return launch_h<float, K, V, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
}

template <bool DELTA>
hipError_t dispatch_f32(int64_t K, int64_t V, const void* k, const void* w, const void* vu, const void* g,
                        const void* h0, void* h, void* vnew, void* ht, int64_t B, int64_t T, int64_t H,
                        hipStream_t s) {
  if (K == 64 && V == 64) return launch_f32<64, 64, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
  if (K == 64 && V == 128) return launch_f32<64, 128, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
  if (K == 128 && V == 64) return launch_f32<128, 64, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
  return launch_f32<128, 128, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
}

}  // namespace

__attribute__((visibility("hidden"))) hipError_t chunk_fwd_h_f32(bool delta, int64_t K, int64_t V, const void* k, const void* w, const void* vu,
                           const void* g, const void* h0, void* h, void* vnew, void* ht, int64_t B, int64_t T,
                           int64_t H, hipStream_t s) {
  return delta ? dispatch_f32<true>(K, V, k, w, vu, g, h0, h, vnew, ht, B, T, H, s)
               : dispatch_f32<false>(K, V, k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
}

}  // namespace thm
