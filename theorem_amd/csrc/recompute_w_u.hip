// Gated DeltaNet WY recompute for MI355X (gfx950):
//   per chunk c of 64 tokens:  w_c = A_c (k_c * beta_c e^{g_c}),  u_c = A_c (v_c * beta_c)
//
// Replaces kernels/recompute_w_u/kernel.py:73-186 (Triton) and its launcher
// kernel.py:192-248; math of reference.py:118-149.
//
// One workgroup (4 wavefronts) per (b, chunk, head) tile, one memory phase:
//   1. Every global load of the tile is issued at once: the 64 x (K+V) tile
//      X = [k | v] (16-byte loads into registers), this wave's 16 rows of A_c
//      (fp32), and beta / g.
//   2. X goes to LDS unchanged for bf16 inputs (fp32 inputs: bf16 hi + lo);
//      beta, g go to LDS; one barrier.
//   3. The per-token scales are folded into A instead of X:
//        w = (A diag(beta e^g)) k,   u = (A diag(beta)) v,
//      each scaled A operand split into bf16 hi + lo (so A, beta and e^g enter
//      at ~fp32 accuracy and bf16 k / v enter exactly).
//   4. Wave wv owns positions t = 16 wv .. 16 wv + 15 and computes the
//      transposed product D[n][t] = sum_j X[j][n] A'[t][j] with
//      v_mfma_f32_16x16x32_bf16; X^T is read from LDS with ds_read_b64_tr_b16.
//      Each lane ends with 4 consecutive features of one token: one 8-byte
//      (bf16) / 16-byte (fp32) store.
// HBM traffic per tile = k, v, A, beta, g read once + w, u written once.
#include <type_traits>

#include "h_layout.h"
#include "mfma.h"

namespace thm {
namespace {

constexpr int kBT = 64;
constexpr int kWuThreads = 256;

template <typename IT, int K, int V>
struct WuCfg {
  static constexpr bool kSplitX = std::is_same<IT, float>::value;
  static constexpr int kN = K + V;
  static constexpr int kRowB = kN * 2;    // LDS row bytes of one bf16 tile (unpadded, h_layout.h xtile_off)
  static constexpr int kTile = kBT * kN;  // bf16 elements
  static constexpr int kNB = kN / 16;
  static constexpr int kVE = 16 / (int)sizeof(IT);  // elements per 16-byte load
  static constexpr int kCPR = kN / kVE;             // 16-byte chunks per row
  static constexpr int kLoads = kBT * kCPR / kWuThreads;
  static_assert(kBT * kCPR % kWuThreads == 0, "staging must divide evenly");
};

template <typename IT, int K, int V>
__global__ void __launch_bounds__(kWuThreads)
recompute_w_u_kernel(const IT* __restrict__ k, const IT* __restrict__ v,
                     const float* __restrict__ beta, const float* __restrict__ A,
                     const float* __restrict__ g, IT* __restrict__ w, IT* __restrict__ u,
                     int64_t T, int64_t H, int64_t NT) {
  using C = WuCfg<IT, K, V>;
  __shared__ __attribute__((aligned(16))) bf16 xs[(C::kSplitX ? 2 : 1) * C::kTile];
  __shared__ float sbeta[kBT], sg[kBT];
  bf16* const xhi = xs;
  bf16* const xlo = xs + (C::kSplitX ? C::kTile : 0);

  // tile -> (b, c, h), head fastest within an XCD: the workgroups of one XCD
  // read one contiguous [64 tokens x H x D] block, and beta / g lines once.
  const TileCoord tc = tile_coord(hl::xcd_tile_order(blockIdx.x, H, (int64_t)gridDim.x / H), H, NT, T);
  const int64_t h = tc.hh;
  const int64_t tok0 = tc.tok0;
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int li = lane & 15;

  // 1. Issue every load.
  u32x4 xr[C::kLoads];
#pragma unroll
  for (int it = 0; it < C::kLoads; ++it) {
    const int q = tid + it * kWuThreads;
    const int j = q / C::kCPR;
    const int col = (q - j * C::kCPR) * C::kVE;
    const int64_t row = (tok0 + j) * H + h;
    // Non-temporal: k and v are read once (measured 2% faster at config 4
    // than cached loads; the A rows stay cached loads, which measured faster).
    xr[it] = ldg16_nt(col < K ? (const void*)(k + row * K + col) : (const void*)(v + row * V + (col - K)));
  }
  const int64_t trow = (tok0 + 16 * wv + li) * H + h;
  const float* arow = A + trow * kBT;
  float av[2][8];
#pragma unroll
  for (int s = 0; s < 2; ++s) load8f(arow + 32 * s + 8 * grp, av[s], false);
  float bj = 0.f, gj = 0.f;
  if (tid < kBT) {
    const int64_t row = (tok0 + tid) * H + h;
    bj = beta[row];
    gj = g ? g[row] : 0.f;
  }

  // 2. Stage X, beta, g.  X rows are unpadded with the chunk-pair swizzle of
  // xtile_off: the fragment reads below are then free of bank conflicts (a
  // 16-byte row pad left ~0.56 conflict cycles per access).
  char* const xhb = reinterpret_cast<char*>(xhi);
  char* const xlb = reinterpret_cast<char*>(xlo);
#pragma unroll
  for (int it = 0; it < C::kLoads; ++it) {
    const int q = tid + it * kWuThreads;
    const int j = q / C::kCPR;
    const int col = (q - j * C::kCPR) * C::kVE;
    const uint32_t off = hl::xtile_off(j, col, C::kRowB);
    if constexpr (C::kSplitX) {
      float vals[4];
      unpack16(xr[it], vals, 0.f);
      lds_put4(reinterpret_cast<bf16*>(xhb + off), reinterpret_cast<bf16*>(xlb + off), vals, true);
    } else {
      *reinterpret_cast<u32x4*>(xhb + off) = xr[it];
    }
  }
  if (tid < kBT) {
    sbeta[tid] = bj;
    sg[tid] = gj;
  }
  lds_barrier();

  // 3. Scaled A operands: A'[t][j] for j = 32 s + 8 grp + 0..7.
  bf16x8 awh[2], awl[2], auh[2], aul[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float fw[8], fu[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 32 * s + 8 * grp + i;
      const float bb = sbeta[j];
      fu[i] = av[s][i] * bb;
      fw[i] = fu[i] * fast_exp(sg[j]);
    }
    split_bf16x8(fw, awh[s], awl[s]);
    split_bf16x8(fu, auh[s], aul[s]);
  }

  // 4. D[n][t] = sum_j X[j][n] A'[t][j].
#pragma unroll
  for (int nb = 0; nb < C::kNB; ++nb) {
    const bool is_w = 16 * nb < K;
    f32x4 acc = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t o0 = hl::xtr_frag_off(32 * s, 0, 16 * nb, lane, C::kRowB);
      const uint32_t o1 = hl::xtr_frag_off(32 * s, 1, 16 * nb, lane, C::kRowB);
      const bf16x8 xh = concat(ds_read_tr16(reinterpret_cast<const bf16*>(xhb + o0)),
                               ds_read_tr16(reinterpret_cast<const bf16*>(xhb + o1)));
      acc = mfma16x16x32(xh, is_w ? awh[s] : auh[s], acc);
      acc = mfma16x16x32(xh, is_w ? awl[s] : aul[s], acc);
      if constexpr (C::kSplitX) {
        const bf16x8 xl = concat(ds_read_tr16(reinterpret_cast<const bf16*>(xlb + o0)),
                                 ds_read_tr16(reinterpret_cast<const bf16*>(xlb + o1)));
        acc = mfma16x16x32(xl, is_w ? awh[s] : auh[s], acc);
      }
    }
    const int n = 16 * nb + 4 * grp;
    if (is_w) {
      store4(w + trow * K + n, acc);
    } else {
      store4(u + trow * V + (n - K), acc);
    }
  }
}

template <typename IT, int K, int V>
hipError_t launch_wu(const void* k, const void* v, const void* beta, const void* A, const void* g,
                     void* w, void* u, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / kBT;
  const int64_t tiles = B * NT * H;
  hipLaunchKernelGGL((recompute_w_u_kernel<IT, K, V>), dim3((unsigned)tiles), dim3(kWuThreads), 0, s,
                     (const IT*)k, (const IT*)v, (const float*)beta, (const float*)A,
                     (const float*)g, (IT*)w, (IT*)u, T, H, NT);
  return hipGetLastError();
}

template <typename IT>
hipError_t dispatch_kv(int64_t K, int64_t V, const void* k, const void* v, const void* beta,
                       const void* A, const void* g, void* w, void* u, int64_t B, int64_t T,
                       int64_t H, hipStream_t s) {
  if (K == 64 && V == 64) return launch_wu<IT, 64, 64>(k, v, beta, A, g, w, u, B, T, H, s);
  if (K == 64 && V == 128) return launch_wu<IT, 64, 128>(k, v, beta, A, g, w, u, B, T, H, s);
  if (K == 128 && V == 64) return launch_wu<IT, 128, 64>(k, v, beta, A, g, w, u, B, T, H, s);
  return launch_wu<IT, 128, 128>(k, v, beta, A, g, w, u, B, T, H, s);
}

}  // namespace
}  // namespace thm

extern "C" int thm_recompute_w_u_fwd(const void* k, const void* v, const void* beta, const void* A,
                                     const void* g, void* w, void* u, int64_t B, int64_t T,
                                     int64_t H, int64_t K, int64_t V, int32_t chunk_size,
                                     int32_t kv_dtype, void* stream) {
  using namespace thm;
  if (chunk_size != kBT) return THM_ERR_BAD_ARGUMENT;
  if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || T % kBT) return THM_ERR_BAD_SHAPE;
  if (kv_dtype != THM_DTYPE_F32 && kv_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) return THM_ERR_UNSUPPORTED;
  if (B == 0 || T == 0) return THM_OK;  // empty: nothing is read or written
  if (!k || !v || !beta || !A || !w || !u) return THM_ERR_NULL_POINTER;
  const void* ptrs[] = {k, v, A, w, u};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return THM_ERR_MISALIGNED;
  if (((uintptr_t)beta % 4) || (g && ((uintptr_t)g % 4))) return THM_ERR_MISALIGNED;
  if (B * (T / kBT) > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
  if (!launch_fits(B * (T / kBT) * H, kWuThreads)) return THM_ERR_BAD_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = (kv_dtype == THM_DTYPE_F32)
                     ? dispatch_kv<float>(K, V, k, v, beta, A, g, w, u, B, T, H, s)
                     : dispatch_kv<bf16>(K, V, k, v, beta, A, g, w, u, B, T, H, s);
  return (int)e;
}
