// Gated DeltaNet chunkwise output for MI355X (gfx950):
//   o_i = scale ( sum_{j<=i in chunk} (q_i . k_j) e^{g_i - g_j} v_j  +  e^{g_i} q_i . h[c] )
//
// Replaces kernels/chunk_fwd_o/kernel.py:52-136 (Triton) and its launcher
// kernel.py:146-212; math of reference.py:80-142, which uses the equivalent
// factored gates q e^{g}, v e^{-g}.  Here only e^{g_i - g_j} with j <= i is
// formed, which cannot overflow for a non-increasing gate.
//
// One workgroup (4 wavefronts) per (b, chunk, head) tile.  v_c [64 x V] and
// h[c] [K x V] are staged in LDS as bf16 (fp32 inputs: bf16 hi + lo).  Wave wv
// owns query positions i = 16 wv .. 16 wv + 15 and computes o^T (features x
// positions), so each lane ends with 4 consecutive features of one token:
//   1. acc[n][i]  = sum_kappa h[kappa][n] q[i][kappa]          (h^T from LDS via
//      ds_read_b64_tr_b16, q straight from HBM), then acc *= e^{g_i};
//   2. S^T[j][i]  = sum_kappa k[j][kappa] q[i][kappa] for key blocks j <= i;
//      P[i][j] = S^T[j][i] e^{g_i - g_j} (0 for j > i), kept in registers;
//   3. acc[n][i] += sum_j v[j][n] P[i][j]: the P accumulator pairs are the B
//      operand in paired order, v^T comes from LDS in the same order;
//   4. o[i][n..n+3] = scale * acc.
#include <type_traits>

#include "mfma.h"

namespace thm {
namespace {

constexpr int kBT = 64;
constexpr int kOThreads = 256;

template <typename IT, int K, int V>
struct OCfg {
  static constexpr bool kSplit = std::is_same<IT, float>::value;
  static constexpr int kPitch = V + 8;  // LDS row pitch (elements) of the v and h tiles
  static constexpr int kVTile = kBT * kPitch;
  static constexpr int kHTile = K * kPitch;
  static constexpr int kLds = (kSplit ? 2 : 1) * (kVTile + kHTile);
  static constexpr int kVE = 16 / (int)sizeof(IT);
};

template <typename IT, int K, int V>
__global__ void __launch_bounds__(kOThreads)
chunk_fwd_o_kernel(const IT* __restrict__ q, const IT* __restrict__ k, const IT* __restrict__ v,
                   const float* __restrict__ g, const float* __restrict__ hs, IT* __restrict__ o,
                   float scale, int64_t T, int64_t H, int64_t NT) {
  using C = OCfg<IT, K, V>;
  __shared__ __attribute__((aligned(16))) bf16 lds[C::kLds];
  __shared__ float gs[kBT];
  bf16* const vhi = lds;
  bf16* const hhi = lds + C::kVTile;
  bf16* const vlo = lds + C::kVTile + C::kHTile;
  bf16* const hlo = vlo + C::kVTile;

  const int64_t tile = blockIdx.x;
  const int64_t hh = tile % H;
  const int64_t bc = tile / H;
  const int64_t c = bc % NT;
  const int64_t b = bc / NT;
  const int64_t tok0 = b * T + c * kBT;
  const int tid = threadIdx.x;

  // Stage v_c (IT) and h[c] (fp32) as bf16 (hi[, lo]).
  {
    constexpr int VCPR = V / C::kVE;
    for (int qi = tid; qi < kBT * VCPR; qi += kOThreads) {
      const int j = qi / VCPR;
      const int col = (qi - j * VCPR) * C::kVE;
      float vals[C::kVE];
      unpack16(ldg16(v + ((tok0 + j) * H + hh) * V + col), vals, IT{});
      if constexpr (C::kSplit) {
        lds_put4(vhi + j * C::kPitch + col, vlo + j * C::kPitch + col, vals, true);
      } else {
        *reinterpret_cast<bf16x8*>(vhi + j * C::kPitch + col) = to_bf16x8(vals);
      }
    }
    const float* hsrc = hs + ((b * NT + c) * H + hh) * (int64_t)(K * V);
    constexpr int HCPR = V / 4;
    for (int qi = tid; qi < K * HCPR; qi += kOThreads) {
      const int r = qi / HCPR;
      const int col = (qi - r * HCPR) * 4;
      float vals[4];
      unpack16(ldg16(hsrc + r * V + col), vals, 0.f);
      lds_put4(hhi + r * C::kPitch + col, hlo + r * C::kPitch + col, vals, C::kSplit);
    }
    if (tid < kBT) gs[tid] = g ? g[(tok0 + tid) * H + hh] : 0.f;
  }
  __syncthreads();

  const int wv = tid >> 6;
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int i = 16 * wv + li;  // this lane's query position (column of every accumulator)
  const int64_t qrow = (tok0 + i) * H + hh;

  // q fragments, natural contraction order: q[i][32 s + 8 grp + 0..7].
  constexpr int KS = K / 32;
  bf16x8 qh[KS], ql[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if constexpr (C::kSplit) {
      float f[8];
      load8f(q + qrow * K + 32 * s + 8 * grp, f);
      split_bf16x8(f, qh[s], ql[s]);
    } else {
      qh[s] = load8(reinterpret_cast<const bf16*>(q) + qrow * K + 32 * s + 8 * grp);
    }
  }

  // 1. Inter-chunk term.
  constexpr int NB = V / 16;
  f32x4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    acc[nb] = zero4();
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int r0 = tr_row_natural(32 * s, 0), r1 = tr_row_natural(32 * s, 1);
      const bf16x8 hf = frag_tr(hhi, C::kPitch, r0, r1, 16 * nb);
      acc[nb] = mfma16x16x32(hf, qh[s], acc[nb]);
      if constexpr (C::kSplit) {
        acc[nb] = mfma16x16x32(hf, ql[s], acc[nb]);
        const bf16x8 hl = frag_tr(hlo, C::kPitch, r0, r1, 16 * nb);
        acc[nb] = mfma16x16x32(hl, qh[s], acc[nb]);
      }
    }
  }
  const float gi = gs[i];
  const float egi = fast_exp(gi);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] *= egi;

  // 2. Gated, causally masked scores for key blocks jb <= wv.
  f32x4 p[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    p[jb] = zero4();
    if (jb > wv) continue;  // wave-uniform
    const int64_t krow = (tok0 + 16 * jb + li) * H + hh;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if constexpr (C::kSplit) {
        float f[8];
        bf16x8 kh, kl;
        load8f(k + krow * K + 32 * s + 8 * grp, f);
        split_bf16x8(f, kh, kl);
        p[jb] = mfma16x16x32(kh, qh[s], p[jb]);
        p[jb] = mfma16x16x32(kh, ql[s], p[jb]);
        p[jb] = mfma16x16x32(kl, qh[s], p[jb]);
      } else {
        const bf16x8 kf = load8(reinterpret_cast<const bf16*>(k) + krow * K + 32 * s + 8 * grp);
        p[jb] = mfma16x16x32(kf, qh[s], p[jb]);
      }
    }
    // lane holds S^T[j = 16 jb + 4 grp + r][i]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * jb + 4 * grp + r;
      p[jb][r] = (j <= i) ? p[jb][r] * fast_exp(gi - gs[j]) : 0.f;
    }
  }

  // 3. Intra-chunk term: key steps of 32 (block pairs 2s, 2s+1).
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (2 * s > wv) continue;  // wave-uniform: both blocks fully masked
    float f[8] = {p[2 * s][0], p[2 * s][1], p[2 * s][2], p[2 * s][3],
                  p[2 * s + 1][0], p[2 * s + 1][1], p[2 * s + 1][2], p[2 * s + 1][3]};
    bf16x8 ph, pl;
    if constexpr (C::kSplit) {
      split_bf16x8(f, ph, pl);
    } else {
      ph = to_bf16x8(f);
    }
    const int r0 = tr_row_paired(32 * s, 0), r1 = tr_row_paired(32 * s, 1);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const bf16x8 vf = frag_tr(vhi, C::kPitch, r0, r1, 16 * nb);
      acc[nb] = mfma16x16x32(vf, ph, acc[nb]);
      if constexpr (C::kSplit) {
        acc[nb] = mfma16x16x32(vf, pl, acc[nb]);
        const bf16x8 vl = frag_tr(vlo, C::kPitch, r0, r1, 16 * nb);
        acc[nb] = mfma16x16x32(vl, ph, acc[nb]);
      }
    }
  }

  // 4. o[i][16 nb + 4 grp + 0..3].
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) store4(o + qrow * V + 16 * nb + 4 * grp, acc[nb] * scale);
}

template <typename IT, int K, int V>
hipError_t launch_o(const void* q, const void* k, const void* v, const void* g, const void* h,
                    void* o, float scale, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / kBT;
  hipLaunchKernelGGL((chunk_fwd_o_kernel<IT, K, V>), dim3((unsigned)(B * NT * H)), dim3(kOThreads),
                     0, s, (const IT*)q, (const IT*)k, (const IT*)v, (const float*)g,
                     (const float*)h, (IT*)o, scale, T, H, NT);
  return hipGetLastError();
}

template <typename IT>
hipError_t dispatch_o(int64_t K, int64_t V, const void* q, const void* k, const void* v,
                      const void* g, const void* h, void* o, float scale, int64_t B, int64_t T,
                      int64_t H, hipStream_t s) {
  if (K == 64 && V == 64) return launch_o<IT, 64, 64>(q, k, v, g, h, o, scale, B, T, H, s);
  if (K == 64 && V == 128) return launch_o<IT, 64, 128>(q, k, v, g, h, o, scale, B, T, H, s);
  if (K == 128 && V == 64) return launch_o<IT, 128, 64>(q, k, v, g, h, o, scale, B, T, H, s);
  return launch_o<IT, 128, 128>(q, k, v, g, h, o, scale, B, T, H, s);
}

}  // namespace
}  // namespace thm

extern "C" int thm_chunk_fwd_o(const void* q, const void* k, const void* v, const void* g,
                               const void* h, void* o, float scale, int64_t B, int64_t T,
                               int64_t H, int64_t K, int64_t V, int32_t chunk_size,
                               int32_t qkv_dtype, void* stream) {
  using namespace thm;
  if (chunk_size != kBT) return THM_ERR_BAD_ARGUMENT;
  if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || T % kBT) return THM_ERR_BAD_SHAPE;
  if (qkv_dtype != THM_DTYPE_F32 && qkv_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) return THM_ERR_UNSUPPORTED;
  if (B == 0 || T == 0) return THM_OK;  // empty: nothing is read or written
  if (!q || !k || !v || !h || !o) return THM_ERR_NULL_POINTER;
  const void* ptrs[] = {q, k, v, h, o};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return THM_ERR_MISALIGNED;
  if (g && ((uintptr_t)g % 4)) return THM_ERR_MISALIGNED;
  if (B * (T / kBT) > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = (qkv_dtype == THM_DTYPE_F32)
                     ? dispatch_o<float>(K, V, q, k, v, g, h, o, scale, B, T, H, s)
                     : dispatch_o<bf16>(K, V, q, k, v, g, h, o, scale, B, T, H, s);
  return (int)e;
}
