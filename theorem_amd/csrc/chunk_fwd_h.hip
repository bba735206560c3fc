// Gated DeltaNet inter-chunk state recurrence for MI355X (gfx950).
//
// For one (b, head), state S [K x V] fp32 (h0 or 0 at chunk 0), per chunk c
// with g_last = g at the chunk's last token:
//   reference form (DELTA = false; vu = v)                kernels/chunk_fwd_h/
//     S <- e^{g_last} S + k_c^T (v_c e^{g_last - g_c});  h[c] = S      reference.py:50-97
//   delta form (DELTA = true; vu = u)
//     h[c] = S;  v_new = u_c - w_c S;  S <- e^{g_last} S + k_c^T (v_new e^{g_last - g_c})
// Replaces kernels/chunk_fwd_h/kernel.py:61-138 (Triton) and its launcher
// kernel.py:141-191.
//
// One workgroup per (b, head, V-tile of BV columns), BV / 16 wavefronts; wave
// wv owns state columns 16 wv .. 16 wv + 15 of the tile for the whole sequence,
// held in MFMA accumulators (K/16 tiles of 16x16 fp32).  Per chunk:
//   P1 (delta)  v_new^[j][n] = sum_kappa w[j][kappa] S[kappa][n]: the S
//               accumulator pairs are the B operand in paired order, w rows
//               come from LDS in the same order;  v_new = u - that.
//   P2          S = e^{g_last} S + sum_j k[j][kappa] (v_new[j][n] e^{g_last-g_j}):
//               the v_new accumulator pairs (gate folded in) are the B
//               operand, k^T comes from LDS with ds_read_b64_tr_b16.
// The next chunk's k, w, u/v and g are loaded into registers while the
// current chunk computes, then written to the other half of a double-buffered
// LDS stage: the only serial dependency is the state itself.
// Workgroups map XCD-aware: the V-tiles of one (b, head) share an XCD (and its
// L2), so k and w are fetched from HBM once per (b, head).
#include <type_traits>

#include "mfma.h"

namespace thm {
namespace {

constexpr int kBT = 64;

template <typename IT, int K, int BV, bool DELTA>
struct HCfg {
  static constexpr bool kSplit = std::is_same<IT, float>::value;
  static constexpr int kWaves = BV / 16;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kVE = 16 / (int)sizeof(IT);   // elements per 16-byte load
  static constexpr int kKPitch = K + 8;              // bf16 elements
  static constexpr int kUPitch = BV + 16 / (int)sizeof(IT);
  static constexpr int kKTile = kBT * kKPitch;       // bf16 elements
  static constexpr int kUTile = kBT * kUPitch;       // IT elements
  // bf16 elements of one stage: k (hi[, lo]), w (hi[, lo]) when DELTA
  static constexpr int kBf16PerStage = (kSplit ? 2 : 1) * (DELTA ? 2 : 1) * kKTile;
  // 16-byte chunks of one chunk's inputs
  static constexpr int kKChunks = kBT * K / kVE;
  static constexpr int kWChunks = DELTA ? kKChunks : 0;
  static constexpr int kUChunks = kBT * BV / kVE;
  static constexpr int kGChunks = kBT / 4;
  static constexpr int kChunks = kKChunks + kWChunks + kUChunks + kGChunks;
  static constexpr int kPer = (kChunks + kThreads - 1) / kThreads;
  static constexpr int kStageBytes =
      kBf16PerStage * 2 + kUTile * (int)sizeof(IT) + kBT * (int)sizeof(float);
  // Double-buffer the stage when two fit in 128 KiB of LDS; otherwise one stage
  // (fp32 inputs with K = 128) and a barrier before it is overwritten.
  static constexpr int kStages = (2 * kStageBytes <= 128 * 1024) ? 2 : 1;
};

template <typename IT, int K, int BV, bool DELTA>
struct HStage {
  using C = HCfg<IT, K, BV, DELTA>;
  bf16* khi;
  bf16* klo;
  bf16* whi;
  bf16* wlo;
  IT* u;
  float* g;
};

template <typename IT, int K, int BV, bool DELTA>
__device__ __forceinline__ void h_prefetch(u32x4* pf, const IT* k,
                                           const IT* w, const IT* vu, const float* g,
                                           int64_t tok0, int64_t H, int64_t hh, int64_t V,
                                           int64_t v0) {
  using C = HCfg<IT, K, BV, DELTA>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < C::kPer; ++it) {
    const int q = tid + it * C::kThreads;
    if (q >= C::kChunks) break;
    if (q < C::kKChunks + C::kWChunks) {
      const bool isw = q >= C::kKChunks;
      const int qq = isw ? q - C::kKChunks : q;
      constexpr int CPR = K / C::kVE;
      const int j = qq / CPR;
      const int col = (qq - j * CPR) * C::kVE;
      const IT* src = (isw ? w : k) + ((tok0 + j) * H + hh) * K + col;
      pf[it] = ldg16(src);
    } else if (q < C::kKChunks + C::kWChunks + C::kUChunks) {
      const int qq = q - C::kKChunks - C::kWChunks;
      constexpr int CPR = BV / C::kVE;
      const int j = qq / CPR;
      const int col = (qq - j * CPR) * C::kVE;
      pf[it] = ldg16(vu + ((tok0 + j) * H + hh) * V + v0 + col);
    } else {
      const int j0 = (q - C::kKChunks - C::kWChunks - C::kUChunks) * 4;
      if (g) {
        u32x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = __float_as_uint(g[(tok0 + j0 + e) * H + hh]);
        pf[it] = r;
      } else {
        pf[it] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
}

template <typename IT, int K, int BV, bool DELTA>
__device__ __forceinline__ void h_commit(const u32x4* pf,
                                         const HStage<IT, K, BV, DELTA>& st) {
  using C = HCfg<IT, K, BV, DELTA>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < C::kPer; ++it) {
    const int q = tid + it * C::kThreads;
    if (q >= C::kChunks) break;
    if (q < C::kKChunks + C::kWChunks) {
      const bool isw = q >= C::kKChunks;
      const int qq = isw ? q - C::kKChunks : q;
      constexpr int CPR = K / C::kVE;
      const int j = qq / CPR;
      const int col = (qq - j * CPR) * C::kVE;
      const int off = j * C::kKPitch + col;
      if constexpr (C::kSplit) {
        float vals[4];
        unpack16(pf[it], vals, 0.f);
        lds_put4((isw ? st.whi : st.khi) + off, (isw ? st.wlo : st.klo) + off, vals, true);
      } else {
        *reinterpret_cast<u32x4*>((isw ? st.whi : st.khi) + off) = pf[it];
      }
    } else if (q < C::kKChunks + C::kWChunks + C::kUChunks) {
      const int qq = q - C::kKChunks - C::kWChunks;
      constexpr int CPR = BV / C::kVE;
      const int j = qq / CPR;
      const int col = (qq - j * CPR) * C::kVE;
      *reinterpret_cast<u32x4*>(st.u + j * C::kUPitch + col) = pf[it];
    } else {
      const int j0 = (q - C::kKChunks - C::kWChunks - C::kUChunks) * 4;
      *reinterpret_cast<u32x4*>(st.g + j0) = pf[it];
    }
  }
}

template <typename IT, int K, int BV, bool DELTA>
__global__ void __launch_bounds__(BV / 16 * 64)
chunk_fwd_h_kernel(const IT* __restrict__ k, const IT* __restrict__ w, const IT* __restrict__ vu,
                   const float* __restrict__ g, const float* __restrict__ h0,
                   float* __restrict__ hout, IT* __restrict__ vnew, float* __restrict__ ht,
                   int64_t T, int64_t H, int64_t V, int64_t NT, int64_t BH, int n_vt) {
  using C = HCfg<IT, K, BV, DELTA>;
  using St = HStage<IT, K, BV, DELTA>;
  __shared__ __attribute__((aligned(16))) bf16 lds_b[C::kStages * C::kBf16PerStage];
  __shared__ __attribute__((aligned(16))) IT lds_u[C::kStages * C::kUTile];
  __shared__ __attribute__((aligned(16))) float lds_g[C::kStages * kBT];

  // XCD-aware block mapping: block i runs on XCD i % 8; give all V-tiles of a
  // (b, head) the same i % 8 when the grid allows it.
  const int64_t blk = blockIdx.x;
  int64_t bh, vt;
  if (BH % 8 == 0) {
    const int64_t xcd = blk % 8, slot = blk / 8;
    bh = (slot / n_vt) * 8 + xcd;
    vt = slot % n_vt;
  } else {
    bh = blk / n_vt;
    vt = blk % n_vt;
  }
  const int64_t b = bh / H, hh = bh % H;
  const int64_t v0 = vt * BV;

  // Stage i's tiles, by pointer arithmetic (no dynamically indexed array).
  auto stage = [&](int i) {
    St st;
    bf16* base = lds_b + i * C::kBf16PerStage;
    st.khi = base;
    st.klo = base + (C::kSplit ? C::kKTile : 0);
    st.whi = base + (C::kSplit ? 2 : 1) * C::kKTile;
    st.wlo = st.whi + (C::kSplit ? C::kKTile : 0);
    st.u = lds_u + i * C::kUTile;
    st.g = lds_g + i * kBT;
    return st;
  };

  const int tid = threadIdx.x;
  const int wv = tid >> 6;
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int ucol = 16 * wv + li;   // column within the V-tile
  const int64_t vcol = v0 + ucol;  // column within V
  constexpr int KB = K / 16;

  // State: S[kappa = 16 kb + 4 grp + r][vcol] in s[kb][r].
  f32x4 S[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[kb][r] = h0 ? h0[(bh * K + 16 * kb + 4 * grp + r) * V + vcol] : 0.f;
  }

  // One chunk of work on the tiles staged in `cs`.
  auto chunk = [&](const St& cs, int64_t c) {
    const int64_t tok0 = b * T + c * kBT;
    float* hc = hout + ((b * NT + c) * H + hh) * (int64_t)K * V;
    if constexpr (DELTA) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) hc[(16 * kb + 4 * grp + r) * V + vcol] = S[kb][r];
    }

    // v_new (or v) for rows j = 16 jb + 4 grp + r of this lane's column.
    f32x4 vn[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) vn[jb][r] = to_f32(cs.u[(16 * jb + 4 * grp + r) * C::kUPitch + ucol]);
    }
    if constexpr (DELTA) {
      // P1: B operand = S pairs (kappa blocks 2s, 2s+1) in paired order.
      bf16x8 sh[K / 32], sl[K / 32];
#pragma unroll
      for (int s = 0; s < K / 32; ++s) {
        const float f[8] = {S[2 * s][0], S[2 * s][1], S[2 * s][2], S[2 * s][3],
                            S[2 * s + 1][0], S[2 * s + 1][1], S[2 * s + 1][2], S[2 * s + 1][3]};
        if constexpr (C::kSplit) split_bf16x8(f, sh[s], sl[s]);
        else sh[s] = to_bf16x8(f);
      }
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        f32x4 a = zero4();
        const bf16* wrow = cs.whi + (16 * jb + li) * C::kKPitch;
#pragma unroll
        for (int s = 0; s < K / 32; ++s) {
          const bf16x8 wf = load8_paired(wrow, 32 * s);
          a = mfma16x16x32(wf, sh[s], a);
          if constexpr (C::kSplit) {
            a = mfma16x16x32(wf, sl[s], a);
            const bf16x8 wl = load8_paired(cs.wlo + (16 * jb + li) * C::kKPitch, 32 * s);
            a = mfma16x16x32(wl, sh[s], a);
          }
        }
        vn[jb] -= a;
      }
      if (vnew) {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            vnew[((tok0 + 16 * jb + 4 * grp + r) * H + hh) * V + vcol] = from_f32<IT>(vn[jb][r]);
      }
    }

    // P2: S = e^{g_last} S + k^T (v_new e^{g_last - g}).
    const float gl = cs.g[kBT - 1];
    bf16x8 vh[2], vl[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float f[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j0 = 32 * s + 4 * grp + r;
        f[r] = vn[2 * s][r] * fast_exp(gl - cs.g[j0]);
        f[4 + r] = vn[2 * s + 1][r] * fast_exp(gl - cs.g[j0 + 16]);
      }
      if constexpr (C::kSplit) split_bf16x8(f, vh[s], vl[s]);
      else vh[s] = to_bf16x8(f);
    }
    const float decay = fast_exp(gl);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      S[kb] *= decay;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int r0 = tr_row_paired(32 * s, 0), r1 = tr_row_paired(32 * s, 1);
        const bf16x8 kf = frag_tr(cs.khi, C::kKPitch, r0, r1, 16 * kb);
        S[kb] = mfma16x16x32(kf, vh[s], S[kb]);
        if constexpr (C::kSplit) {
          S[kb] = mfma16x16x32(kf, vl[s], S[kb]);
          const bf16x8 kl = frag_tr(cs.klo, C::kKPitch, r0, r1, 16 * kb);
          S[kb] = mfma16x16x32(kl, vh[s], S[kb]);
        }
      }
    }
    if constexpr (!DELTA) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) hc[(16 * kb + 4 * grp + r) * V + vcol] = S[kb][r];
    }

  };

  // The next chunk's loads are issued before the current chunk computes and
  // written to the other LDS stage after it.
  u32x4 pf[C::kPer];
  if (NT > 0) {
    h_prefetch<IT, K, BV, DELTA>(pf, k, w, vu, g, b * T, H, hh, V, v0);
    h_commit<IT, K, BV, DELTA>(pf, stage(0));
    __syncthreads();
  }
  for (int64_t c = 0; c < NT; ++c) {
    if (c + 1 < NT) h_prefetch<IT, K, BV, DELTA>(pf, k, w, vu, g, b * T + (c + 1) * kBT, H, hh, V, v0);
    chunk(stage((int)(c % C::kStages)), c);
    if (c + 1 < NT) {
      if constexpr (C::kStages == 1) __syncthreads();  // every wave is done with the stage
      h_commit<IT, K, BV, DELTA>(pf, stage((int)((c + 1) % C::kStages)));
    }
    __syncthreads();
  }

  if (ht) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) ht[(bh * K + 16 * kb + 4 * grp + r) * V + vcol] = S[kb][r];
  }
}

template <typename IT, int K, int BV, bool DELTA>
hipError_t launch_h(const void* k, const void* w, const void* vu, const void* g, const void* h0,
                    void* h, void* vnew, void* ht, int64_t B, int64_t T, int64_t H, int64_t V,
                    hipStream_t s) {
  using C = HCfg<IT, K, BV, DELTA>;
  const int64_t NT = T / kBT;
  const int n_vt = (int)(V / BV);
  const int64_t BH = B * H;
  hipLaunchKernelGGL((chunk_fwd_h_kernel<IT, K, BV, DELTA>), dim3((unsigned)(BH * n_vt)),
                     dim3(C::kThreads), 0, s, (const IT*)k, (const IT*)w, (const IT*)vu,
                     (const float*)g, (const float*)h0, (float*)h, (IT*)vnew, (float*)ht, T, H, V,
                     NT, BH, n_vt);
  return hipGetLastError();
}

// V-tiles of 64 columns (4 wavefronts): the four waves share the staging of
// each chunk's k / w / u, which keeps the per-thread prefetch buffer small.
template <typename IT, int K, bool DELTA>
hipError_t dispatch_bv(int64_t V, const void* k, const void* w, const void* vu, const void* g,
                       const void* h0, void* h, void* vnew, void* ht, int64_t B, int64_t T,
                       int64_t H, hipStream_t s) {
  return launch_h<IT, K, 64, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, V, s);
}

template <typename IT>
hipError_t dispatch_h(int64_t K, bool delta, int64_t V, const void* k, const void* w,
                      const void* vu, const void* g, const void* h0, void* h, void* vnew,
                      void* ht, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  if (K == 64) {
    return delta ? dispatch_bv<IT, 64, true>(V, k, w, vu, g, h0, h, vnew, ht, B, T, H, s)
                 : dispatch_bv<IT, 64, false>(V, k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
  }
  return delta ? dispatch_bv<IT, 128, true>(V, k, w, vu, g, h0, h, vnew, ht, B, T, H, s)
               : dispatch_bv<IT, 128, false>(V, k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
}

}  // namespace
}  // namespace thm

extern "C" int thm_chunk_fwd_h(const void* k, const void* w, const void* vu, const void* g,
                               const void* h0, void* h, void* v_new, void* ht, int64_t B,
                               int64_t T, int64_t H, int64_t K, int64_t V, int32_t chunk_size,
                               int32_t kv_dtype, int32_t flags, void* stream) {
  using namespace thm;
  if (flags & ~THM_H_DELTA) return THM_ERR_BAD_ARGUMENT;
  const bool delta = (flags & THM_H_DELTA) != 0;
  if (!delta && v_new) return THM_ERR_BAD_ARGUMENT;  // v_new exists only in the delta form
  if (chunk_size != kBT) return THM_ERR_BAD_ARGUMENT;
  if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || T % kBT) return THM_ERR_BAD_SHAPE;
  if (kv_dtype != THM_DTYPE_F32 && kv_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) return THM_ERR_UNSUPPORTED;
  if (B == 0) return THM_OK;
  if (T == 0 && !ht) return THM_OK;  // no chunks and no final state: nothing to write
  // With T == 0 only h0 (optional) is read and ht written.
  if (T > 0 && (!k || !vu || !h || (delta && !w))) return THM_ERR_NULL_POINTER;
  const void* ptrs16[] = {k, vu, w};
  for (const void* p : ptrs16)
    if (p && ((uintptr_t)p % 16)) return THM_ERR_MISALIGNED;
  const void* ptrs4[] = {g, h0, h, v_new, ht};
  for (const void* p : ptrs4)
    if (p && ((uintptr_t)p % 4)) return THM_ERR_MISALIGNED;
  if (v_new && kv_dtype == THM_DTYPE_BF16 && ((uintptr_t)v_new % 2)) return THM_ERR_MISALIGNED;
  if (B > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = (kv_dtype == THM_DTYPE_F32)
                     ? dispatch_h<float>(K, delta, V, k, w, vu, g, h0, h, v_new, ht, B, T, H, s)
                     : dispatch_h<bf16>(K, delta, V, k, w, vu, g, h0, h, v_new, ht, B, T, H, s);
  return (int)e;
}
