// Gated DeltaNet inter-chunk state recurrence, register-prefetch kernel
// (included by chunk_fwd_h.hip for bf16 inputs and by chunk_fwd_h_f32.hip for
// fp32 inputs; the two are compiled with different code-generation options).
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
// One workgroup per (b, head, V-tile of 64 columns), 4 wavefronts; wave wv
// owns state columns 16 wv .. 16 wv + 15 of the tile for the whole sequence,
// held in MFMA accumulators (K/16 tiles of 16x16 fp32).  Per chunk:
//   P1 (delta)  v_new^[j][n] = sum_kappa w[j][kappa] S[kappa][n]: the S
//               accumulator pairs are the B operand in paired order, w rows
//               come from LDS in the same order;  v_new = u - that.
//   P2          S = e^{g_last} S + sum_j k[j][kappa] (v_new[j][n] e^{g_last-g_j}):
//               the v_new accumulator pairs (gate folded in) are the B
//               operand, k^T comes from LDS with ds_read_b64_tr_b16.
// The next chunk's k, w, u/v and g are loaded into registers while the
// current chunk computes, then written to the other half of a double-buffered
// LDS stage: the only serial dependency is the state itself.  Every address
// in the chunk loop is a wave-uniform chunk base plus a per-lane 32-bit offset
// fixed before the loop, so the loop spends no VALU on address arithmetic.
// Workgroups map XCD-aware: the V-tiles of one (b, head) share an XCD (and its
// L2), so k and w are fetched from HBM once per (b, head).
//
// bf16 inputs on grids that fill the GPU use a second kernel
// (chunk_fwd_h.hip): chunk tiles arrive by global -> LDS DMA instead of
// through registers, and the K rows of the state are split over two waves per
// SIMD.
#pragma once

#include <type_traits>

#include "h_layout.h"
#include "mfma.h"
#include "vmem.h"

namespace thm {
namespace {

constexpr int kBT = 64;
constexpr int kHBV = 64;        // V-tile width
constexpr int kHThreads = 256;  // 4 wavefronts x 16 state columns

template <typename IT, int K, int V, bool DELTA>
struct HCfg {
  static constexpr bool kSplit = std::is_same<IT, float>::value;
  static constexpr int kEB = (int)sizeof(IT);
  static constexpr int kVE = 16 / kEB;               // elements per 16-byte load
  static constexpr int kKPitch = K + 8;              // bf16 elements (16-byte pad)
  static constexpr int kUPitch = kHBV + kVE;         // IT elements (16-byte pad)
  static constexpr int kKTile = kBT * kKPitch;       // bf16 elements
  static constexpr int kUTile = kBT * kUPitch;       // IT elements
  // bf16 elements of one stage: k (hi[, lo]), w (hi[, lo]) when DELTA
  static constexpr int kBf16PerStage = (kSplit ? 2 : 1) * (DELTA ? 2 : 1) * kKTile;
  // per-thread 16-byte load slots of one chunk
  static constexpr int kKCPR = K / kVE;              // 16-byte chunks per k / w row
  static constexpr int kKLoads = kBT * kKCPR / kHThreads;
  static constexpr int kUCPR = kHBV / kVE;           // 16-byte chunks per u row of the tile
  static constexpr int kULoads = kBT * kUCPR / kHThreads;
  static_assert(kHThreads % kKCPR == 0 && kHThreads % kUCPR == 0, "slot mapping");
  static_assert(kBT * kKCPR % kHThreads == 0 && kBT * kUCPR % kHThreads == 0, "slot count");
  static constexpr int kStageBytes =
      kBf16PerStage * 2 + kUTile * kEB + kBT * (int)sizeof(float);
  // Double-buffer the stage when two fit in 128 KiB of LDS; otherwise one stage
  // (fp32 inputs with K = 128) and a barrier before it is overwritten.
  static constexpr int kStages = (2 * kStageBytes <= 128 * 1024) ? 2 : 1;
};

template <typename IT>
struct HStage {
  bf16* khi;
  bf16* klo;
  bf16* whi;
  bf16* wlo;
  IT* u;
  float* g;
};

// One chunk's loads, in registers.
template <typename IT, int K, int V, bool DELTA>
struct HPrefetch {
  using C = HCfg<IT, K, V, DELTA>;
  u32x4 k[C::kKLoads];
  u32x4 w[DELTA ? C::kKLoads : 1];
  u32x4 u[C::kULoads];
  float g;  // gate of token lane_id() of the chunk
};

__device__ __forceinline__ const char* cptr(const void* p, int64_t byte_off) {
  return reinterpret_cast<const char*>(p) + byte_off;
}

// DEEP: two register sets, two chunks ahead (see the chunk loop below).
template <typename IT, int K, int V, bool DELTA, bool HAS_G, bool DEEP>
__global__ void __launch_bounds__(kHThreads)
chunk_fwd_h_kernel(const IT* __restrict__ k, const IT* __restrict__ w, const IT* __restrict__ vu,
                   const float* __restrict__ g, const float* __restrict__ h0,
                   float* __restrict__ hout, IT* __restrict__ vnew, float* __restrict__ ht,
                   int64_t T, int64_t H, int64_t NT, int64_t BH) {
  using C = HCfg<IT, K, V, DELTA>;
  using St = HStage<IT>;
  using Pf = HPrefetch<IT, K, V, DELTA>;
  constexpr int KB = K / 16;
  constexpr int NVT = V / kHBV;
  constexpr int EB = C::kEB;
  __shared__ __attribute__((aligned(16))) bf16 lds_b[C::kStages * C::kBf16PerStage];
  __shared__ __attribute__((aligned(16))) IT lds_u[C::kStages * C::kUTile];
  __shared__ __attribute__((aligned(16))) float lds_g[C::kStages * kBT];

  // XCD-aware block mapping: block i runs on XCD i % 8; give all V-tiles of a
  // (b, head) the same i % 8 when the grid allows it.
  const int64_t blk = blockIdx.x;
  int64_t bh, vt;
  if (BH % 8 == 0) {
    const int64_t xcd = blk % 8, slot = blk / 8;
    bh = (slot / NVT) * 8 + xcd;
    vt = slot % NVT;
  } else {
    bh = blk / NVT;
    vt = blk % NVT;
  }
  const int64_t b = bh / H, hh = bh % H;
  const int v0 = (int)vt * kHBV;

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
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int ucol = 16 * wv + li;  // column within the V-tile
  const int vcol = v0 + ucol;     // column within V

  // ---- per-lane offsets, fixed for the whole sequence ----------------------
  // Token t of chunk c, head hh lives at element ((b*T + c*64 + t) * H + hh) * D.
  const int64_t tok_stride_k = H * K * EB;  // bytes between tokens of k / w
  const int64_t tok_stride_v = H * V * EB;  // bytes between tokens of u / v / v_new
  const int kj0 = tid / C::kKCPR, kcol = (tid % C::kKCPR) * C::kVE;
  const int uj0 = tid / C::kUCPR, ucol0 = (tid % C::kUCPR) * C::kVE;
  const uint32_t koff0 = (uint32_t)(kj0 * tok_stride_k + kcol * EB);
  const uint32_t kstep = (uint32_t)((kHThreads / C::kKCPR) * tok_stride_k);
  const uint32_t uoff0 = (uint32_t)(uj0 * tok_stride_v + (v0 + ucol0) * EB);
  const uint32_t ustep = (uint32_t)((kHThreads / C::kUCPR) * tok_stride_v);
  const uint32_t goff = (uint32_t)(lane * H * 4);  // every wave: token `lane` of the chunk
  // chunk bases (bytes from the tensor start), advanced per chunk
  const int64_t kc0 = ((b * T) * H + hh) * K * EB;
  const int64_t uc0 = ((b * T) * H + hh) * V * EB;
  const int64_t gc0 = ((b * T) * H + hh) * 4;
  const int64_t kcs = kBT * tok_stride_k, ucs = kBT * tok_stride_v, gcs = kBT * H * 4;

  auto prefetch = [&](Pf& pf, int64_t c) {
    const char* kb = cptr(k, kc0 + c * kcs);
#pragma unroll
    for (int it = 0; it < C::kKLoads; ++it) pf.k[it] = ldg16(kb + koff0 + it * kstep);
    if constexpr (DELTA) {
      const char* wb = cptr(w, kc0 + c * kcs);
#pragma unroll
      for (int it = 0; it < C::kKLoads; ++it) pf.w[it] = ldg16(wb + koff0 + it * kstep);
    }
    const char* ub = cptr(vu, uc0 + c * ucs);
#pragma unroll
    for (int it = 0; it < C::kULoads; ++it) pf.u[it] = ldg16(ub + uoff0 + it * ustep);
    // Every wave loads the chunk's 64 gates (one per lane): no branch around a
    // memory operation, so the chunk loop issues the same VMEM sequence on
    // every path and the waits at the commit cover exactly the prefetch.
    if constexpr (HAS_G) pf.g = *reinterpret_cast<const float*>(cptr(g, gc0 + c * gcs) + goff);
    else pf.g = 0.f;
  };
  auto commit = [&](const Pf& pf, const St& st) {
#pragma unroll
    for (int it = 0; it < C::kKLoads; ++it) {
      const int off = (kj0 + it * (kHThreads / C::kKCPR)) * C::kKPitch + kcol;
      if constexpr (C::kSplit) {
        float vals[4];
        unpack16(pf.k[it], vals, 0.f);
        lds_put4(st.khi + off, st.klo + off, vals, true);
        if constexpr (DELTA) {
          unpack16(pf.w[it], vals, 0.f);
          lds_put4(st.whi + off, st.wlo + off, vals, true);
        }
      } else {
        *reinterpret_cast<u32x4*>(st.khi + off) = pf.k[it];
        if constexpr (DELTA) *reinterpret_cast<u32x4*>(st.whi + off) = pf.w[it];
      }
    }
#pragma unroll
    for (int it = 0; it < C::kULoads; ++it) {
      const int off = (uj0 + it * (kHThreads / C::kUCPR)) * C::kUPitch + ucol0;
      *reinterpret_cast<u32x4*>(st.u + off) = pf.u[it];
    }
    if (wv == 0) st.g[lane] = pf.g;
  };

  // State: S[kappa = 16 kb + 4 grp + r][vcol] in S[kb][r].
  f32x4 S[KB];
  const uint32_t s_off = (uint32_t)((4 * grp * V + vcol) * 4);  // + (16 kb + r) * V * 4
  const int64_t st_base = bh * (int64_t)(K * V) * 4;             // h0 / ht (bytes)
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[kb][r] = h0 ? *reinterpret_cast<const float*>(cptr(h0, st_base) + s_off + (16 * kb + r) * V * 4) : 0.f;

  // v_new rows j = 16 jb + 4 grp + r of this lane's column, relative to the chunk base.
  // (h and v_new are stored one element per lane: 16 consecutive lanes cover
  // 64 / 32 contiguous bytes of a row.  The row-quad re-layout of the DMA
  // kernel below is slower here: 31.0 against 25.6 us at config 3.)
  const uint32_t vn_off = (uint32_t)(4 * grp * tok_stride_v + vcol * EB);
  auto store_state = [&](int64_t c) {
    char* hb = reinterpret_cast<char*>(hout) + ((b * NT + c) * H + hh) * (int64_t)(K * V) * 4;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<float*>(hb + s_off + (16 * kb + r) * V * 4) = S[kb][r];
  };

  // With DEEP, two register sets run two chunks ahead: at chunk c `cur`
  // holds chunk c + 1 (its loads issued during chunk c - 1) and `nxt`
  // receives chunk c + 2, so the commit at the end of chunk c waits for loads
  // a whole chunk old.  Without it one set is loaded at the top of chunk c
  // and committed at its end.  DEEP is faster on large grids (fp32 at config
  // 4: 890 -> 779 us) and slower on small ones (fp32 config 3: 38.9 -> 46.7
  // us), where the chunk's own latency chain, not the loads, sets the period.
  Pf pa, pb;
  if (NT > 0) {
    prefetch(pa, 0);
    commit(pa, stage(0));
    if (DEEP && NT > 1) prefetch(pa, 1);
    lds_barrier();
  }
  auto chunk = [&](int64_t c, Pf& cur, Pf& nxt) {
    const St cs = stage((int)(c % C::kStages));
    {
      const int64_t pc = DEEP ? c + 2 : c + 1;
      if (pc < NT) prefetch(nxt, pc);
    }
    if constexpr (DELTA) store_state(c);  // state before chunk c

    // v_new (or v) for rows j = 16 jb + 4 grp + r of this lane's column.
    f32x4 vn[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int r = 0; r < 4; ++r) vn[jb][r] = to_f32(cs.u[(16 * jb + 4 * grp + r) * C::kUPitch + ucol]);

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
    if constexpr (!DELTA) store_state(c);  // state after chunk c

    if (c + 1 < NT) {
      if constexpr (C::kStages == 1) lds_barrier();  // every wave is done with the stage
      commit(cur, stage((int)((c + 1) % C::kStages)));
    }
    lds_barrier();
    // v_new after the commit: stores queued behind the prefetch would make its
    // wait cover them too (loads and stores share one in-order counter).
    if constexpr (DELTA) {
      if (vnew) {
        char* vb = reinterpret_cast<char*>(vnew) + (((b * T + c * kBT) * H + hh) * V) * EB;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            *reinterpret_cast<IT*>(vb + vn_off + (16 * jb + r) * tok_stride_v) = from_f32<IT>(vn[jb][r]);
      }
    }
  };
  if constexpr (DEEP) {
    for (int64_t c = 0; c < NT; c += 2) {
      chunk(c, pa, pb);
      if (c + 1 < NT) chunk(c + 1, pb, pa);
    }
  } else {
    for (int64_t c = 0; c < NT; ++c) chunk(c, pa, pa);
  }

  if (ht) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<float*>(reinterpret_cast<char*>(ht) + st_base + s_off + (16 * kb + r) * V * 4) = S[kb][r];
  }
}

// Grids of at least this many workgroups are bandwidth-bound: the register
// kernel then prefetches two chunks ahead (DEEP), and bf16 inputs take the
// DMA pipeline of chunk_fwd_h.hip instead.
constexpr int64_t kHDmaMinGrid = 256;

template <typename IT, int K, int V, bool DELTA>
hipError_t launch_h(const void* k, const void* w, const void* vu, const void* g, const void* h0,
                    void* h, void* vnew, void* ht, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / kBT;
  const int64_t BH = B * H;
  const dim3 grid((unsigned)(BH * (V / kHBV)));
  const bool deep = BH * (V / kHBV) >= kHDmaMinGrid;  // bandwidth-bound regime
#define THM_H_LAUNCH(HG, DP)                                                                      \
  hipLaunchKernelGGL((chunk_fwd_h_kernel<IT, K, V, DELTA, HG, DP>), grid, dim3(kHThreads), 0, s,  \
                     (const IT*)k, (const IT*)w, (const IT*)vu, (const float*)g, (const float*)h0, \
                     (float*)h, (IT*)vnew, (float*)ht, T, H, NT, BH)
  if (g) {
    if (deep) THM_H_LAUNCH(true, true);
    else THM_H_LAUNCH(true, false);
  } else {
    if (deep) THM_H_LAUNCH(false, true);
    else THM_H_LAUNCH(false, false);
  }
#undef THM_H_LAUNCH
  return hipGetLastError();
}

// fp32 inputs, defined in chunk_fwd_h_f32.hip: the register kernel for every
// (K, V) and form.
}  // namespace
__attribute__((visibility("hidden"))) hipError_t chunk_fwd_h_f32(bool delta, int64_t K, int64_t V, const void* k, const void* w, const void* vu,
                           const void* g, const void* h0, void* h, void* vnew, void* ht, int64_t B, int64_t T,
                           int64_t H, hipStream_t s);
}  // namespace thm
