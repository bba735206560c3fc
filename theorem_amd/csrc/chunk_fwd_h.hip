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
// bf16 inputs on grids that fill the GPU use a second kernel (below): chunk
// tiles arrive by global -> LDS DMA instead of through registers, and the K
// rows of the state are split over two waves per SIMD.
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
  const int wv = tid >> 6;
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

// ---------------------------------------------------------------------------
// bf16 inputs: DMA pipeline.
//
// One workgroup per (b, head, V-tile of 64 columns) of 4 KS wavefronts: wave
// w = 4 kh + wq owns state rows [kh K/KS, (kh + 1) K/KS) and columns
// 16 wq .. 16 wq + 15 of the tile.  Chunk tiles (k, w, u or v, g) are copied
// global -> LDS by DMA into a ring of NS stages, NS - 1 chunks ahead of use,
// with no registers held for them; the tiles are stored unpadded with the XOR
// swizzle of h_layout.h.  Per chunk c:
//   wait for this wave's DMA of chunk c, barrier A, issue the DMA of chunk
//   c + NS - 1 into the stage chunk c - 1 used;
//   P1 (delta form) v_new = u - w S (with KS = 2 each K half forms a partial
//   sum, exchanged through LDS behind barrier B);  v_new stored;
//   P2: S = e^{g_last} S + k^T (v_new e^{g_last - g}) on this wave's rows,
//   one 16-row tile at a time; h[c] = S is stored tile by tile inside P2,
//   before each tile's update (delta form) or after it (reference form).
// h and v_new are written as 16- / 8-byte lane stores after the accumulators
// are re-laid out so that each quad of lanes covers one contiguous piece of a
// row (vmem.h acc_to_row_quads); only wave 0 loads the chunk's gates (a
// strided 64-lane gather is the costliest DMA instruction per byte).  The
// address unit of a CU, not HBM, bounded the earlier layout: at B = 1 (32
// workgroups) a chunk took ~5800 cycles, of which ~4600 were address-unit
// time for the chunk's DMA and stores.  Every DMA and store of the chunk loop is
// issued through vmem.h, so the wait at the top of the loop is an exact count:
// after this wave's DMA of chunk c it has issued NS - 1 chunks of stores and
// NS - 2 chunks of DMA.
template <int K, int KS, int NS, bool DELTA, bool HAS_G, bool STORE_VN>
struct PCfg {
  static constexpr int kWaves = 4 * KS;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kRowK = K * 2;                   // bytes per k / w row
  static constexpr int kTileK = kBT * kRowK;            // bytes per k / w tile
  static constexpr int kRowU = kHBV * 2;                // bytes per u row of the V-tile
  static constexpr int kTileU = kBT * kRowU;
  static constexpr int kGBytes = 1024;                  // the chunk's 64 gates (wave 0's DMA), padded
  static constexpr int kStage = kTileK * (DELTA ? 2 : 1) + kTileU + (HAS_G ? kGBytes : 0);
  static constexpr int kXBytes = (DELTA && KS == 2) ? kWaves * 4 * 64 * 16 : 0;  // P1 partials
  static constexpr int kLds = NS * kStage + kXBytes;
  static constexpr int kRows = K / KS;                  // state rows per wave
  static constexpr int KBH = kRows / 16;                // 16-row accumulator tiles per wave
  static constexpr int kKDma = kTileK / 1024 / kWaves;  // 1 KiB DMA instructions per wave per k tile
  static constexpr int kUDma = kTileU / 1024 / kWaves;
  static constexpr int kJbStore = 4 / KS;               // v_new row tiles stored per wave
  // DMA instructions per chunk: every wave's share of the k, w, u tiles, plus
  // the gate load that only wave 0 issues.
  static constexpr int kDma = kKDma * (DELTA ? 2 : 1) + kUDma;
  static constexpr int kDma0 = kDma + (HAS_G ? 1 : 0);
  static constexpr int kStores = KBH + ((DELTA && STORE_VN) ? kJbStore : 0);
  static constexpr int kWaitFirst = (NS - 2) * kDma;
  static constexpr int kWaitFirst0 = (NS - 2) * kDma0;
  static constexpr int kWaitSteady = (NS - 1) * kStores + (NS - 2) * kDma;
  static constexpr int kWaitSteady0 = (NS - 1) * kStores + (NS - 2) * kDma0;
  static_assert(KS == 1 || KS == 2, "K split");
  static_assert(NS >= 2, "at least double buffering");
  static_assert(kKDma >= 1 && kUDma >= 1, "whole DMA instructions per wave");
  static_assert(kStage % 1024 == 0, "1 KiB aligned stages");
  static_assert(kLds <= 160 * 1024, "LDS budget");
  static_assert(kWaitSteady0 <= 63, "vmcnt range");
};

template <int K, int V, int KS, int NS, bool DELTA, bool HAS_G, bool STORE_VN>
__global__ void __launch_bounds__(256 * KS)
chunk_fwd_h_dma_kernel(const bf16* __restrict__ k, const bf16* __restrict__ w,
                       const bf16* __restrict__ vu, const float* __restrict__ g,
                       const float* __restrict__ h0, float* __restrict__ hout,
                       bf16* __restrict__ vnew, float* __restrict__ ht, int64_t T, int64_t H,
                       int64_t NT, int64_t BH) {
  using C = PCfg<K, KS, NS, DELTA, HAS_G, STORE_VN>;
  constexpr int NVT = V / kHBV;
  __shared__ __attribute__((aligned(1024))) char lds[C::kLds];

  const int64_t blk = blockIdx.x;
  int64_t bh, vt;
  if (BH % 8 == 0) {  // the V-tiles of one (b, head) on one XCD (block i runs on XCD i % 8)
    const int64_t xcd = blk % 8, slot = blk / 8;
    bh = (slot / NVT) * 8 + xcd;
    vt = slot % NVT;
  } else {
    bh = blk / NVT;
    vt = blk % NVT;
  }
  const int64_t b = bh / H, hh = bh % H;
  const int v0 = (int)vt * kHBV;

  const int tid = threadIdx.x;
  const int wi = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kh = wi >> 2, wq = wi & 3;
  const int lane = tid & 63, grp = lane >> 4, li = lane & 15;
  const int kap0 = kh * C::kRows;

  auto stage_k = [&](int s) { return lds + s * C::kStage; };
  auto stage_w = [&](int s) { return lds + s * C::kStage + C::kTileK; };
  auto stage_u = [&](int s) { return lds + s * C::kStage + C::kTileK * (DELTA ? 2 : 1); };
  auto stage_g = [&](int s) {
    return reinterpret_cast<float*>(lds + s * C::kStage + C::kTileK * (DELTA ? 2 : 1) + C::kTileU);
  };
  float* const xbuf = reinterpret_cast<float*>(lds + NS * C::kStage);

  // Global geometry in bytes.  Token t of chunk c, head hh: ((b T + 64 c + t) H + hh) D.
  const int64_t tsk = H * K * 2, tsv = H * V * 2;
  const int64_t kc0 = ((b * T) * H + hh) * K * 2;
  const int64_t uc0 = ((b * T) * H + hh) * V * 2 + v0 * 2;
  const int64_t gc0 = ((b * T) * H + hh) * 4;
  const int64_t kcs = kBT * tsk, ucs = kBT * tsv, gcs = kBT * H * 4;

  // Per-lane DMA source offsets within a chunk (fixed for the sequence).
  uint32_t koff[C::kKDma], uoff[C::kUDma];
#pragma unroll
  for (int i = 0; i < C::kKDma; ++i) {
    const int P = (wi * C::kKDma + i) * 64 + lane;
    koff[i] = (uint32_t)(hl::dma_row(P, C::kRowK) * tsk + hl::dma_chunk(P, C::kRowK) * 16);
  }
#pragma unroll
  for (int i = 0; i < C::kUDma; ++i) {
    const int P = (wi * C::kUDma + i) * 64 + lane;
    uoff[i] = (uint32_t)(hl::dma_row(P, C::kRowU) * tsv + hl::dma_chunk(P, C::kRowU) * 16);
  }
  const uint32_t goff = (uint32_t)(lane * H * 4);

  auto issue = [&](int64_t cc, int s) {
    const char* kb = reinterpret_cast<const char*>(k) + kc0 + cc * kcs;
    const uint32_t lk = lds_address(stage_k(s)) + wi * C::kKDma * 1024;
#pragma unroll
    for (int i = 0; i < C::kKDma; ++i) dma_b128(kb, koff[i], __builtin_amdgcn_readfirstlane(lk + i * 1024));
    if constexpr (DELTA) {
      const char* wb = reinterpret_cast<const char*>(w) + kc0 + cc * kcs;
      const uint32_t lw = lds_address(stage_w(s)) + wi * C::kKDma * 1024;
#pragma unroll
      for (int i = 0; i < C::kKDma; ++i) dma_b128(wb, koff[i], __builtin_amdgcn_readfirstlane(lw + i * 1024));
    }
    const char* ub = reinterpret_cast<const char*>(vu) + uc0 + cc * ucs;
    const uint32_t lu = lds_address(stage_u(s)) + wi * C::kUDma * 1024;
#pragma unroll
    for (int i = 0; i < C::kUDma; ++i) dma_b128(ub, uoff[i], __builtin_amdgcn_readfirstlane(lu + i * 1024));
    if constexpr (HAS_G) {
      // One copy of the gates for the workgroup: a 64-lane gather at a
      // 4 H-byte stride costs the address unit ~60 cycles per instruction.
      if (wi == 0) {
        const char* gb = reinterpret_cast<const char*>(g) + gc0 + cc * gcs;
        dma_b32(gb, goff, __builtin_amdgcn_readfirstlane(lds_address(stage_g(s))));
      }
    }
  };

  // State S[kappa = kap0 + 16 kb + 4 grp + r][n = v0 + 16 wq + li] in S[kb][r].
  f32x4 S[C::KBH];
  const int ncol = v0 + 16 * wq + li;
  const int64_t st_base = bh * (int64_t)(K * V);
#pragma unroll
  for (int kb = 0; kb < C::KBH; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[kb][r] = h0 ? h0[st_base + (int64_t)(kap0 + 16 * kb + 4 * grp + r) * V + ncol] : 0.f;
  // Retire the h0 loads here: a load still pending at the loop entry would
  // make the compiler wait for every outstanding operation inside the loop.
  wait_vmcnt<0>();

  // Store offsets after acc_to_row_quads: lane (grp, 4 ra + cb) holds row
  // 4 grp + ra of a 16-row tile at columns 16 wq + 4 cb .. + 3.
  const int ra = li >> 2, cb = li & 3;
  const uint32_t hoff0 = (uint32_t)(((kap0 + 4 * grp + ra) * V + v0 + 16 * wq + 4 * cb) * 4);
  const uint32_t vnoff0 = (uint32_t)((4 * grp + ra) * tsv + (v0 + 16 * wq + 4 * cb) * 2);
  // One 16-row tile of h[c] (this wave's rows 16 kb .. 16 kb + 15).  The tiles
  // are stored one at a time inside P2, each next to the MFMAs that update
  // it, instead of as a burst after the chunk's DMA issue: 441 against 483 us
  // at config 4, the stores no longer queue ahead of the next chunk's loads.
  auto store_h_tile = [&](int64_t c, int kb) {
    float* hb = hout + ((b * NT + c) * H + hh) * (int64_t)(K * V);
    st_b128(hb, hoff0 + (uint32_t)(kb * 16 * V * 4), __builtin_bit_cast(u32x4, acc_to_row_quads(S[kb])));
  };

  if (NT > 0) {
#pragma unroll
    for (int i = 0; i < NS - 1; ++i) issue(i < NT ? i : NT - 1, i);
  }
  for (int64_t c = 0; c < NT; ++c) {
    const int s = (int)(c % NS);
    if (wi == 0) {
      if (c < NS - 1) wait_vmcnt<C::kWaitFirst0>();
      else wait_vmcnt<C::kWaitSteady0>();
    } else {
      if (c < NS - 1) wait_vmcnt<C::kWaitFirst>();
      else wait_vmcnt<C::kWaitSteady>();
    }
    lds_barrier();  // A: chunk c is in LDS; every wave is done with chunk c - 1
    {
      const int64_t cn = c + NS - 1;
      issue(cn < NT ? cn : NT - 1, (int)(cn % NS));
    }

    const char* tk = stage_k(s);
    const char* tu = stage_u(s);
    // Every LDS read of the chunk is issued here, before any of the work that
    // uses it, so the reads' latencies overlap each other and the VALU work
    // below (at one LDS round trip per MFMA pair the chunk body took ~2900
    // cycles).  The compiler keeps this order: the sched_barrier stops it from
    // sinking the reads next to their uses.
    // u (or v) rows j = 16 jb + 4 grp + r of column 16 wq + li.
    bf16x4 ur[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
      ur[jb] = ds_read_tr16(reinterpret_cast<const bf16*>(
          tu + hl::tile_off(16 * jb + 4 * grp + (li >> 2), 16 * wq + 4 * (li & 3), C::kRowU)));
    // w rows 16 jb + li, this wave's K elements, paired order (A operand of P1).
    bf16x4 wa[DELTA ? 4 : 1][C::KBH / 2][2];
    if constexpr (DELTA) {
      const char* tw = stage_w(s);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int s2 = 0; s2 < C::KBH / 2; ++s2) {
          const int e0 = kap0 + 32 * s2 + 4 * grp;
          wa[jb][s2][0] = *reinterpret_cast<const bf16x4*>(tw + hl::tile_off(16 * jb + li, e0, C::kRowK));
          wa[jb][s2][1] = *reinterpret_cast<const bf16x4*>(tw + hl::tile_off(16 * jb + li, e0 + 16, C::kRowK));
        }
    }
    // k^T fragments of this wave's state rows (A operand of P2), paired order.
    bf16x4 ka[C::KBH][2][2];
#pragma unroll
    for (int kb = 0; kb < C::KBH; ++kb)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int col = kap0 + 16 * kb + 4 * (li & 3);
        ka[kb][s2][0] = ds_read_tr16(reinterpret_cast<const bf16*>(
            tk + hl::tile_off(32 * s2 + 4 * grp + (li >> 2), col, C::kRowK)));
        ka[kb][s2][1] = ds_read_tr16(reinterpret_cast<const bf16*>(
            tk + hl::tile_off(32 * s2 + 16 + 4 * grp + (li >> 2), col, C::kRowK)));
      }
    // Gates of this lane's rows j0 = 32 s2 + 4 grp + r and j0 + 16.
    float gl = 0.f;
    f32x4 gr[2][2];
    if constexpr (HAS_G) {
      const float* gs = stage_g(s);
      gl = gs[kBT - 1];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        gr[s2][0] = *reinterpret_cast<const f32x4*>(gs + 32 * s2 + 4 * grp);
        gr[s2][1] = *reinterpret_cast<const f32x4*>(gs + 32 * s2 + 16 + 4 * grp);
      }
    }
    __builtin_amdgcn_sched_barrier(0);

    f32x4 vn[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int r = 0; r < 4; ++r) vn[jb][r] = (float)ur[jb][r];

    if constexpr (DELTA) {
      bf16x8 sb[C::KBH / 2];
#pragma unroll
      for (int s2 = 0; s2 < C::KBH / 2; ++s2) {
        const float f[8] = {S[2 * s2][0], S[2 * s2][1], S[2 * s2][2], S[2 * s2][3],
                            S[2 * s2 + 1][0], S[2 * s2 + 1][1], S[2 * s2 + 1][2], S[2 * s2 + 1][3]};
        sb[s2] = to_bf16x8(f);
      }
      // P1: this wave's K half of w S for v_new rows 16 jb .. 16 jb + 15.
      f32x4 part[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        f32x4 acc = zero4();
#pragma unroll
        for (int s2 = 0; s2 < C::KBH / 2; ++s2) acc = mfma16x16x32(concat(wa[jb][s2][0], wa[jb][s2][1]), sb[s2], acc);
        part[jb] = acc;
      }
      if constexpr (KS == 2) {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) *reinterpret_cast<f32x4*>(xbuf + ((wi * 4 + jb) * 64 + lane) * 4) = part[jb];
        lds_barrier();  // B: both K halves' partials are in LDS
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const f32x4 o = *reinterpret_cast<const f32x4*>(xbuf + (((wi ^ 4) * 4 + jb) * 64 + lane) * 4);
          vn[jb] -= part[jb] + o;
        }
      } else {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) vn[jb] -= part[jb];
      }
      if constexpr (STORE_VN) {
        bf16* vb = vnew + ((b * T + c * kBT) * H + hh) * V;
        // Row tiles kJbStore kh .. + kJbStore - 1.  One branch per K half
        // (kh is wave-uniform) keeps the register indices static: indexing
        // vn by kh itself compiled to relative register moves.
        auto store_vn = [&](auto kh_c) {
#pragma unroll
          for (int jj = 0; jj < C::kJbStore; ++jj) {
            constexpr int kOff = C::kJbStore * decltype(kh_c)::value;
            st_b64(vb, vnoff0 + (uint32_t)(16 * (kOff + jj) * tsv), acc_to_row_quads_bf16(vn[kOff + jj]));
          }
        };
        if (kh == 0) store_vn(std::integral_constant<int, 0>{});
        else if constexpr (KS == 2) store_vn(std::integral_constant<int, 1>{});
      }
    }

    // P2: S = e^{g_last} S + k^T (v_new e^{g_last - g}).
    bf16x8 vh[2];
    float decay = 1.f;
    if constexpr (HAS_G) {
      decay = fast_exp(gl);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        float f[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          f[r] = vn[2 * s2][r] * fast_exp(gl - gr[s2][0][r]);
          f[4 + r] = vn[2 * s2 + 1][r] * fast_exp(gl - gr[s2][1][r]);
        }
        vh[s2] = to_bf16x8(f);
      }
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const float f[8] = {vn[2 * s2][0], vn[2 * s2][1], vn[2 * s2][2], vn[2 * s2][3],
                            vn[2 * s2 + 1][0], vn[2 * s2 + 1][1], vn[2 * s2 + 1][2], vn[2 * s2 + 1][3]};
        vh[s2] = to_bf16x8(f);
      }
    }
#pragma unroll
    for (int kb = 0; kb < C::KBH; ++kb) {
      if constexpr (DELTA) store_h_tile(c, kb);  // state before chunk c
      if constexpr (HAS_G) S[kb] *= decay;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) S[kb] = mfma16x16x32(concat(ka[kb][s2][0], ka[kb][s2][1]), vh[s2], S[kb]);
      if constexpr (!DELTA) store_h_tile(c, kb);  // state after chunk c
    }
  }
  // Drain: no DMA may still target this workgroup's LDS when it exits.
  wait_vmcnt<0>();

  if (ht) {
#pragma unroll
    for (int kb = 0; kb < C::KBH; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ht[st_base + (int64_t)(kap0 + 16 * kb + 4 * grp + r) * V + ncol] = S[kb][r];
  }
}

// Measured on MI355X at B=8, T=8192, H=16, K=V=128 (256 workgroups): the K
// split with a 2-stage ring is the fastest form (3 stages and the unsplit form
// are slower); every form is bound by HBM traffic, 2.16 GB per launch.
constexpr int kHKSplit = 2;  // K split of the bf16 pipeline
constexpr int kHStages = 2;  // DMA ring depth of the bf16 pipeline
// The DMA pipeline serves grids that fill the GPU (bandwidth-bound); below
// that, fewer and serial chunks are latency-bound and the register-prefetch
// kernel (shorter chunk-to-chunk latency) is faster.
constexpr int64_t kHDmaMinGrid = 256;

template <int K, int V, bool DELTA>
hipError_t launch_h_dma(const void* k, const void* w, const void* vu, const void* g, const void* h0,
                        void* h, void* vnew, void* ht, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / kBT;
  const int64_t BH = B * H;
  const dim3 grid((unsigned)(BH * (V / kHBV)));
  constexpr int KS = kHKSplit, NS = kHStages;
#define THM_H_DMA_LAUNCH(HG, SV)                                                               \
  hipLaunchKernelGGL((chunk_fwd_h_dma_kernel<K, V, KS, NS, DELTA, HG, SV>), grid,              \
                     dim3(PCfg<K, KS, NS, DELTA, HG, SV>::kThreads), 0, s, (const bf16*)k,     \
                     (const bf16*)w, (const bf16*)vu, (const float*)g, (const float*)h0,       \
                     (float*)h, (bf16*)vnew, (float*)ht, T, H, NT, BH)
  const bool sv = DELTA && vnew != nullptr;
  if (g) {
    if (sv) THM_H_DMA_LAUNCH(true, DELTA);
    else THM_H_DMA_LAUNCH(true, false);
  } else {
    if (sv) THM_H_DMA_LAUNCH(false, DELTA);
    else THM_H_DMA_LAUNCH(false, false);
  }
#undef THM_H_DMA_LAUNCH
  return hipGetLastError();
}

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

template <typename IT, bool DELTA, int K, int V>
hipError_t launch_kv(const void* k, const void* w, const void* vu, const void* g, const void* h0,
                     void* h, void* vnew, void* ht, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  if constexpr (std::is_same<IT, bf16>::value) {
    if (B * H * (V / kHBV) >= kHDmaMinGrid)
      return launch_h_dma<K, V, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
  }
  return launch_h<IT, K, V, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
}

template <typename IT, bool DELTA>
hipError_t dispatch_kv(int64_t K, int64_t V, const void* k, const void* w, const void* vu,
                       const void* g, const void* h0, void* h, void* vnew, void* ht, int64_t B,
                       int64_t T, int64_t H, hipStream_t s) {
  if (K == 64 && V == 64) return launch_kv<IT, DELTA, 64, 64>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
  if (K == 64 && V == 128) return launch_kv<IT, DELTA, 64, 128>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
  if (K == 128 && V == 64) return launch_kv<IT, DELTA, 128, 64>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
  return launch_kv<IT, DELTA, 128, 128>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
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
  // k, w, u/v are read and h, v_new written as 16-byte vectors per lane.
  const void* ptrs16[] = {k, vu, w, h, v_new};
  for (const void* p : ptrs16)
    if (p && ((uintptr_t)p % 16)) return THM_ERR_MISALIGNED;
  const void* ptrs4[] = {g, h0, ht};
  for (const void* p : ptrs4)
    if (p && ((uintptr_t)p % 4)) return THM_ERR_MISALIGNED;
  if (B > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
  // Per-lane offsets within one chunk's token block are 32-bit.
  if (64 * H * (K > V ? K : V) * (kv_dtype == THM_DTYPE_F32 ? 4 : 2) > (INT64_C(1) << 31))
    return THM_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (kv_dtype == THM_DTYPE_F32) {
    e = delta ? dispatch_kv<float, true>(K, V, k, w, vu, g, h0, h, v_new, ht, B, T, H, s)
              : dispatch_kv<float, false>(K, V, k, w, vu, g, h0, h, v_new, ht, B, T, H, s);
  } else {
    e = delta ? dispatch_kv<bf16, true>(K, V, k, w, vu, g, h0, h, v_new, ht, B, T, H, s)
              : dispatch_kv<bf16, false>(K, V, k, w, vu, g, h0, h, v_new, ht, B, T, H, s);
  }
  return (int)e;
}
