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
// Two kernels:
//   * the register-prefetch kernel (chunk_fwd_h_reg.h): every fp32 call (its
//     instantiations are in chunk_fwd_h_f32.hip) and bf16 on grids under
//     kHDmaMinGrid workgroups;
//   * the DMA pipeline below: bf16 on grids that fill the GPU.
// This unit is compiled with MFMA accumulators forced into VGPRs
// (theorem_amd/build.py): the bf16 register kernel at config 3 takes 24.4
// against 25.5 us with them in AGPRs, and the DMA kernel uses no AGPRs either way.
#include "chunk_fwd_h_reg.h"
#include "chunk_fwd_h_small.h"

#include "pipe_cfg.h"

namespace thm {
namespace {

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
using pipe::PCfg;
static_assert(pipe::kBT == kBT && pipe::kTileV == kHBV, "one chunk length and V-tile width");

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

  const hl::BhTile bt = hl::xcd_tile(blockIdx.x, BH, NVT);
  const int64_t bh = bt.bh;
  const int64_t b = bh / H, hh = bh % H;
  const int v0 = (int)bt.vt * kHBV;

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
    koff[i] = hl::dma_src_off(P, C::kRowK, tsk);
  }
#pragma unroll
  for (int i = 0; i < C::kUDma; ++i) {
    const int P = (wi * C::kUDma + i) * 64 + lane;
    uoff[i] = hl::dma_src_off(P, C::kRowU, tsv);
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

  // Store offsets of the row-quad layout (acc_to_row_quads) for this wave's
  // first 16-row tile of h and of v_new; later tiles add 16 rows.
  const uint32_t hoff0 = hl::rowquad_off(kap0, v0 + 16 * wq, lane, V * 4, 4);
  const uint32_t vnoff0 = hl::rowquad_off(0, v0 + 16 * wq, lane, tsv, 2);
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
      ur[jb] = ds_read_tr16(reinterpret_cast<const bf16*>(tu + hl::tr_frag_off(16 * jb, 16 * wq, lane, C::kRowU)));
    // w rows 16 jb + li, this wave's K elements, paired order (A operand of P1).
    bf16x4 wa[DELTA ? 4 : 1][C::KBH / 2][2];
    if constexpr (DELTA) {
      const char* tw = stage_w(s);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int s2 = 0; s2 < C::KBH / 2; ++s2) {
          const int e0 = kap0 + 32 * s2;
          wa[jb][s2][0] = *reinterpret_cast<const bf16x4*>(tw + hl::pair_frag_off(16 * jb, e0, lane, C::kRowK));
          wa[jb][s2][1] = *reinterpret_cast<const bf16x4*>(tw + hl::pair_frag_off(16 * jb, e0 + 16, lane, C::kRowK));
        }
    }
    // k^T fragments of this wave's state rows (A operand of P2), paired order.
    bf16x4 ka[C::KBH][2][2];
#pragma unroll
    for (int kb = 0; kb < C::KBH; ++kb)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int col = kap0 + 16 * kb;
        ka[kb][s2][0] = ds_read_tr16(reinterpret_cast<const bf16*>(tk + hl::tr_frag_off(32 * s2, col, lane, C::kRowK)));
        ka[kb][s2][1] = ds_read_tr16(reinterpret_cast<const bf16*>(tk + hl::tr_frag_off(32 * s2 + 16, col, lane, C::kRowK)));
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
using pipe::kHKSplit;  // K split of the bf16 pipeline
using pipe::kHStages;  // DMA ring depth of the bf16 pipeline

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

template <typename IT, bool DELTA, int K, int V>
hipError_t launch_kv(const void* k, const void* w, const void* vu, const void* g, const void* h0,
                     void* h, void* vnew, void* ht, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  if constexpr (std::is_same<IT, bf16>::value) {
    if (B * H * (V / kHBV) >= kHDmaMinGrid)
      return launch_h_dma<K, V, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
    return launch_h_small<bf16, K, V, kHSmallNW, DELTA>(k, w, vu, g, h0, h, vnew, ht, B, T, H, s);
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
  if (!launch_fits(B * H * (V / kHBV), 64 * 4 * kHKSplit)) return THM_ERR_BAD_SHAPE;  // the DMA kernel's block
  // Per-lane offsets within one chunk's token block are 32-bit.
  if (64 * H * (K > V ? K : V) * (kv_dtype == THM_DTYPE_F32 ? 4 : 2) > (INT64_C(1) << 31))
    return THM_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (kv_dtype == THM_DTYPE_F32) {
    e = chunk_fwd_h_f32(delta, K, V, k, w, vu, g, h0, h, v_new, ht, B, T, H, s);
  } else {
    e = delta ? dispatch_kv<bf16, true>(K, V, k, w, vu, g, h0, h, v_new, ht, B, T, H, s)
              : dispatch_kv<bf16, false>(K, V, k, w, vu, g, h0, h, v_new, ht, B, T, H, s);
  }
  return (int)e;
}
