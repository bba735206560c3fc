// Gated DeltaNet inter-chunk state recurrence on small grids (fewer
// workgroups than CUs): a role-split kernel for the chunk latency.  Included
// by chunk_fwd_h.hip (bf16 inputs) and chunk_fwd_h_f32.hip (fp32 inputs).
//
// The math is the register kernel's (chunk_fwd_h_reg.h), operation for
// operation, so h, v_new and the final state are bit-identical to it (fp32
// inputs: k and w staged as bf16 hi + lo, S and the gated v_new split the
// same way, three MFMAs per product):
//   reference form (DELTA = false; vu = v)                kernels/chunk_fwd_h/
//     S <- e^{g_last} S + k_c^T (v_c e^{g_last - g_c});  h[c] = S      reference.py:50-97
//   delta form (DELTA = true; vu = u)
//     h[c] = S;  v_new = u_c - w_c S;  S <- e^{g_last} S + k_c^T (v_new e^{g_last - g_c})
// Replaces kernels/chunk_fwd_h/kernel.py:61-138 (Triton) on small grids.
//
// One workgroup per (b, head, V-tile of 16 NW columns), 2 NW wavefronts in
// two roles:
//   state waves 0 .. NW-1: wave wq owns state columns 16 wq .. + 15 of the
//     tile for the whole sequence, in MFMA accumulators.  Per chunk they only
//     read the staged chunk from LDS, run P1 (v_new = u - w S) and P2 (the
//     state update), and write h and v_new (fp32) into an LDS out buffer: no
//     global memory access and no transcendental in their chain.
//   memory waves NW .. 2 NW-1: per chunk they store the previous chunk's h
//     and v_new from the out buffer (16-byte rows), stage the next chunk's
//     k, w, u and its gate factors e^{g_last - g_j}, e^{g_last} into the
//     other LDS stage, and issue the loads of the chunk three ahead into one
//     of two register sets (two chunk periods to arrive).
// One barrier per chunk.  Stage s = c % 2 holds chunk c; out buffer c % 2
// holds chunk c's h and v_new.  Between barriers B_c and B_{c+1} the state
// waves read stage c % 2 and write out buffer c % 2, while the memory waves
// read out buffer (c - 1) % 2 and write stage (c + 1) % 2: each buffer is
// written and read on opposite sides of a barrier.
//
// Why: in the register kernel each wave issues, per chunk, 7 loads and 32
// stores of one element per lane (each store instruction covers 4 rows), the
// LDS staging of the next chunk and 16 exponentials, all in the chain between
// its state updates (~2,800 cycles per chunk at config 3).  Narrower V-tiles
// (16 NW columns) also spread a small grid over more CUs: each CU then moves
// fewer bytes through its LDS and address unit per chunk.
#pragma once

#include "h_layout.h"
#include "mfma.h"
#include "pipe_cfg.h"
#include "vmem.h"

namespace thm {
namespace {

using pipe::SCfg;

// State waves per workgroup (V-tile of 32 columns).  At config 3 (B=2,
// T=1024, H=3, K=V=64, bf16), per launch with HIP events: 1 state wave
// 15.9 us, 2 15.6, 4 21.6; the register kernel 26.8.
constexpr int kHSmallNW = 2;

template <typename IT, int K, int V, int NW, bool DELTA, bool HAS_G>
__global__ void __launch_bounds__(128 * NW)
chunk_fwd_h_small_kernel(const IT* __restrict__ k, const IT* __restrict__ w,
                         const IT* __restrict__ vu, const float* __restrict__ g,
                         const float* __restrict__ h0, float* __restrict__ hout,
                         IT* __restrict__ vnew, float* __restrict__ ht, int64_t T, int64_t H,
                         int64_t NT, int64_t BH) {
  constexpr int EB = (int)sizeof(IT);
  using C = SCfg<K, NW, DELTA, EB>;
  static_assert(C::kFits, "LDS budget");
  constexpr bool SPLIT = C::kSplit;
  constexpr int KB = K / 16;
  constexpr int NVT = V / C::kCols;
  __shared__ __attribute__((aligned(16))) char lds[C::kLds];

  const hl::BhTile bt = hl::xcd_tile(blockIdx.x, BH, NVT);
  const int64_t bh = bt.bh, b = bh / H, hh = bh % H;
  const int v0 = (int)bt.vt * C::kCols;
  const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // wave-uniform
  const int lane = (int)threadIdx.x & 63;
  const int grp = lane >> 4;
  const int li = lane & 15;

  // Stage s: k hi[, lo], w hi[, lo] (delta form), u, gate factors.  The lo
  // tile of a split operand follows its hi tile.
  auto st_k = [&](int s) { return reinterpret_cast<bf16*>(lds + s * C::kStageB); };
  auto st_w = [&](int s) { return reinterpret_cast<bf16*>(lds + s * C::kStageB + C::kKPartB); };
  auto lo_of = [](const bf16* hi) { return hi + C::kKTileB / 2; };
  auto st_u = [&](int s) {
    return reinterpret_cast<IT*>(lds + s * C::kStageB + C::kKPartB * (DELTA ? 2 : 1));
  };
  auto st_f = [&](int s) {
    return reinterpret_cast<float*>(lds + s * C::kStageB + C::kKPartB * (DELTA ? 2 : 1) + C::kUTileB);
  };
  char* const hob = lds + 2 * C::kStageB;     // out buffers: h [2][kHOutB]
  char* const vob = hob + 2 * C::kHOutB;      // v_new [2][kVOutB]

  const int64_t tok_k = H * K;   // elements between tokens of k / w
  const int64_t tok_v = H * V;   // elements between tokens of u / v / v_new
  const int64_t st_base = bh * (int64_t)(K * V);  // h0 / ht (elements)

  if (wv < NW) {
    // ---------------------------------------------------------------- state waves
    const int ucol = 16 * wv + li;  // column within the V-tile
    const int vcol = v0 + ucol;     // column within V
    f32x4 S[KB];  // S[kappa = 16 kb + 4 grp + r][vcol] in S[kb][r]
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[kb][r] = h0 ? h0[st_base + (16 * kb + 4 * grp + r) * V + vcol] : 0.f;
    // Rows 16 b + 4 grp + r of this lane's column of an out buffer.
    auto put_out = [&](char* buf, int blk, f32x4 v) {
      float* const p = reinterpret_cast<float*>(buf);
#pragma unroll
      for (int r = 0; r < 4; ++r) p[hl::sout_put(blk, r, lane, wv, C::kOutPitch)] = v[r];
    };
    lds_barrier();  // B_0: chunk 0 staged
    for (int64_t c = 0; c < NT; ++c) {
      const int s = (int)(c & 1);
      const bf16* const ks = st_k(s);
      const IT* const us = st_u(s);
      const float* const fs = st_f(s);
      char* const ho = hob + s * C::kHOutB;
      if constexpr (DELTA) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) put_out(ho, kb, S[kb]);  // h[c]: state before chunk c
      }
      // v_new (or v) for rows j = 16 jb + 4 grp + r of this lane's column: one
      // transposed read per 16-row block (lane li of a 16-lane group receives
      // the 4 rows of column 16 wq + li).
      f32x4 vn[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        if constexpr (SPLIT) {
#pragma unroll
          for (int r = 0; r < 4; ++r) vn[jb][r] = us[(16 * jb + 4 * grp + r) * C::kUPitch + ucol];
        } else {
          const bf16x4 u4 = ds_read_tr16(us + (16 * jb + 4 * grp + (li >> 2)) * C::kUPitch + 16 * wv + 4 * (li & 3));
#pragma unroll
          for (int r = 0; r < 4; ++r) vn[jb][r] = to_f32(u4[r]);
        }
      }
      if constexpr (DELTA) {
        // P1: B operand = S pairs (kappa blocks 2t, 2t+1) in paired order.
        const bf16* const ws = st_w(s);
        bf16x8 sh[K / 32], sl[SPLIT ? K / 32 : 1];
#pragma unroll
        for (int t = 0; t < K / 32; ++t) {
          const float f[8] = {S[2 * t][0], S[2 * t][1], S[2 * t][2], S[2 * t][3],
                              S[2 * t + 1][0], S[2 * t + 1][1], S[2 * t + 1][2], S[2 * t + 1][3]};
          if constexpr (SPLIT) split_bf16x8(f, sh[t], sl[t]);
          else sh[t] = to_bf16x8(f);
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          f32x4 a = zero4();
          const bf16* const wrow = ws + (16 * jb + li) * C::kKPitch;
#pragma unroll
          for (int t = 0; t < K / 32; ++t) {
            const bf16x8 wf = load8_paired(wrow, 32 * t);
            a = mfma16x16x32(wf, sh[t], a);
            if constexpr (SPLIT) {
              a = mfma16x16x32(wf, sl[t], a);
              a = mfma16x16x32(load8_paired(lo_of(wrow), 32 * t), sh[t], a);
            }
          }
          vn[jb] -= a;
        }
        char* const vo = vob + s * C::kVOutB;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) put_out(vo, jb, vn[jb]);
      }
      // P2: S = e^{g_last} S + k^T (v_new e^{g_last - g}), the factors staged by
      // the memory waves.
      bf16x8 vh[2], vl[SPLIT ? 2 : 1];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f32x4 fa = *reinterpret_cast<const f32x4*>(fs + 32 * t + 4 * grp);
        const f32x4 fb = *reinterpret_cast<const f32x4*>(fs + 32 * t + 16 + 4 * grp);
        float f[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          f[r] = vn[2 * t][r] * fa[r];
          f[4 + r] = vn[2 * t + 1][r] * fb[r];
        }
        if constexpr (SPLIT) split_bf16x8(f, vh[t], vl[t]);
        else vh[t] = to_bf16x8(f);
      }
      const float decay = fs[64];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        S[kb] *= decay;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int r0 = tr_row_paired(32 * t, 0), r1 = tr_row_paired(32 * t, 1);
          const bf16x8 kf = frag_tr(ks, C::kKPitch, r0, r1, 16 * kb);
          S[kb] = mfma16x16x32(kf, vh[t], S[kb]);
          if constexpr (SPLIT) {
            S[kb] = mfma16x16x32(kf, vl[t], S[kb]);
            S[kb] = mfma16x16x32(frag_tr(lo_of(ks), C::kKPitch, r0, r1, 16 * kb), vh[t], S[kb]);
          }
        }
      }
      if constexpr (!DELTA) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) put_out(ho, kb, S[kb]);  // h[c]: state after chunk c
      }
      lds_barrier();  // B_{c+1}
    }
    if (ht) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) ht[st_base + (16 * kb + 4 * grp + r) * V + vcol] = S[kb][r];
    }
    return;
  }

  // ------------------------------------------------------------------ memory waves
  const int m = wv - NW;
  const int tid = (int)threadIdx.x - C::kML;  // 0 .. kML - 1
  // Loads: piece it of this lane is row hl::spiece_row(tid, it, n, kML, kVE),
  // elements hl::spiece_col(tid, n, kVE) .. + kVE - 1 of the k / w (n = K) or
  // u / v (n = kCols) tile; successive pieces are kKRows / kURows rows apart.
  constexpr int VE = C::kVE;
  constexpr int kKRows = C::kML / C::kKCPR, kURows = C::kML / C::kUCPR;
  const int kj0 = hl::spiece_row(tid, 0, K, C::kML, VE), kcol = hl::spiece_col(tid, K, VE);
  const int uj0 = hl::spiece_row(tid, 0, C::kCols, C::kML, VE), ucol0 = hl::spiece_col(tid, C::kCols, VE);
  const uint32_t koff = (uint32_t)(kj0 * tok_k + kcol) * EB;        // bytes from the chunk base
  const uint32_t kstep = (uint32_t)(kKRows * tok_k) * EB;
  const uint32_t uoff = (uint32_t)(uj0 * tok_v + v0 + ucol0) * EB;
  const uint32_t ustep = (uint32_t)(kURows * tok_v) * EB;
  const int64_t kc0 = ((b * T) * H + hh) * K * EB;  // bytes: chunk 0 of this (b, head)
  const int64_t uc0 = ((b * T) * H + hh) * V * EB;
  const int64_t kcs = 64 * tok_k * EB, ucs = 64 * tok_v * EB;
  auto cbytes = [](const void* p, int64_t off) { return reinterpret_cast<const char*>(p) + off; };

  // Two register sets: the loads of chunk c + 3 are issued during chunk c and
  // staged during chunk c + 2, so each has two chunk periods to arrive.
  struct Regs {
    u32x4 k[C::kKLoads], w[DELTA ? C::kKLoads : 1], u[C::kULoads];
    float g;
  };
  Regs ra, rb;
  auto load = [&](Regs& r, int64_t c) {
    const char* const kb_ = cbytes(k, kc0 + c * kcs);
#pragma unroll
    for (int it = 0; it < C::kKLoads; ++it) r.k[it] = ldg16(kb_ + koff + it * kstep);
    if constexpr (DELTA) {
      const char* const wb = cbytes(w, kc0 + c * kcs);
#pragma unroll
      for (int it = 0; it < C::kKLoads; ++it) r.w[it] = ldg16(wb + koff + it * kstep);
    }
    const char* const ub = cbytes(vu, uc0 + c * ucs);
#pragma unroll
    for (int it = 0; it < C::kULoads; ++it) r.u[it] = ldg16(ub + uoff + it * ustep);
    // Every memory wave loads the chunk's 64 gates (one per lane), so all of
    // them issue the same loads; wave 4 stages the factors.
    if constexpr (HAS_G) r.g = g[(b * T + c * 64 + lane) * H + hh];
    else r.g = 0.f;
  };
  // A k / w piece into its tile: as loaded (bf16), or split into bf16 hi and
  // lo halves at the same offset of the hi and lo tiles (fp32).
  auto put_piece = [&](bf16* tile, int off, u32x4 v) {
    if constexpr (SPLIT) {
      float f[4];
      unpack16(v, f, 0.f);
      lds_put4(tile + off, tile + C::kKTileB / 2 + off, f, true);
    } else {
      *reinterpret_cast<u32x4*>(tile + off) = v;
    }
  };
  auto commit = [&](const Regs& r, int s) {
    bf16* const ks = st_k(s);
#pragma unroll
    for (int it = 0; it < C::kKLoads; ++it) put_piece(ks, (kj0 + it * kKRows) * C::kKPitch + kcol, r.k[it]);
    if constexpr (DELTA) {
      bf16* const ws = st_w(s);
#pragma unroll
      for (int it = 0; it < C::kKLoads; ++it) put_piece(ws, (kj0 + it * kKRows) * C::kKPitch + kcol, r.w[it]);
    }
    IT* const us = st_u(s);
#pragma unroll
    for (int it = 0; it < C::kULoads; ++it)
      *reinterpret_cast<u32x4*>(us + (uj0 + it * kURows) * C::kUPitch + ucol0) = r.u[it];
    if (m == 0) {  // wave-uniform: the gate factors of the chunk, one per lane
      float* const fs = st_f(s);
      if constexpr (HAS_G) {
        const float gl = readlane(r.g, 63);
        fs[lane] = fast_exp(gl - r.g);
        if (lane == 0) fs[64] = fast_exp(gl);
      } else {
        fs[lane] = 1.f;
        if (lane == 0) fs[64] = 1.f;
      }
    }
  };
  // h[c] and v_new[c] from out buffer s: piece p = i * kML + tid (row
  // hl::sout_row, columns hl::sout_col .. + 3) is read as one 16-byte LDS
  // block and stored as 16 bytes of h or 8 of v_new.  All of a chunk's blocks
  // are read before the first store.
  constexpr int kHPieces = K / 16, kVPieces = 4;  // per memory lane
  auto store_out = [&](int64_t c, int s) {
    const float* const ho = reinterpret_cast<const float*>(hob + s * C::kHOutB);
    const float* const vo = reinterpret_cast<const float*>(vob + s * C::kVOutB);
    f32x4 hv[kHPieces], vv[DELTA ? kVPieces : 1];
#pragma unroll
    for (int i = 0; i < kHPieces; ++i) {
      const int p = i * C::kML + tid;
      hv[i] = *reinterpret_cast<const f32x4*>(ho + hl::sout_row(p, C::kCols) * C::kOutPitch + hl::sout_col(p, C::kCols));
    }
    if constexpr (DELTA) {
#pragma unroll
      for (int i = 0; i < kVPieces; ++i) {
        const int p = i * C::kML + tid;
        vv[i] = *reinterpret_cast<const f32x4*>(vo + hl::sout_row(p, C::kCols) * C::kOutPitch + hl::sout_col(p, C::kCols));
      }
    }
    float* const hb = hout + ((b * NT + c) * H + hh) * (int64_t)(K * V) + v0;
#pragma unroll
    for (int i = 0; i < kHPieces; ++i) {
      const int p = i * C::kML + tid;
      *reinterpret_cast<f32x4*>(hb + hl::sout_row(p, C::kCols) * V + hl::sout_col(p, C::kCols)) = hv[i];
    }
    if constexpr (DELTA) {
      if (vnew) {  // uniform
        IT* const vb = vnew + ((b * T + c * 64) * H + hh) * V + v0;
#pragma unroll
        for (int i = 0; i < kVPieces; ++i) {
          const int p = i * C::kML + tid;
          IT* const dst = vb + hl::sout_row(p, C::kCols) * tok_v + hl::sout_col(p, C::kCols);
          if constexpr (SPLIT) {
            *reinterpret_cast<f32x4*>(dst) = vv[i];
          } else {
            bf16x4 o;
            o[0] = (bf16)vv[i][0]; o[1] = (bf16)vv[i][1]; o[2] = (bf16)vv[i][2]; o[3] = (bf16)vv[i][3];
            *reinterpret_cast<bf16x4*>(dst) = o;
          }
        }
      }
    }
  };

  // Chunk j > 0 arrives in set ra when j is odd, rb when j is even.
  if (NT > 0) {
    load(ra, 0);
    commit(ra, 0);
    if (NT > 1) load(ra, 1);
    if (NT > 2) load(rb, 2);
  }
  lds_barrier();  // B_0
  auto step = [&](int64_t c, Regs& r) {  // r holds chunk c + 1
    if (c >= 1) store_out(c - 1, (int)((c - 1) & 1));
    if (c + 1 < NT) {
      commit(r, (int)((c + 1) & 1));
      if (c + 3 < NT) load(r, c + 3);
    }
    lds_barrier();  // B_{c+1}
  };
  for (int64_t c = 0; c < NT; c += 2) {
    step(c, ra);
    if (c + 1 < NT) step(c + 1, rb);
  }
  if (NT > 0) store_out(NT - 1, (int)((NT - 1) & 1));
}

template <typename IT, int K, int V, int NW, bool DELTA>
hipError_t launch_h_small(const void* k, const void* w, const void* vu, const void* g, const void* h0,
                          void* h, void* vnew, void* ht, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / 64;
  const int64_t BH = B * H;
  const dim3 grid((unsigned)(BH * (V / (16 * NW))));
#define THM_H_SMALL_LAUNCH(HG)                                                                            \
  hipLaunchKernelGGL((chunk_fwd_h_small_kernel<IT, K, V, NW, DELTA, HG>), grid, dim3(128 * NW), 0, s, \
                     (const IT*)k, (const IT*)w, (const IT*)vu, (const float*)g,                         \
                     (const float*)h0, (float*)h, (IT*)vnew, (float*)ht, T, H, NT, BH)
  if (g) THM_H_SMALL_LAUNCH(true);
  else THM_H_SMALL_LAUNCH(false);
#undef THM_H_SMALL_LAUNCH
  return hipGetLastError();
}

}  // namespace
}  // namespace thm
