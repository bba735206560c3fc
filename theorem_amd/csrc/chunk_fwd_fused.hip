// Fused chunked Gated DeltaNet forward for MI355X (gfx950): the state
// recurrence of chunk_fwd_h (delta form) and the output of chunk_fwd_o in one
// pass, so the per-chunk states h never travel through HBM.
//
// For one (b, head, V-tile of 64 columns), state S [K x 64] fp32 (h0 or 0),
// per chunk c with g_last = g at the chunk's last token:
//   v_new = u_c - w_c S
//   o_c   = scale ( e^{g_i} q_i . S  +  sum_{j <= i} (q_i . k_j) e^{g_i - g_j} v_new_j )
//   S    <- e^{g_last} S + (k_c e^{g_last - g_c})^T v_new
// which is chunk_fwd_h (kernels/chunk_fwd_h/kernel.py:61-138 in its delta form)
// followed by chunk_fwd_o (kernels/chunk_fwd_o/kernel.py:52-136) with h[c] the
// state before chunk c; nothing of either reference kernel's output but o
// (and optionally v_new and the final state) is written.
//
// The A form (FROM_A, thm_chunk_gated_delta_fwd_a) takes the chunk's WY
// matrix A, v and beta instead of w and u:
//   v_new = A (beta (v - e^{g} k S))
// equals u - w S for the recompute_w_u outputs u = A (v beta), w =
// A (k beta e^g) (kernels/recompute_w_u/reference.py:118-149), so the chunked
// forward needs neither w nor u in HBM: A (64 fp32 per token-head) replaces
// w (K bf16) in the w slot and v replaces u in the u slot.  P1 forms
// k S as the w form forms w S, t = beta (v - e^g k S) as bf16 B-operand
// pairs, then A t with A as bf16 hi + lo operands (converted in place once
// per chunk, see prepare below).
//
// Structure: one 512-thread workgroup per (b, head, V-tile), 8 wavefronts in
// two roles that share SIMDs pairwise; wave role and column group wq (columns
// 16 wq .. 16 wq + 15 of the tile) are wave-uniform:
//   * k, w, q, u and g of a chunk arrive by global -> LDS DMA into a 2-stage
//     ring (XOR-swizzled tiles of h_layout.h), issued by the state waves: k, q
//     and g in P1 of the chunk before, w and u (read by P1 only) after the
//     mid-chunk barrier of the chunk two before, into the slots that chunk's
//     P1 has just finished with;
//   * state waves (0-3) hold S[K x 16 columns] in fp32 registers.  Phase 1:
//     hand S to the output waves as bf16 B-operand pairs (LDS), P1 v_new =
//     u - w S (the S pairs as the B operand, paired contraction order), hand
//     v_new over the same way.  Phase 2: P2 S = e^{g_last} S +
//     k^T (v_new e^{g_last - g});
//   * output waves (4-7).  Phase 1: the scores P[i][j] = (q_i . k_j)
//     e^{g_i - g_j}, j <= i (diagonal included), each wave 2 or 3 of the ten
//     16 x 16 lower-triangle blocks, written to LDS as bf16.  Phase 2, per
//     16-row query block: global term q S from the handed-over S pairs,
//     local term P v_new (P rows as the A operand, the v_new pairs as B),
//     o = scale (e^{g_i} q S + P v_new) as one 8-byte store per lane after a
//     4x4 quad transpose;
//   * a barrier at the top of each chunk (its tiles are in LDS, chunk c - 1
//     is finished) and one between the phases.
// All DMA and stores of the chunk loop go through vmem.h, and the state waves'
// wait at the top of the loop is an exact count of the ops they issue after
// the chunk's k / q DMA (pipe_cfg.h FCfg); the output waves issue stores only.
// HBM traffic per token-head: k, w and q (K eb each), u (V eb) and g (4 B)
// read once; o (V eb) written once (+ v_new when requested).  The A form
// reads A (256 B) in place of w and beta (4 B) besides.  The V-tiles of
// one (b, head) run on one XCD, so their second read of k, w, q is meant to
// hit that XCD's L2.
#include "h_layout.h"
#include "mfma.h"
#include "pipe_cfg.h"
#include "vmem.h"

namespace thm {
namespace {

using pipe::FCfg;
using pipe::kBT;
using pipe::kFStages;
using pipe::kFThreads;
constexpr int kFBV = pipe::kTileV;  // V-tile width

template <int K, int V, bool HAS_G, bool STORE_VN, bool FROM_A>
__global__ void __launch_bounds__(kFThreads)
chunk_fwd_fused_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                       const bf16* __restrict__ w, const bf16* __restrict__ u,
                       const float* __restrict__ A, const float* __restrict__ beta,
                       const float* __restrict__ g, const float* __restrict__ h0,
                       bf16* __restrict__ o, bf16* __restrict__ vnew, float* __restrict__ ht,
                       float scale, int64_t T, int64_t H, int64_t NT, int64_t BH) {
  // FROM_A: w = nullptr, u = v (the u slot holds v), A and beta given.
  using C = FCfg<K, HAS_G, STORE_VN, FROM_A>;
  constexpr int NVT = V / kFBV;
  constexpr int KB2 = C::KB / 2;
  __shared__ __attribute__((aligned(1024))) char lds[C::kLds];

  const hl::BhTile bt = hl::xcd_tile(blockIdx.x, BH, NVT);
  const int64_t bh = bt.bh;
  const int64_t b = bh / H, hh = bh % H;
  const int v0 = (int)bt.vt * kFBV;

  const int tid = threadIdx.x;
  const int wi = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool state_wave = wi < 4;  // waves 0-3: recurrence; waves 4-7: output
  const int wq = wi & 3;           // column group 16 wq .. 16 wq + 15 of the tile
  const int lane = tid & 63, grp = lane >> 4, li = lane & 15;

  auto stage_k = [&](int s) { return lds + s * C::kStage; };
  auto stage_w = [&](int s) { return lds + s * C::kStage + C::kTileK; };  // w, or A (FROM_A)
  auto stage_q = [&](int s) { return lds + s * C::kStage + C::kTileK + C::kTileW; };
  auto stage_u = [&](int s) { return lds + s * C::kStage + 2 * C::kTileK + C::kTileW; };  // u, or v
  auto stage_g = [&](int s) {
    return reinterpret_cast<float*>(lds + s * C::kStage + 2 * C::kTileK + C::kTileW + C::kTileU);
  };
  char* const lp = lds + kFStages * C::kStage;  // P[i][j], 128-byte rows, swizzled
  // Hand-over slots, lane-major: 16 bytes per lane per B-operand pair.
  bf16x8* const ls = reinterpret_cast<bf16x8*>(lp + C::kPBytes) + wq * KB2 * 64 + lane;
  bf16x8* const lv = reinterpret_cast<bf16x8*>(lp + C::kPBytes + C::kSBytes) + wq * 2 * 64 + lane;

  // Global geometry in bytes.  Token t of chunk c, head hh: ((b T + 64 c + t) H + hh) D.
  const int64_t tsk = H * K * 2, tsv = H * V * 2;
  const int64_t kc0 = ((b * T) * H + hh) * K * 2;
  const int64_t uc0 = ((b * T) * H + hh) * V * 2 + v0 * 2;
  const int64_t gc0 = ((b * T) * H + hh) * 4;
  const int64_t kcs = kBT * tsk, ucs = kBT * tsv, gcs = kBT * H * 4;
  // A rows (FROM_A): 64 fp32 per token-head.
  const int64_t tsa = H * kBT * 4, ac0 = ((b * T) * H + hh) * kBT * 4, acs = kBT * tsa;

  uint32_t koff[C::kKDma], uoff[C::kUDma], aoff[FROM_A ? C::kWDma : 1];
#pragma unroll
  for (int i = 0; i < C::kKDma; ++i) {
    const int P = (wq * C::kKDma + i) * 64 + lane;
    koff[i] = hl::dma_src_off(P, C::kRowK, tsk);
  }
#pragma unroll
  for (int i = 0; i < C::kUDma; ++i) {
    const int P = (wq * C::kUDma + i) * 64 + lane;
    uoff[i] = hl::dma_src_off(P, C::kRowU, tsv);
  }
  if constexpr (FROM_A) {
#pragma unroll
    for (int i = 0; i < C::kWDma; ++i) {
      const int P = (wq * C::kWDma + i) * 64 + lane;
      aoff[i] = hl::dma_src_off(P, C::kRowW, tsa);
    }
  }
  const uint32_t goff = (uint32_t)(lane * H * 4);

  // DMA of chunk cc's [64 x K] tile of src (k, w or q) into dst.
  auto issue_tile = [&](const bf16* src, int64_t cc, char* dst) {
    const char* sb = reinterpret_cast<const char*>(src) + kc0 + cc * kcs;
    const uint32_t l0 = lds_address(dst) + wq * C::kKDma * 1024;
#pragma unroll
    for (int i = 0; i < C::kKDma; ++i) dma_b128(sb, koff[i], __builtin_amdgcn_readfirstlane(l0 + i * 1024));
  };
  // Part m of the DMA of chunk cc's k, q and gates into stage s (P1 of the
  // chunk before): m = 0 the k tile, 1 the q tile, 2 the gates.  One copy of
  // the gates (state wave 0): a 64-lane gather at a 4 H-byte stride is the
  // costliest DMA instruction per byte.
  auto issue_part = [&](int64_t cc, int s, int m) {
    if (m == 0) {
      issue_tile(k, cc, stage_k(s));
    } else if (m == 1) {
      issue_tile(q, cc, stage_q(s));
    } else if (m == 2) {
      if constexpr (HAS_G) {
        if (wq == 0) {
          const char* gb = reinterpret_cast<const char*>(g) + gc0 + cc * gcs;
          dma_b32(gb, goff, __builtin_amdgcn_readfirstlane(lds_address(stage_g(s))));
        }
      }
      if constexpr (FROM_A) {
        if (wq == 1) {  // beta, after the gate factors
          const char* bb = reinterpret_cast<const char*>(beta) + gc0 + cc * gcs;
          dma_b32(bb, goff, __builtin_amdgcn_readfirstlane(lds_address(stage_g(s) + 192)));
        }
      }
    }
  };
  // DMA of chunk cc's w and u (A and v) tiles into stage s.
  auto issue_wu = [&](int64_t cc, int s) {
    if constexpr (FROM_A) {
      const char* ab = reinterpret_cast<const char*>(A) + ac0 + cc * acs;
      const uint32_t la = lds_address(stage_w(s)) + wq * C::kWDma * 1024;
#pragma unroll
      for (int i = 0; i < C::kWDma; ++i) dma_b128(ab, aoff[i], __builtin_amdgcn_readfirstlane(la + i * 1024));
    } else {
      issue_tile(w, cc, stage_w(s));
    }
    const char* ub = reinterpret_cast<const char*>(u) + uc0 + cc * ucs;
    const uint32_t lu = lds_address(stage_u(s)) + wq * C::kUDma * 1024;
#pragma unroll
    for (int i = 0; i < C::kUDma; ++i) dma_b128(ub, uoff[i], __builtin_amdgcn_readfirstlane(lu + i * 1024));
  };

  // rows x S for a 16-row block of a [64 x K] tile (w or q): A = tile rows,
  // B = the S pairs sbv, paired contraction order.
  auto rows_times_S = [&](const char* tile, int ib, const bf16x8* sbv) {
    f32x4 acc = zero4();
#pragma unroll
    for (int s2 = 0; s2 < KB2; ++s2) {
      const bf16x4 a0 = *reinterpret_cast<const bf16x4*>(tile + hl::pair_frag_off(16 * ib, 32 * s2, lane, C::kRowK));
      const bf16x4 a1 = *reinterpret_cast<const bf16x4*>(tile + hl::pair_frag_off(16 * ib, 32 * s2 + 16, lane, C::kRowK));
      acc = mfma16x16x32(concat(a0, a1), sbv[s2], acc);
    }
    return acc;
  };

  // Row-tile stores after the quad transpose: lane (grp, 4 m4 + qq) holds row
  // 4 grp + qq of a 16-row tile at columns 16 wq + 4 m4 .. + 3.  (The
  // row-contiguous layout of vmem.h acc_to_row_quads, which chunk_fwd_h's
  // stores use, is slower here: 366 against 356 us at config 4; the lane
  // transpose lengthens the output waves' path, which bounds this kernel.)
  const uint32_t rowoff0 = hl::quadT_off(0, v0 + 16 * wq, lane, tsv, 2);
  auto store_rows = [&](bf16* base, int ib, f32x4 val) {
    const f32x4 t = quad_transpose(val);
    bf16x4 ov;
    ov[0] = (bf16)t[0]; ov[1] = (bf16)t[1]; ov[2] = (bf16)t[2]; ov[3] = (bf16)t[3];
    st_b64(base, rowoff0 + (uint32_t)(16 * ib * tsv), __builtin_bit_cast(u32x2, ov));
  };

  // State S[kappa = 16 kb + 4 grp + r][n = v0 + 16 wq + li] in S[kb][r] (state waves).
  f32x4 S[C::KB];
  const int ncol = v0 + 16 * wq + li;
  const int64_t st_base = bh * (int64_t)(K * V);
#pragma unroll
  for (int kb = 0; kb < C::KB; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[kb][r] = (state_wave && h0) ? h0[st_base + (int64_t)(16 * kb + 4 * grp + r) * V + ncol] : 0.f;
  wait_vmcnt<0>();  // retire the h0 loads before the counted loop

  // Once a chunk's tiles are in LDS (this wave has waited for its own DMA of
  // them), before the barrier that opens the chunk (state waves):
  //   * the chunk's gate factors, once per workgroup (state wave 0, one token
  //     per lane), into the stage's gate block after the gates (which the DMA
  //     fills, bytes 0-255): e^{g_i} at +64 floats (the output's global term
  //     and, in the A form, P1), e^{g_last - g_j} at +128 (the state update);
  //   * A form: each state wave turns the 16 rows of A it loaded (4 KiB of
  //     the tile) into bf16 hi / lo in place, each 16-byte piece of 4 fp32
  //     becoming 4 hi then 4 lo, so P1 reads MFMA operands directly.
  // Both happen at the end of the chunk before, where the state waves wait
  // for the output waves anyway, rather than at the top of P1.
  auto prepare = [&](int sp) {
    if constexpr (HAS_G) {
      if (wq == 0) {
        float* const ge = stage_g(sp);
        const float gt = ge[lane];
        ge[64 + lane] = fast_exp(gt);
        ge[128 + lane] = fast_exp(ge[kBT - 1] - gt);
      }
    }
    if constexpr (FROM_A) {
      char* const ta = stage_w(sp) + wq * (C::kTileW / 4);
#pragma unroll
      for (int i = 0; i < C::kTileW / 4 / 16 / 64; ++i) {
        u32x4* const pc = reinterpret_cast<u32x4*>(ta + 16 * (lane + 64 * i));
        const f32x4 x = __builtin_bit_cast(f32x4, *pc);
        bf16x4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hi[e] = (bf16)x[e];
          lo[e] = (bf16)(x[e] - (float)hi[e]);
        }
        const u32x2 h2 = __builtin_bit_cast(u32x2, hi), l2 = __builtin_bit_cast(u32x2, lo);
        *pc = u32x4{h2[0], h2[1], l2[0], l2[1]};
      }
    }
  };

  if (state_wave && NT > 0) {
    issue_wu(0, 0);
#pragma unroll
    for (int m = 0; m < 3; ++m) issue_part(0, 0, m);
#pragma unroll
    for (int x = 1; x < C::kWuLead; ++x) issue_wu(x < NT ? x : NT - 1, x % kFStages);
    wait_vmcnt<C::kWaitFirst>();  // chunk 0's tiles are in
    prepare(0);
  }
  for (int64_t c = 0; c < NT; ++c) {
    const int s = (int)(c % kFStages);
    lds_barrier();  // A: chunk c is in LDS and prepared; every wave is done with chunk c - 1
    const char* tk = stage_k(s);
    const char* tq = stage_q(s);
    const float* gs = C::kGates ? stage_g(s) : nullptr;

    f32x4 vn[4];    // state waves: v_new rows j = 16 jb + 4 grp + r of column 16 wq + li
    bf16x8 vp[2];   // state waves: v_new as bf16 B-operand pairs
    if (state_wave) {
      // The next chunk's k / q / g DMA is issued in parts between P1's row
      // blocks, so the address unit drains between parts while the MFMAs run.
      const int64_t cn = c + C::kKqLead;
      const int64_t cnc = cn < NT ? cn : NT - 1;
      const int cns = (int)(cn % kFStages);
      // S as the B operand (pairs of 16-row tiles), also handed to the output wave.
      bf16x8 sb[KB2];
#pragma unroll
      for (int s2 = 0; s2 < KB2; ++s2) {
        const float f[8] = {S[2 * s2][0], S[2 * s2][1], S[2 * s2][2], S[2 * s2][3],
                            S[2 * s2 + 1][0], S[2 * s2 + 1][1], S[2 * s2 + 1][2], S[2 * s2 + 1][3]};
        sb[s2] = to_bf16x8(f);
        ls[s2 * 64] = sb[s2];
      }
      // P1: v_new = u - w S.
      const char* tw = stage_w(s);
      const char* tu = stage_u(s);
      if constexpr (FROM_A) {
        // v_new = A t with t_j = beta_j (v_j - e^{g_j} k_j . S) = (v beta - k
        // beta e^g S)_j: A (v beta) = u, A (k beta e^g) = w.  t as bf16
        // B-operand pairs; A (fp32) as bf16 hi + lo A operands.
        f32x4 t4[4];
        // A fragments of row blocks 0 and 1 read before the products with S
        // (those of blocks 2 and 3 after them: all of them up front spilled),
        // so the first products with t do not wait on LDS.
        u32x4 af[4][2][2];
#pragma unroll
        for (int ib = 0; ib < 2; ++ib)
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            if (2 * s2 > ib) continue;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
              af[ib][s2][hf] = *reinterpret_cast<const u32x4*>(tw + hl::tile_off(16 * ib + li, 2 * (32 * s2 + 16 * hf + 4 * grp), C::kRowW));
          }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          issue_part(cnc, cns, jb);
          const bf16x4 t = ds_read_tr16(reinterpret_cast<const bf16*>(tu + hl::tr_frag_off(16 * jb, 16 * wq, lane, C::kRowU)));
          const f32x4 ks = rows_times_S(tk, jb, sb);
          const f32x4 bt = *reinterpret_cast<const f32x4*>(gs + 192 + 16 * jb + 4 * grp);  // beta_j
          f32x4 eg = {1.f, 1.f, 1.f, 1.f};
          if constexpr (HAS_G) eg = *reinterpret_cast<const f32x4*>(gs + 64 + 16 * jb + 4 * grp);  // e^{g_j}
#pragma unroll
          for (int r = 0; r < 4; ++r) t4[jb][r] = bt[r] * ((float)t[r] - eg[r] * ks[r]);
        }
        bf16x8 tp[2];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const float f[8] = {t4[2 * s2][0], t4[2 * s2][1], t4[2 * s2][2], t4[2 * s2][3],
                              t4[2 * s2 + 1][0], t4[2 * s2 + 1][1], t4[2 * s2 + 1][2], t4[2 * s2 + 1][3]};
          tp[s2] = to_bf16x8(f);
        }
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          vn[ib] = zero4();
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            if (2 * s2 > ib) continue;  // A is lower triangular
            // Each 16-byte piece holds 4 elements as bf16 hi then lo (prepare).
            if (ib >= 2)
#pragma unroll
              for (int hf = 0; hf < 2; ++hf)
                af[ib][s2][hf] = *reinterpret_cast<const u32x4*>(tw + hl::tile_off(16 * ib + li, 2 * (32 * s2 + 16 * hf + 4 * grp), C::kRowW));
            const u32x4 x0 = af[ib][s2][0], x1 = af[ib][s2][1];
            const bf16x8 ah = __builtin_bit_cast(bf16x8, u32x4{x0[0], x0[1], x1[0], x1[1]});
            const bf16x8 al = __builtin_bit_cast(bf16x8, u32x4{x0[2], x0[3], x1[2], x1[3]});
            vn[ib] = mfma16x16x32(ah, tp[s2], vn[ib]);
            vn[ib] = mfma16x16x32(al, tp[s2], vn[ib]);
          }
        }
      } else {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          issue_part(cnc, cns, jb);
          const bf16x4 t = ds_read_tr16(reinterpret_cast<const bf16*>(tu + hl::tr_frag_off(16 * jb, 16 * wq, lane, C::kRowU)));
#pragma unroll
          for (int r = 0; r < 4; ++r) vn[jb][r] = (float)t[r];
          vn[jb] -= rows_times_S(tw, jb, sb);
        }
      }
      if constexpr (STORE_VN) {
        bf16* vb = vnew + ((b * T + c * kBT) * H + hh) * V;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) store_rows(vb, jb, vn[jb]);
      }
      // v_new as the B operand of the local term (paired order over j), to the output wave.
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const float f[8] = {vn[2 * s2][0], vn[2 * s2][1], vn[2 * s2][2], vn[2 * s2][3],
                            vn[2 * s2 + 1][0], vn[2 * s2 + 1][1], vn[2 * s2 + 1][2], vn[2 * s2 + 1][3]};
        vp[s2] = to_bf16x8(f);
        lv[s2 * 64] = vp[s2];
      }
    } else {
      // Scores, once per workgroup: P[i][j] = (q_i . k_j) e^{g_i - g_j} for
      // j <= i (0 above the diagonal), as bf16 rows of lp.  The ten 16 x 16
      // blocks (ib, jb <= ib) are shared out 3 / 3 / 2 / 2 over the output
      // waves; the accumulator of block (ib, jb) holds
      // P^T[j = 16 jb + 4 grp + r][i = 16 ib + li], so each lane stores 4
      // consecutive j of row i as one 8-byte write.
      // Each wave's blocks are fixed (wq is wave-uniform), so every k and q
      // fragment a wave needs is read from LDS before its first MFMA, and
      // only diagonal blocks are masked.  (A loop over runtime block ids
      // read each block's fragments after the previous block's products.)
      constexpr int KS = K / 32;
      auto frags = [&](const char* tile, int rb, bf16x8* f) {
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2)
          f[s2] = load8(reinterpret_cast<const bf16*>(tile + hl::row8_frag_off(16 * rb, 32 * s2, lane, C::kRowK)));
      };
      auto block = [&](int ib, int jb, const bf16x8* kf, const bf16x8* qf) {
        f32x4 pt = zero4();
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2) pt = mfma16x16x32(kf[s2], qf[s2], pt);
        const int i = 16 * ib + li;
        const float gi = HAS_G ? gs[i] : 0.f;
        bf16x4 pv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * jb + 4 * grp + r;
          float gate = 1.f;
          if constexpr (HAS_G) gate = fast_exp(gi - gs[j]);
          pv[r] = (bf16)((jb < ib || j <= i) ? pt[r] * gate : 0.f);
        }
        *reinterpret_cast<bf16x4*>(lp + hl::pair_frag_off(16 * ib, 16 * jb, lane, 128)) = pv;
      };
      bf16x8 fa[KS], fb[KS], fc[KS], fd[KS];
      if (wq == 0) {  // (3, 0), (3, 1), (3, 2)
        frags(tq, 3, fa); frags(tk, 0, fb); frags(tk, 1, fc); frags(tk, 2, fd);
        block(3, 0, fb, fa); block(3, 1, fc, fa); block(3, 2, fd, fa);
      } else if (wq == 1) {  // (2, 0), (2, 1), (2, 2)
        frags(tq, 2, fa); frags(tk, 0, fb); frags(tk, 1, fc); frags(tk, 2, fd);
        block(2, 0, fb, fa); block(2, 1, fc, fa); block(2, 2, fd, fa);
      } else if (wq == 2) {  // (3, 3), (1, 0)
        frags(tq, 3, fa); frags(tk, 3, fb); frags(tq, 1, fc); frags(tk, 0, fd);
        block(3, 3, fb, fa); block(1, 0, fd, fc);
      } else {  // (1, 1), (0, 0)
        frags(tq, 1, fa); frags(tk, 1, fb); frags(tq, 0, fc); frags(tk, 0, fd);
        block(1, 1, fb, fa); block(0, 0, fd, fc);
      }
    }
    lds_barrier();  // M: P, the S pairs and the v_new pairs of chunk c are in LDS

    if (state_wave) {
      // P1 of this chunk is done with its w and u: chunk c + kWuLead's go to
      // that chunk's stage (clamped re-loads at the end land in slots no later
      // chunk reads).
      const int64_t cw = c + C::kWuLead;
      issue_wu(cw < NT ? cw : NT - 1, (int)(cw % kFStages));
      // P2: S = e^{g_last} S + k^T (v_new e^{g_last - g}).
      bf16x8 vh[2];
      float decay = 1.f;
      if constexpr (HAS_G) {
        decay = fast_exp(gs[kBT - 1]);
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const f32x4 fa = *reinterpret_cast<const f32x4*>(gs + 128 + 32 * s2 + 4 * grp);  // e^{g_last - g_j}
          const f32x4 fb = *reinterpret_cast<const f32x4*>(gs + 128 + 32 * s2 + 16 + 4 * grp);
          float f[8];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            f[r] = vn[2 * s2][r] * fa[r];
            f[4 + r] = vn[2 * s2 + 1][r] * fb[r];
          }
          vh[s2] = to_bf16x8(f);
        }
      } else {
        vh[0] = vp[0];
        vh[1] = vp[1];
      }
#pragma unroll
      for (int kb = 0; kb < C::KB; ++kb) {
        if constexpr (HAS_G) S[kb] *= decay;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x4 a = ds_read_tr16(reinterpret_cast<const bf16*>(tk + hl::tr_frag_off(32 * s2, 16 * kb, lane, C::kRowK)));
          const bf16x4 bq = ds_read_tr16(reinterpret_cast<const bf16*>(tk + hl::tr_frag_off(32 * s2 + 16, 16 * kb, lane, C::kRowK)));
          S[kb] = mfma16x16x32(concat(a, bq), vh[s2], S[kb]);
        }
      }
      // Chunk c + 1's tiles (this wave's DMA of them) are in: prepare its stage.
      if (c + 1 < NT) {
        wait_vmcnt<C::kWaitSteady>();
        prepare((int)((c + 1) % kFStages));
      }
    } else {
      // Output, one 16-row query block at a time: o = scale (e^{g_i} q S + P v_new).
      bf16x8 sb[KB2];
#pragma unroll
      for (int s2 = 0; s2 < KB2; ++s2) sb[s2] = ls[s2 * 64];
      const bf16x8 vb16[2] = {lv[0], lv[64]};
      bf16* ob = o + ((b * T + c * kBT) * H + hh) * V;
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        f32x4 acc = rows_times_S(tq, ib, sb);  // q S
        if constexpr (HAS_G) {
          const f32x4 e = *reinterpret_cast<const f32x4*>(gs + 64 + 16 * ib + 4 * grp);  // e^{g_i}
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] *= e[r];
        }
        // Local term: A = P[i][j] rows of lp, B = v_new (pairs), paired order
        // over j; key blocks above the diagonal block contribute zero.
        f32x4 loc = zero4();
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          if (2 * s2 > ib) continue;
          const bf16x4 lo = *reinterpret_cast<const bf16x4*>(lp + hl::pair_frag_off(16 * ib, 32 * s2, lane, 128));
          bf16x4 hi = {};
          if (2 * s2 + 1 <= ib) hi = *reinterpret_cast<const bf16x4*>(lp + hl::pair_frag_off(16 * ib, 32 * s2 + 16, lane, 128));
          loc = mfma16x16x32(concat(lo, hi), vb16[s2], loc);
        }
        store_rows(ob, ib, (acc + loc) * scale);
      }
    }
  }
  wait_vmcnt<0>();  // no DMA may still target this workgroup's LDS when it exits

  if (state_wave && ht) {
#pragma unroll
    for (int kb = 0; kb < C::KB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) ht[st_base + (int64_t)(16 * kb + 4 * grp + r) * V + ncol] = S[kb][r];
  }
}

template <int K, int V, bool FROM_A>
hipError_t launch_fused(const void* q, const void* k, const void* w, const void* u, const void* A,
                        const void* beta, const void* g, const void* h0, void* o, void* vnew, void* ht,
                        float scale, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / kBT, BH = B * H;
  const dim3 grid((unsigned)(BH * (V / kFBV)));
#define THM_FUSED_LAUNCH(HG, SV)                                                                   \
  hipLaunchKernelGGL((chunk_fwd_fused_kernel<K, V, HG, SV, FROM_A>), grid, dim3(kFThreads), 0, s,  \
                     (const bf16*)q, (const bf16*)k, (const bf16*)w, (const bf16*)u, (const float*)A, \
                     (const float*)beta, (const float*)g, (const float*)h0, (bf16*)o, (bf16*)vnew,  \
                     (float*)ht, scale, T, H, NT, BH)
  if (g) {
    if (vnew) THM_FUSED_LAUNCH(true, true);
    else THM_FUSED_LAUNCH(true, false);
  } else {
    if (vnew) THM_FUSED_LAUNCH(false, true);
    else THM_FUSED_LAUNCH(false, false);
  }
#undef THM_FUSED_LAUNCH
  return hipGetLastError();
}

// Shared argument checks and dispatch of both entry points (FROM_A: w = A,
// u = v, beta given).
template <bool FROM_A>
int fused_entry(const void* q, const void* k, const void* w, const void* u, const void* beta,
                const void* g, const void* h0, void* o, void* v_new, void* ht, float scale, int64_t B,
                int64_t T, int64_t H, int64_t K, int64_t V, int32_t chunk_size, int32_t qkv_dtype,
                void* stream) {
  if (chunk_size != kBT) return THM_ERR_BAD_ARGUMENT;
  if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || T % kBT) return THM_ERR_BAD_SHAPE;
  if (qkv_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;  // the fused path is bf16-only
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) return THM_ERR_UNSUPPORTED;
  if (B == 0) return THM_OK;
  if (T == 0 && !ht) return THM_OK;
  if (T > 0 && (!q || !k || !w || !u || !o || (FROM_A && !beta))) return THM_ERR_NULL_POINTER;
  const void* p16[] = {q, k, w, u};
  for (const void* p : p16)
    if (p && ((uintptr_t)p % 16)) return THM_ERR_MISALIGNED;
  const void* p4[] = {g, h0, ht, beta};
  for (const void* p : p4)
    if (p && ((uintptr_t)p % 4)) return THM_ERR_MISALIGNED;
  if (((uintptr_t)o % 8) || (v_new && ((uintptr_t)v_new % 8))) return THM_ERR_MISALIGNED;
  if (B > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
  if (!launch_fits(B * H * (V / kFBV), kFThreads)) return THM_ERR_BAD_SHAPE;
  // 32-bit lane offsets (A rows are 256 bytes for any K).
  const int64_t row_max = (K > V ? K : V) * 2 > 256 || !FROM_A ? (K > V ? K : V) * 2 : 256;
  if (64 * H * row_max > (INT64_C(1) << 31)) return THM_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  const void* wp = FROM_A ? nullptr : w;
  const void* ap = FROM_A ? w : nullptr;
  hipError_t e;
  if (K == 64 && V == 64) e = launch_fused<64, 64, FROM_A>(q, k, wp, u, ap, beta, g, h0, o, v_new, ht, scale, B, T, H, s);
  else if (K == 64 && V == 128) e = launch_fused<64, 128, FROM_A>(q, k, wp, u, ap, beta, g, h0, o, v_new, ht, scale, B, T, H, s);
  else if (K == 128 && V == 64) e = launch_fused<128, 64, FROM_A>(q, k, wp, u, ap, beta, g, h0, o, v_new, ht, scale, B, T, H, s);
  else e = launch_fused<128, 128, FROM_A>(q, k, wp, u, ap, beta, g, h0, o, v_new, ht, scale, B, T, H, s);
  return (int)e;
}

}  // namespace
}  // namespace thm

extern "C" int thm_chunk_gated_delta_fwd(const void* q, const void* k, const void* w, const void* u,
                                         const void* g, const void* h0, void* o, void* v_new,
                                         void* ht, float scale, int64_t B, int64_t T, int64_t H,
                                         int64_t K, int64_t V, int32_t chunk_size,
                                         int32_t qkv_dtype, void* stream) {
  return thm::fused_entry<false>(q, k, w, u, nullptr, g, h0, o, v_new, ht, scale, B, T, H, K, V, chunk_size,
                                 qkv_dtype, stream);
}

extern "C" int thm_chunk_gated_delta_fwd_a(const void* q, const void* k, const void* v, const void* beta,
                                           const void* A, const void* g, const void* h0, void* o,
                                           void* v_new, void* ht, float scale, int64_t B, int64_t T,
                                           int64_t H, int64_t K, int64_t V, int32_t chunk_size,
                                           int32_t qkv_dtype, void* stream) {
  return thm::fused_entry<true>(q, k, A, v, beta, g, h0, o, v_new, ht, scale, B, T, H, K, V, chunk_size,
                                qkv_dtype, stream);
}
