// Blocked inversion of the WY matrix of one 64-token chunk (gfx950), shared by
// the A-builder (wy_build_A.hip) and the fused WY forward (wy_fwd.hip).
//
// With L = sign M strictly lower triangular, M[i][j] = beta_i (k_i . k_j)
// e^{g_i - g_j}, the chunk's A = (I + L)^{-1} is block lower triangular in
// 16 x 16 blocks:
//   X_ii = (I + L_ii)^{-1}                        (forward substitution)
//   X_ij = -X_ii sum_{m=j}^{i-1} L_im X_mj        (i > j, by distance i - j)
// Lower blocks (i, j), j <= i < 4, are stored packed (blk(i, j)) in LDS with
// row pitch kBP floats.  The math follows the reference's `_build_A`
// (kernels/recompute_w_u/reference.py:48-91: a torch matmul for M and
// solve_triangular for the inverse).
#pragma once

#include "h_layout.h"
#include "mfma.h"

namespace thm {
namespace wy {

constexpr int kBT = 64;
constexpr int kBP = hl::kWyPitch;  // LDS pitch (floats) of a 16x16 block (h_layout.h)
constexpr int kBlk = 16 * kBP;  // floats per block
constexpr int kLdsFloats = 10 * kBlk + 10 * kBlk + 3 * kBlk;  // L, X, per-level T

// Packed index of lower block (i, j), j <= i < 4.
__host__ __device__ constexpr int blk(int i, int j) { return i * (i + 1) / 2 + j; }

__device__ __forceinline__ f32x4 mfma16x16x4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// acc += P Q for 16x16 blocks P, Q in LDS (pitch kBP): lane (g, l) feeds
// P[l][4q + g] and Q[4q + g][l] at k-step q; acc[r] = row 4g + r, column l.
__device__ __forceinline__ f32x4 block_mm(const float* P, const float* Q, f32x4 acc) {
  const int lane = lane_id();
#pragma unroll
  for (int q = 0; q < 4; ++q) acc = mfma16x16x4f32(P[hl::wy_a_off(lane, q)], Q[hl::wy_b_off(lane, q)], acc);
  return acc;
}

__device__ __forceinline__ void block_put(float* D, f32x4 acc, float sgn) {
  const int lane = lane_id();
#pragma unroll
  for (int r = 0; r < 4; ++r) D[hl::wy_put_off(lane, r)] = sgn * acc[r];
}

// L blocks of one chunk from k fragments fh[tb][s] = k[16 tb + li][32 s + 8 grp .. + 7]
// (fp32 k: bf16 hi fh + lo fl, three products): wave wv forms the lower blocks
// p = wv, wv + 4, wv + 8 of the packed order (compile-time block indices, so
// the fragments stay in registers); sb, sg hold beta and g of the chunk.
template <int SIGN, int KS, bool kSplit>
__device__ __forceinline__ void form_L(const bf16x8 (&fh)[4][KS], const bf16x8 (&fl)[4][kSplit ? KS : 1],
                                       const float* sb, const float* sg, float* Lb, int wv) {
  const int lane = lane_id(), grp = lane >> 4, li = lane & 15;
#pragma unroll
  for (int p = 0; p < 10; ++p) {
    if ((p & 3) != wv) continue;  // wave-uniform
    constexpr int kIb[10] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3};
    const int ib = kIb[p], jb = p - ib * (ib + 1) / 2;
    f32x4 acc = zero4();
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      acc = mfma16x16x32(fh[ib][s], fh[jb][s], acc);
      if constexpr (kSplit) {
        acc = mfma16x16x32(fh[ib][s], fl[jb][s], acc);
        acc = mfma16x16x32(fl[ib][s], fh[jb][s], acc);
      }
    }
    const int j = 16 * jb + li;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * ib + 4 * grp + r;
      Lb[p * kBlk + hl::wy_put_off(lane, r)] =
          (j < i) ? (float)SIGN * sb[i] * acc[r] * fast_exp(sg[i] - sg[j]) : 0.f;
    }
  }
}

// form_L for bf16 k with the fragments read from LDS per block (frag(tb, s)
// returns k[16 tb + li][32 s + 8 grp .. + 7]) instead of held in registers
// for the whole chunk: the same products in the same order, ~40 fewer VGPRs
// at K = 128 (the A-builder's pipelined kernel, 4 workgroups per CU).
template <int SIGN, int KS, typename Frag>
__device__ __forceinline__ void form_L_lds(Frag frag, const float* sb, const float* sg, float* Lb, int wv) {
  const int lane = lane_id(), grp = lane >> 4, li = lane & 15;
#pragma unroll
  for (int p = 0; p < 10; ++p) {
    if ((p & 3) != wv) continue;  // wave-uniform
    constexpr int kIb[10] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3};
    const int ib = kIb[p], jb = p - ib * (ib + 1) / 2;
    bf16x8 fi[KS], fj[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      fi[s] = frag(ib, s);
      fj[s] = frag(jb, s);
    }
    f32x4 acc = zero4();
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma16x16x32(fi[s], fj[s], acc);
    const int j = 16 * jb + li;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * ib + 4 * grp + r;
      Lb[p * kBlk + hl::wy_put_off(lane, r)] =
          (j < i) ? (float)SIGN * sb[i] * acc[r] * fast_exp(sg[i] - sg[j]) : 0.f;
    }
  }
}

// X = (I + L)^{-1} from the L blocks (all four waves; ends with a barrier):
//   diagonal blocks: wave w, lane c < 16 owns column c of X_ww (16-row
//   forward substitution), then one barrier;
//   off-diagonal blocks: wave j forms column j of X, X_{j+1,j} .. X_{3,j}
//   (3, 2, 1 and 0 blocks), each two fp32 MFMA products (exact fp32
//   multiplies): T = sum L_im X_mj, then X_ij = -X_ii T, T passing through
//   the wave's own LDS block to change from the accumulator to the operand
//   layout.  One barrier at the end (a barrier per level measured 266 against
//   251 us for the fused WY kernel at config 4, 146 against 141 for the
//   A-builder, bit-identical).
__device__ __forceinline__ void invert_L(const float* Lb, float* Xb, float* Tb, int wv) {
  const int lane = lane_id();
  {
    const float* L = Lb + blk(wv, wv) * kBlk;
    float* X = Xb + blk(wv, wv) * kBlk;
    if (lane < 16) {
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float a0 = (r == lane) ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
        for (int s = 0; s < r; ++s) {
          if (s & 1) a1 = fmaf(-L[r * kBP + s], x[s], a1);
          else a0 = fmaf(-L[r * kBP + s], x[s], a0);
        }
        x[r] = a0 + a1;
        X[r * kBP + lane] = x[r];
      }
    }
  }
  lds_barrier();
  // Column j of X is wave j's alone: X_ij needs X_mj (m < i, this wave's own
  // earlier blocks), the L blocks and X_ii (both behind the barrier above), so
  // the levels need no workgroup barrier.  Each block a wave writes (T, then
  // X_ij) is read back by other lanes of the same wave, so every write is
  // followed by a wave-scope sync.
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    const int j = wv, i = wv + d;
    if (i < 4) {  // wave-uniform
      f32x4 acc = zero4();
#pragma unroll
      for (int m = 0; m < 3; ++m) {
        const int mm = j + m;
        if (mm < i) acc = block_mm(Lb + blk(i, mm) * kBlk, Xb + blk(mm, j) * kBlk, acc);
      }
      block_put(Tb + wv * kBlk, acc, 1.f);
      wave_lds_sync();
      acc = block_mm(Xb + blk(i, i) * kBlk, Tb + wv * kBlk, zero4());
      block_put(Xb + blk(i, j) * kBlk, acc, -1.f);
      wave_lds_sync();
    }
  }
  lds_barrier();
}

}  // namespace wy
}  // namespace thm
