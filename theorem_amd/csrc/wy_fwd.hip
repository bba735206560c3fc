// Fused WY forward of the Gated DeltaNet chunk forward for MI355X (gfx950):
// per chunk c of 64 tokens,
//   A_c = (I + sign M)^{-1},  M[i][j] = beta_i (k_i . k_j) e^{g_i - g_j}  (j < i),
//   w_c = A_c (k_c * beta_c e^{g_c}),   u_c = A_c (v_c * beta_c),
// i.e. the A-builder (wy_build_A.hip; the reference's `_build_A`,
// kernels/recompute_w_u/reference.py:48-91) followed by recompute_w_u
// (recompute_w_u.hip; reference.py:118-149) in one kernel, so A never travels
// through HBM (its fp32 write and read are half of the two kernels' bytes).
//
// One workgroup (4 wavefronts) per (b, chunk, head) tile, head fastest:
//   1. k fragments (16-byte row loads, every wave all 64 rows), beta and g;
//   2. the L blocks (wy_blocks.h); then the [k | v] tile loads are issued
//      into registers (the k rows hit L2), in flight during the inversion;
//   3. X = A_c = (I + L)^{-1}, blocked (wy_blocks.h);
//   4. wave wv forms its scaled A operands A'[t][j] (t = 16 wv + li) from X:
//      A diag(beta e^g) for w and A diag(beta) for u, each split into bf16
//      hi + lo, as recompute_w_u does with A read from HBM;
//   5. barrier; the [k | v] tile is staged in LDS over the inversion's blocks;
//      barrier;
//   6. D[n][t] = sum_j X[j][n] A'[t][j] on v_mfma_f32_16x16x32_bf16 (X^T
//      fragments by ds_read_b64_tr_b16), stored as 16-byte pieces of 8
//      features after a lane-pair exchange.
// A is the same fp32 value the A-builder writes, and the products are
// recompute_w_u's, so w and u equal the two-kernel path's bit for bit.
// bf16 inputs only.  HBM traffic per tile: k, v, beta, g read once, w, u
// written once.
#include "h_layout.h"
#include "vmem.h"
#include "wy_blocks.h"

namespace thm {
namespace {

using wy::blk;
using wy::kBlk;
using wy::kBP;
constexpr int kBT = wy::kBT;
constexpr int kWyThreads = 256;

template <int K, int V>
struct WyCfg {
  static constexpr int kN = K + V;
  // [k | v] tile: row pitch in bytes, rows stored in the nat_row order
  // (h_layout.h wy_tile_pitch, ntile_off, ntr_frag_off).
  static constexpr int kPitch = hl::wy_tile_pitch(kN);
  static constexpr int kTileBytes = kBT * kPitch;
  static constexpr int kInvBytes = wy::kLdsFloats * 4;
  static constexpr int kUnion = kTileBytes > kInvBytes ? kTileBytes : kInvBytes;
  static constexpr int kNB = kN / 16;
  static constexpr int kCPR = kN / 8;                      // 16-byte chunks per row
  static constexpr int kLoads = kBT * kCPR / kWyThreads;   // per thread
  static constexpr int KS = K / 32;
  static_assert(kBT * kCPR % kWyThreads == 0, "staging must divide evenly");
};

// Scaled A operands of wave wv from the inverted blocks Xb: A'[t][j] for
// t = 16 wv + li, j = 32 s + 8 grp + 0..7, in X's block (wv, jb = 2 s + grp / 2),
// columns 8 (grp & 1) + 0..7: A diag(beta e^g) for w and A diag(beta) for u,
// each split into bf16 hi + lo, as recompute_w_u does with A read from HBM.
struct WyOperands {
  bf16x8 awh[2], awl[2], auh[2], aul[2];
};
__device__ __forceinline__ WyOperands wy_operands(const float* Xb, const float* sb, const float* sg, int wv) {
  const int lane = lane_id(), grp = lane >> 4, li = lane & 15;
  WyOperands op;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int jb = 2 * s + (grp >> 1);
    const float* X = Xb + blk(wv, jb < wv ? jb : wv) * kBlk + li * kBP + 8 * (grp & 1);
    float fw[8], fu[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 32 * s + 8 * grp + i;
      const float a = (jb <= wv) ? X[i] : 0.f;
      fu[i] = a * sb[j];
      fw[i] = fu[i] * fast_exp(sg[j]);
    }
    split_bf16x8(fw, op.awh[s], op.awl[s]);
    split_bf16x8(fu, op.auh[s], op.aul[s]);
  }
  return op;
}

// D[n][t] = sum_j X[j][n] A'[t][j] for this wave's 16 tokens, stored to w / u:
// the [k | v] tile xs (`pitch` bytes per row, rows in the nat_row order)
// gives the X^T fragments by ds_read_b64_tr_b16 in the natural order; each
// lane ends with features 16 nb + 4 grp .. + 3 of token t = 16 wv + li.  The
// products are recompute_w_u's.  Column blocks are taken in pairs
// (2 m, 2 m + 1) and stored as 16-byte pieces of 8 consecutive features
// (vmem.h acc_pair_to_b128): 8-byte stores of 4 features put 32-byte runs of
// 16 rows in one store instruction, which the memory path takes far more
// slowly.
template <int K, int V>
__device__ __forceinline__ void wy_products(const char* xs, int pitch, const WyOperands& op, bf16* w, bf16* u,
                                            int64_t trow) {
  const int lane = lane_id(), grp = lane >> 4;
  static_assert(K % 32 == 0 && V % 32 == 0, "column pairs do not straddle w and u");
#pragma unroll
  for (int m = 0; m < (K + V) / 32; ++m) {
    const bool is_w = 32 * m < K;
    f32x4 acc[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int nb = 2 * m + p;
      acc[p] = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const bf16x8 xh =
            concat(ds_read_tr16(reinterpret_cast<const bf16*>(xs + hl::ntr_frag_off(32 * s, 0, 16 * nb, lane, pitch))),
                   ds_read_tr16(reinterpret_cast<const bf16*>(xs + hl::ntr_frag_off(32 * s, 1, 16 * nb, lane, pitch))));
        acc[p] = mfma16x16x32(xh, is_w ? op.awh[s] : op.auh[s], acc[p]);
        acc[p] = mfma16x16x32(xh, is_w ? op.awl[s] : op.aul[s], acc[p]);
      }
    }
    const u32x4 piece = acc_pair_to_b128(acc[0], acc[1]);
    if (is_w) *reinterpret_cast<u32x4*>(w + trow * K + 32 * m + pair_col(grp)) = piece;
    else *reinterpret_cast<u32x4*>(u + trow * V + 32 * m - K + pair_col(grp)) = piece;
  }
}

template <int K, int V, int SIGN>
__global__ void __launch_bounds__(kWyThreads)
wy_fwd_kernel(const bf16* __restrict__ k, const bf16* __restrict__ v,
              const float* __restrict__ beta, const float* __restrict__ g, bf16* __restrict__ w,
              bf16* __restrict__ u, int64_t T, int64_t H, int64_t NT) {
  using C = WyCfg<K, V>;
  constexpr int KS = C::KS;
  __shared__ __attribute__((aligned(16))) char lds[C::kUnion];
  __shared__ float sb[kBT], sg[kBT];
  float* const Lb = reinterpret_cast<float*>(lds);  // L = sign M, lower blocks
  float* const Xb = Lb + 10 * kBlk;                  // X = A_c, lower blocks
  float* const Tb = Xb + 10 * kBlk;                  // per-level partial products
  char* const xs = lds;                              // [k | v] tile, after the inversion

  const TileCoord tc = tile_coord(blockIdx.x, H, NT, T);
  const int64_t h = tc.hh;
  const int64_t tok0 = tc.tok0;
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int lane = tid & 63;
  const int grp = lane >> 4, li = lane & 15;

  // 1. k fragments: fh[tb][s] = k[tok0 + 16 tb + li][32 s + 8 grp .. + 7].
  bf16x8 fh[4][KS], fl[4][1];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const bf16* row = k + ((tok0 + 16 * tb + li) * H + h) * K + 8 * grp;
#pragma unroll
    for (int s = 0; s < KS; ++s) fh[tb][s] = load8(row + 32 * s);
  }
  if (tid < kBT) {
    sb[tid] = beta[(tok0 + tid) * H + h];
    sg[tid] = g ? g[(tok0 + tid) * H + h] : 0.f;
  }
  lds_barrier();

  // 2. L blocks, then the [k | v] tile loads (thread q: row q / kCPR, chunk q % kCPR).
  wy::form_L<SIGN, KS, false>(fh, fl, sb, sg, Lb, wv);
  u32x4 xr[C::kLoads];
#pragma unroll
  for (int it = 0; it < C::kLoads; ++it) {
    const int q = tid + it * kWyThreads;
    const int j = q / C::kCPR;
    const int col = (q - j * C::kCPR) * 8;
    const int64_t row = (tok0 + j) * H + h;
    // Non-temporal: read once here (measured 1% faster at config 4).
    xr[it] = ldg16_nt(col < K ? (const void*)(k + row * K + col) : (const void*)(v + row * V + (col - K)));
  }
  lds_barrier();

  // 3. X = (I + L)^{-1}.
  wy::invert_L(Lb, Xb, Tb, wv);

  // 4. Scaled A operands of this wave (read from X before the tile overwrites it).
  const WyOperands op = wy_operands(Xb, sb, sg, wv);

  // 5. Stage the tile over the inversion's blocks.
  lds_barrier();  // every wave has read its A operands
#pragma unroll
  for (int it = 0; it < C::kLoads; ++it) {
    const int q = tid + it * kWyThreads;
    const int j = q / C::kCPR;
    const int col = (q - j * C::kCPR) * 8;
    *reinterpret_cast<u32x4*>(xs + hl::ntile_off(j, col, C::kPitch)) = xr[it];
  }
  lds_barrier();

  // 6. Products and stores.
  wy_products<K, V>(xs, C::kPitch, op, w, u, (tok0 + 16 * wv + li) * H + h);
}

// ---------------------------------------------------------------------------
// Grids of at least two tiles per persistent workgroup: software-pipelined.
//
// With one tile per workgroup, every resident workgroup of a CU moves through
// the same phases at about the same time: a burst of loads, then the latency
// of form_L and the inversion (seven barriers) with no memory traffic, then
// the stores.  Here 2 workgroups per CU walk the tiles t, t + G, t + 2G, ...
// (G = the grid) and each issues the next tile's [k | v], beta and g loads into
// registers before computing the current tile, so those loads are in flight
// through the current tile's form_L, inversion and products.  The [k | v]
// tile is staged in LDS once and form_L takes its k fragments from there (the
// one-tile kernel loads them separately from global memory).  The tile and
// the inversion blocks have separate LDS (59 KB per workgroup).  The
// arithmetic is the one-tile kernel's (wy_blocks.h, wy_operands,
// wy_products), so w and u are bit-identical to it.
constexpr int kWyPipeWGsPerCU = 2;

template <int K, int V, int SIGN>
__global__ void __launch_bounds__(kWyThreads, 2)
wy_fwd_pipe_kernel(const bf16* __restrict__ k, const bf16* __restrict__ v,
                   const float* __restrict__ beta, const float* __restrict__ g, bf16* __restrict__ w,
                   bf16* __restrict__ u, int64_t T, int64_t H, int64_t NT, int64_t tiles) {
  using C = WyCfg<K, V>;
  constexpr int KS = C::KS;
  __shared__ __attribute__((aligned(16))) char xs[kBT * C::kPitch];  // [k | v] tile
  __shared__ float Lb[10 * kBlk];  // L = sign M, lower blocks
  __shared__ float Xb[10 * kBlk];  // X = A_c, lower blocks
  __shared__ float Tb[3 * kBlk];   // per-level partial products
  __shared__ float sb[kBT], sg[kBT];

  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int lane = tid & 63;
  const int grp = lane >> 4, li = lane & 15;

  // Tile -> (b, c, head), head fastest within an XCD (h_layout.h
  // xcd_tile_order, a bijection; workgroup w runs on XCD w % 8, and with a
  // grid that is a multiple of 8, as 2 workgroups on each of 256 CUs, its
  // tiles t = w + i G stay on that XCD): the 16 heads of one (b, chunk) share
  // an L2, and the beta / g lines they share are fetched once.  HBM reads at config 4: 545.5 MB, the algorithmic bytes, against
  // 604 MB with the plain head-fastest order (230.9 against 231.8 us, w and u
  // bit-identical).
  auto tok_of = [&](int64_t tile, int64_t& h) {
    const TileCoord tc = tile_coord(hl::xcd_tile_order((uint32_t)tile, H, tiles / H), H, NT, T);
    h = tc.hh;
    return tc.tok0;
  };

  // Prefetched registers of one tile: the k block, then the v block, each
  // loaded as in chunk_fwd_o (h_layout.h o_blk_lane / o_blk_step: a 32-bit
  // per-lane offset on a wave-uniform base; thread tid's load it is token
  // tid / (n / 8) + it 256 / (n / 8), elements 8 (tid % (n / 8)) .. + 7).
  constexpr int kLK = K / 32, kLV = V / 32;
  static_assert(kLK + kLV == C::kLoads && kWyThreads == 256, "load split");
  const uint32_t k_off = hl::o_blk_lane(tid, K, H * K), v_off = hl::o_blk_lane(tid, V, H * V);
  u32x4 xr[C::kLoads];
  float br = 0.f, gr = 0.f;
  auto prefetch = [&](int64_t tile) {
    int64_t h;
    const int64_t tok0 = tok_of(tile, h);
    const char* const kb = reinterpret_cast<const char*>(k + (tok0 * H + h) * K);
    const char* const vb = reinterpret_cast<const char*>(v + (tok0 * H + h) * V);
#pragma unroll
    for (int it = 0; it < kLK; ++it) xr[it] = ldg16_nt(kb + hl::o_blk_step(it, K, H * K) + k_off);
#pragma unroll
    for (int it = 0; it < kLV; ++it) xr[kLK + it] = ldg16_nt(vb + hl::o_blk_step(it, V, H * V) + v_off);
    if (tid < kBT) {
      const int64_t row = (tok0 + tid) * H + h;
      br = beta[row];
      gr = g ? g[row] : 0.f;
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int it = 0; it < kLK; ++it) {
      const int q = tid + it * kWyThreads, j = q / (K / 8), col = (q % (K / 8)) * 8;
      *reinterpret_cast<u32x4*>(xs + hl::ntile_off(j, col, C::kPitch)) = xr[it];
    }
#pragma unroll
    for (int it = 0; it < kLV; ++it) {
      const int q = tid + it * kWyThreads, j = q / (V / 8), col = (q % (V / 8)) * 8;
      *reinterpret_cast<u32x4*>(xs + hl::ntile_off(j, K + col, C::kPitch)) = xr[kLK + it];
    }
    if (tid < kBT) {
      sb[tid] = br;
      sg[tid] = gr;
    }
  };

  int64_t t = blockIdx.x;
  if (t >= tiles) return;  // whole workgroup
  prefetch(t);
  stage();
  lds_barrier();
  for (;;) {
    const int64_t tn = t + gridDim.x;
    if (tn < tiles) prefetch(tn);  // in flight while tile t computes
    int64_t h;
    const int64_t tok0 = tok_of(t, h);

    // k fragments from the staged tile: fh[tb][s] = k[16 tb + li][32 s + 8 grp .. + 7].
    bf16x8 fh[4][KS], fl[4][1];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int s = 0; s < KS; ++s)
        fh[tb][s] = load8(reinterpret_cast<const bf16*>(xs + hl::ntile_off(16 * tb + li, 32 * s + 8 * grp, C::kPitch)));
    wy::form_L<SIGN, KS, false>(fh, fl, sb, sg, Lb, wv);
    lds_barrier();
    wy::invert_L(Lb, Xb, Tb, wv);  // ends with a barrier
    const WyOperands op = wy_operands(Xb, sb, sg, wv);
    wy_products<K, V>(xs, C::kPitch, op, w, u, (tok0 + 16 * wv + li) * H + h);

    if (tn >= tiles) break;
    lds_barrier();  // every wave is done with tile t's LDS
    stage();
    lds_barrier();
    t = tn;
  }
}

template <int K, int V>
hipError_t launch_wy(const void* k, const void* v, const void* beta, const void* g, void* w, void* u,
                     int64_t B, int64_t T, int64_t H, int sign, hipStream_t s) {
  const int64_t NT = T / kBT;
  const int64_t tiles = B * NT * H;
  const int64_t pgrid = (int64_t)device_cu_count() * kWyPipeWGsPerCU;
  if (pgrid > 0 && tiles >= 2 * pgrid) {
#define THM_WY_PIPE_LAUNCH(SG)                                                                        \
  hipLaunchKernelGGL((wy_fwd_pipe_kernel<K, V, SG>), dim3((unsigned)pgrid), dim3(kWyThreads), 0, s,   \
                     (const bf16*)k, (const bf16*)v, (const float*)beta, (const float*)g, (bf16*)w, \
                     (bf16*)u, T, H, NT, tiles)
    if (sign < 0) THM_WY_PIPE_LAUNCH(-1);
    else THM_WY_PIPE_LAUNCH(1);
#undef THM_WY_PIPE_LAUNCH
    return hipGetLastError();
  }
  const dim3 grid((unsigned)tiles);
#define THM_WY_LAUNCH(SG)                                                                        \
  hipLaunchKernelGGL((wy_fwd_kernel<K, V, SG>), grid, dim3(kWyThreads), 0, s, (const bf16*)k,    \
                     (const bf16*)v, (const float*)beta, (const float*)g, (bf16*)w, (bf16*)u, T, H, NT)
  if (sign < 0) THM_WY_LAUNCH(-1);
  else THM_WY_LAUNCH(1);
#undef THM_WY_LAUNCH
  return hipGetLastError();
}

}  // namespace
}  // namespace thm

extern "C" int thm_wy_fwd(const void* k, const void* v, const void* beta, const void* g, void* w,
                          void* u, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                          int32_t chunk_size, int32_t kv_dtype, int32_t sign, void* stream) {
  using namespace thm;
  if (chunk_size != kBT) return THM_ERR_BAD_ARGUMENT;
  if (sign != 1 && sign != -1) return THM_ERR_BAD_ARGUMENT;
  if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || T % kBT) return THM_ERR_BAD_SHAPE;
  if (kv_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;  // the fused path is bf16-only
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) return THM_ERR_UNSUPPORTED;
  if (B == 0 || T == 0) return THM_OK;  // empty: nothing is read or written
  if (!k || !v || !beta || !w || !u) return THM_ERR_NULL_POINTER;
  if (((uintptr_t)k % 16) || ((uintptr_t)v % 16)) return THM_ERR_MISALIGNED;
  if (((uintptr_t)w % 16) || ((uintptr_t)u % 16)) return THM_ERR_MISALIGNED;
  if (((uintptr_t)beta % 4) || (g && ((uintptr_t)g % 4))) return THM_ERR_MISALIGNED;
  if (B * (T / kBT) > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
  if (!launch_fits(B * (T / kBT) * H, kWyThreads)) return THM_ERR_BAD_SHAPE;
  // 32-bit per-lane offsets of the pipelined kernel's loads: 64 tokens x H heads.
  if (kBT * H * (K > V ? K : V) * 2 >= (INT64_C(1) << 32)) return THM_ERR_BAD_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (K == 64 && V == 64) e = launch_wy<64, 64>(k, v, beta, g, w, u, B, T, H, sign, s);
  else if (K == 64 && V == 128) e = launch_wy<64, 128>(k, v, beta, g, w, u, B, T, H, sign, s);
  else if (K == 128 && V == 64) e = launch_wy<128, 64>(k, v, beta, g, w, u, B, T, H, sign, s);
  else e = launch_wy<128, 128>(k, v, beta, g, w, u, B, T, H, sign, s);
  return (int)e;
}
