// Gated DeltaNet chunkwise output for MI355X (gfx950):
//   o_i = scale ( sum_{j<=i in chunk} (q_i . k_j) e^{g_i - g_j} v_j  +  e^{g_i} q_i . h[c] )
//
// Replaces kernels/chunk_fwd_o/kernel.py:52-136 (Triton) and its launcher
// kernel.py:146-212; math of reference.py:80-142, which uses the equivalent
// factored gates q e^{g}, v e^{-g}.  Here only e^{g_i - g_j} with j <= i is
// formed, which cannot overflow for a non-increasing gate.
//
// Three kernels: for bf16 inputs, the one-tile kernel below and, on grids
// of two or more tiles per persistent workgroup, a software-pipelined form;
// for fp32 inputs, chunk_fwd_o_f32_kernel (h read from memory, further below).
//
// One-tile kernel: one workgroup (4 wavefronts) per (b, chunk, head) tile,
// one memory phase: every global load of the tile (v_c, h[c], this wave's q
// rows and the k rows of its key blocks, g) is issued before the first wait.
// v_c [64 x V] and h[c] [K x V] are then staged in LDS as bf16.
// Wave wv owns query positions i = 16 wv .. 16 wv + 15 and computes o^T
// (features x positions), so each lane ends with 4 consecutive features of
// one token:
//   1. acc[n][i]  = sum_kappa h[kappa][n] q[i][kappa]          (h^T from LDS via
//      ds_read_b64_tr_b16, q fragments from registers), then acc *= e^{g_i};
//   2. S^T[j][i]  = sum_kappa k[j][kappa] q[i][kappa] for key blocks j <= i;
//      P[i][j] = S^T[j][i] e^{g_i - g_j} (0 for j > i), kept in registers;
//   3. acc[n][i] += sum_j v[j][n] P[i][j]: the P accumulator pairs are the B
//      operand in paired order, v^T comes from LDS in the same order;
//   4. o[i][n..n+3] = scale * acc.
#include <type_traits>

#include "h_layout.h"
#include "handout.h"
#include "mfma.h"
#include "vmem.h"

namespace thm {
namespace {

constexpr int kBT = 64;
constexpr int kOThreads = 256;

// LDS tiles of v [64 x V] and h [K x V] (bf16), rows padded by 32 bytes
// (h_layout.h tr_pitch): v fragments are read in the paired order, h in the
// natural order with its rows stored in the nat_row order; both are read
// without bank conflicts at constant offsets.  A 16-byte row pad left ~0.59
// conflict cycles per access.
template <int K, int V>
struct OCfg {
  static constexpr int kPitchB = hl::tr_pitch(V * 2);  // bytes per v / h row
  static constexpr int kVTile = kBT * kPitchB / 2;     // bf16 elements
  static constexpr int kHTile = K * kPitchB / 2;
  static constexpr int kLds = kVTile + kHTile;
  static constexpr int kVCPR = V / 8;                           // 16-byte chunks per v row
  static constexpr int kVLoads = kBT * kVCPR / kOThreads;
  static constexpr int kHLoads = K * (V / 4) / kOThreads;       // h is fp32
  static constexpr int KS = K / 32;                             // contraction steps over K
  static_assert(kBT * kVCPR % kOThreads == 0 && K * (V / 4) % kOThreads == 0, "staging split");
};

// h^T fragment for contraction step s (rows 32 s .. 32 s + 31, natural order)
// and output columns 16 nb .. + 15.
template <int P>
__device__ __forceinline__ bf16x8 h_frag(const char* tile, int s, int nb, int lane) {
  return concat(ds_read_tr16(reinterpret_cast<const bf16*>(tile + hl::ntr_frag_off(32 * s, 0, 16 * nb, lane, P))),
                ds_read_tr16(reinterpret_cast<const bf16*>(tile + hl::ntr_frag_off(32 * s, 1, 16 * nb, lane, P))));
}
// v^T fragment for key step s (rows 32 s .. 32 s + 31, paired order) and
// output columns 16 nb .. + 15.
template <int P>
__device__ __forceinline__ bf16x8 v_frag(const char* tile, int s, int nb, int lane) {
  return concat(ds_read_tr16(reinterpret_cast<const bf16*>(tile + hl::ptr_frag_off(32 * s, 16 * nb, lane, P))),
                ds_read_tr16(reinterpret_cast<const bf16*>(tile + hl::ptr_frag_off(32 * s + 16, 16 * nb, lane, P))));
}

template <int K, int V>
__global__ void __launch_bounds__(kOThreads)
chunk_fwd_o_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
                   const float* __restrict__ g, const float* __restrict__ hs, bf16* __restrict__ o,
                   float scale, int64_t T, int64_t H, int64_t NT) {
  using C = OCfg<K, V>;
  constexpr int KS = C::KS;
  __shared__ __attribute__((aligned(16))) bf16 lds[C::kLds];
  __shared__ float gs[kBT];
  char* const vhi = reinterpret_cast<char*>(lds);
  char* const hhi = reinterpret_cast<char*>(lds + C::kVTile);

  const int64_t tile = blockIdx.x;
  const TileCoord tc = tile_coord(tile, H, NT, T);
  const int64_t hh = tc.hh;
  const int64_t tok0 = tc.tok0;
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int i = 16 * wv + li;  // this lane's query position (column of every accumulator)
  const int64_t qrow = (tok0 + i) * H + hh;

  // 1. Issue every global load of the tile.
  u32x4 vr[C::kVLoads], hr[C::kHLoads];
#pragma unroll
  for (int it = 0; it < C::kVLoads; ++it) {
    const int qi = tid + it * kOThreads;
    const int j = qi / C::kVCPR;
    const int col = (qi - j * C::kVCPR) * 8;
    vr[it] = ldg16_nt(v + ((tok0 + j) * H + hh) * V + col);
  }
  const float* hsrc = hs + (int64_t)tile * (K * V);  // h[b, c, hh]: the state of this tile
#pragma unroll
  for (int it = 0; it < C::kHLoads; ++it) {
    const int qi = tid + it * kOThreads;
    const int r = qi / (V / 4);
    const int col = (qi - r * (V / 4)) * 4;
    hr[it] = ldg16_nt(hsrc + r * V + col);
  }
  // q fragments q[i][32 s + 8 grp + 0..7] and k fragments of key blocks jb <= wv.
  bf16x8 qh[KS], kf[4][KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qh[s] = __builtin_bit_cast(bf16x8, ldg16_nt(q + qrow * K + 32 * s + 8 * grp));
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    if (jb > wv) continue;  // wave-uniform
    const int64_t krow = (tok0 + 16 * jb + li) * H + hh;
#pragma unroll
    for (int s = 0; s < KS; ++s) kf[jb][s] = __builtin_bit_cast(bf16x8, ldg16_nt(k + krow * K + 32 * s + 8 * grp));
  }
  const float gload = (tid < kBT && g) ? g[(tok0 + tid) * H + hh] : 0.f;

  // 2. Stage v_c and h[c] (as bf16) and g.
#pragma unroll
  for (int it = 0; it < C::kVLoads; ++it) {
    const int qi = tid + it * kOThreads;
    const int j = qi / C::kVCPR;
    const int col = (qi - j * C::kVCPR) * 8;
    *reinterpret_cast<u32x4*>(vhi + hl::ptile_off(j, col, C::kPitchB)) = vr[it];
  }
#pragma unroll
  for (int it = 0; it < C::kHLoads; ++it) {
    const int qi = tid + it * kOThreads;
    const int r = qi / (V / 4);
    const int col = (qi - r * (V / 4)) * 4;
    float vals[4];
    unpack16(hr[it], vals, 0.f);
    lds_put4(reinterpret_cast<bf16*>(hhi + hl::ntile_off(r, col, C::kPitchB)), nullptr, vals, false);
  }
  if (tid < kBT) gs[tid] = gload;
  lds_barrier();

  // 3. Inter-chunk term, then scaled by e^{g_i}.
  constexpr int NB = V / 16;
  f32x4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    acc[nb] = zero4();
#pragma unroll
    for (int s = 0; s < KS; ++s) acc[nb] = mfma16x16x32(h_frag<C::kPitchB>(hhi, s, nb, lane), qh[s], acc[nb]);
  }
  const float gi = gs[i];
  const float egi = fast_exp(gi);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] *= egi;

  // 4. Gated, causally masked scores S^T[j][i] for key blocks jb <= wv.
  f32x4 p[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    p[jb] = zero4();
    if (jb > wv) continue;  // wave-uniform
#pragma unroll
    for (int s = 0; s < KS; ++s) p[jb] = mfma16x16x32(kf[jb][s], qh[s], p[jb]);
    // lane holds S^T[j = 16 jb + 4 grp + r][i]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * jb + 4 * grp + r;
      p[jb][r] = (j <= i) ? p[jb][r] * fast_exp(gi - gs[j]) : 0.f;
    }
  }

  // 5. Intra-chunk term: key steps of 32 (block pairs 2s, 2s+1), paired order.
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (2 * s > wv) continue;  // wave-uniform: both blocks fully masked
    const float f[8] = {p[2 * s][0], p[2 * s][1], p[2 * s][2], p[2 * s][3],
                        p[2 * s + 1][0], p[2 * s + 1][1], p[2 * s + 1][2], p[2 * s + 1][3]};
    const bf16x8 ph = to_bf16x8(f);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma16x16x32(v_frag<C::kPitchB>(vhi, s, nb, lane), ph, acc[nb]);
  }

  // 6. o[i][16 nb + 4 grp + 0..3], as 16-byte pieces of 8 consecutive
  // columns (vmem.h acc_pair_to_b128).
#pragma unroll
  for (int m = 0; m < NB / 2; ++m)
    *reinterpret_cast<u32x4*>(o + qrow * V + 32 * m + pair_col(grp)) =
        acc_pair_to_b128(acc[2 * m] * scale, acc[2 * m + 1] * scale);
}

// ---------------------------------------------------------------------------
// bf16 inputs on grids larger than the GPU: persistent, software-pipelined.
//
// With one tile per workgroup the loads of a tile are all in flight before
// its compute, but nothing loads while it computes; at 3 resident workgroups
// per CU that leaves HBM idle for a large part of each tile (the kernel with
// its MFMA work removed runs in 60 % of the time).  Here G = 2 workgroups per
// CU stay resident and take the tiles of a sequence (chunks in descending
// order) one after another: each issues the next tile's global loads into
// registers before computing the current tile from LDS, then stages them to
// LDS behind a barrier.  k is staged in LDS as well (its fragments are plain
// 16-byte row reads), which keeps the prefetched set to 28 16-byte loads per
// thread.  The arithmetic is the kernel above's.
//
// The tiles are handed out at run time (handout.h): workgroups on the XCDs
// that run slower (XCDs 1 and 5 on every box measured) take fewer tiles; the
// fixed walk t, t + G, ... waited for them (419.1-419.9 against 400.1-401.5
// us alone at config 4, interleaved, o bit-identical).
constexpr int kOPipeWGsPerCU = 2;

// The hand-out counters of this kernel (handout.h): slot s = {next ticket,
// workgroups finished}.
__device__ __align__(256) unsigned int g_o_tiles[kTileSlots][2];

// The host side of those slots (handout.h TileSlots): one table for every
// instantiation of the kernel, since they share g_o_tiles.
TileSlots& o_tile_slots() {
  static TileSlots slots;
  return slots;
}

template <int K, int V>
struct OPCfg {
  static constexpr int kPitchB = hl::tr_pitch(V * 2);    // bytes per v / h row (layouts as in OCfg)
  static constexpr int kKPitchB = hl::tr_pitch(K * 2);  // bytes per k row (16-byte row reads)
  static constexpr int kVTile = kBT * kPitchB / 2;       // bf16 elements
  static constexpr int kHTile = K * kPitchB / 2;
  static constexpr int kKTile = kBT * kKPitchB / 2;
  static constexpr int kVLoads = kBT * (V / 8) / kOThreads;  // 16-byte loads per thread
  static constexpr int kHLoads = K * (V / 4) / kOThreads;    // h is fp32
  static constexpr int kKLoads = kBT * (K / 8) / kOThreads;
  static constexpr int KS = K / 32;
  static_assert(kBT * (V / 8) % kOThreads == 0 && K * (V / 4) % kOThreads == 0 &&
                kBT * (K / 8) % kOThreads == 0, "staging split");
};

template <int K, int V>
__global__ void __launch_bounds__(kOThreads, 2)
chunk_fwd_o_pipe_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                        const bf16* __restrict__ v, const float* __restrict__ g,
                        const float* __restrict__ hs, bf16* __restrict__ o, float scale, int64_t T,
                        int64_t H, int64_t NT, int64_t tiles, uint32_t slot) {
  using C = OPCfg<K, V>;
  constexpr int KS = C::KS;
  constexpr int NB = V / 16;
  __shared__ __attribute__((aligned(16))) bf16 lv[C::kVTile];
  __shared__ __attribute__((aligned(16))) bf16 lh[C::kHTile];
  __shared__ __attribute__((aligned(16))) bf16 lk[C::kKTile];
  __shared__ float gs[kBT];

  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int i = 16 * wv + li;  // this lane's query position

  // Walk order (h_layout.h desc_walk_at): head fastest, chunks in descending
  // order.  This kernel takes the same time in either order, but the kernel
  // that runs after it does not: the next step's recompute_w_u (after the
  // conv or directly after this kernel, with its own or shared k and g)
  // takes 263-266 us instead of 271-278 at config 4, from the write-back of
  // this kernel's output overlapping it in a different address order.  The
  // walk index is decomposed once per tile, on wave-uniform values.
  const uint32_t Hu = (uint32_t)H, Bu = (uint32_t)(tiles / (NT * H)), ntiles = (uint32_t)tiles;
  TileHandout ho(g_o_tiles, slot);
  char* const lvb = reinterpret_cast<char*>(lv);
  char* const lhb = reinterpret_cast<char*>(lh);
  char* const lkb = reinterpret_cast<char*>(lk);

  // Per-lane byte offsets of the tile's loads (the entry point checks
  // 64 H max(K, V) 2 < 2^32), added to wave-uniform 64-bit bases.
  const uint32_t h_off = hl::o_h_lane(tid, V);
  const uint32_t v_off = hl::o_blk_lane(tid, V, H * V);
  const uint32_t k_off = hl::o_blk_lane(tid, K, H * K);
  const uint32_t q_off = hl::o_q_lane(i, grp, H * K);

  // Prefetched registers of one tile, and its coordinates.
  u32x4 vr[C::kVLoads], hr[C::kHLoads], kr[C::kKLoads], qr[KS];
  float gr = 0.f;
  int64_t nx_hh = 0, nx_tok0 = 0;
  auto prefetch = [&](uint32_t t) {  // the tile at walk index t
    const hl::DescWalk walk = hl::desc_walk_at(t, Bu, Hu);
    const int64_t c = (int64_t)NT - 1 - walk.cq;
    const int64_t hh = walk.hh, tile = ((int64_t)walk.b * NT + c) * H + hh;
    const int64_t tok0 = (int64_t)walk.b * T + c * 64;
    nx_hh = hh;
    nx_tok0 = tok0;
    const char* const hb = reinterpret_cast<const char*>(hs + tile * (int64_t)(K * V));
    const char* const vb = reinterpret_cast<const char*>(v + (tok0 * H + hh) * V);
    const char* const kb = reinterpret_cast<const char*>(k + (tok0 * H + hh) * K);
    const char* const qb = reinterpret_cast<const char*>(q + (tok0 * H + hh) * K);
    static_assert(kOThreads == 256, "h_layout.h o_* offsets assume 256 threads");
#pragma unroll
    for (int it = 0; it < C::kHLoads; ++it) hr[it] = ldg16_nt(hb + hl::o_h_step(it, V) + h_off);
#pragma unroll
    for (int it = 0; it < C::kVLoads; ++it) vr[it] = ldg16_nt(vb + hl::o_blk_step(it, V, H * V) + v_off);
#pragma unroll
    for (int it = 0; it < C::kKLoads; ++it) kr[it] = ldg16_nt(kb + hl::o_blk_step(it, K, H * K) + k_off);
#pragma unroll
    for (int s = 0; s < KS; ++s) qr[s] = ldg16_nt(qb + 64 * s + q_off);
    gr = (tid < kBT && g) ? g[(tok0 + tid) * H + hh] : 0.f;
  };
  auto stage = [&]() {
#pragma unroll
    for (int it = 0; it < C::kVLoads; ++it) {
      const int qi = tid + it * kOThreads;
      const int j = qi / (V / 8), col = (qi - j * (V / 8)) * 8;
      *reinterpret_cast<u32x4*>(lvb + hl::ptile_off(j, col, C::kPitchB)) = vr[it];
    }
#pragma unroll
    for (int it = 0; it < C::kHLoads; ++it) {
      const int qi = tid + it * kOThreads;
      const int r = qi / (V / 4), col = (qi - r * (V / 4)) * 4;
      float vals[4];
      unpack16(hr[it], vals, 0.f);
      lds_put4(reinterpret_cast<bf16*>(lhb + hl::ntile_off(r, col, C::kPitchB)), nullptr, vals, false);
    }
#pragma unroll
    for (int it = 0; it < C::kKLoads; ++it) {
      const int qi = tid + it * kOThreads;
      const int j = qi / (K / 8), col = (qi - j * (K / 8)) * 8;
      *reinterpret_cast<u32x4*>(lkb + hl::ptile_off(j, col, C::kKPitchB)) = kr[it];
    }
    if (tid < kBT) gs[tid] = gr;
  };

  __shared__ uint32_t s_next;
  uint32_t t = blockIdx.x;
  if (t >= ntiles) {  // whole workgroup
    ho.finish(tid);
    return;
  }
  ho.start(&s_next, tid);
  prefetch(t);
  stage();
  lds_barrier();
  uint32_t tn = __builtin_amdgcn_readfirstlane(s_next);  // the tile after t
  for (;;) {
    bf16x8 qh[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) qh[s] = __builtin_bit_cast(bf16x8, qr[s]);
    const int64_t hh = nx_hh, tok0 = nx_tok0;  // tile t
    if (tn < ntiles) prefetch(tn);  // in flight while tile t computes

    // Inter-chunk term, scaled by e^{g_i}.
    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      acc[nb] = zero4();
#pragma unroll
      for (int s = 0; s < KS; ++s) acc[nb] = mfma16x16x32(h_frag<C::kPitchB>(lhb, s, nb, lane), qh[s], acc[nb]);
    }
    const float gi = gs[i];
    const float egi = fast_exp(gi);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] *= egi;
    // Gated, causally masked scores S^T[j][i] for key blocks jb <= wv.
    f32x4 p[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      p[jb] = zero4();
      if (jb > wv) continue;  // wave-uniform
#pragma unroll
      for (int s = 0; s < KS; ++s)
        p[jb] = mfma16x16x32(load8(reinterpret_cast<const bf16*>(lkb + hl::prow8_frag_off(16 * jb, 32 * s, lane, C::kKPitchB))),
                             qh[s], p[jb]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * jb + 4 * grp + r;
        p[jb][r] = (j <= i) ? p[jb][r] * fast_exp(gi - gs[j]) : 0.f;
      }
    }
    // Intra-chunk term, paired order.
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (2 * s > wv) continue;  // wave-uniform: both blocks fully masked
      const float f[8] = {p[2 * s][0], p[2 * s][1], p[2 * s][2], p[2 * s][3],
                          p[2 * s + 1][0], p[2 * s + 1][1], p[2 * s + 1][2], p[2 * s + 1][3]};
      const bf16x8 ph = to_bf16x8(f);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma16x16x32(v_frag<C::kPitchB>(lvb, s, nb, lane), ph, acc[nb]);
    }
    const int64_t orow = (tok0 + i) * H + hh;
#pragma unroll
    for (int m = 0; m < NB / 2; ++m)
      *reinterpret_cast<u32x4*>(o + orow * V + 32 * m + pair_col(grp)) =
          acc_pair_to_b128(acc[2 * m] * scale, acc[2 * m + 1] * scale);

    if (tn >= ntiles) break;
    lds_barrier();  // every wave is done with tile t's LDS
    stage();
    ho.advance(&s_next, tid);  // every thread read s_next before the barrier above
    lds_barrier();
    t = tn;
    tn = __builtin_amdgcn_readfirstlane(s_next);
  }
  ho.finish(tid);
}

template <int K, int V>
hipError_t launch_o_pipe(const void* q, const void* k, const void* v, const void* g, const void* h,
                         void* o, float scale, int64_t B, int64_t T, int64_t H, int64_t grid,
                         hipStream_t s) {
  const int64_t NT = T / kBT;
  TileSlots& slots = o_tile_slots();
  const uint32_t slot = slots.acquire(s);
  hipLaunchKernelGGL((chunk_fwd_o_pipe_kernel<K, V>), dim3((unsigned)grid), dim3(kOThreads), 0, s,
                     (const bf16*)q, (const bf16*)k, (const bf16*)v, (const float*)g, (const float*)h,
                     (bf16*)o, scale, T, H, NT, B * NT * H, slot);
  const hipError_t e = hipGetLastError();
  slots.release(slot, s, e == hipSuccess);
  return e;
}

// ---------------------------------------------------------------------------
// fp32 inputs: the inter-chunk term with h read from memory.
//
// Staging h as bf16 hi + lo beside v took 104 KB of LDS (one workgroup per
// CU).  Here h is read straight from memory: the output columns are taken in
// column sets (q, c) holding features 64 q + 4 li + c, so one 16-byte load of
// h row kappa at columns 64 q + 4 li .. + 3 gives a lane its B-operand value
// in 4 sets (4 rows x 256 bytes per instruction; the tile's 4 waves share h
// through L2).  For kappa = 32 a + 8 grp + e, e = 0..7, a set's 8 values are
// split into bf16 hi + lo in registers and contracted with the q fragments
// on v_mfma_f32_16x16x32_bf16 (hi hi + lo hi + hi lo, as for every fp32
// product here).  Only v and k are staged (bf16 hi + lo, 70 KB at K = V =
// 128: two workgroups per CU); v's columns are stored in set order.  Both
// products are formed untransposed, D[i][n] (rows i = 16 wv + 4 grp + r):
// the intra-chunk term takes the score accumulator pairs as its A operand and
// the v^T fragments of a set as its B operand, so each lane ends with 4
// consecutive features of a row (one 16-byte store).
template <int K, int V>
struct OFCfg {
  static constexpr int kPitch = V + 8;   // v rows (bf16 elements, 16-byte pad)
  static constexpr int kKPitch = K + 8;  // k rows
  static constexpr int kVTile = kBT * kPitch;
  static constexpr int kKTile = kBT * kKPitch;
  static constexpr int kVLoads = kBT * (V / 4) / kOThreads;  // fp32 16-byte loads per thread
  static constexpr int kKLoads = kBT * (K / 4) / kOThreads;
  static constexpr int KS = K / 32;
  static_assert(kBT * (V / 4) % kOThreads == 0 && kBT * (K / 4) % kOThreads == 0, "staging split");
};

template <int K, int V>
__global__ void __launch_bounds__(kOThreads, 2)
chunk_fwd_o_f32_kernel(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                       const float* __restrict__ g, const float* __restrict__ hs, float* __restrict__ o,
                       float scale, int64_t T, int64_t H, int64_t NT) {
  using C = OFCfg<K, V>;
  constexpr int KS = C::KS, NQ = V / 64;
  __shared__ __attribute__((aligned(16))) bf16 lv[2 * C::kVTile];  // v hi, v lo
  __shared__ __attribute__((aligned(16))) bf16 lk[2 * C::kKTile];  // k hi, k lo
  __shared__ float gs[kBT];
  bf16* const vhi = lv;
  bf16* const vlo = lv + C::kVTile;
  bf16* const khi = lk;
  bf16* const klo = lk + C::kKTile;

  const TileCoord tc = tile_coord(blockIdx.x, H, NT, T);
  const int64_t hh = tc.hh;
  const int64_t tok0 = tc.tok0;
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int iq = 16 * wv + li;  // this lane's q row (A-operand row of both products)

  // 1. Every load of the tile but h: v and k (16-byte pieces), this lane's q
  // fragments q[iq][32 a + 8 grp + 0..7], g.
  u32x4 vr[C::kVLoads], kr[C::kKLoads];
#pragma unroll
  for (int it = 0; it < C::kVLoads; ++it) {
    const int qi = tid + it * kOThreads;
    const int j = qi / (V / 4), col = (qi - j * (V / 4)) * 4;
    vr[it] = ldg16_nt(v + ((tok0 + j) * H + hh) * V + col);
  }
#pragma unroll
  for (int it = 0; it < C::kKLoads; ++it) {
    const int qi = tid + it * kOThreads;
    const int j = qi / (K / 4), col = (qi - j * (K / 4)) * 4;
    kr[it] = ldg16_nt(k + ((tok0 + j) * H + hh) * K + col);
  }
  float qv[KS][8];
#pragma unroll
  for (int a = 0; a < KS; ++a) load8f(q + ((tok0 + iq) * H + hh) * K + 32 * a + 8 * grp, qv[a], true);
  const float gload = (tid < kBT && g) ? g[(tok0 + tid) * H + hh] : 0.f;

  // 2. Stage v and k as bf16 hi + lo, and g.
  // v columns are stored in the order of the output column sets: feature
  // n = 64 q + 4 m + c at position 64 q + 16 c + m, so the 16 consecutive
  // positions 64 q + 16 c + li hold the features 64 q + 4 li + c.
#pragma unroll
  for (int it = 0; it < C::kVLoads; ++it) {
    const int qi = tid + it * kOThreads;
    const int j = qi / (V / 4), m4 = qi - j * (V / 4);
    const int base = j * C::kPitch + 64 * (m4 >> 4) + (m4 & 15);
    float vals[4];
    unpack16(vr[it], vals, 0.f);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bf16 hi = (bf16)vals[c];
      vhi[base + 16 * c] = hi;
      vlo[base + 16 * c] = (bf16)(vals[c] - (float)hi);
    }
  }
#pragma unroll
  for (int it = 0; it < C::kKLoads; ++it) {
    const int qi = tid + it * kOThreads;
    const int j = qi / (K / 4), col = (qi - j * (K / 4)) * 4;
    float vals[4];
    unpack16(kr[it], vals, 0.f);
    lds_put4(khi + j * C::kKPitch + col, klo + j * C::kKPitch + col, vals, true);
  }
  if (tid < kBT) gs[tid] = gload;

  // 3. Inter-chunk term D[i][n] = sum_kappa q[i][kappa] h[kappa][n] (runs
  // while the staging stores drain; h is not in LDS): kappa = 32 a + 8 grp + e
  // in the q fragment's order.
  // Column set (q, c) holds features n = 64 q + 4 li + c: one 16-byte load per
  // row gives a lane its 4 column sets' values.
  const float* hb = hs + (int64_t)blockIdx.x * (K * V) + 4 * li;  // h[b, c, hh]: the state of this tile
  f32x4 acc[NQ][4];
#pragma unroll
  for (int q4 = 0; q4 < NQ; ++q4)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[q4][c] = zero4();
  bf16x8 qh[KS], ql[KS];
#pragma unroll
  for (int a = 0; a < KS; ++a) split_bf16x8(qv[a], qh[a], ql[a]);
#pragma unroll
  for (int a = 0; a < KS; ++a)
#pragma unroll
    for (int q4 = 0; q4 < NQ; ++q4) {
      float hv[8][4];
#pragma unroll
      for (int e = 0; e < 8; ++e) unpack16(ldg16(hb + (32 * a + 8 * grp + e) * V + 64 * q4), hv[e], 0.f);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float col[8] = {hv[0][c], hv[1][c], hv[2][c], hv[3][c], hv[4][c], hv[5][c], hv[6][c], hv[7][c]};
        bf16x8 hh, hl;
        split_bf16x8(col, hh, hl);
        acc[q4][c] = mfma16x16x32(qh[a], hh, acc[q4][c]);
        acc[q4][c] = mfma16x16x32(ql[a], hh, acc[q4][c]);
        acc[q4][c] = mfma16x16x32(qh[a], hl, acc[q4][c]);
      }
    }
  lds_barrier();
  // acc[nb][r] holds row i = 16 wv + 4 grp + r: scale it by e^{g_i}.
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float egi = fast_exp(gs[16 * wv + 4 * grp + r]);
#pragma unroll
    for (int q4 = 0; q4 < NQ; ++q4)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[q4][c][r] *= egi;
  }

  // 4. Gated, causally masked scores S^T[j][iq] for key blocks jb <= wv (as
  // the kernel above, with k from LDS).
  const float gq = gs[iq];
  f32x4 p[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    p[jb] = zero4();
    if (jb > wv) continue;  // wave-uniform
#pragma unroll
    for (int a = 0; a < KS; ++a) {
      const int off = (16 * jb + li) * C::kKPitch + 32 * a + 8 * grp;
      const bf16x8 kh = load8(khi + off), kl = load8(klo + off);
      p[jb] = mfma16x16x32(kh, qh[a], p[jb]);
      p[jb] = mfma16x16x32(kh, ql[a], p[jb]);
      p[jb] = mfma16x16x32(kl, qh[a], p[jb]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * jb + 4 * grp + r;
      p[jb][r] = (j <= iq) ? p[jb][r] * fast_exp(gq - gs[j]) : 0.f;
    }
  }

  // 5. Intra-chunk term D[i][n] += sum_j P[i][j] v[j][n]: A = the score
  // accumulator pairs (paired order over j), B = v^T fragments in the same order.
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    if (2 * s2 > wv) continue;  // wave-uniform: both key blocks fully masked
    const float f[8] = {p[2 * s2][0], p[2 * s2][1], p[2 * s2][2], p[2 * s2][3],
                        p[2 * s2 + 1][0], p[2 * s2 + 1][1], p[2 * s2 + 1][2], p[2 * s2 + 1][3]};
    bf16x8 ph, pl;
    split_bf16x8(f, ph, pl);
    const int r0 = tr_row_paired(32 * s2, 0), r1 = tr_row_paired(32 * s2, 1);
#pragma unroll
    for (int q4 = 0; q4 < NQ; ++q4)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const bf16x8 vh = frag_tr(vhi, C::kPitch, r0, r1, 64 * q4 + 16 * c);
        const bf16x8 vl = frag_tr(vlo, C::kPitch, r0, r1, 64 * q4 + 16 * c);
        acc[q4][c] = mfma16x16x32(ph, vh, acc[q4][c]);
        acc[q4][c] = mfma16x16x32(pl, vh, acc[q4][c]);
        acc[q4][c] = mfma16x16x32(ph, vl, acc[q4][c]);
      }
  }

  // 6. o[i][64 q + 4 li .. + 3] for i = 16 wv + 4 grp + r: one 16-byte store
  // per lane, 16 lanes cover 256 contiguous bytes of a row.
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float* orow = o + ((tok0 + 16 * wv + 4 * grp + r) * H + hh) * V + 4 * li;
#pragma unroll
    for (int q4 = 0; q4 < NQ; ++q4)
      store4(orow + 64 * q4, f32x4{acc[q4][0][r], acc[q4][1][r], acc[q4][2][r], acc[q4][3][r]} * scale);
  }
}

template <int K, int V>
hipError_t launch_o_f32(const void* q, const void* k, const void* v, const void* g, const void* h, void* o,
                        float scale, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / kBT;
  hipLaunchKernelGGL((chunk_fwd_o_f32_kernel<K, V>), dim3((unsigned)(B * NT * H)), dim3(kOThreads), 0, s,
                     (const float*)q, (const float*)k, (const float*)v, (const float*)g, (const float*)h,
                     (float*)o, scale, T, H, NT);
  return hipGetLastError();
}

template <int K, int V>
hipError_t launch_o(const void* q, const void* k, const void* v, const void* g, const void* h,
                    void* o, float scale, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / kBT;
  hipLaunchKernelGGL((chunk_fwd_o_kernel<K, V>), dim3((unsigned)(B * NT * H)), dim3(kOThreads),
                     0, s, (const bf16*)q, (const bf16*)k, (const bf16*)v, (const float*)g,
                     (const float*)h, (bf16*)o, scale, T, H, NT);
  return hipGetLastError();
}

template <typename IT>
hipError_t dispatch_o(int64_t K, int64_t V, const void* q, const void* k, const void* v,
                      const void* g, const void* h, void* o, float scale, int64_t B, int64_t T,
                      int64_t H, hipStream_t s) {
  if constexpr (std::is_same<IT, float>::value) {
    if (K == 64 && V == 64) return launch_o_f32<64, 64>(q, k, v, g, h, o, scale, B, T, H, s);
    if (K == 64 && V == 128) return launch_o_f32<64, 128>(q, k, v, g, h, o, scale, B, T, H, s);
    if (K == 128 && V == 64) return launch_o_f32<128, 64>(q, k, v, g, h, o, scale, B, T, H, s);
    return launch_o_f32<128, 128>(q, k, v, g, h, o, scale, B, T, H, s);
  } else {
    const int64_t tiles = B * (T / kBT) * H;
    const int64_t grid = (int64_t)device_cu_count() * kOPipeWGsPerCU;
    if (grid > 0 && tiles >= 2 * grid) {
      if (K == 64 && V == 64) return launch_o_pipe<64, 64>(q, k, v, g, h, o, scale, B, T, H, grid, s);
      if (K == 64 && V == 128) return launch_o_pipe<64, 128>(q, k, v, g, h, o, scale, B, T, H, grid, s);
      if (K == 128 && V == 64) return launch_o_pipe<128, 64>(q, k, v, g, h, o, scale, B, T, H, grid, s);
      return launch_o_pipe<128, 128>(q, k, v, g, h, o, scale, B, T, H, grid, s);
    }
    if (K == 64 && V == 64) return launch_o<64, 64>(q, k, v, g, h, o, scale, B, T, H, s);
    if (K == 64 && V == 128) return launch_o<64, 128>(q, k, v, g, h, o, scale, B, T, H, s);
    if (K == 128 && V == 64) return launch_o<128, 64>(q, k, v, g, h, o, scale, B, T, H, s);
    return launch_o<128, 128>(q, k, v, g, h, o, scale, B, T, H, s);
  }
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
  if (!launch_fits(B * (T / kBT) * H, kOThreads)) return THM_ERR_BAD_SHAPE;
  // 32-bit per-lane offsets of the pipelined kernel: 64 tokens x H heads.
  if (kBT * H * (K > V ? K : V) * 2 >= (INT64_C(1) << 32)) return THM_ERR_BAD_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = (qkv_dtype == THM_DTYPE_F32)
                     ? dispatch_o<float>(K, V, q, k, v, g, h, o, scale, B, T, H, s)
                     : dispatch_o<bf16>(K, V, q, k, v, g, h, o, scale, B, T, H, s);
  return (int)e;
}
