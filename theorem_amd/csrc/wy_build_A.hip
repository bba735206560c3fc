// WY matrix of the Gated DeltaNet chunk forward for MI355X (gfx950):
//   per chunk c of 64 tokens:  M[i][j] = beta_i (k_i . k_j) e^{g_i - g_j}  (j < i),
//                              A_c = (I + sign M)^{-1}
// sign = -1 is the reference's (I - M)^{-1} (kernels/recompute_w_u/reference.py:48-91,
// `_build_A`, a torch matmul + solve_triangular); sign = +1 is the gated delta
// rule's (I + M)^{-1}.  A [B, T, H, 64] fp32 holds row r of A_c at token c*64 + r.
//
// One workgroup (4 wavefronts) per (b, chunk, head) tile, head fastest.  With
// L = sign M (strictly lower) and 16x16 blocks L_ij, X = (I + L)^{-1} is block
// lower triangular:
//   X_ii = (I + L_ii)^{-1}                        (forward substitution)
//   X_ij = -X_ii sum_{m=j}^{i-1} L_im X_mj        (i > j, by distance i - j)
//   1. k k^T on v_mfma_f32_16x16x32_bf16: lane (g, j) holds features
//      8g .. 8g+7 of token j of a 16-token block, so the A fragment of block ib
//      and the B fragment of block jb are the same kind of 16-byte row load
//      (fp32 k: bf16 hi + lo, three products).  The 10 lower blocks are spread
//      over the 4 waves; every wave loads the tile's k (the repeats hit L2).
//   2. L blocks (scaled by beta_i e^{g_i - g_j}, strict lower part) go to LDS.
//   3. Wave w inverts the diagonal block w: lane c (< 16) owns column c and runs
//      the 16-row substitution.
//   4. The 6 off-diagonal blocks, 3 levels of independent blocks (3, 2, 1
//      waves), each two fp32 MFMA products (v_mfma_f32_16x16x4_f32, exact fp32
//      multiplies): T = sum L_im X_mj, then X_ij = -X_ii T, T passing through
//      LDS to change from the accumulator to the operand layout.
//   5. All 256 threads write A_c: 16-byte stores, 4 full 256-byte rows per
//      wavefront instruction.
// HBM traffic per tile: k, beta, g read once, A written once.
#include <type_traits>

#include "h_layout.h"
#include "wy_blocks.h"

namespace thm {
namespace {

using wy::blk;
using wy::kBlk;
using wy::kBP;
constexpr int kBT = wy::kBT;
constexpr int kABThreads = 256;

// A_c rows of the inverted blocks Xb: thread (r = q / 16, chunk j4 = q % 16)
// writes A[r][4 j4 .. + 3]; 16-byte stores, 4 full 256-byte rows per
// wavefront instruction.
__device__ __forceinline__ void store_A(const float* Xb, float* out, int64_t H) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < kBT * 16 / kABThreads; ++it) {
    const int q = tid + it * kABThreads;
    const int r = q >> 4, j0 = (q & 15) * 4;
    const int ib = r >> 4, jb = j0 >> 4;
    f32x4 v = zero4();
    if (jb <= ib) {
      const float* X = Xb + blk(ib, jb) * kBlk + (r & 15) * kBP + (j0 & 15);
      v[0] = X[0]; v[1] = X[1]; v[2] = X[2]; v[3] = X[3];
    }
    *reinterpret_cast<f32x4*>(out + (int64_t)r * H * kBT + j0) = v;
  }
}

template <typename IT, int K, int SIGN>
__global__ void __launch_bounds__(kABThreads)
wy_build_A_kernel(const IT* __restrict__ k, const float* __restrict__ beta,
                  const float* __restrict__ g, float* __restrict__ A, int64_t T, int64_t H,
                  int64_t NT) {
  constexpr bool kSplit = std::is_same<IT, float>::value;
  constexpr int KS = K / 32;  // contraction steps
  __shared__ float Lb[10 * kBlk];  // L = sign M, lower blocks (diagonal blocks: strict lower part)
  __shared__ float Xb[10 * kBlk];  // X = A_c, lower blocks
  __shared__ float Tb[3 * kBlk];   // per-level partial products
  __shared__ float sb[kBT], sg[kBT];

  const TileCoord tc = tile_coord(blockIdx.x, H, NT, T);
  const int64_t h = tc.hh;
  const int64_t tok0 = tc.tok0;
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int lane = tid & 63;
  const int grp = lane >> 4, li = lane & 15;

  // 1. k fragments: fh[tb][s] = k[tok0 + 16 tb + li][32 s + 8 grp .. + 7].
  bf16x8 fh[4][KS], fl[4][kSplit ? KS : 1];
  {
    float v[8];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const IT* row = k + ((tok0 + 16 * tb + li) * H + h) * K + 8 * grp;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        if constexpr (kSplit) {
          load8f(row + 32 * s, v);
          split_bf16x8(v, fh[tb][s], fl[tb][s]);
        } else {
          fh[tb][s] = load8(row + 32 * s);
        }
      }
    }
  }
  if (tid < kBT) {
    sb[tid] = beta[(tok0 + tid) * H + h];
    sg[tid] = g ? g[(tok0 + tid) * H + h] : 0.f;
  }
  lds_barrier();

  // 2. L blocks; 3.-4. X = (I + L)^{-1}.
  wy::form_L<SIGN, KS, kSplit>(fh, fl, sb, sg, Lb, wv);
  lds_barrier();
  wy::invert_L(Lb, Xb, Tb, wv);

  // 5. A_c rows.
  store_A(Xb, A + (tok0 * H + h) * kBT, H);
}

// ---------------------------------------------------------------------------
// bf16 k on grids of at least two tiles per persistent workgroup:
// software-pipelined, as the fused WY kernel (wy_fwd.hip).  Workgroups walk
// the tiles t, t + G, ... and issue the next tile's k rows (16-byte row-major
// loads), beta and g into registers before computing the current tile, so the
// loads are in flight through form_L and the inversion; the k tile is staged
// in LDS and the MFMA fragments are read from there.  The arithmetic is the
// one-tile kernel's, so A is bit-identical.
// Workgroups per CU: 4.  The inversion's latency chain, not memory, sets this
// kernel's time (timing-only copies at config 4: 105.4 us; without the
// inversion 26.6, without the next tile's loads 99.5, without the stores of
// A 95.2), so the more tiles a CU inverts at once the better:
//   * the k loads go through one 32-bit per-lane offset on a wave-uniform
//     base (h_layout.h o_blk_lane / o_blk_step; 64-bit addresses spilled at
//     3 workgroups): 2 -> 3 per CU, 140 -> 116 us;
//   * the X and T blocks share the k tile's LDS (31.7 KB per workgroup
//     instead of 48.6) and form_L reads its k fragments per block
//     (wy::form_L_lds; 120 VGPRs at K = 128, no scratch): 3 -> 4 per CU,
//     105.7 -> 96.3 us.  5 per CU spill (140 us).
// A is bit-identical throughout.
template <int K>
constexpr int ab_pipe_wgs_per_cu() { return 4; }

template <int K, int SIGN>
__global__ void __launch_bounds__(kABThreads, ab_pipe_wgs_per_cu<K>())
wy_build_A_pipe_kernel(const bf16* __restrict__ k, const float* __restrict__ beta,
                       const float* __restrict__ g, float* __restrict__ A, int64_t T, int64_t H,
                       int64_t NT, int64_t tiles) {
  constexpr int KS = K / 32;
  // bf16 elements per k row: a 32-byte pad (h_layout.h tr_pitch), under which
  // the 16-byte fragment reads of 16 rows are conflict-free on gfx950.
  constexpr int kPitch = hl::tr_pitch(2 * K) / 2;
  constexpr int kCPR = K / 8;                         // 16-byte chunks per k row
  constexpr int kLoads = kBT * kCPR / kABThreads;     // per thread
  static_assert(kBT * kCPR % kABThreads == 0, "staging split");
  // The k tile is read only up to the barrier after form_L and restaged
  // after the barrier that follows the store of A, so the inversion's X and T
  // blocks share its LDS.
  constexpr int kKBytes = kBT * kPitch * 2, kXTBytes = 13 * kBlk * 4;
  __shared__ __attribute__((aligned(16))) char kxt[kKBytes > kXTBytes ? kKBytes : kXTBytes];
  bf16* const ks = reinterpret_cast<bf16*>(kxt);
  float* const Xb = reinterpret_cast<float*>(kxt);
  float* const Tb = Xb + 10 * kBlk;
  __shared__ float Lb[10 * kBlk];
  __shared__ float sb[kBT], sg[kBT];

  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int lane = tid & 63;
  const int grp = lane >> 4, li = lane & 15;

  // XCD-aware walk (h_layout.h xcd_tile_order, a bijection of the tiles;
  // with a grid that is a multiple of 8, 1024 on MI355X, sequence index t runs
  // on XCD t % 8): the 16 heads of a (b, chunk) share
  // one XCD's L2, so each 64-byte line of beta and g is fetched once, not once
  // per XCD.  Measured traffic 1.108 -> 1.00 of the algorithmic bytes, at
  // +1.4 % time (115.2 -> 116.8 us at config 4, A bit-identical).
  const int64_t BNT = tiles / H;
  auto tok_of = [&](int64_t tile, int64_t& h) {
    const TileCoord tc = tile_coord(hl::xcd_tile_order((uint32_t)tile, H, BNT), H, NT, T);
    h = tc.hh;
    return tc.tok0;
  };
  u32x4 kr[kLoads];
  float br = 0.f, gr = 0.f;
  const uint32_t k_off = hl::o_blk_lane(tid, K, H * K);
  auto prefetch = [&](int64_t tile) {
    int64_t h;
    const int64_t tok0 = tok_of(tile, h);
    const char* const kb = reinterpret_cast<const char*>(k + (tok0 * H + h) * K);
#pragma unroll
    for (int it = 0; it < kLoads; ++it) kr[it] = ldg16_nt(kb + hl::o_blk_step(it, K, H * K) + k_off);
    if (tid < kBT) {
      const int64_t row = (tok0 + tid) * H + h;
      br = beta[row];
      gr = g ? g[row] : 0.f;
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int it = 0; it < kLoads; ++it) {
      const int q = tid + it * kABThreads;
      const int j = q / kCPR, col = (q - j * kCPR) * 8;
      *reinterpret_cast<u32x4*>(ks + j * kPitch + col) = kr[it];
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
    wy::form_L_lds<SIGN, KS>([&](int tb, int s) { return load8(ks + (16 * tb + li) * kPitch + 32 * s + 8 * grp); },
                             sb, sg, Lb, wv);
    lds_barrier();  // every wave's k fragment reads are done: X may overwrite ks
    wy::invert_L(Lb, Xb, Tb, wv);  // ends with a barrier
    store_A(Xb, A + (tok0 * H + h) * kBT, H);

    if (tn >= tiles) break;
    lds_barrier();  // every wave is done with tile t's LDS
    stage();
    lds_barrier();
    t = tn;
  }
}

template <typename IT, int K>
hipError_t launch_A(const void* k, const void* beta, const void* g, void* A, int64_t B, int64_t T,
                    int64_t H, int sign, hipStream_t s) {
  const int64_t NT = T / kBT;
  const int64_t tiles = B * NT * H;
  if constexpr (std::is_same<IT, bf16>::value) {
    const int64_t pgrid = (int64_t)device_cu_count() * ab_pipe_wgs_per_cu<K>();
    if (pgrid > 0 && tiles >= 2 * pgrid) {
      if (sign < 0)
        hipLaunchKernelGGL((wy_build_A_pipe_kernel<K, -1>), dim3((unsigned)pgrid), dim3(kABThreads), 0, s,
                           (const bf16*)k, (const float*)beta, (const float*)g, (float*)A, T, H, NT, tiles);
      else
        hipLaunchKernelGGL((wy_build_A_pipe_kernel<K, 1>), dim3((unsigned)pgrid), dim3(kABThreads), 0, s,
                           (const bf16*)k, (const float*)beta, (const float*)g, (float*)A, T, H, NT, tiles);
      return hipGetLastError();
    }
  }
  const dim3 grid((unsigned)tiles);
  if (sign < 0)
    hipLaunchKernelGGL((wy_build_A_kernel<IT, K, -1>), grid, dim3(kABThreads), 0, s, (const IT*)k,
                       (const float*)beta, (const float*)g, (float*)A, T, H, NT);
  else
    hipLaunchKernelGGL((wy_build_A_kernel<IT, K, 1>), grid, dim3(kABThreads), 0, s, (const IT*)k,
                       (const float*)beta, (const float*)g, (float*)A, T, H, NT);
  return hipGetLastError();
}

}  // namespace
}  // namespace thm

extern "C" int thm_wy_build_A(const void* k, const void* beta, const void* g, void* A, int64_t B,
                              int64_t T, int64_t H, int64_t K, int32_t chunk_size,
                              int32_t k_dtype, int32_t sign, void* stream) {
  using namespace thm;
  if (chunk_size != kBT) return THM_ERR_BAD_ARGUMENT;
  if (sign != 1 && sign != -1) return THM_ERR_BAD_ARGUMENT;
  if (B < 0 || T < 0 || H <= 0 || K <= 0 || T % kBT) return THM_ERR_BAD_SHAPE;
  if (k_dtype != THM_DTYPE_F32 && k_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if (K != 64 && K != 128) return THM_ERR_UNSUPPORTED;
  if (B == 0 || T == 0) return THM_OK;  // empty: nothing is read or written
  if (!k || !beta || !A) return THM_ERR_NULL_POINTER;
  if (((uintptr_t)k % 16) || ((uintptr_t)A % 16)) return THM_ERR_MISALIGNED;
  if (((uintptr_t)beta % 4) || (g && ((uintptr_t)g % 4))) return THM_ERR_MISALIGNED;
  if (B * (T / kBT) > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
  if (!launch_fits(B * (T / kBT) * H, kABThreads)) return THM_ERR_BAD_SHAPE;
  // 32-bit per-lane offsets of the pipelined kernel's k loads: 64 tokens x H heads.
  if (kBT * H * K * 2 >= (INT64_C(1) << 32)) return THM_ERR_BAD_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (k_dtype == THM_DTYPE_F32)
    e = (K == 64) ? launch_A<float, 64>(k, beta, g, A, B, T, H, sign, s)
                  : launch_A<float, 128>(k, beta, g, A, B, T, H, sign, s);
  else
    e = (K == 64) ? launch_A<bf16, 64>(k, beta, g, A, B, T, H, sign, s)
                  : launch_A<bf16, 128>(k, beta, g, A, B, T, H, sign, s);
  return (int)e;
}
