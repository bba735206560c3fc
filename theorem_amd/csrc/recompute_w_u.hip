// Gated DeltaNet WY recompute for MI355X (gfx950):
//   per chunk c of 64 tokens:  w_c = A_c (k_c * beta_c e^{g_c}),  u_c = A_c (v_c * beta_c)
//
// Replaces kernels/recompute_w_u/kernel.py:73-186 (Triton) and its launcher
// kernel.py:192-248; math of reference.py:118-149.
//
// One workgroup per (b, chunk, HP adjacent heads) tile, 4 wavefronts per head
// (HP = 2 for bf16 with an even head count, else 1), one memory phase:
//   1. Every global load of the tile is issued at once: the 64 x (K+V) tile
//      X = [k | v] of each head (16-byte loads into registers; a token's k of
//      the HP heads is one contiguous run, as is its v), this wave's 16 rows
//      of A_c (fp32), and beta / g.
//   2. X goes to LDS unchanged for bf16 inputs (fp32 inputs: bf16 hi + lo);
//      beta, g go to LDS; one barrier.
//   3. The per-token scales are folded into A instead of X:
//        w = (A diag(beta e^g)) k,   u = (A diag(beta)) v,
//      each scaled A operand split into bf16 hi + lo (so A, beta and e^g enter
//      at ~fp32 accuracy and bf16 k / v enter exactly).
//   4. Wave wv owns positions t = 16 wv .. 16 wv + 15 and computes the
//      transposed product D[n][t] = sum_j X[j][n] A'[t][j] with
//      v_mfma_f32_16x16x32_bf16; X^T is read from LDS with ds_read_b64_tr_b16.
//      Each lane ends with 4 consecutive features of one token.
//   5. w and u go through LDS (the X tiles' space) and out as 16-byte
//      stores of consecutive token rows.
// HBM traffic per tile = k, v, A, beta, g read once + w, u written once.
#include <type_traits>

#include "h_layout.h"
#include "mfma.h"

namespace thm {
namespace {

constexpr int kBT = 64;
constexpr int kWuThreads = 256;  // per head of a tile

// A tile is (b, chunk, HP adjacent heads): 4 HP waves, 4 per head.  HP = 2
// (bf16, even H) reads each token row of k and v as one contiguous run of
// 2 heads (512 bytes at K = V = 128) instead of one 256-byte run per head.
template <typename IT, int K, int V, int HP>
struct WuCfg {
  static constexpr bool kSplitX = std::is_same<IT, float>::value;
  static constexpr int kN = K + V;
  static constexpr int kThreads = kWuThreads * HP;
  static constexpr int kRowB = kN * 2;    // LDS row bytes of one bf16 tile (unpadded, h_layout.h xtile_off)
  static constexpr int kTile = kBT * kN;  // bf16 elements per head
  static constexpr int kNB = kN / 16;
  static constexpr int kVE = 16 / (int)sizeof(IT);  // elements per 16-byte load
  // k (then v) pieces: a token row of the tile's HP heads is HP K / kVE
  // 16-byte pieces; thread tid takes pieces tid, tid + kThreads, ...
  static constexpr int kKLoads = kBT * HP * (K / kVE) / kThreads;
  static constexpr int kVLoads = kBT * HP * (V / kVE) / kThreads;
  static_assert(kBT * HP * (K / kVE) % kThreads == 0 && kBT * HP * (V / kVE) % kThreads == 0,
                "staging must divide evenly");
};

template <typename IT, int K, int V, int HP>
__global__ void __launch_bounds__(kWuThreads * HP)
recompute_w_u_kernel(const IT* __restrict__ k, const IT* __restrict__ v,
                     const float* __restrict__ beta, const float* __restrict__ A,
                     const float* __restrict__ g, IT* __restrict__ w, IT* __restrict__ u,
                     int64_t T, int64_t H, int64_t NT) {
  using C = WuCfg<IT, K, V, HP>;
  __shared__ __attribute__((aligned(16))) bf16 xs[HP][(C::kSplitX ? 2 : 1) * C::kTile];
  __shared__ float sbeta[HP][kBT], sg[HP][kBT];

  // tile -> (b, c, head group), head groups fastest within an XCD: the
  // workgroups of one XCD read one contiguous [64 tokens x H x D] block, and
  // beta / g lines once.
  const int64_t HG = H / HP;
  const TileCoord tc = tile_coord(hl::xcd_tile_order(blockIdx.x, HG, (int64_t)gridDim.x / HG), HG, NT, T);
  const int64_t h0 = tc.hh * HP;  // first head of the tile
  const int64_t tok0 = tc.tok0;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int hs = wave >> 2;  // this wave's head within the tile
  const int wv = wave & 3;   // its 16 positions t = 16 wv ..
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int li = lane & 15;

  // 1. Issue every load: the tile's k rows, then its v rows (HP heads
  // contiguous per token), this wave's 16 rows of A, beta and g.
  // Non-temporal k and v: read once (measured 2% faster at config 4 than
  // cached loads; the A rows stay cached loads, which measured faster).
  u32x4 kr[C::kKLoads], vr[C::kVLoads];
#pragma unroll
  for (int it = 0; it < C::kKLoads; ++it) {
    const int q = tid + it * C::kThreads;
    const int j = q / (HP * K / C::kVE), c = q - j * (HP * K / C::kVE);
    kr[it] = ldg16_nt(k + ((tok0 + j) * H + h0) * K + c * C::kVE);
  }
#pragma unroll
  for (int it = 0; it < C::kVLoads; ++it) {
    const int q = tid + it * C::kThreads;
    const int j = q / (HP * V / C::kVE), c = q - j * (HP * V / C::kVE);
    vr[it] = ldg16_nt(v + ((tok0 + j) * H + h0) * V + c * C::kVE);
  }
  const float* arow = A + ((tok0 + 16 * wv + li) * H + h0 + hs) * kBT;
  float av[2][8];
#pragma unroll
  for (int s = 0; s < 2; ++s) load8f(arow + 32 * s + 8 * grp, av[s], false);
  float bj = 0.f, gj = 0.f;
  if (tid < kBT * HP) {  // token tid / HP, head tid % HP: HP adjacent values per token
    const int64_t row = (tok0 + tid / HP) * H + h0 + tid % HP;
    bj = beta[row];
    gj = g ? g[row] : 0.f;
  }

  // 2. Stage X = [k | v] per head, beta, g.  X rows are unpadded with the
  // chunk-pair swizzle of xtile_off: the fragment reads below are then free
  // of bank conflicts (a 16-byte row pad left ~0.56 conflict cycles per access).
  auto put = [&](u32x4 val, int hsub, int j, int col) {
    char* const xhb = reinterpret_cast<char*>(xs[hsub]);
    const uint32_t off = hl::xtile_off(j, col, C::kRowB);
    if constexpr (C::kSplitX) {
      float vals[4];
      unpack16(val, vals, 0.f);
      lds_put4(reinterpret_cast<bf16*>(xhb + off), reinterpret_cast<bf16*>(xhb + 2 * C::kTile + off), vals, true);
    } else {
      *reinterpret_cast<u32x4*>(xhb + off) = val;
    }
  };
#pragma unroll
  for (int it = 0; it < C::kKLoads; ++it) {
    const int q = tid + it * C::kThreads;
    const int j = q / (HP * K / C::kVE), c = q - j * (HP * K / C::kVE);
    put(kr[it], c / (K / C::kVE), j, (c % (K / C::kVE)) * C::kVE);
  }
#pragma unroll
  for (int it = 0; it < C::kVLoads; ++it) {
    const int q = tid + it * C::kThreads;
    const int j = q / (HP * V / C::kVE), c = q - j * (HP * V / C::kVE);
    put(vr[it], c / (V / C::kVE), j, K + (c % (V / C::kVE)) * C::kVE);
  }
  if (tid < kBT * HP) {
    sbeta[tid % HP][tid / HP] = bj;
    sg[tid % HP][tid / HP] = gj;
  }
  lds_barrier();

  // 3. Scaled A operands: A'[t][j] for j = 32 s + 8 grp + 0..7.
  bf16x8 awh[2], awl[2], auh[2], aul[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float fw[8], fu[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 32 * s + 8 * grp + i;
      const float bb = sbeta[hs][j];
      fu[i] = av[s][i] * bb;
      fw[i] = fu[i] * fast_exp(sg[hs][j]);
    }
    split_bf16x8(fw, awh[s], awl[s]);
    split_bf16x8(fu, auh[s], aul[s]);
  }

  // 4. D[n][t] = sum_j X[j][n] A'[t][j].
  const char* const xhb = reinterpret_cast<const char*>(xs[hs]);
  const char* const xlb = xhb + 2 * C::kTile;
  f32x4 acc[C::kNB];
#pragma unroll
  for (int nb = 0; nb < C::kNB; ++nb) {
    const bool is_w = 16 * nb < K;
    acc[nb] = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t o0 = hl::xtr_frag_off(32 * s, 0, 16 * nb, lane, C::kRowB);
      const uint32_t o1 = hl::xtr_frag_off(32 * s, 1, 16 * nb, lane, C::kRowB);
      const bf16x8 xh = concat(ds_read_tr16(reinterpret_cast<const bf16*>(xhb + o0)),
                               ds_read_tr16(reinterpret_cast<const bf16*>(xhb + o1)));
      acc[nb] = mfma16x16x32(xh, is_w ? awh[s] : auh[s], acc[nb]);
      acc[nb] = mfma16x16x32(xh, is_w ? awl[s] : aul[s], acc[nb]);
      if constexpr (C::kSplitX) {
        const bf16x8 xl = concat(ds_read_tr16(reinterpret_cast<const bf16*>(xlb + o0)),
                                 ds_read_tr16(reinterpret_cast<const bf16*>(xlb + o1)));
        acc[nb] = mfma16x16x32(xl, is_w ? awh[s] : auh[s], acc[nb]);
      }
    }
  }

  // 5. Stage w and u through LDS (the X tiles' space, once every wave is done
  // with them) so that the global stores are whole 16-byte pieces of
  // consecutive token rows, the HP heads of a token contiguous: 64 HP rows of
  // K (V) features per tile, in global order (h_layout.h otile_off; bf16
  // pieces with the half swap that keeps the 8-byte writes conflict-free).
  // Stores of 4 features per lane straight from the accumulators touch 16
  // rows per instruction (249 against 226 us for the same bytes stored
  // contiguously, config 4).
  constexpr bool kHalf = !C::kSplitX;  // 8-byte (bf16) pieces
  char* const owb = reinterpret_cast<char*>(&xs[0][0]);  // w rows
  constexpr int kWRow = K * (int)sizeof(IT), kURow = V * (int)sizeof(IT);
  char* const oub = owb + HP * kBT * kWRow;  // u rows
  lds_barrier();  // every wave is done reading X
  const int t = 16 * wv + li;
#pragma unroll
  for (int nb = 0; nb < C::kNB; ++nb) {
    const int n = 16 * nb + 4 * grp;
    if (16 * nb < K) {
      lds_store4(owb + hl::otile_off(t, hs, HP, n * (int)sizeof(IT), kWRow, kHalf), acc[nb], (const IT*)nullptr);
    } else {
      lds_store4(oub + hl::otile_off(t, hs, HP, (n - K) * (int)sizeof(IT), kURow, kHalf), acc[nb], (const IT*)nullptr);
    }
  }
  lds_barrier();
  // Thread q: 16-byte piece c of token j's HP contiguous w (u) rows.
  auto piece = [&](const char* base, int j, int c, int row) {
    u32x4 val = *reinterpret_cast<const u32x4*>(base + hl::otile_chunk(j, c / (row / 16), HP, c % (row / 16), row));
    if (hl::otile_half_swapped(j, kHalf)) val = u32x4{val[2], val[3], val[0], val[1]};
    return val;
  };
  constexpr int kWPieces = kBT * HP * kWRow / 16, kUPieces = kBT * HP * kURow / 16;
  static_assert(kWPieces % C::kThreads == 0 && kUPieces % C::kThreads == 0, "store split");
#pragma unroll
  for (int it = 0; it < kWPieces / C::kThreads; ++it) {
    const int q = tid + it * C::kThreads;
    const int j = q / (HP * kWRow / 16), c = q - j * (HP * kWRow / 16);
    *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(w + ((tok0 + j) * H + h0) * K) + c * 16) = piece(owb, j, c, kWRow);
  }
#pragma unroll
  for (int it = 0; it < kUPieces / C::kThreads; ++it) {
    const int q = tid + it * C::kThreads;
    const int j = q / (HP * kURow / 16), c = q - j * (HP * kURow / 16);
    *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(u + ((tok0 + j) * H + h0) * V) + c * 16) = piece(oub, j, c, kURow);
  }
}

template <typename IT, int K, int V, int HP>
hipError_t launch_wu(const void* k, const void* v, const void* beta, const void* A, const void* g,
                     void* w, void* u, int64_t B, int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / kBT;
  const int64_t tiles = B * NT * H / HP;
  hipLaunchKernelGGL((recompute_w_u_kernel<IT, K, V, HP>), dim3((unsigned)tiles), dim3(kWuThreads * HP), 0, s,
                     (const IT*)k, (const IT*)v, (const float*)beta, (const float*)A,
                     (const float*)g, (IT*)w, (IT*)u, T, H, NT);
  return hipGetLastError();
}

template <typename IT, int HP>
hipError_t dispatch_kv_hp(int64_t K, int64_t V, const void* k, const void* v, const void* beta,
                          const void* A, const void* g, void* w, void* u, int64_t B, int64_t T,
                          int64_t H, hipStream_t s) {
  if (K == 64 && V == 64) return launch_wu<IT, 64, 64, HP>(k, v, beta, A, g, w, u, B, T, H, s);
  if (K == 64 && V == 128) return launch_wu<IT, 64, 128, HP>(k, v, beta, A, g, w, u, B, T, H, s);
  if (K == 128 && V == 64) return launch_wu<IT, 128, 64, HP>(k, v, beta, A, g, w, u, B, T, H, s);
  return launch_wu<IT, 128, 128, HP>(k, v, beta, A, g, w, u, B, T, H, s);
}

// bf16 with an even head count takes tiles of 2 heads (66 KB of LDS at
// K = V = 128, 2 workgroups per CU): at config 4 the memory-only floor of
// that pattern moves the kernel's bytes in 238.9 against 255.9 us for
// 1-head tiles.  fp32 rows are already 512 bytes per head, and a 2-head fp32
// tile (hi + lo) would not leave room for 2 workgroups per CU.
template <typename IT>
hipError_t dispatch_kv(int64_t K, int64_t V, const void* k, const void* v, const void* beta,
                       const void* A, const void* g, void* w, void* u, int64_t B, int64_t T,
                       int64_t H, hipStream_t s) {
  if constexpr (!std::is_same<IT, float>::value) {
    if (H % 2 == 0) return dispatch_kv_hp<IT, 2>(K, V, k, v, beta, A, g, w, u, B, T, H, s);
  }
  return dispatch_kv_hp<IT, 1>(K, V, k, v, beta, A, g, w, u, B, T, H, s);
}

}  // namespace
}  // namespace thm

extern "C" int thm_recompute_w_u_fwd(const void* k, const void* v, const void* beta, const void* A,
                                     const void* g, void* w, void* u, int64_t B, int64_t T,
                                     int64_t H, int64_t K, int64_t V, int32_t chunk_size,
                                     int32_t kv_dtype, void* stream) {
  using namespace thm;
  if (chunk_size != kBT) return THM_ERR_BAD_ARGUMENT;
  if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || T % kBT) return THM_ERR_BAD_SHAPE;
  if (kv_dtype != THM_DTYPE_F32 && kv_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) return THM_ERR_UNSUPPORTED;
  if (B == 0 || T == 0) return THM_OK;  // empty: nothing is read or written
  if (!k || !v || !beta || !A || !w || !u) return THM_ERR_NULL_POINTER;
  const void* ptrs[] = {k, v, A, w, u};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return THM_ERR_MISALIGNED;
  if (((uintptr_t)beta % 4) || (g && ((uintptr_t)g % 4))) return THM_ERR_MISALIGNED;
  if (B * (T / kBT) > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
  if (!launch_fits(B * (T / kBT) * H, kWuThreads)) return THM_ERR_BAD_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = (kv_dtype == THM_DTYPE_F32)
                     ? dispatch_kv<float>(K, V, k, v, beta, A, g, w, u, B, T, H, s)
                     : dispatch_kv<bf16>(K, V, k, v, beta, A, g, w, u, B, T, H, s);
  return (int)e;
}
