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
// Structure (the bf16 DMA pipeline of chunk_fwd_h.hip, 4 wavefronts, wave wq
// owns state columns 16 wq .. 16 wq + 15 of the tile for all K rows):
//   * k, w, q, u and g of a chunk arrive by global -> LDS DMA into a 2-stage
//     ring (XOR-swizzled tiles of h_layout.h), one chunk ahead of use;
//   * P1: v_new = u - w S, the S accumulator pairs as the B operand (paired
//     contraction order), w rows from LDS in the same order;
//   * per 16-row query block ib:
//       global term  q S     -- the same product as P1 with q rows;
//       scores P^T[j][i] = k_j . q_i (natural order), gated and masked
//       (diagonal included); their accumulator pairs are directly the A
//       operand of the local term P v_new, whose B operand is the v_new
//       accumulator pairs; each wave forms the scores it needs itself;
//       o = scale (e^{g_i} q S + P v_new), an 8-byte store per lane after a
//       4x4 quad transpose;
//   * P2: S = e^{g_last} S + k^T (v_new e^{g_last - g}).
// All DMA and stores of the chunk loop go through vmem.h, and the wait at the
// top of the loop is an exact count (one chunk of stores is issued after each
// chunk's DMA).
// HBM traffic per token-head: k, w and q (K eb each), u (V eb) and g (4 B)
// read once; o (V eb) written once (+ v_new when requested).  The V-tiles of
// one (b, head) run on one XCD, so their second read of k, w, q is meant to
// hit that XCD's L2.
#include "h_layout.h"
#include "mfma.h"
#include "vmem.h"

namespace thm {
namespace {

constexpr int kBT = 64;
constexpr int kFBV = 64;        // V-tile width
constexpr int kFThreads = 256;  // 4 wavefronts x 16 state columns
constexpr int kFStages = 2;

template <int K, bool HAS_G, bool STORE_VN>
struct FCfg {
  static constexpr int kRowK = K * 2;             // bytes per k / w / q row
  static constexpr int kTileK = kBT * kRowK;
  static constexpr int kRowU = kFBV * 2;          // bytes per u row of the V-tile
  static constexpr int kTileU = kBT * kRowU;
  static constexpr int kGBytes = 4 * kBT * 4;     // one gate copy per wave
  static constexpr int kStage = 3 * kTileK + kTileU + (HAS_G ? kGBytes : 0);
  static constexpr int kLds = kFStages * kStage;
  static constexpr int KB = K / 16;               // 16-row state tiles per wave
  static constexpr int kKDma = kTileK / 1024 / 4; // 1 KiB DMA instructions per wave per k / w / q tile
  static constexpr int kUDma = kTileU / 1024 / 4;
  static constexpr int kDma = 3 * kKDma + kUDma + (HAS_G ? 1 : 0);
  static constexpr int kStores = 4 + (STORE_VN ? 4 : 0);  // o (+ v_new) row tiles per wave
  static constexpr int kWaitFirst = (kFStages - 2) * kDma;
  static constexpr int kWaitSteady = (kFStages - 1) * kStores + (kFStages - 2) * kDma;
  static_assert(kStage % 1024 == 0, "1 KiB aligned stages");
  static_assert(kLds <= 160 * 1024, "LDS budget");
  static_assert(kWaitSteady <= 63, "vmcnt range");
};

template <int K, int V, bool HAS_G, bool STORE_VN>
__global__ void __launch_bounds__(kFThreads)
chunk_fwd_fused_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                       const bf16* __restrict__ w, const bf16* __restrict__ u,
                       const float* __restrict__ g, const float* __restrict__ h0,
                       bf16* __restrict__ o, bf16* __restrict__ vnew, float* __restrict__ ht,
                       float scale, int64_t T, int64_t H, int64_t NT, int64_t BH) {
  using C = FCfg<K, HAS_G, STORE_VN>;
  constexpr int NVT = V / kFBV;
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
  const int v0 = (int)vt * kFBV;

  const int tid = threadIdx.x;
  const int wq = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, grp = lane >> 4, li = lane & 15;

  auto stage_k = [&](int s) { return lds + s * C::kStage; };
  auto stage_w = [&](int s) { return lds + s * C::kStage + C::kTileK; };
  auto stage_q = [&](int s) { return lds + s * C::kStage + 2 * C::kTileK; };
  auto stage_u = [&](int s) { return lds + s * C::kStage + 3 * C::kTileK; };
  auto stage_g = [&](int s) {
    return reinterpret_cast<float*>(lds + s * C::kStage + 3 * C::kTileK + C::kTileU);
  };

  // Global geometry in bytes.  Token t of chunk c, head hh: ((b T + 64 c + t) H + hh) D.
  const int64_t tsk = H * K * 2, tsv = H * V * 2;
  const int64_t kc0 = ((b * T) * H + hh) * K * 2;
  const int64_t uc0 = ((b * T) * H + hh) * V * 2 + v0 * 2;
  const int64_t gc0 = ((b * T) * H + hh) * 4;
  const int64_t kcs = kBT * tsk, ucs = kBT * tsv, gcs = kBT * H * 4;

  uint32_t koff[C::kKDma], uoff[C::kUDma];
#pragma unroll
  for (int i = 0; i < C::kKDma; ++i) {
    const int P = (wq * C::kKDma + i) * 64 + lane;
    koff[i] = (uint32_t)(hl::dma_row(P, C::kRowK) * tsk + hl::dma_chunk(P, C::kRowK) * 16);
  }
#pragma unroll
  for (int i = 0; i < C::kUDma; ++i) {
    const int P = (wq * C::kUDma + i) * 64 + lane;
    uoff[i] = (uint32_t)(hl::dma_row(P, C::kRowU) * tsv + hl::dma_chunk(P, C::kRowU) * 16);
  }
  const uint32_t goff = (uint32_t)(lane * H * 4);

  auto issue = [&](int64_t cc, int s) {
    const int64_t off = kc0 + cc * kcs;
    const char* srcs[3] = {reinterpret_cast<const char*>(k) + off, reinterpret_cast<const char*>(w) + off,
                           reinterpret_cast<const char*>(q) + off};
    char* dsts[3] = {stage_k(s), stage_w(s), stage_q(s)};
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      const uint32_t l0 = lds_address(dsts[m]) + wq * C::kKDma * 1024;
#pragma unroll
      for (int i = 0; i < C::kKDma; ++i) dma_b128(srcs[m], koff[i], __builtin_amdgcn_readfirstlane(l0 + i * 1024));
    }
    const char* ub = reinterpret_cast<const char*>(u) + uc0 + cc * ucs;
    const uint32_t lu = lds_address(stage_u(s)) + wq * C::kUDma * 1024;
#pragma unroll
    for (int i = 0; i < C::kUDma; ++i) dma_b128(ub, uoff[i], __builtin_amdgcn_readfirstlane(lu + i * 1024));
    if constexpr (HAS_G) {
      const char* gb = reinterpret_cast<const char*>(g) + gc0 + cc * gcs;
      dma_b32(gb, goff, __builtin_amdgcn_readfirstlane(lds_address(stage_g(s)) + wq * 256));
    }
  };

  // State S[kappa = 16 kb + 4 grp + r][n = v0 + 16 wq + li] in S[kb][r].
  f32x4 S[C::KB];
  const int ncol = v0 + 16 * wq + li;
  const int64_t st_base = bh * (int64_t)(K * V);
#pragma unroll
  for (int kb = 0; kb < C::KB; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[kb][r] = h0 ? h0[st_base + (int64_t)(16 * kb + 4 * grp + r) * V + ncol] : 0.f;
  wait_vmcnt<0>();  // retire the h0 loads before the counted loop

  // Row-tile stores after the quad transpose: lane (grp, 4 m4 + qq) holds row
  // 4 grp + qq of a 16-row tile at columns 16 wq + 4 m4 .. + 3.
  const int m4 = li >> 2, qq = li & 3;
  const uint32_t rowoff0 = (uint32_t)((4 * grp + qq) * tsv + (v0 + 16 * wq + 4 * m4) * 2);
  auto store_rows = [&](bf16* base, int ib, f32x4 val) {
    const f32x4 t = quad_transpose(val);
    bf16x4 ov;
    ov[0] = (bf16)t[0]; ov[1] = (bf16)t[1]; ov[2] = (bf16)t[2]; ov[3] = (bf16)t[3];
    st_b64(base, rowoff0 + (uint32_t)(16 * ib * tsv), __builtin_bit_cast(u32x2, ov));
  };

  if (NT > 0) issue(0, 0);
  for (int64_t c = 0; c < NT; ++c) {
    const int s = (int)(c % kFStages);
    if (c < kFStages - 1) wait_vmcnt<C::kWaitFirst>();
    else wait_vmcnt<C::kWaitSteady>();
    lds_barrier();  // chunk c is in LDS; every wave is done with chunk c - 1
    {
      const int64_t cn = c + kFStages - 1;
      issue(cn < NT ? cn : NT - 1, (int)(cn % kFStages));
    }
    const char* tk = stage_k(s);
    const char* tw = stage_w(s);
    const char* tq = stage_q(s);
    const char* tu = stage_u(s);
    const float* gs = HAS_G ? stage_g(s) + wq * kBT : nullptr;

    // S as the B operand: pairs of 16-row tiles, paired contraction order.
    bf16x8 sb[C::KB / 2];
#pragma unroll
    for (int s2 = 0; s2 < C::KB / 2; ++s2) {
      const float f[8] = {S[2 * s2][0], S[2 * s2][1], S[2 * s2][2], S[2 * s2][3],
                          S[2 * s2 + 1][0], S[2 * s2 + 1][1], S[2 * s2 + 1][2], S[2 * s2 + 1][3]};
      sb[s2] = to_bf16x8(f);
    }
    // rows x S for a 16-row block of a [64 x K] tile (w or q).
    auto rows_times_S = [&](const char* tile, int ib) {
      f32x4 acc = zero4();
      const int row = 16 * ib + li;
#pragma unroll
      for (int s2 = 0; s2 < C::KB / 2; ++s2) {
        const int e0 = 32 * s2 + 4 * grp;
        const bf16x4 a0 = *reinterpret_cast<const bf16x4*>(tile + hl::tile_off(row, e0, C::kRowK));
        const bf16x4 a1 = *reinterpret_cast<const bf16x4*>(tile + hl::tile_off(row, e0 + 16, C::kRowK));
        acc = mfma16x16x32(concat(a0, a1), sb[s2], acc);
      }
      return acc;
    };

    // v_new rows j = 16 jb + 4 grp + r of column 16 wq + li.
    f32x4 vn[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const bf16x4 t = ds_read_tr16(reinterpret_cast<const bf16*>(
          tu + hl::tile_off(16 * jb + 4 * grp + (li >> 2), 16 * wq + 4 * (li & 3), C::kRowU)));
#pragma unroll
      for (int r = 0; r < 4; ++r) vn[jb][r] = (float)t[r];
      vn[jb] -= rows_times_S(tw, jb);
    }
    if constexpr (STORE_VN) {
      bf16* vb = vnew + ((b * T + c * kBT) * H + hh) * V;
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) store_rows(vb, jb, vn[jb]);
    }
    // v_new as the B operand of the local term (paired order over j).
    bf16x8 vb16[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const float f[8] = {vn[2 * s2][0], vn[2 * s2][1], vn[2 * s2][2], vn[2 * s2][3],
                          vn[2 * s2 + 1][0], vn[2 * s2 + 1][1], vn[2 * s2 + 1][2], vn[2 * s2 + 1][3]};
      vb16[s2] = to_bf16x8(f);
    }

    // Output, one 16-row query block at a time.
    bf16* ob = o + ((b * T + c * kBT) * H + hh) * V;
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      f32x4 acc = rows_times_S(tq, ib);  // q S
      if constexpr (HAS_G) {
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= fast_exp(gs[16 * ib + 4 * grp + r]);
      }
      // Scores P^T[j][i] for key blocks jb <= ib, i = 16 ib + li.
      f32x4 pt[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        pt[jb] = zero4();
        if (jb > ib) continue;
#pragma unroll
        for (int s2 = 0; s2 < K / 32; ++s2) {
          const bf16x8 kf = load8(reinterpret_cast<const bf16*>(tk + hl::tile_off(16 * jb + li, 32 * s2 + 8 * grp, C::kRowK)));
          const bf16x8 qf = load8(reinterpret_cast<const bf16*>(tq + hl::tile_off(16 * ib + li, 32 * s2 + 8 * grp, C::kRowK)));
          pt[jb] = mfma16x16x32(kf, qf, pt[jb]);
        }
        const int i = 16 * ib + li;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * jb + 4 * grp + r;
          float gate = 1.f;
          if constexpr (HAS_G) gate = fast_exp(gs[i] - gs[j]);
          pt[jb][r] = (j <= i) ? pt[jb][r] * gate : 0.f;
        }
      }
      // Local term: A = P[i][j] (the P^T pairs), B = v_new (pairs), paired order over j.
      f32x4 loc = zero4();
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        if (2 * s2 > ib) continue;
        const float f[8] = {pt[2 * s2][0], pt[2 * s2][1], pt[2 * s2][2], pt[2 * s2][3],
                            pt[2 * s2 + 1][0], pt[2 * s2 + 1][1], pt[2 * s2 + 1][2], pt[2 * s2 + 1][3]};
        loc = mfma16x16x32(to_bf16x8(f), vb16[s2], loc);
      }
      store_rows(ob, ib, (acc + loc) * scale);
    }

    // P2: S = e^{g_last} S + k^T (v_new e^{g_last - g}).
    bf16x8 vh[2];
    float decay = 1.f;
    if constexpr (HAS_G) {
      const float gl = gs[kBT - 1];
      decay = fast_exp(gl);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        float f[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j0 = 32 * s2 + 4 * grp + r;
          f[r] = vn[2 * s2][r] * fast_exp(gl - gs[j0]);
          f[4 + r] = vn[2 * s2 + 1][r] * fast_exp(gl - gs[j0 + 16]);
        }
        vh[s2] = to_bf16x8(f);
      }
    } else {
      vh[0] = vb16[0];
      vh[1] = vb16[1];
    }
#pragma unroll
    for (int kb = 0; kb < C::KB; ++kb) {
      if constexpr (HAS_G) S[kb] *= decay;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int col = 16 * kb + 4 * (li & 3);
        const bf16x4 a = ds_read_tr16(reinterpret_cast<const bf16*>(
            tk + hl::tile_off(32 * s2 + 4 * grp + (li >> 2), col, C::kRowK)));
        const bf16x4 bq = ds_read_tr16(reinterpret_cast<const bf16*>(
            tk + hl::tile_off(32 * s2 + 16 + 4 * grp + (li >> 2), col, C::kRowK)));
        S[kb] = mfma16x16x32(concat(a, bq), vh[s2], S[kb]);
      }
    }
  }
  wait_vmcnt<0>();  // no DMA may still target this workgroup's LDS when it exits

  if (ht) {
#pragma unroll
    for (int kb = 0; kb < C::KB; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) ht[st_base + (int64_t)(16 * kb + 4 * grp + r) * V + ncol] = S[kb][r];
  }
}

template <int K, int V>
hipError_t launch_fused(const void* q, const void* k, const void* w, const void* u, const void* g,
                        const void* h0, void* o, void* vnew, void* ht, float scale, int64_t B,
                        int64_t T, int64_t H, hipStream_t s) {
  const int64_t NT = T / kBT, BH = B * H;
  const dim3 grid((unsigned)(BH * (V / kFBV)));
#define THM_FUSED_LAUNCH(HG, SV)                                                                  \
  hipLaunchKernelGGL((chunk_fwd_fused_kernel<K, V, HG, SV>), grid, dim3(kFThreads), 0, s,         \
                     (const bf16*)q, (const bf16*)k, (const bf16*)w, (const bf16*)u, (const float*)g, \
                     (const float*)h0, (bf16*)o, (bf16*)vnew, (float*)ht, scale, T, H, NT, BH)
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

}  // namespace
}  // namespace thm

extern "C" int thm_chunk_gated_delta_fwd(const void* q, const void* k, const void* w, const void* u,
                                         const void* g, const void* h0, void* o, void* v_new,
                                         void* ht, float scale, int64_t B, int64_t T, int64_t H,
                                         int64_t K, int64_t V, int32_t chunk_size,
                                         int32_t qkv_dtype, void* stream) {
  using namespace thm;
  if (chunk_size != kBT) return THM_ERR_BAD_ARGUMENT;
  if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || T % kBT) return THM_ERR_BAD_SHAPE;
  if (qkv_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;  // the fused path is bf16-only
  if ((K != 64 && K != 128) || (V != 64 && V != 128)) return THM_ERR_UNSUPPORTED;
  if (B == 0) return THM_OK;
  if (T == 0 && !ht) return THM_OK;
  if (T > 0 && (!q || !k || !w || !u || !o)) return THM_ERR_NULL_POINTER;
  const void* p16[] = {q, k, w, u};
  for (const void* p : p16)
    if (p && ((uintptr_t)p % 16)) return THM_ERR_MISALIGNED;
  const void* p4[] = {g, h0, ht};
  for (const void* p : p4)
    if (p && ((uintptr_t)p % 4)) return THM_ERR_MISALIGNED;
  if (((uintptr_t)o % 8) || (v_new && ((uintptr_t)v_new % 8))) return THM_ERR_MISALIGNED;
  if (B > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
  if (64 * H * (K > V ? K : V) * 2 > (INT64_C(1) << 31)) return THM_ERR_UNSUPPORTED;  // 32-bit lane offsets
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (K == 64 && V == 64) e = launch_fused<64, 64>(q, k, w, u, g, h0, o, v_new, ht, scale, B, T, H, s);
  else if (K == 64 && V == 128) e = launch_fused<64, 128>(q, k, w, u, g, h0, o, v_new, ht, scale, B, T, H, s);
  else if (K == 128 && V == 64) e = launch_fused<128, 64>(q, k, w, u, g, h0, o, v_new, ht, scale, B, T, H, s);
  else e = launch_fused<128, 128>(q, k, w, u, g, h0, o, v_new, ht, scale, B, T, H, s);
  return (int)e;
}
