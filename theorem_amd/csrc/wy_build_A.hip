// WY matrix of the Gated DeltaNet chunk forward for MI355X (gfx950):
//   per chunk c of 64 tokens:  M[i][j] = beta_i (k_i . k_j) e^{g_i - g_j}  (j < i),
//                              A_c = (I + sign M)^{-1}
// sign = -1 is the reference's (I - M)^{-1} (kernels/recompute_w_u/reference.py:48-91,
// `_build_A`, a torch matmul + solve_triangular); sign = +1 is the gated delta
// rule's (I + M)^{-1}.  A [B, T, H, 64] fp32 holds row r of A_c at token c*64 + r.
//
// One wavefront per (b, chunk, head) tile, head fastest:
//   1. k k^T on v_mfma_f32_16x16x32_bf16.  With lane (g, j) holding features
//      8g .. 8g+7 of token j of a 16-token block, the A fragment of block ib
//      and the B fragment of block jb are the same kind of 16-byte row load, so
//      the tile's k is read from HBM exactly once, straight into registers
//      (fp32 k: bf16 hi + lo, three products).  Only the 10 lower 16x16 tiles
//      are formed.
//   2. sign * M (strict lower part, scaled by beta_i e^{g_i - g_j}) goes to LDS
//      as a packed triangle: row r holds its r entries, padded to a multiple of
//      4 floats so it is read with 16-byte broadcast loads.
//   3. Forward substitution in fp32: lane c holds column c of X = A_c and
//      computes X[r][c] = delta_rc - sum_{s<r} (sign M)[r][s] X[s][c] for
//      r = 0..63, fully unrolled (2016 FMAs per lane, two partial sums).
//      The coefficient reads are LDS broadcasts whose latency the unrolled
//      chain exposes: this step, not HBM, bounds the kernel.
//   4. Row r of A_c is one 256-byte store (lane c writes column c).
// HBM traffic per tile: k, beta, g read once, A written once.
#include <type_traits>

#include "mfma.h"

namespace thm {
namespace {

constexpr int kBT = 64;

// Offset (floats) of packed row r: rows padded to multiples of 4.
__host__ __device__ constexpr int tri_off(int r) {
  int o = 0;
  for (int q = 0; q < r; ++q) o += (q + 3) & ~3;
  return o;
}
constexpr int kTriFloats = tri_off(kBT);

template <typename IT, int K, int SIGN>
__global__ void __launch_bounds__(64)
wy_build_A_kernel(const IT* __restrict__ k, const float* __restrict__ beta,
                  const float* __restrict__ g, float* __restrict__ A, int64_t T, int64_t H,
                  int64_t NT) {
  constexpr bool kSplit = std::is_same<IT, float>::value;
  constexpr int KS = K / 32;  // contraction steps
  __shared__ __attribute__((aligned(16))) float lm[kTriFloats];
  __shared__ float sb[kBT], sg[kBT];

  const int64_t tile = blockIdx.x;
  const int64_t h = tile % H;
  const int64_t bc = tile / H;
  const int64_t c = bc % NT;
  const int64_t b = bc / NT;
  const int64_t tok0 = b * T + c * kBT;
  const int lane = threadIdx.x;
  const int grp = lane >> 4, li = lane & 15;

  // k fragments: fr[tb][s] = k[tok0 + 16 tb + li][32 s + 8 grp .. + 7].
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
  sb[lane] = beta[(tok0 + lane) * H + h];
  sg[lane] = g ? g[(tok0 + lane) * H + h] : 0.f;
  lds_barrier();

  // sign * M into the packed triangle.
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) {
#pragma unroll
    for (int jb = 0; jb <= ib; ++jb) {
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
        if (j < i) lm[tri_off(i) + j] = (float)SIGN * sb[i] * acc[r] * fast_exp(sg[i] - sg[j]);
      }
    }
  }
  lds_barrier();

  // Forward substitution, lane = column; coefficients are 16-byte LDS
  // broadcasts, two partial sums per row.
  float X[kBT];
#pragma unroll
  for (int r = 0; r < kBT; ++r) {
    float a0 = (r == lane) ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
    for (int s4 = 0; s4 < (r + 3) / 4; ++s4) {
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(lm + tri_off(r) + 4 * s4);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int s = 4 * s4 + q;
        if (s < r) {
          if (q & 1) a1 = fmaf(-l4[q], X[s], a1);
          else a0 = fmaf(-l4[q], X[s], a0);
        }
      }
    }
    X[r] = a0 + a1;
  }

  float* out = A + (tok0 * H + h) * kBT + lane;
#pragma unroll
  for (int r = 0; r < kBT; ++r) out[r * H * kBT] = X[r];
}

template <typename IT, int K>
hipError_t launch_A(const void* k, const void* beta, const void* g, void* A, int64_t B, int64_t T,
                    int64_t H, int sign, hipStream_t s) {
  const int64_t NT = T / kBT;
  const dim3 grid((unsigned)(B * NT * H));
  if (sign < 0)
    hipLaunchKernelGGL((wy_build_A_kernel<IT, K, -1>), grid, dim3(64), 0, s, (const IT*)k,
                       (const float*)beta, (const float*)g, (float*)A, T, H, NT);
  else
    hipLaunchKernelGGL((wy_build_A_kernel<IT, K, 1>), grid, dim3(64), 0, s, (const IT*)k,
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
  if ((uintptr_t)k % 16) return THM_ERR_MISALIGNED;
  if (((uintptr_t)beta % 4) || ((uintptr_t)A % 4) || (g && ((uintptr_t)g % 4))) return THM_ERR_MISALIGNED;
  if (B * (T / kBT) > (INT64_C(1) << 31) / H) return THM_ERR_BAD_SHAPE;
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
