// Depthwise causal 1-D convolution for MI355X (gfx950).
//
//   out[b,d,t] = act( bias[d] + sum_{k<W} w[d,k] * x[b,d,t-W+1+k] ),  x[t<0] = 0
//
// Replaces kernels/causal_conv1d/kernel.py:44-117 (Triton) and its launcher
// kernel.py:170-230; arithmetic order (acc = bias, then taps k = 0..W-1) of
// kernel.py:85-110.
//
// HBM-bound design: x and out are streamed exactly once.
//   * A row r = b*D + d is a contiguous run of S elements.  Each wavefront owns
//     one segment of one row: NV groups of 64 lanes x VEC elements, where VEC
//     elements are one 16-byte vector (4 fp32 / 8 bf16) per lane, so every
//     wave-wide load/store moves 1 KiB of contiguous memory.
//   * The W-1 inputs left of a lane's vector live in the previous lane's
//     registers: they are passed with a DPP whole-wave shift (wave_shr:1), and
//     lane 0 takes lane 63's value of the previous group (v_readlane).  Only the
//     W-1 elements before each segment are re-read (wave-uniform loads).
//   * Weights and bias are wave-uniform; accumulation is fp32 FMA.
//   * Stores are non-temporal: the output is not re-read by this kernel.
#include "common.h"

namespace thm {
namespace {

constexpr int kConvWaves = 4;  // wavefronts per workgroup
constexpr int kConvNV = 4;     // 64-lane vector groups per wavefront segment

template <typename XT, int VEC>
__device__ __forceinline__ void load_vec(const XT* p, float* v) {
  if constexpr (VEC * sizeof(XT) == 16) {
    unpack16(ldg16_nt(p), v, XT{});
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = to_f32(p[i]);
  }
}

template <typename XT, int VEC>
__device__ __forceinline__ void store_vec(XT* p, const float* v) {
  if constexpr (VEC * sizeof(XT) == 16) {
    stg16_nt(p, pack16(v, XT{}));
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) p[i] = from_f32<XT>(v[i]);
  }
}

template <typename WT>
__device__ __forceinline__ float load_param(const void* p, int64_t i) {
  return to_f32(reinterpret_cast<const WT*>(p)[i]);
}

template <typename XT, typename WT, int VEC, int W, int NV>
__global__ void __launch_bounds__(kConvWaves * kWave)
causal_conv1d_kernel(const XT* __restrict__ x, const void* __restrict__ weight,
                     const void* __restrict__ bias, XT* __restrict__ out, int64_t n_rows,
                     int64_t dim, int64_t seqlen, int64_t segs_per_row, int act) {
  constexpr int SEG = NV * kWave * VEC;
  constexpr int P = (W - 1 + VEC - 1) / VEC;  // previous vectors a lane needs
  constexpr int PA = P > 0 ? P : 1;

  const int lane = lane_id();
  // The wave index is uniform; saying so makes the row, its weights and the
  // halo scalar (s_load) rather than per-lane loads behind divergent branches.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t seg = (int64_t)blockIdx.x * kConvWaves + wave;
  if (seg >= n_rows * segs_per_row) return;  // wave-uniform exit
  const int64_t row = seg / segs_per_row;
  const int64_t s0 = (seg - row * segs_per_row) * SEG;
  const int64_t d = row % dim;

  const XT* __restrict__ xr = x + row * seqlen;
  XT* __restrict__ orow = out + row * seqlen;

  float cur[NV][VEC];   // this lane's vectors
  float halo[PA][VEC];  // vectors just left of the segment (stream index -1-q), wave-uniform
  if constexpr (VEC * sizeof(XT) == 16) {
    // Every load of the wave is issued before the first use: the segment's
    // vectors (a lane past the row end reads the row start and is zeroed) and
    // the P vectors left of the segment (uniform; none for the row's first
    // segment, where they are the causal zero padding).
    u32x4 raw[NV], hraw[PA];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e0 = s0 + (int64_t)(j * kWave + lane) * VEC;
      raw[j] = ldg16_nt(xr + (e0 < seqlen ? e0 : 0));
    }
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      const int64_t pos = s0 - (int64_t)(q + 1) * VEC;
      hraw[q] = (q < P && pos >= 0) ? ldg16(xr + pos) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e0 = s0 + (int64_t)(j * kWave + lane) * VEC;
      unpack16(raw[j], cur[j], XT{});
      if (e0 >= seqlen) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) cur[j][i] = 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < PA; ++q) unpack16(hraw[q], halo[q], XT{});
  } else {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e0 = s0 + (int64_t)(j * kWave + lane) * VEC;
      if (e0 < seqlen) {
        load_vec<XT, VEC>(xr + e0, cur[j]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) cur[j][i] = 0.f;
      }
    }
    // Only the elements within W-1 of the segment start are read.
#pragma unroll
    for (int q = 0; q < PA; ++q) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int64_t pos = s0 - (int64_t)(q + 1) * VEC + e;
        const bool needed = (q < P) && ((q + 1) * VEC - e <= W - 1);
        halo[q][e] = (needed && pos >= 0) ? to_f32(xr[pos]) : 0.f;
      }
    }
  }
  float wk[W];
#pragma unroll
  for (int k = 0; k < W; ++k) wk[k] = load_param<WT>(weight, d * W + k);
  const float b0 = bias ? load_param<WT>(bias, d) : 0.f;

  // prev[p-1][j] = vector at stream index (j*64 + lane - p); only the elements
  // e >= p*VEC - (W-1) are used.
  float prev[PA][NV][VEC];
#pragma unroll
  for (int p = 1; p <= P; ++p) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      if (e < p * VEC - (W - 1)) continue;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const float src = (p == 1) ? cur[j][e] : prev[p - 2][j][e];
        float fill;
        if (j == 0) {
          fill = halo[p - 1][e];
        } else {
          fill = readlane((p == 1) ? cur[j - 1][e] : prev[p - 2][j - 1][e], kWave - 1);
        }
        prev[p - 1][j][e] = wave_shr1(src, fill);
      }
    }
  }

#pragma unroll
  for (int j = 0; j < NV; ++j) {
    float res[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      float acc = b0;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const int rel = v - (W - 1) + k;
        float xv;
        if (rel >= 0) {
          xv = cur[j][rel];
        } else {
          const int m = -rel;
          const int p = (m + VEC - 1) / VEC;
          xv = prev[p - 1][j][p * VEC - m];
        }
        acc = __builtin_fmaf(wk[k], xv, acc);
      }
      if (act == THM_ACT_SILU) acc = acc / (1.f + fast_exp(-acc));
      res[v] = acc;
    }
    const int64_t e0 = s0 + (int64_t)(j * kWave + lane) * VEC;
    if (e0 < seqlen) store_vec<XT, VEC>(orow + e0, res);
  }
}

template <typename XT, typename WT, int VEC, int W>
hipError_t launch_conv(const void* x, const void* weight, const void* bias, void* out,
                       int64_t n_rows, int64_t dim, int64_t seqlen, int act, hipStream_t stream) {
  constexpr int SEG = kConvNV * kWave * VEC;
  const int64_t segs_per_row = (seqlen + SEG - 1) / SEG;
  const int64_t n_seg = n_rows * segs_per_row;
  const int64_t blocks = (n_seg + kConvWaves - 1) / kConvWaves;
  hipLaunchKernelGGL((causal_conv1d_kernel<XT, WT, VEC, W, kConvNV>), dim3((unsigned)blocks),
                     dim3(kConvWaves * kWave), 0, stream, (const XT*)x, weight, bias, (XT*)out,
                     n_rows, dim, seqlen, segs_per_row, act);
  return hipGetLastError();
}

template <typename XT, int VEC, typename WT>
hipError_t dispatch_width_w(int width, const void* x, const void* weight, const void* bias,
                            void* out, int64_t n_rows, int64_t dim, int64_t seqlen, int act,
                            hipStream_t s) {
  switch (width) {
#define THM_CONV_W(WV)                                                                           \
  case WV:                                                                                       \
    return launch_conv<XT, WT, VEC, WV>(x, weight, bias, out, n_rows, dim, seqlen, act, s);
    THM_CONV_W(1)
    THM_CONV_W(2)
    THM_CONV_W(3)
    THM_CONV_W(4)
    THM_CONV_W(5)
    THM_CONV_W(6)
    THM_CONV_W(7)
    THM_CONV_W(8)
#undef THM_CONV_W
    default:
      return hipErrorInvalidValue;
  }
}

template <typename XT, int VEC>
hipError_t dispatch_width(int width, const void* x, const void* weight, const void* bias,
                          void* out, int64_t n_rows, int64_t dim, int64_t seqlen, int w_is_bf16,
                          int act, hipStream_t s) {
  return w_is_bf16 ? dispatch_width_w<XT, VEC, bf16>(width, x, weight, bias, out, n_rows, dim, seqlen, act, s)
                   : dispatch_width_w<XT, VEC, float>(width, x, weight, bias, out, n_rows, dim, seqlen, act, s);
}

}  // namespace
}  // namespace thm

extern "C" int thm_causal_conv1d_fwd(const void* x, const void* weight, const void* bias,
                                     void* out, int64_t batch, int64_t dim, int64_t seqlen,
                                     int32_t width, int32_t x_dtype, int32_t w_dtype,
                                     int32_t activation, void* stream) {
  using namespace thm;
  if (batch < 0 || dim <= 0 || seqlen < 0) return THM_ERR_BAD_SHAPE;
  if (x_dtype != THM_DTYPE_F32 && x_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if (w_dtype != THM_DTYPE_F32 && w_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if (width < 1 || width > 8) return THM_ERR_UNSUPPORTED;
  if (activation != THM_ACT_NONE && activation != THM_ACT_SILU) return THM_ERR_BAD_ARGUMENT;
  if (batch == 0 || seqlen == 0) return THM_OK;  // empty: nothing is read or written
  if (!x || !weight || !out) return THM_ERR_NULL_POINTER;
  const int64_t xe = (x_dtype == THM_DTYPE_F32) ? 4 : 2;
  const int64_t we = (w_dtype == THM_DTYPE_F32) ? 4 : 2;
  if (((uintptr_t)x % xe) || ((uintptr_t)out % xe) || ((uintptr_t)weight % we) ||
      (bias && ((uintptr_t)bias % we)))
    return THM_ERR_MISALIGNED;
  if (batch > (INT64_C(1) << 40) / dim || batch * dim > (INT64_C(1) << 46) / seqlen)
    return THM_ERR_BAD_SHAPE;
  const int64_t n_rows = batch * dim;
  // Largest grid: the scalar path's 256-element segments, kConvWaves per block.
  if (!launch_fits((n_rows * ((seqlen + 255) / 256) + kConvWaves - 1) / kConvWaves, kConvWaves * kWave))
    return THM_ERR_BAD_SHAPE;
  const int vec = (int)(16 / xe);
  // 16-byte vectors need every row start 16-byte aligned.
  const bool vec_ok = ((uintptr_t)x % 16 == 0) && ((uintptr_t)out % 16 == 0) && (seqlen % vec == 0);
  const int wb = (w_dtype == THM_DTYPE_BF16);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (x_dtype == THM_DTYPE_F32) {
    e = vec_ok ? dispatch_width<float, 4>(width, x, weight, bias, out, n_rows, dim, seqlen, wb,
                                          activation, s)
               : dispatch_width<float, 1>(width, x, weight, bias, out, n_rows, dim, seqlen, wb,
                                          activation, s);
  } else {
    e = vec_ok ? dispatch_width<bf16, 8>(width, x, weight, bias, out, n_rows, dim, seqlen, wb,
                                         activation, s)
               : dispatch_width<bf16, 1>(width, x, weight, bias, out, n_rows, dim, seqlen, wb,
                                         activation, s);
  }
  return (int)e;
}
