// Depthwise causal 1-D convolution, two extensions of causal_conv1d.hip for
// MI355X (gfx950), same arithmetic (acc = bias, then taps 0..W-1 in fp32 FMA,
// optional SiLU):
//
// 1. Channels-last layout: x, out [B, S, D] with D contiguous (the layout of a
//    [B, D, S] tensor that is a transposed view of [B, S, D]).  Vectors run
//    along D: a lane owns VEC channels (one 16-byte vector) and walks a segment
//    of kClSeg timesteps, keeping the last W-1 input vectors of its channels in
//    registers; only the W-1 rows before each segment are read twice.  A
//    wavefront reads and writes 1 KiB of one row per step, and x and out are
//    streamed once.
//
// 2. Decode step (rolling state): for each (b, d), with state s[0..L_s) and
//    the new samples x[0..L):  window = s ++ x,
//      out[t] = act(bias + sum_k w[k] window[L_s - (W-1) + t + k]),  t < L,
//    and the state becomes the last L_s samples of the window (in place).
//    One lane per (b, d); a decode step moves a few bytes per channel, so this
//    is latency-, not bandwidth-, bound.
#include "common.h"

namespace thm {
namespace {

constexpr int kClThreads = 256;
constexpr int kClSeg = 64;  // timesteps per lane

constexpr int kClDepth = 16;  // time steps whose loads are in flight ahead of use

__device__ __forceinline__ float conv_param(const void* p, int64_t i, int is_bf16) {
  return is_bf16 ? (float)reinterpret_cast<const bf16*>(p)[i] : reinterpret_cast<const float*>(p)[i];
}

template <typename WT>
__device__ __forceinline__ float conv_param_t(const void* p, int64_t i) {
  return to_f32(reinterpret_cast<const WT*>(p)[i]);
}

template <typename XT, int VEC>
__device__ __forceinline__ void cl_load(const XT* p, float* v) {
  if constexpr (VEC * sizeof(XT) == 16) {
    unpack16(ldg16_nt(p), v, XT{});
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = to_f32(p[i]);
  }
}

template <typename XT, int VEC>
__device__ __forceinline__ void cl_store(XT* p, const float* v) {
  if constexpr (VEC * sizeof(XT) == 16) {
    stg16_nt(p, pack16(v, XT{}));
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) p[i] = from_f32<XT>(v[i]);
  }
}

template <typename XT, typename WT, int VEC, int W, bool SILU>
__global__ void __launch_bounds__(kClThreads)
causal_conv1d_cl_kernel(const XT* __restrict__ x, const void* __restrict__ weight,
                        const void* __restrict__ bias, XT* __restrict__ out, int64_t seqlen,
                        int64_t dim, int64_t groups, int64_t blocks_per_seg, int64_t segs) {
  const int64_t blk = blockIdx.x;
  const int64_t cb = blk % blocks_per_seg;
  const int64_t bs = blk / blocks_per_seg;
  const int64_t seg = bs % segs, b = bs / segs;
  const int64_t cg = cb * kClThreads + threadIdx.x;  // channel group
  if (cg >= groups) return;                           // no barriers follow
  const int64_t d0 = cg * VEC;
  const int64_t t0 = seg * kClSeg;
  const int64_t tend = (t0 + kClSeg < seqlen) ? t0 + kClSeg : seqlen;

  const XT* __restrict__ xb = x + b * seqlen * dim + d0;
  XT* __restrict__ ob = out + b * seqlen * dim + d0;
  // A whole segment of 16-byte vectors runs as straight-line code with
  // kClDepth loads in flight ahead of use (no loop, so the compiler's wait
  // counts stay exact); a partial last segment, or scalar lanes, loop.
  const bool pipelined = VEC * sizeof(XT) == 16 && tend - t0 == kClSeg;
  u32x4 pf[kClDepth];
  if constexpr (VEC * sizeof(XT) == 16) {
    if (pipelined) {
#pragma unroll
      for (int i = 0; i < kClDepth; ++i) pf[i] = ldg16_nt(xb + (t0 + i) * dim);
    }
  }
  // win[k] = input at t - (W-1) + k for k < W-1 (zero before t = 0): loaded
  // from a clamped row, then zeroed, so every load is issued before any use.
  float win[W > 1 ? W - 1 : 1][VEC];
#pragma unroll
  for (int k = 0; k < W - 1; ++k) {
    const int64_t t = t0 - (W - 1) + k;
    cl_load<XT, VEC>(xb + (t >= 0 ? t : 0) * dim, win[k]);
    if (t < 0) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) win[k][v] = 0.f;
    }
  }
  // Weights and bias (bias absent: read the weights, then zero).
  const WT* __restrict__ wp = reinterpret_cast<const WT*>(weight);
  const WT* __restrict__ bp = bias ? reinterpret_cast<const WT*>(bias) : wp;
  float wk[W][VEC], bv[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
#pragma unroll
    for (int k = 0; k < W; ++k) wk[k][v] = to_f32(wp[(d0 + v) * W + k]);
    bv[v] = to_f32(bp[d0 + v]);
  }
  if (!bias) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) bv[v] = 0.f;
  }

  auto step = [&](int64_t t, const float* cur) {
    float res[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      float acc = bv[v];
#pragma unroll
      for (int k = 0; k < W - 1; ++k) acc = __builtin_fmaf(wk[k][v], win[k][v], acc);
      acc = __builtin_fmaf(wk[W - 1][v], cur[v], acc);
      if constexpr (SILU) acc = acc / (1.f + fast_exp(-acc));
      res[v] = acc;
    }
    cl_store<XT, VEC>(ob + t * dim, res);
#pragma unroll
    for (int k = 0; k + 1 < W - 1; ++k)
#pragma unroll
      for (int v = 0; v < VEC; ++v) win[k][v] = win[k + 1][v];
    if constexpr (W > 1) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) win[W - 2][v] = cur[v];
    }
  };

  if constexpr (VEC * sizeof(XT) == 16) {
    if (pipelined) {
#pragma unroll
      for (int i = 0; i < kClSeg; ++i) {
        float cur[VEC];
        unpack16(pf[i % kClDepth], cur, XT{});
        if (i + kClDepth < kClSeg) pf[i % kClDepth] = ldg16_nt(xb + (t0 + i + kClDepth) * dim);
        step(t0 + i, cur);
      }
      return;
    }
  }
  for (int64_t t = t0; t < tend; ++t) {
    float cur[VEC];
    cl_load<XT, VEC>(xb + t * dim, cur);
    step(t, cur);
  }
}

template <typename XT, typename WT, int VEC>
hipError_t launch_cl_w(int width, const void* x, const void* weight, const void* bias, void* out,
                       int64_t batch, int64_t seqlen, int64_t dim, int act, hipStream_t s) {
  const int64_t groups = dim / VEC;
  const int64_t blocks_per_seg = (groups + kClThreads - 1) / kClThreads;
  const int64_t segs = (seqlen + kClSeg - 1) / kClSeg;
  const dim3 grid((unsigned)(batch * segs * blocks_per_seg));
  switch (width) {
#define THM_CL_W(WV)                                                                          \
  case WV:                                                                                    \
    if (act == THM_ACT_SILU)                                                                       \
      hipLaunchKernelGGL((causal_conv1d_cl_kernel<XT, WT, VEC, WV, true>), grid, dim3(kClThreads), 0, \
                         s, (const XT*)x, weight, bias, (XT*)out, seqlen, dim, groups,             \
                         blocks_per_seg, segs);                                                    \
    else                                                                                           \
      hipLaunchKernelGGL((causal_conv1d_cl_kernel<XT, WT, VEC, WV, false>), grid, dim3(kClThreads), 0,\
                         s, (const XT*)x, weight, bias, (XT*)out, seqlen, dim, groups,             \
                         blocks_per_seg, segs);                                                    \
    break;
    THM_CL_W(1)
    THM_CL_W(2)
    THM_CL_W(3)
    THM_CL_W(4)
    THM_CL_W(5)
    THM_CL_W(6)
    THM_CL_W(7)
    THM_CL_W(8)
#undef THM_CL_W
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename XT, int VEC>
hipError_t launch_cl(int width, const void* x, const void* weight, const void* bias, void* out,
                     int64_t batch, int64_t seqlen, int64_t dim, int wb, int act, hipStream_t s) {
  return wb ? launch_cl_w<XT, bf16, VEC>(width, x, weight, bias, out, batch, seqlen, dim, act, s)
            : launch_cl_w<XT, float, VEC>(width, x, weight, bias, out, batch, seqlen, dim, act, s);
}

template <typename XT>
__global__ void __launch_bounds__(256)
causal_conv1d_update_kernel(const XT* __restrict__ x, XT* __restrict__ state,
                            const void* __restrict__ weight, const void* __restrict__ bias,
                            XT* __restrict__ out, int64_t rows, int64_t dim, int64_t seqlen,
                            int64_t state_len, int width, int w_is_bf16, int act) {
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // b * dim + d
  if (row >= rows) return;
  const int64_t d = row % dim;
  float wk[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) wk[k] = (k < width) ? conv_param(weight, d * width + k, w_is_bf16) : 0.f;
  const float b0 = bias ? conv_param(bias, d, w_is_bf16) : 0.f;
  XT* __restrict__ st = state + row * state_len;
  const XT* __restrict__ xr = x + row * seqlen;
  XT* __restrict__ orow = out + row * seqlen;
  // window = st ++ xr;  window index i is st[i] for i < L_s, else xr[i - L_s].
  auto at = [&](int64_t i) { return to_f32(i < state_len ? st[i] : xr[i - state_len]); };
  for (int64_t t = 0; t < seqlen; ++t) {
    float acc = b0;
    const int64_t base = state_len - (width - 1) + t;
    for (int k = 0; k < width; ++k) acc = __builtin_fmaf(wk[k], at(base + k), acc);
    if (act == THM_ACT_SILU) acc = acc / (1.f + fast_exp(-acc));
    orow[t] = from_f32<XT>(acc);
  }
  // New state: the last L_s window samples, written front to back (the
  // source index i + seqlen is never below the destination i).
  for (int64_t i = 0; i < state_len; ++i) st[i] = i + seqlen < state_len ? st[i + seqlen] : xr[i + seqlen - state_len];
}

template <typename XT>
hipError_t launch_update(const void* x, void* state, const void* weight, const void* bias, void* out,
                         int64_t batch, int64_t dim, int64_t seqlen, int64_t state_len, int width,
                         int wb, int act, hipStream_t s) {
  const int64_t rows = batch * dim;
  const dim3 grid((unsigned)((rows + 255) / 256));
  hipLaunchKernelGGL((causal_conv1d_update_kernel<XT>), grid, dim3(256), 0, s, (const XT*)x,
                     (XT*)state, weight, bias, (XT*)out, rows, dim, seqlen, state_len, width, wb, act);
  return hipGetLastError();
}

}  // namespace
}  // namespace thm

extern "C" int thm_causal_conv1d_fwd_channels_last(const void* x, const void* weight,
                                                   const void* bias, void* out, int64_t batch,
                                                   int64_t seqlen, int64_t dim, int32_t width,
                                                   int32_t x_dtype, int32_t w_dtype,
                                                   int32_t activation, void* stream) {
  using namespace thm;
  if (batch < 0 || dim <= 0 || seqlen < 0) return THM_ERR_BAD_SHAPE;
  if (x_dtype != THM_DTYPE_F32 && x_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if (w_dtype != THM_DTYPE_F32 && w_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if (width < 1 || width > 8) return THM_ERR_UNSUPPORTED;
  if (activation != THM_ACT_NONE && activation != THM_ACT_SILU) return THM_ERR_BAD_ARGUMENT;
  if (batch == 0 || seqlen == 0) return THM_OK;
  if (!x || !weight || !out) return THM_ERR_NULL_POINTER;
  const int64_t xe = (x_dtype == THM_DTYPE_F32) ? 4 : 2;
  const int64_t we = (w_dtype == THM_DTYPE_F32) ? 4 : 2;
  if (((uintptr_t)x % xe) || ((uintptr_t)out % xe) || ((uintptr_t)weight % we) ||
      (bias && ((uintptr_t)bias % we)))
    return THM_ERR_MISALIGNED;
  if (batch > (INT64_C(1) << 40) / dim || batch * dim > (INT64_C(1) << 46) / seqlen)
    return THM_ERR_BAD_SHAPE;
  const int vec = (int)(16 / xe);
  const bool vec_ok = ((uintptr_t)x % 16 == 0) && ((uintptr_t)out % 16 == 0) && (dim % vec == 0);
  const int64_t groups = vec_ok ? dim / vec : dim;
  if (!launch_fits(batch * ((seqlen + kClSeg - 1) / kClSeg) * ((groups + kClThreads - 1) / kClThreads), kClThreads))
    return THM_ERR_BAD_SHAPE;
  const int wb = (w_dtype == THM_DTYPE_BF16);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (x_dtype == THM_DTYPE_F32)
    e = vec_ok ? launch_cl<float, 4>(width, x, weight, bias, out, batch, seqlen, dim, wb, activation, s)
               : launch_cl<float, 1>(width, x, weight, bias, out, batch, seqlen, dim, wb, activation, s);
  else
    e = vec_ok ? launch_cl<bf16, 8>(width, x, weight, bias, out, batch, seqlen, dim, wb, activation, s)
               : launch_cl<bf16, 1>(width, x, weight, bias, out, batch, seqlen, dim, wb, activation, s);
  return (int)e;
}

extern "C" int thm_causal_conv1d_update(const void* x, void* conv_state, const void* weight,
                                        const void* bias, void* out, int64_t batch, int64_t dim,
                                        int64_t seqlen, int64_t state_len, int32_t width,
                                        int32_t x_dtype, int32_t w_dtype, int32_t activation,
                                        void* stream) {
  using namespace thm;
  if (batch < 0 || dim <= 0 || seqlen < 0 || state_len < 0) return THM_ERR_BAD_SHAPE;
  if (x_dtype != THM_DTYPE_F32 && x_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if (w_dtype != THM_DTYPE_F32 && w_dtype != THM_DTYPE_BF16) return THM_ERR_BAD_DTYPE;
  if (width < 1 || width > 8) return THM_ERR_UNSUPPORTED;
  if (state_len < width - 1) return THM_ERR_BAD_SHAPE;  // the window must cover the taps
  if (activation != THM_ACT_NONE && activation != THM_ACT_SILU) return THM_ERR_BAD_ARGUMENT;
  if (batch == 0 || seqlen == 0) return THM_OK;  // nothing new: the state is unchanged
  if (!x || !weight || !out || (state_len > 0 && !conv_state)) return THM_ERR_NULL_POINTER;
  const int64_t xe = (x_dtype == THM_DTYPE_F32) ? 4 : 2;
  const int64_t we = (w_dtype == THM_DTYPE_F32) ? 4 : 2;
  if (((uintptr_t)x % xe) || ((uintptr_t)out % xe) || ((uintptr_t)conv_state % xe) ||
      ((uintptr_t)weight % we) || (bias && ((uintptr_t)bias % we)))
    return THM_ERR_MISALIGNED;
  if (batch > (INT64_C(1) << 38) / dim || !launch_fits((batch * dim + 255) / 256, 256)) return THM_ERR_BAD_SHAPE;
  const int wb = (w_dtype == THM_DTYPE_BF16);
  hipStream_t s = (hipStream_t)stream;
  const hipError_t e =
      (x_dtype == THM_DTYPE_F32)
          ? launch_update<float>(x, conv_state, weight, bias, out, batch, dim, seqlen, state_len, width, wb, activation, s)
          : launch_update<bf16>(x, conv_state, weight, bias, out, batch, dim, seqlen, state_len, width, wb, activation, s);
  return (int)e;
}
