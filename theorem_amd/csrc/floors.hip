// Memory-only floors of the hot-path kernels' access patterns (measurement
// tooling for bench.py, built as a separate library, libtheorem_floors.so).
//
// Each kernel here moves exactly the algorithmic bytes of one hot-path kernel
// with that kernel's tile pattern, and computes nothing: its time is the
// fastest this box moves those bytes in that pattern.  bench.py reports each
// hot-path kernel against it beside the 8 TB/s published peak, because the
// achievable HBM rate on MI355X depends strongly on the read / write mix
// (a read-only stream reaches ~7 TB/s, a write-only one ~5.8 TB/s, and a
// few percent of writes mixed into a read stream cost far more than their
// own bytes).
//
// Layouts are the hot path's, at K = V = 128, bf16 (the config-4 shapes):
//   q, k, w, v, u, o, v_new, w/u outputs: [B, T, H, 128] bf16 (256 B per token-head)
//   A: [B, T, H, 64] fp32 (256 B per token-head);  h: [B, T/64, H, 128, 128] fp32
//   beta, g: [B, T, H] fp32
// One 256-thread workgroup per (b, chunk of 64 tokens, head) tile, head
// fastest, every load of the tile issued before the first store, as the
// tile-parallel hot-path kernels do.  Outputs hold XOR mixes of the inputs.
//
// A second reference point, floor_mfma_kernel, measures the box's bf16 MFMA
// throughput (v_mfma_f32_16x16x32_bf16 on register operands, no memory
// traffic) for the compute side of the roofline.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kRow = 256;      // bytes per token-head row of every [B, T, H, 128] bf16 tensor
constexpr int kHTile = 65536;  // bytes of one fp32 128 x 128 state

__device__ __forceinline__ u32x4 ld_nt(const char* p) { return __builtin_nontemporal_load((const u32x4*)p); }
__device__ __forceinline__ u32x4 ld(const char* p) { return *(const u32x4*)p; }
__device__ __forceinline__ void st(char* p, u32x4 v) { *(u32x4*)p = v; }

// Tile (b, chunk of 64 tokens, group of HPT adjacent heads) of a
// 256 HPT-thread workgroup, head groups fastest.  HPT = 1 is the hot-path
// kernels' tile; HPT = 2 and 4 read each token row of a tensor as one 512 B
// or 1 KB contiguous run instead of 256 B.
struct Tile {
  int64_t tile, hh, tok0;
};
template <int HPT>
__device__ __forceinline__ Tile tile_of(int64_t T, int64_t H) {
  Tile t;
  t.tile = blockIdx.x;
  const int64_t HG = H / HPT;
  t.hh = (t.tile % HG) * HPT;
  const int64_t bc = t.tile / HG, NT = T / 64;
  t.tok0 = (bc / NT) * T + (bc % NT) * 64;
  return t;
}
// Byte offset of 16-byte piece i (0..3) of this thread within a tile's 64 rows
// of HPT heads (16 HPT pieces per row).
template <int HPT>
__device__ __forceinline__ int64_t row_off(const Tile& t, int64_t H, int i) {
  const int q = threadIdx.x + i * 256 * HPT, j = q / (16 * HPT), col = (q % (16 * HPT)) * 16;
  return ((t.tok0 + j) * H + t.hh) * kRow + col;
}
// Index of this thread's beta / g value: token tid / HPT, head tid % HPT of
// the tile (threads below 64 HPT).
template <int HPT>
__device__ __forceinline__ int64_t tok_idx(const Tile& t, int64_t H) {
  return (t.tok0 + threadIdx.x / HPT) * H + t.hh + threadIdx.x % HPT;
}

// causal_conv1d: a streaming copy of the same bytes (x read once, out written once).
__global__ void __launch_bounds__(256) floor_copy_kernel(const char* __restrict__ src, char* __restrict__ dst,
                                                         int64_t n16) {
  // Piece i of thread t: 16-byte index (block * 4 + i) * 256 + t, so every
  // load and store instruction covers 4 KiB of contiguous memory.
  const int64_t i0 = (int64_t)blockIdx.x * 1024 + threadIdx.x;
  u32x4 r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (i0 + i * 256 < n16) r[i] = ld_nt(src + (i0 + i * 256) * 16);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (i0 + i * 256 < n16) __builtin_nontemporal_store(r[i], (u32x4*)(dst + (i0 + i * 256) * 16));
}

// bf16 MFMA throughput: each wave runs kMfmaChains independent accumulator
// chains of v_mfma_f32_16x16x32_bf16 (16384 flops each) for `iters` rounds,
// then writes one sum per lane so nothing is dead code.  16 chains: with 8
// the MFMA pipe waits on each chain's accumulator (1.2-1.4 PFLOP/s on the box
// against 2.0-2.1 with 16 at 2-8 waves per SIMD).
constexpr int kMfmaChains = 16;
__global__ void __launch_bounds__(256) floor_mfma_kernel(float* __restrict__ out, int64_t iters) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(1e-3f * (float)(lane + i));
    b[i] = (__bf16)(1e-3f * (float)(lane - i));
  }
  f32x4 acc[kMfmaChains];
#pragma unroll
  for (int c = 0; c < kMfmaChains; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kMfmaChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
  }
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < kMfmaChains; ++c) sum += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = sum;
}

// recompute_w_u: k, v, A rows, beta, g in; w, u rows out.
template <int HPT>
__global__ void __launch_bounds__(256 * HPT) floor_wu_kernel(const char* __restrict__ k, const char* __restrict__ v,
                                                             const char* __restrict__ A, const float* __restrict__ beta,
                                                             const float* __restrict__ g, char* __restrict__ w,
                                                             char* __restrict__ u, int64_t T, int64_t H) {
  const Tile t = tile_of<HPT>(T, H);
  u32x4 kr[4], vr[4], ar[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t off = row_off<HPT>(t, H, i);
    kr[i] = ld_nt(k + off);
    vr[i] = ld_nt(v + off);
    ar[i] = ld(A + off);
  }
  float s = 0.f;
  if (threadIdx.x < 64 * HPT) {
    const int64_t r = tok_idx<HPT>(t, H);
    s = beta[r] + g[r];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t off = row_off<HPT>(t, H, i);
    u32x4 a = ar[i];
    a[0] ^= __float_as_uint(s);
    st(w + off, kr[i] ^ a);
    st(u + off, vr[i] ^ a);
  }
}

// chunk_fwd_h (delta form): k, w, u rows and g in; the 64 KB states of the
// tile's heads (HPT adjacent states, one contiguous run) and the v_new rows out.
template <int HPT>
__global__ void __launch_bounds__(256 * HPT) floor_h_kernel(const char* __restrict__ k, const char* __restrict__ w,
                                                            const char* __restrict__ u, const float* __restrict__ g,
                                                            char* __restrict__ h, char* __restrict__ vn, int64_t T,
                                                            int64_t H) {
  const Tile t = tile_of<HPT>(T, H);
  u32x4 kr[4], wr[4], ur[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t off = row_off<HPT>(t, H, i);
    kr[i] = ld_nt(k + off);
    wr[i] = ld_nt(w + off);
    ur[i] = ld_nt(u + off);
  }
  u32x4 x = kr[0] ^ kr[1] ^ kr[2] ^ kr[3] ^ wr[0] ^ wr[1] ^ wr[2] ^ wr[3];
  if (threadIdx.x < 64 * HPT) x[0] ^= __float_as_uint(g[tok_idx<HPT>(t, H)]);
  char* hb = h + t.tile * (int64_t)HPT * kHTile;
#pragma unroll
  for (int i = 0; i < 16; ++i) st(hb + (threadIdx.x + i * 256 * HPT) * 16, x ^ ur[i & 3]);
#pragma unroll
  for (int i = 0; i < 4; ++i) st(vn + row_off<HPT>(t, H, i), ur[i] ^ x);
}

// chunk_fwd_o: q, k, v rows, the tile's 64 KB states and g in; o rows out.
template <int HPT>
__global__ void __launch_bounds__(256 * HPT) floor_o_kernel(const char* __restrict__ q, const char* __restrict__ k,
                                                            const char* __restrict__ v, const char* __restrict__ h,
                                                            const float* __restrict__ g, char* __restrict__ o,
                                                            int64_t T, int64_t H) {
  const Tile t = tile_of<HPT>(T, H);
  u32x4 hr[16], qr[4], kr[4], vr[4];
  const char* hb = h + t.tile * (int64_t)HPT * kHTile;
#pragma unroll
  for (int i = 0; i < 16; ++i) hr[i] = ld_nt(hb + (threadIdx.x + i * 256 * HPT) * 16);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t off = row_off<HPT>(t, H, i);
    qr[i] = ld_nt(q + off);
    kr[i] = ld_nt(k + off);
    vr[i] = ld_nt(v + off);
  }
  u32x4 x = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 16; ++i) x ^= hr[i];
  if (threadIdx.x < 64 * HPT) x[0] ^= __float_as_uint(g[tok_idx<HPT>(t, H)]);
#pragma unroll
  for (int i = 0; i < 4; ++i) st(o + row_off<HPT>(t, H, i), qr[i] ^ kr[i] ^ vr[i] ^ x);
}

// Fused WY forward (A-builder + recompute_w_u, A kept on chip): k, v rows,
// beta, g in; w, u rows out.
__global__ void __launch_bounds__(256) floor_wy_kernel(const char* __restrict__ k, const char* __restrict__ v,
                                                       const float* __restrict__ beta, const float* __restrict__ g,
                                                       char* __restrict__ w, char* __restrict__ u, int64_t T,
                                                       int64_t H) {
  const Tile t = tile_of<1>(T, H);
  u32x4 kr[4], vr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t off = row_off<1>(t, H, i);
    kr[i] = ld_nt(k + off);
    vr[i] = ld_nt(v + off);
  }
  u32x4 x = {0, 0, 0, 0};
  if (threadIdx.x < 64) {
    const int64_t r = tok_idx<1>(t, H);
    x[0] = __float_as_uint(beta[r] + g[r]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t off = row_off<1>(t, H, i);
    st(w + off, kr[i] ^ x);
    st(u + off, vr[i] ^ x);
  }
}

// Fused h + o (the per-chunk states stay on chip): q, k, w, u rows and g in;
// o rows out.
__global__ void __launch_bounds__(256) floor_ho_kernel(const char* __restrict__ q, const char* __restrict__ k,
                                                       const char* __restrict__ w, const char* __restrict__ u,
                                                       const float* __restrict__ g, char* __restrict__ o,
                                                       int64_t T, int64_t H) {
  const Tile t = tile_of<1>(T, H);
  u32x4 qr[4], kr[4], wr[4], ur[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t off = row_off<1>(t, H, i);
    qr[i] = ld_nt(q + off);
    kr[i] = ld_nt(k + off);
    wr[i] = ld_nt(w + off);
    ur[i] = ld_nt(u + off);
  }
  u32x4 x = {0, 0, 0, 0};
  if (threadIdx.x < 64) x[0] = __float_as_uint(g[tok_idx<1>(t, H)]);
#pragma unroll
  for (int i = 0; i < 4; ++i) st(o + row_off<1>(t, H, i), qr[i] ^ kr[i] ^ wr[i] ^ ur[i] ^ x);
}

// Contiguous ceiling of a read / write byte mix: nr16 16-byte pieces read
// from src and nw16 written to dst, both as one contiguous stream.  Block b
// reads pieces [b rper, (b + 1) rper) and writes [b wper, (b + 1) wper)
// (rper, wper <= 1024: at most 4 pieces per thread and direction, every load
// issued before the first store, ordinary stores as in the hot-path kernels),
// so the blocks in flight move the two directions in the given ratio.
__global__ void __launch_bounds__(256) floor_mix_kernel(const char* __restrict__ src, int64_t nr16, int64_t rper,
                                                        char* __restrict__ dst, int64_t nw16, int64_t wper) {
  const int64_t r0 = (int64_t)blockIdx.x * rper, w0 = (int64_t)blockIdx.x * wper;
  u32x4 r[4];
  u32x4 x = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t p = threadIdx.x + i * 256;
    r[i] = (p < rper && r0 + p < nr16) ? ld_nt(src + (r0 + p) * 16) : x;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) x ^= r[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t p = threadIdx.x + i * 256;
    if (p < wper && w0 + p < nw16) st(dst + (w0 + p) * 16, x ^ r[i]);
  }
}

bool tile_shape_ok(int64_t B, int64_t T, int64_t H, int heads = 1) {
  return B > 0 && T > 0 && H > 0 && T % 64 == 0 && (heads == 1 || heads == 2 || heads == 4) && H % heads == 0 &&
         B * (T / 64) * H <= (INT64_C(1) << 31) - 1;
}

}  // namespace

// All pointers are device pointers; 16-byte aligned for the row tensors and
// states, 4-byte for beta and g.  Return 0, -1 for a bad shape or pointer, or
// the positive hipError_t of the launch.
extern "C" int thm_floor_copy(const void* src, void* dst, int64_t nbytes, void* stream) {
  if (!src || !dst || nbytes <= 0 || nbytes % 16 || ((uintptr_t)src | (uintptr_t)dst) % 16) return -1;
  const int64_t n16 = nbytes / 16, per_block = 256 * 4;
  hipLaunchKernelGGL(floor_copy_kernel, dim3((unsigned)((n16 + per_block - 1) / per_block)), dim3(256), 0,
                     (hipStream_t)stream, (const char*)src, (char*)dst, n16);
  return (int)hipGetLastError();
}

// Contiguous read / write mix: nread bytes from src, nwrite bytes to dst
// (multiples of 16; dst's contents are overwritten with XOR mixes of src).
extern "C" int thm_floor_mix(const void* src, int64_t nread, void* dst, int64_t nwrite, void* stream) {
  if (!src || !dst || nread <= 0 || nwrite <= 0 || nread % 16 || nwrite % 16 ||
      ((uintptr_t)src | (uintptr_t)dst) % 16)
    return -1;
  const int64_t nr16 = nread / 16, nw16 = nwrite / 16, per_block = 256 * 4;
  const int64_t big = nr16 > nw16 ? nr16 : nw16;
  const int64_t blocks = (big + per_block - 1) / per_block;
  if (blocks > (INT64_C(1) << 31) - 1) return -1;
  const int64_t rper = (nr16 + blocks - 1) / blocks, wper = (nw16 + blocks - 1) / blocks;
  hipLaunchKernelGGL(floor_mix_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const char*)src, nr16, rper, (char*)dst, nw16, wper);
  return (int)hipGetLastError();
}

// bf16 MFMA throughput: `nblocks` workgroups of 256 threads (out holds
// nblocks * 256 floats); flops = nblocks * 4 waves * iters * kMfmaChains * 16384.
extern "C" int thm_floor_mfma(void* out, int64_t nblocks, int64_t iters, void* stream) {
  if (!out || nblocks <= 0 || nblocks > (INT64_C(1) << 31) - 1 || iters <= 0 || (uintptr_t)out % 4) return -1;
  hipLaunchKernelGGL(floor_mfma_kernel, dim3((unsigned)nblocks), dim3(256), 0, (hipStream_t)stream, (float*)out,
                     iters);
  return (int)hipGetLastError();
}

// The tile floors take `heads` = 1, 2 or 4 adjacent heads per workgroup
// (256 heads threads; H must be a multiple of heads).
#define THM_FLOOR_HPT(KERNEL, HEADS, GRID, S, ...)                                               \
  do {                                                                                          \
    if ((HEADS) == 1)                                                                           \
      hipLaunchKernelGGL(KERNEL<1>, dim3((unsigned)(GRID)), dim3(256), 0, S, __VA_ARGS__);      \
    else if ((HEADS) == 2)                                                                      \
      hipLaunchKernelGGL(KERNEL<2>, dim3((unsigned)((GRID) / 2)), dim3(512), 0, S, __VA_ARGS__); \
    else                                                                                        \
      hipLaunchKernelGGL(KERNEL<4>, dim3((unsigned)((GRID) / 4)), dim3(1024), 0, S, __VA_ARGS__); \
  } while (0)

extern "C" int thm_floor_wu_heads(const void* k, const void* v, const void* A, const void* beta, const void* g,
                                  void* w, void* u, int64_t B, int64_t T, int64_t H, int32_t heads, void* stream) {
  if (!tile_shape_ok(B, T, H, heads) || !k || !v || !A || !beta || !g || !w || !u) return -1;
  THM_FLOOR_HPT(floor_wu_kernel, heads, B * (T / 64) * H, (hipStream_t)stream, (const char*)k, (const char*)v,
                (const char*)A, (const float*)beta, (const float*)g, (char*)w, (char*)u, T, H);
  return (int)hipGetLastError();
}

extern "C" int thm_floor_wu(const void* k, const void* v, const void* A, const void* beta, const void* g,
                            void* w, void* u, int64_t B, int64_t T, int64_t H, void* stream) {
  return thm_floor_wu_heads(k, v, A, beta, g, w, u, B, T, H, 1, stream);
}

extern "C" int thm_floor_h_heads(const void* k, const void* w, const void* u, const void* g, void* h, void* vn,
                                 int64_t B, int64_t T, int64_t H, int32_t heads, void* stream) {
  if (!tile_shape_ok(B, T, H, heads) || !k || !w || !u || !g || !h || !vn) return -1;
  THM_FLOOR_HPT(floor_h_kernel, heads, B * (T / 64) * H, (hipStream_t)stream, (const char*)k, (const char*)w,
                (const char*)u, (const float*)g, (char*)h, (char*)vn, T, H);
  return (int)hipGetLastError();
}

extern "C" int thm_floor_h(const void* k, const void* w, const void* u, const void* g, void* h, void* vn,
                           int64_t B, int64_t T, int64_t H, void* stream) {
  return thm_floor_h_heads(k, w, u, g, h, vn, B, T, H, 1, stream);
}

extern "C" int thm_floor_wy(const void* k, const void* v, const void* beta, const void* g, void* w, void* u,
                            int64_t B, int64_t T, int64_t H, void* stream) {
  if (!tile_shape_ok(B, T, H) || !k || !v || !beta || !g || !w || !u) return -1;
  hipLaunchKernelGGL(floor_wy_kernel, dim3((unsigned)(B * (T / 64) * H)), dim3(256), 0, (hipStream_t)stream,
                     (const char*)k, (const char*)v, (const float*)beta, (const float*)g, (char*)w, (char*)u, T, H);
  return (int)hipGetLastError();
}

extern "C" int thm_floor_ho(const void* q, const void* k, const void* w, const void* u, const void* g, void* o,
                            int64_t B, int64_t T, int64_t H, void* stream) {
  if (!tile_shape_ok(B, T, H) || !q || !k || !w || !u || !g || !o) return -1;
  hipLaunchKernelGGL(floor_ho_kernel, dim3((unsigned)(B * (T / 64) * H)), dim3(256), 0, (hipStream_t)stream,
                     (const char*)q, (const char*)k, (const char*)w, (const char*)u, (const float*)g, (char*)o, T,
                     H);
  return (int)hipGetLastError();
}

extern "C" int thm_floor_o_heads(const void* q, const void* k, const void* v, const void* h, const void* g, void* o,
                                 int64_t B, int64_t T, int64_t H, int32_t heads, void* stream) {
  if (!tile_shape_ok(B, T, H, heads) || !q || !k || !v || !h || !g || !o) return -1;
  THM_FLOOR_HPT(floor_o_kernel, heads, B * (T / 64) * H, (hipStream_t)stream, (const char*)q, (const char*)k,
                (const char*)v, (const char*)h, (const float*)g, (char*)o, T, H);
  return (int)hipGetLastError();
}

extern "C" int thm_floor_o(const void* q, const void* k, const void* v, const void* h, const void* g, void* o,
                           int64_t B, int64_t T, int64_t H, void* stream) {
  return thm_floor_o_heads(q, k, v, h, g, o, B, T, H, 1, stream);
}
