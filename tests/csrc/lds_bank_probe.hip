// Measures LDS bank conflicts per instruction on the GPU, to pin the model in
// lds_banks.h that the layout check (dma_check.cpp) applies.  Each pattern is
// one kernel launch: 256 single-wave workgroups, each repeating one LDS
// instruction kind 4096 times at fixed per-lane offsets into a 64 KiB LDS
// array.  Run under rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE
// SQ_INSTS_LDS; lds_bank_summary.py divides the counters by the instruction
// count and sets them beside the model's verdict, which this program prints
// (one line per launch, in launch order).
//
// Build: hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature
//   -Xclang -packed-fp32-ops -Itheorem_amd/csrc tests/csrc/lds_bank_probe.hip
//   -o <exe>
// Every offset is checked on the host (aligned, inside the array) before any
// launch.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <string>
#include <vector>

#include "h_layout.h"
#include "lds_banks.h"

namespace hl = thm::hl;

namespace {

typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) unsigned lds_u;
typedef __attribute__((address_space(3))) v2u lds_v2u;
typedef __attribute__((address_space(3))) v4u lds_v4u;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kLdsBytes = 65536;
constexpr int kGrid = 256, kIters = 4096;

enum Op { kW4, kW8, kW16, kR4, kR8, kR16, kTr };
constexpr int kBytes[] = {4, 8, 16, 4, 8, 16, 8};
constexpr const char* kOpName[] = {"ds_write_b32", "ds_write_b64", "ds_write_b128", "ds_read_b32",
                                   "ds_read_b64", "ds_read_b128", "ds_read_b64_tr_b16"};

template <int OP>
__global__ __launch_bounds__(64) void lds_probe(const uint32_t* offs, uint32_t* out) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  const uint32_t off = offs[threadIdx.x];
  uint32_t acc = threadIdx.x;
  for (int i = 0; i < kIters; ++i) {
    if constexpr (OP == kW4) {
      *(volatile lds_u*)(lds + off) = acc + i;
    } else if constexpr (OP == kW8) {
      *(volatile lds_v2u*)(lds + off) = v2u{(unsigned)i, acc};
    } else if constexpr (OP == kW16) {
      *(volatile lds_v4u*)(lds + off) = v4u{(unsigned)i, acc, (unsigned)i, acc};
    } else if constexpr (OP == kR4) {
      acc += *(volatile lds_u*)(lds + off);
    } else if constexpr (OP == kR8) {
      const v2u v = *(volatile lds_v2u*)(lds + off);
      acc += v.x ^ v.y;
    } else if constexpr (OP == kR16) {
      const v4u v = *(volatile lds_v4u*)(lds + off);
      acc += v.x ^ v.y ^ v.z ^ v.w;
    } else {
      const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds + off));
      acc += (uint32_t)(v[0] ^ v[1] ^ v[2] ^ v[3]);
      asm volatile("" ::: "memory");
    }
  }
  out[blockIdx.x * 64 + threadIdx.x] = acc;
}

struct Pattern {
  std::string name;
  Op op;
  std::vector<uint32_t> off;
};

template <class F>
void add(std::vector<Pattern>& ps, const std::string& name, Op op, F f) {
  Pattern p{name, op, std::vector<uint32_t>(64)};
  for (int l = 0; l < 64; ++l) p.off[l] = (uint32_t)f(l);
  ps.push_back(p);
}

std::vector<Pattern> patterns() {
  std::vector<Pattern> ps;
  for (int op = 0; op < 7; ++op) {
    const int w = kBytes[op];
    const Op o = (Op)op;
    const std::string n = kOpName[op];
    add(ps, n + " contiguous", o, [&](int l) { return l * w; });
    add(ps, n + " all lanes 512 B apart", o, [&](int l) { return l * 512 % kLdsBytes; });
    // Runs of r lanes, contiguous, runs `gap` bytes apart.
    for (int r : {4, 8, 16, 32})
      for (int gap : {128, 256, 512}) {
        if (r * w > gap) continue;
        add(ps, n + " runs of " + std::to_string(r) + " lanes " + std::to_string(gap) + " B apart", o,
            [&](int l) { return (l % r) * w + (l / r) * gap; });
      }
  }
  // Runs of 8 (16) lanes; runs 1-4 (lanes 0-31) 512 B apart, lanes 32-63 128 B
  // further: whole-instruction bank counts would be even, per-pass ones not.
  add(ps, "ds_read_b128 runs of 8 lanes, halves 128 B apart", kR16,
      [](int l) { return (l % 8) * 16 + ((l / 8) % 4) * 512 + (l / 32) * 128; });
  add(ps, "ds_read_b64 runs of 16 lanes, halves 128 B apart", kR8,
      [](int l) { return (l % 16) * 8 + ((l / 16) % 2) * 512 + (l / 32) * 128; });
  // 16 rows `pitch` apart, 16 lanes per 16-byte column (chunk_fwd_o's k reads).
  for (int pitch : {256, 272, 288})
    add(ps, "ds_read_b128 16 rows " + std::to_string(pitch) + " B apart", kR16,
        [&](int l) { return pitch * (l & 15) + 16 * (l >> 4); });
  // recompute_w_u's output staging at K = 128 bf16 (256-byte rows): writes of
  // one 8-byte piece per token, 16 tokens per pass, with and without the half
  // swap; reads of 16-byte pieces of the two heads' rows.
  add(ps, "ds_write_b64 recompute_w_u staging, half swap", kW8,
      [](int l) { return hl::otile_off(l & 15, 0, 2, 8 * (l >> 4), 256, true); });
  add(ps, "ds_write_b64 recompute_w_u staging, no half swap", kW8,
      [](int l) { return hl::otile_off(l & 15, 0, 2, 8 * (l >> 4), 256, false); });
  add(ps, "ds_read_b128 recompute_w_u staging rows", kR16,
      [](int l) { return hl::otile_chunk(l / 32, (l / 16) % 2, 2, l % 16, 256); });
  add(ps, "ds_read_b64_tr_b16 recompute_w_u [k | v] fragments", kTr,
      [](int l) { return hl::xtr_frag_off(0, 0, 16, l, 512); });
  // The DMA pipelines' swizzled chunk tiles (h_layout.h tile_off): 256-byte
  // k / w / q rows and the fused kernel's 128-byte score rows.
  for (int e0 : {0, 32})
    add(ps, "ds_read_b128 row fragments, 256-B swizzled rows, e0 " + std::to_string(e0), kR16,
        [&](int l) { return hl::row8_frag_off(16, e0, l, 256); });
  for (int e0 : {0, 16})
    add(ps, "ds_read_b64 paired fragments, 256-B swizzled rows, e0 " + std::to_string(e0), kR8,
        [&](int l) { return hl::pair_frag_off(16, e0, l, 256); });
  add(ps, "ds_read_b64_tr_b16 transposed fragments, 256-B swizzled rows", kTr,
      [](int l) { return hl::tr_frag_off(32, 16, l, 256); });
  for (int jb : {0, 1})
    add(ps, "ds_write_b64 score blocks, 128-B swizzled rows, jb " + std::to_string(jb), kW8,
        [&](int l) { return hl::pair_frag_off(48, 16 * jb, l, 128); });
  add(ps, "ds_read_b64 score pairs, 128-B swizzled rows", kR8, [](int l) { return hl::pair_frag_off(48, 32, l, 128); });
  // 16 rows of 256 bytes, lane (g, r) at chunk (q + g) ^ (r & 14): rows 2m
  // and 2m + 1 share a chunk.  The model calls this conflict-free and the
  // hardware serves it 2-way, so the model is a fit to the patterns above,
  // not the hardware's rule.
  for (int q : {0, 8})
    add(ps, "ds_read_b128 16 rows, row pairs at one chunk, q " + std::to_string(q), kR16,
        [&](int l) { return (uint32_t)(4096 + (l & 15) * 256 + (((q + (l >> 4)) ^ (l & 14)) << 4)); });
  // Minimal pairs (ds_read_b128): every lane of pass 0 but lane 1 reads one
  // base address (a broadcast), lanes 16-63 read a contiguous run elsewhere;
  // lane 1 reads (block, chunk) at 256 bytes per block, 16 bytes per chunk.
  add(ps, "b128 broadcast, all 64 lanes one address", kR16, [](int) { return 0; });
  add(ps, "b128 broadcast pass 0, rest contiguous", kR16, [](int l) { return l < 16 ? 0 : 0x8000 + (l - 16) * 16; });
  const int pairs[][4] = {{0, 0, 1, 0},  {0, 0, 2, 0},  {0, 0, 3, 0},  {0, 0, 4, 0},  {0, 0, 8, 0},
                          {0, 0, 9, 0},  {0, 0, 16, 0}, {0, 0, 17, 0}, {0, 0, 32, 0}, {0, 0, 1, 15},
                          {0, 0, 1, 1},  {0, 0, 1, 14}, {0, 0, 2, 1},  {0, 0, 3, 15}, {0, 0, 0, 1},
                          {16, 0, 17, 0}, {16, 0, 18, 0}, {16, 0, 24, 0}, {16, 0, 25, 0}, {16, 0, 17, 15},
                          {16, 0, 17, 1}, {1, 0, 3, 0},  {1, 0, 2, 0},  {0, 1, 1, 0},  {8, 0, 9, 0}};
  for (const auto& q : pairs) {
    const int b0 = q[0], c0 = q[1], b1 = q[2], c1 = q[3];
    add(ps, "b128 pair (" + std::to_string(b0) + "," + std::to_string(c0) + ") vs (" + std::to_string(b1) + "," +
                std::to_string(c1) + ")",
        kR16, [=](int l) {
          if (l >= 16) return 0x8000 + (l - 16) * 16;
          return l == 1 ? b1 * 256 + c1 * 16 : b0 * 256 + c0 * 16;
        });
  }
  return ps;
}

}  // namespace

int main(int argc, char** argv) {
  const std::vector<Pattern> ps = patterns();
  for (const Pattern& p : ps)
    for (int l = 0; l < 64; ++l)
      if (p.off[l] % kBytes[p.op] || p.off[l] + kBytes[p.op] > (uint32_t)kLdsBytes) {
        std::fprintf(stderr, "bad offset: %s lane %d at %u\n", p.name.c_str(), l, p.off[l]);
        return 1;
      }
  // --model: the model's verdicts only, no GPU (to set beside a stored run).
  if (argc > 1 && std::string(argv[1]) == "--model") {
    for (size_t i = 0; i < ps.size(); ++i) {
      const Access acc = ps[i].op <= kW16 ? kLdsWrite : kLdsRead;
      std::printf("%zu\t%s\t%d\n", i, ps[i].name.c_str(), bank_ways(ps[i].off.data(), kBytes[ps[i].op], acc));
    }
    return 0;
  }
  // --addresses: each pattern's 64 lane offsets (to fit other models to a stored run).
  if (argc > 1 && std::string(argv[1]) == "--addresses") {
    for (size_t i = 0; i < ps.size(); ++i) {
      std::printf("%zu\t%s\t%d\t%d", i, ps[i].name.c_str(), kBytes[ps[i].op], ps[i].op <= kW16 ? 1 : 0);
      for (int l = 0; l < 64; ++l) std::printf("%c%u", l ? ',' : '\t', ps[i].off[l]);
      std::printf("\n");
    }
    return 0;
  }
  uint32_t *doff = nullptr, *dout = nullptr;
  if (hipMalloc(&doff, 64 * sizeof(uint32_t)) != hipSuccess ||
      hipMalloc(&dout, kGrid * 64 * sizeof(uint32_t)) != hipSuccess) {
    std::fprintf(stderr, "hipMalloc failed\n");
    return 2;
  }
  for (size_t i = 0; i < ps.size(); ++i) {
    const Pattern& p = ps[i];
    if (hipMemcpy(doff, p.off.data(), 64 * sizeof(uint32_t), hipMemcpyHostToDevice) != hipSuccess) return 3;
    switch (p.op) {
      case kW4: lds_probe<kW4><<<kGrid, 64>>>(doff, dout); break;
      case kW8: lds_probe<kW8><<<kGrid, 64>>>(doff, dout); break;
      case kW16: lds_probe<kW16><<<kGrid, 64>>>(doff, dout); break;
      case kR4: lds_probe<kR4><<<kGrid, 64>>>(doff, dout); break;
      case kR8: lds_probe<kR8><<<kGrid, 64>>>(doff, dout); break;
      case kR16: lds_probe<kR16><<<kGrid, 64>>>(doff, dout); break;
      default: lds_probe<kTr><<<kGrid, 64>>>(doff, dout); break;
    }
    if (hipDeviceSynchronize() != hipSuccess) {
      std::fprintf(stderr, "launch %zu failed\n", i);
      return 4;
    }
    const Access acc = p.op <= kW16 ? kLdsWrite : kLdsRead;
    std::printf("%zu\t%s\t%d\n", i, p.name.c_str(), bank_ways(p.off.data(), kBytes[p.op], acc));
    std::fflush(stdout);
  }
  return 0;
}
