// Index maps of the two global -> LDS DMA pipelines (the bf16 chunk_fwd_h
// kernel of chunk_fwd_h.hip and the fused kernel of chunk_fwd_fused.hip),
// shared by the kernels and by the host-side check of their addressing
// (tests/csrc/dma_check.cpp, run by tests/test_dma_layout.py).
//
// A chunk tile is 64 rows (tokens) of `row_bytes` = 128 or 256 bytes (64 / 128
// bf16 features), stored in LDS without padding.  The 16-byte chunks of row r
// are XOR-swizzled: logical chunk q sits at physical chunk q ^ swz(r).  The
// swizzle makes the two read patterns of the kernel conflict-free per 256-byte
// pass:
//   * 16 consecutive rows (16-aligned), one 16-byte chunk each (w rows as the
//     A operand, paired order): swz takes 16 distinct values over those rows
//     (row_bytes 256), or distinct values per row parity (row_bytes 128, two
//     rows per 256 bytes);
//   * 8 consecutive rows (8-aligned), one aligned 32-byte chunk pair each
//     (ds_read_b64_tr_b16 fragments of k^T and of the u tile): swz >> 1 takes 8
//     distinct values (row_bytes 256) or 4 per row parity (row_bytes 128).
// A DMA instruction writes 1 KiB = 64 lanes x 16 bytes at consecutive physical
// chunks; lane data is fetched from the logical chunk that belongs there.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#define THM_HD __host__ __device__
#else
#define THM_HD
#endif

namespace thm {
namespace hl {

THM_HD constexpr int swz(int r, int row_bytes) {
  return row_bytes == 256 ? (((r & 7) << 1) | ((r >> 3) & 1))
                          : ((((r >> 1) & 3) << 1) | ((r >> 3) & 1));
}

// Byte offset within the tile of bf16 element e of row r.
THM_HD constexpr uint32_t tile_off(int r, int e, int row_bytes) {
  return (uint32_t)(r * row_bytes + (((e >> 3) ^ swz(r, row_bytes)) << 4) + ((e & 7) << 1));
}

// Physical chunk P of a tile (P = 16-byte slot index) holds logical row
// dma_row(P) and logical chunk dma_chunk(P).
THM_HD constexpr int dma_row(int P, int row_bytes) { return P / (row_bytes / 16); }
THM_HD constexpr int dma_chunk(int P, int row_bytes) {
  return (P % (row_bytes / 16)) ^ swz(P / (row_bytes / 16), row_bytes);
}

// Source of physical chunk P within one chunk's token block in global memory,
// rows (tokens) `tok_stride` bytes apart: a per-lane offset from the block's
// wave-uniform base (the entry points check that it fits in 32 bits).
THM_HD constexpr uint32_t dma_src_off(int P, int row_bytes, int64_t tok_stride) {
  return (uint32_t)(dma_row(P, row_bytes) * tok_stride + dma_chunk(P, row_bytes) * 16);
}

// LDS fragment reads of a swizzled tile, per lane (grp = lane / 16, li =
// lane % 16).  Each returns the byte offset the lane addresses.
//
// ds_read_b64_tr_b16 source of the 16 x 16 block at (r0, c0): lane (grp, li)
// addresses row r0 + 4 grp + li / 4, elements c0 + 4 (li % 4) .. + 3; output
// lane j of the group then holds rows r0 + 4 grp .. + 3 of column c0 + j.
THM_HD constexpr uint32_t tr_frag_off(int r0, int c0, int lane, int row_bytes) {
  return tile_off(r0 + 4 * (lane >> 4) + ((lane & 15) >> 2), c0 + 4 * (lane & 3), row_bytes);
}
// 8-byte read of half a paired-order operand: row r0 + li, elements
// e0 + 4 grp .. + 3 (the other half is the same at e0 + 16).
THM_HD constexpr uint32_t pair_frag_off(int r0, int e0, int lane, int row_bytes) {
  return tile_off(r0 + (lane & 15), e0 + 4 * (lane >> 4), row_bytes);
}
// 16-byte read of a natural-order operand: row r0 + li, elements e0 + 8 grp .. + 7.
THM_HD constexpr uint32_t row8_frag_off(int r0, int e0, int lane, int row_bytes) {
  return tile_off(r0 + (lane & 15), e0 + 8 * (lane >> 4), row_bytes);
}

// L2 prefetch of a chunk's token block: line L (64 bytes) of row
// (L / lines) % 64, lines = row_bytes / 64; indices past the block wrap.
THM_HD constexpr uint32_t l2_line_off(int L, int row_bytes, int64_t tok_stride) {
  return (uint32_t)(((L / (row_bytes / 64)) % 64) * tok_stride + (L % (row_bytes / 64)) * 64);
}

// Global stores of a 16 x 16 accumulator tile at (r0, c0) of a row-major array
// (rows `row_stride` bytes apart, `eb` bytes per element), 4 elements per lane.
// Row-quad layout (after vmem.h acc_to_row_quads): lane (grp, 4 a + b) holds
// row r0 + 4 grp + a, elements c0 + 4 b .. + 3.
THM_HD constexpr uint32_t rowquad_off(int r0, int c0, int lane, int64_t row_stride, int eb) {
  return (uint32_t)((r0 + 4 * (lane >> 4) + ((lane & 15) >> 2)) * row_stride + (c0 + 4 * (lane & 3)) * eb);
}
// Quad-transposed layout (after vmem.h quad_transpose): lane (grp, 4 m + q)
// holds row r0 + 4 grp + q, elements c0 + 4 m .. + 3.
THM_HD constexpr uint32_t quadT_off(int r0, int c0, int lane, int64_t row_stride, int eb) {
  return (uint32_t)((r0 + 4 * (lane >> 4) + (lane & 3)) * row_stride + (c0 + 4 * ((lane & 15) >> 2)) * eb);
}

// Workgroup -> (b * H + head, V-tile) of the recurrence kernels.  Workgroup i
// runs on XCD i % 8; when B * H is a multiple of 8 the V-tiles of one
// (b, head) land on one XCD (and its L2), so k, w and q are fetched from HBM
// once per (b, head).
struct BhTile {
  int64_t bh, vt;
};
THM_HD inline BhTile xcd_tile(int64_t blk, int64_t BH, int nvt) {
  if (BH % 8 == 0) {
    const int64_t xcd = blk % 8, slot = blk / 8;
    return {(slot / nvt) * 8 + xcd, slot % nvt};
  }
  return {blk / nvt, blk % nvt};
}

}  // namespace hl
}  // namespace thm
