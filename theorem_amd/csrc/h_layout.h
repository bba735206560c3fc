// Index maps of the two global -> LDS DMA pipelines (the bf16 chunk_fwd_h
// kernel of chunk_fwd_h.hip and the fused kernel of chunk_fwd_fused.hip),
// shared by the kernels and by the host-side check of their addressing
// (tests/csrc/dma_check.cpp, run by tests/test_dma_layout.py).
//
// A chunk tile is 64 rows (tokens) of `row_bytes` = 128 or 256 bytes (64 / 128
// bf16 features), stored in LDS without padding.  The 16-byte chunks of row r
// are XOR-swizzled: logical chunk q sits at physical chunk q ^ swz(r).  The
// swizzle serves the three read patterns of the kernels:
//   * 16 consecutive rows (16-aligned), one 16-byte chunk each (w rows as the
//     A operand, paired order, two 8-byte reads per 256-byte pass): swz takes
//     16 distinct values over those rows (row_bytes 256), or distinct values
//     per row parity (row_bytes 128, two rows per 256 bytes);
//   * 8 consecutive rows (8-aligned), one aligned 32-byte chunk pair each
//     (ds_read_b64_tr_b16 fragments of k^T and of the u tile): swz >> 1 takes 8
//     distinct values (row_bytes 256) or 4 per row parity (row_bytes 128);
//   * 16-byte reads of 16 consecutive rows at one chunk per 16-lane pass (the
//     fused kernel's score fragments and the A form's A fragments): 2-way as
//     measured on gfx950 (tests/csrc/lds_bank_probe.hip).  Freeing them (a
//     timing-only lane-order copy of the scores, a row-pair swizzle of the A
//     tile) did not speed the kernel up.
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
  return row_bytes == 256 ? ((((r & 7) ^ ((r >> 3) & 1)) << 1) | ((r >> 3) & 1))
                          : (((((r >> 1) & 3) ^ ((r >> 3) & 1)) << 1) | ((r >> 3) & 1));
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

// recompute_w_u's [k | v] tile: 64 rows of row_bytes = 2 (K + V) bytes (256,
// 384 or 512), unpadded, read only as ds_read_b64_tr_b16 fragments in the
// natural contraction order (rows k0 + 8 grp + 4 half + li / 4, elements
// c0 + 4 (li % 4)).  A 16-lane quarter reads one aligned 32-byte chunk pair
// of 4 rows; a 256-byte pass reads the pair at the same logical position in 8
// rows {r0 .. r0 + 3, r0 + 8 .. r0 + 11}.  Logical pair p of row r sits at
// p ^ xswz(r), which spreads those 8 rows over the 8 pair positions of a
// 256-byte bank window: for row_bytes a multiple of 256 xswz takes 8 distinct
// values over them; for an odd multiple of 128 (384: rows alternating between
// the two 128-byte halves of the window) it takes 4 per row parity and stays
// inside aligned groups of 4 pairs, so no row is pushed past its last pair.
// (Measured at config 4 against the padded layout below: 265 against 269 us,
// both free of bank conflicts, outputs bit-identical.)
THM_HD constexpr int xswz(int r, int row_bytes) {
  return row_bytes % 256 == 0 ? ((r & 3) | (((r >> 3) & 1) << 2)) : (((r >> 1) & 1) | (((r >> 3) & 1) << 1));
}
THM_HD constexpr uint32_t xtile_off(int r, int e, int row_bytes) {
  return (uint32_t)(r * row_bytes + (((e >> 3) ^ (xswz(r, row_bytes) << 1)) << 4) + ((e & 7) << 1));
}
// Lane address of the natural-order fragment half `half` at contraction step
// k0 (a multiple of 32) for output columns c0 .. c0 + 15.
THM_HD constexpr uint32_t xtr_frag_off(int k0, int half, int c0, int lane, int row_bytes) {
  return xtile_off(k0 + 8 * (lane >> 4) + 4 * half + ((lane & 15) >> 2), c0 + 4 * (lane & 3), row_bytes);
}

// The WY inversion's 16x16 fp32 blocks in LDS (wy_blocks.h), rows kWyPitch
// floats apart.  Under gfx950's LDS bank model (4-byte writes and reads in
// 32-lane passes over 32 banks) a pitch of 20 makes the accumulator writes
// (block_put, form_L) conflict-free and leaves block_mm's operand reads
// 2-way; no pitch makes all three conflict-free (17 left all three 2-way:
// A-builder 110.8 -> 105.5 us at config 4, fused WY 233.2 -> 231.4,
// bit-identical).
// Float offsets within a block, lane (g = lane / 16, l = lane % 16):
//   accumulator row 4 g + r, column l;  A operand row l, column 4 q + g;
//   B operand row 4 q + g, column l.
constexpr int kWyPitch = 20;
THM_HD constexpr int wy_put_off(int lane, int r) { return (4 * (lane >> 4) + r) * kWyPitch + (lane & 15); }
THM_HD constexpr int wy_a_off(int lane, int q) { return (lane & 15) * kWyPitch + 4 * q + (lane >> 4); }
THM_HD constexpr int wy_b_off(int lane, int q) { return (4 * q + (lane >> 4)) * kWyPitch + (lane & 15); }

// recompute_w_u's output staging tile: the w (or u) rows of the tile's 64
// tokens x hp heads in their global order (physical row t hp + head), each
// row_bytes = n eb (128 to 512 bytes: 64 or 128 features, bf16 or fp32),
// unpadded.  The MFMA result of a lane is 4 consecutive features of one
// token, written as one 8-byte (bf16) or 16-byte (fp32) piece.  LDS writes go
// in passes of 128 bytes over 32 banks (16 lanes of 8 bytes, 8 of 16); a pass
// holds 16 (8) consecutive tokens of one head at one logical 16-byte chunk
// and, for 8-byte pieces, one half of it.  Logical chunk q of token t sits at
// q ^ (t & 7), and with half_swz the two 8-byte halves of the chunk swap for
// t & 8: the pass then covers 16 distinct 8-byte slots (8 distinct chunks) of
// a 128-byte window, conflict-free.  The global stores read whole 16-byte
// chunks of consecutive physical rows (reads go in passes of 16 lanes over
// 128 banks: one row of 256 or 512 bytes or two of 128, conflict-free) and
// swap the halves back where otile_half_swapped.
THM_HD constexpr uint32_t otile_chunk(int t, int head, int hp, int q, int row_bytes) {
  return (uint32_t)((t * hp + head) * row_bytes + ((q ^ (t & 7)) << 4));
}
THM_HD constexpr bool otile_half_swapped(int t, bool half_swz) { return half_swz && ((t >> 3) & 1); }
THM_HD constexpr uint32_t otile_off(int t, int head, int hp, int byte, int row_bytes, bool half_swz) {
  return otile_chunk(t, head, hp, byte >> 4, row_bytes) +
         (uint32_t)((byte & 15) ^ (otile_half_swapped(t, half_swz) ? 8 : 0));
}

// chunk_fwd_o's register-staged v, h and k tiles are padded instead of
// swizzled: a fragment address is then one per-lane base plus a constant,
// folded into the LDS instruction's offset field, where an XOR swizzle needs
// a register per fragment (chunk_fwd_o's pipelined kernel, at 252 VGPRs,
// spilled with it).  Rows are `pitch` bytes apart.
//   * ds_read_b64_tr_b16 fragments read one aligned 32-byte chunk pair from
//     each of 8 rows per 256-byte pass.  In the paired contraction order those
//     are 8 consecutive rows, which land in 8 distinct 32-byte bank groups
//     when pitch / 32 is odd: tr_pitch.  In the natural order they are rows
//     r0 .. r0 + 3 and r0 + 8 .. r0 + 11, which no linear pitch separates, so
//     natural-order tiles store logical row r at physical row nat_row(r) (bits
//     2 and 3 of r swapped): each pass then reads 8 consecutive physical rows.
//   * 16-byte row reads of 16 consecutive rows (chunk_fwd_o's k fragments)
//     are served 16 lanes at a time over 128 banks (512 bytes), as measured
//     on gfx950: a pitch of row_bytes + 32 puts the 16 rows on distinct
//     16-byte positions of that window (a 16-byte pad measured 0.11 conflict
//     cycles per access in chunk_fwd_o; at V = 64 it also makes the
//     transposed reads of the h and v tiles 2-way).
THM_HD constexpr int tr_pitch(int row_bytes) { return row_bytes + 32; }
// The fused WY kernel's [k | v] tile (64 rows of n = K + V bf16): natural-order
// transposed reads in its products and 16-byte row reads (form_L's k
// fragments) of 16 consecutive rows, so the natural-order layout above, which
// serves both without bank conflicts.
THM_HD constexpr int wy_tile_pitch(int n) { return tr_pitch(2 * n); }
THM_HD constexpr int nat_row(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }
// Element e of row r: plain (paired-order and row-read tiles) and with the
// natural-order row permutation.
THM_HD constexpr uint32_t ptile_off(int r, int e, int pitch) { return (uint32_t)(r * pitch + 2 * e); }
THM_HD constexpr uint32_t ntile_off(int r, int e, int pitch) { return (uint32_t)(nat_row(r) * pitch + 2 * e); }
// ds_read_b64_tr_b16 sources of the 16 x 16 block of output columns c0 ..
// c0 + 15: lane (grp, li) addresses elements c0 + 4 (li % 4) .. + 3 of row
//   paired order:  r0 + 4 grp + li / 4             (r0 = 32 s + 16 half)
//   natural order: k0 + 8 grp + 4 half + li / 4    (k0 = 32 s)
// and output lane j of the group receives rows base .. base + 3 of column c0 + j.
THM_HD constexpr uint32_t ptr_frag_off(int r0, int c0, int lane, int pitch) {
  return ptile_off(r0 + 4 * (lane >> 4) + ((lane & 15) >> 2), c0 + 4 * (lane & 3), pitch);
}
// (For k0 a multiple of 16, nat_row(k0 + 4 half + x) = k0 + 8 half + nat_row(x)
// for the lane part x = 8 grp + li / 4: written so, the address is one
// per-lane base plus a constant.)
THM_HD constexpr uint32_t ntr_frag_off(int k0, int half, int c0, int lane, int pitch) {
  return (uint32_t)((k0 + 8 * half + nat_row(8 * (lane >> 4) + ((lane & 15) >> 2))) * pitch + 2 * (c0 + 4 * (lane & 3)));
}
// 16-byte natural-order row read: row r0 + li, elements e0 + 8 grp .. + 7.
THM_HD constexpr uint32_t prow8_frag_off(int r0, int e0, int lane, int pitch) {
  return ptile_off(r0 + (lane & 15), e0 + 8 * (lane >> 4), pitch);
}

// XCD-aware order of the tile-parallel kernels' [B, T / 64, H] tile grid.
// Workgroup i runs on XCD i % 8, each XCD with its own L2.  Launch index t
// maps to a tile index such that, when the (b, chunk) count BNT is a multiple
// of 8, the H heads of one (b, chunk) all get launch indices of one residue
// mod 8 (one XCD): per-token arrays laid out [B, T, H] (beta, g: one cache
// line holds the values of 16 or 32 heads of a token) are then fetched into
// one L2 instead of eight.  Otherwise it is the identity.  A bijection of
// [0, BNT H).
THM_HD inline uint32_t xcd_tile_order(uint32_t t, int64_t H, int64_t BNT) {
  if (BNT % 8 != 0) return t;
  const uint32_t h = (uint32_t)H, slot = t >> 3, sq = slot / h;
  return (sq * 8u + (t & 7u)) * h + (slot - sq * h);
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

// Small-grid chunk_fwd_h kernel (chunk_fwd_h_small.h).  Memory lane m of ml
// loads 16-byte pieces of e elements (8 bf16 or 4 fp32) of a [64 x n] tile
// (k, w: n = K; u: n = the V-tile width): its piece it is row
// spiece_row(m, it, n, ml, e), elements spiece_col(m, n, e) .. + e - 1.
THM_HD constexpr int spiece_row(int m, int it, int n, int ml, int e = 8) { return m / (n / e) + it * (ml / (n / e)); }
THM_HD constexpr int spiece_col(int m, int n, int e = 8) { return (m % (n / e)) * e; }
// Out buffer (fp32, row-major, `pitch` floats per row): lane `lane` of state
// wave wq writes rows 16 blk + 4 (lane / 16) + r (r = 0..3) of column
// 16 wq + lane % 16, one float each.
THM_HD constexpr int sout_put(int blk, int r, int lane, int wq, int pitch) {
  return (16 * blk + 4 * (lane >> 4) + r) * pitch + 16 * wq + (lane & 15);
}
// Memory piece p of an out buffer of `cols` columns: row sout_row, columns
// sout_col .. + 3 (one 16-byte block).
THM_HD constexpr int sout_row(int p, int cols) { return p / (cols / 4); }
THM_HD constexpr int sout_col(int p, int cols) { return 4 * (p % (cols / 4)); }

// chunk_fwd_o's pipelined kernel.
//
// Walk: sequence index t = cq (B H) + b H + hh visits tile (b, chunk
// NT - 1 - cq, head hh): head fastest, chunks in descending order.
// Workgroups take walk indices dynamically: workgroup w first takes t = w,
// then t = dyn_tile(G, n) for each ticket n = 0, 1, ... it draws from the
// launch's counter (G = the grid size), until a t is past the end.  A
// workgroup on a slower XCD so takes fewer tiles.
struct DescWalk {
  uint32_t cq, b, hh;
};
THM_HD inline DescWalk desc_walk_at(uint32_t t, uint32_t B, uint32_t H) {
  const uint32_t bh = B * H, cq = t / bh, r = t - cq * bh, b = r / H;
  return {cq, b, r - b * H};
}
THM_HD constexpr uint32_t dyn_tile(uint32_t grid, uint32_t ticket) { return grid + ticket; }
// Loads of one tile, byte offsets = a per-lane part (loop-invariant, 32-bit)
// plus a wave-uniform step per load `it` (256 threads):
//   h [K x V] fp32: thread tid's load it is row tid / (V / 4) + it 256 / (V / 4),
//     elements 4 (tid % (V / 4)) .. + 3;
//   a [64 x n] bf16 token block (v: n = V, k: n = K; tokens `row_elems`
//     elements apart): token tid / (n / 8) + it 256 / (n / 8), elements
//     8 (tid % (n / 8)) .. + 7;
//   q: lane (i, grp) reads token i, elements 32 s + 8 grp .. + 7 (step 64 s bytes).
THM_HD constexpr uint32_t o_h_lane(int tid, int V) {
  return ((uint32_t)(tid / (V / 4)) * (uint32_t)V + (uint32_t)(tid % (V / 4)) * 4u) * 4u;
}
THM_HD constexpr int64_t o_h_step(int it, int V) { return (int64_t)it * (256 / (V / 4)) * V * 4; }
THM_HD constexpr uint32_t o_blk_lane(int tid, int n, int64_t row_elems) {
  return ((uint32_t)(tid / (n / 8)) * (uint32_t)row_elems + (uint32_t)(tid % (n / 8)) * 8u) * 2u;
}
THM_HD constexpr int64_t o_blk_step(int it, int n, int64_t row_elems) {
  return (int64_t)it * (256 / (n / 8)) * row_elems * 2;
}
THM_HD constexpr uint32_t o_q_lane(int i, int grp, int64_t row_elems) {
  return ((uint32_t)i * (uint32_t)row_elems + 8u * (uint32_t)grp) * 2u;
}

}  // namespace hl
}  // namespace thm
