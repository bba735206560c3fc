// Index maps of the bf16 chunk_fwd_h pipeline (chunk tiles copied global -> LDS
// by DMA), shared by the kernel and a host-side check of the addressing.
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

}  // namespace hl
}  // namespace thm
