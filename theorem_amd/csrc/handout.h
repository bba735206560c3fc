// Run-time tile hand-out of a persistent pipelined kernel (chunk_fwd_o).  (The
// fused WY kernel took 249.6-250.9 against 240.0-240.7 us at config 4 with it,
// so it keeps its fixed walk.)
//
// G workgroups stay resident and walk a sequence of tiles.  Workgroup w takes
// walk index w first; after that, thread 0 draws a ticket n from the launch's
// counter for each further tile and the workgroup takes walk index
// h_layout.h dyn_tile(G, n), until one is past the end.  Each draw is made
// one tile ahead of need (the workgroup knows its next tile while it computes
// the current one and has already drawn the one after), so the atomic's
// latency is hidden.  Workgroups on the XCDs that run slower take fewer
// tiles; a fixed walk t, t + G, ... waits for them.
//
// The counters sit in a static device array of kTileSlots slots in the kernel's
// unit, {next ticket, workgroups finished}, one slot per launch in rotation
// (next_tile_slot).  Every workgroup counts itself finished, after its own
// draws have returned; the last one resets the slot, so it is zero again for
// its next use.  Up to kTileSlots launches of one kernel may be in flight on
// a device at once (across streams) before two of them could share a slot.
// Device code names the array; host code only passes the slot index.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

#include "h_layout.h"

namespace thm {

constexpr int kTileSlots = 256;

inline uint32_t next_tile_slot() {
  static std::atomic<uint32_t> launches{0};
  return launches.fetch_add(1, std::memory_order_relaxed) % kTileSlots;
}

struct TileHandout {
  unsigned int* ticket;
  unsigned int* finished;
  uint32_t pend = 0;  // thread 0: the walk index drawn for the tile after next

  __device__ explicit TileHandout(unsigned int* slot) : ticket(slot), finished(slot + 1) {}

  // Thread 0, before the first tile: the walk indices of the second tile (to
  // *s_next, read by every thread after the next barrier) and the third.
  __device__ void start(uint32_t* s_next, int tid) {
    if (tid == 0) {
      *s_next = hl::dyn_tile(gridDim.x, atomicAdd(ticket, 1u));
      pend = hl::dyn_tile(gridDim.x, atomicAdd(ticket, 1u));
    }
  }
  // Thread 0, after every thread has read *s_next and before the barrier
  // that publishes the new value: hand on the drawn index, draw the next.
  __device__ void advance(uint32_t* s_next, int tid) {
    if (tid == 0) {
      *s_next = pend;
      pend = hl::dyn_tile(gridDim.x, atomicAdd(ticket, 1u));
    }
  }
  // Every workgroup once, at its end (also one that had no tile).
  __device__ void finish(int tid) {
    if (tid == 0) {
      asm volatile("" : : "v"(pend));  // wait for this workgroup's last draw
      if (atomicAdd(finished, 1u) == gridDim.x - 1) {
        atomicExch(ticket, 0u);
        atomicExch(finished, 0u);
      }
    }
  }
};

}  // namespace thm
