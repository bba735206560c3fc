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
// unit, {next ticket, workgroups finished}.  Every workgroup counts itself
// finished, after its own draws have returned; the last one resets the slot,
// so it is zero again for its next use.  Device code names the array; host
// code only passes the slot index.
//
// Slot rules (TileSlots below, on the host):
//   * a slot is given to a launch only when its previous launch is known to
//     be complete: each slot has an event, recorded on the launch's stream
//     right after the launch, and is taken only once that event has
//     completed.  Launches in flight on any streams therefore never share a
//     slot; with all slots busy a launch takes the fixed walk;
//   * a launch on a stream that is being captured into a graph takes the
//     fixed walk (kNoTileSlot) and touches no counter, so a captured graph
//     holds no state and may be replayed any number of times, on any streams,
//     also concurrently;
//   * the fixed walk processes the same tiles with the same arithmetic, so
//     the output is the same either way.
//
// HandoutCore holds the protocol with the atomics as a hook (Ops), so the
// host check (tests/csrc/dma_check.cpp) drives this same code through
// interleaved workgroups, the reset and slot reuse included.
#pragma once

#include <stdint.h>

#include "h_layout.h"

#ifdef __HIPCC__
#include <hip/hip_runtime.h>

#include <mutex>
#endif

namespace thm {

constexpr int kTileSlots = 256;
constexpr uint32_t kNoTileSlot = 0xffffffffu;  // the launch takes the fixed walk

// The protocol of one workgroup (run by its thread 0).  `slot` = {ticket,
// finished} of the launch, or null for the fixed walk.  Ops::add returns the
// old value; Ops::wait(v) returns once v (an earlier add's result) is there.
template <class Ops>
struct HandoutCore {
  unsigned int* ticket;
  unsigned int* finished;
  uint32_t grid;
  uint32_t pend = 0;  // the walk index drawn for the tile after next

  THM_HD HandoutCore(unsigned int* slot, uint32_t grid_)
      : ticket(slot), finished(slot ? slot + 1 : nullptr), grid(grid_) {}

  THM_HD uint32_t draw(uint32_t prev) { return ticket ? hl::dyn_tile(grid, Ops::add(ticket, 1u)) : prev + grid; }
  // Before the first tile (walk index `wg`, the workgroup's index): returns
  // the walk index of the second tile and draws the third.
  THM_HD uint32_t start(uint32_t wg) {
    const uint32_t n = draw(wg);
    pend = draw(n);
    return n;
  }
  // After a tile: returns the walk index drawn before, draws the next one.
  THM_HD uint32_t advance() {
    const uint32_t n = pend;
    pend = draw(n);
    return n;
  }
  // Once per workgroup, at its end (also one that had no tile).  The last
  // workgroup of the launch resets the slot and returns true.
  THM_HD bool finish() {
    if (!ticket) return false;
    Ops::wait(pend);  // this workgroup's last draw has returned
    if (Ops::add(finished, 1u) == grid - 1) {
      Ops::exch(ticket, 0u);
      Ops::exch(finished, 0u);
      return true;
    }
    return false;
  }
};

#ifdef __HIPCC__
struct DeviceAtomics {
  __device__ static unsigned int add(unsigned int* p, unsigned int v) { return atomicAdd(p, v); }
  __device__ static void exch(unsigned int* p, unsigned int v) { atomicExch(p, v); }
  __device__ static void wait(uint32_t v) { asm volatile("" : : "v"(v)); }
};

// The kernel side: thread 0 runs the protocol; the walk index of the next
// tile goes through *s_next (LDS) to the other threads.
struct TileHandout {
  HandoutCore<DeviceAtomics> core;

  __device__ TileHandout(unsigned int (*slots)[2], uint32_t slot)
      : core(slot == kNoTileSlot ? nullptr : slots[slot], gridDim.x) {}
  // Before the first tile: the walk index of the second tile to *s_next, read
  // by every thread after the next barrier.
  __device__ void start(uint32_t* s_next, int tid) {
    if (tid == 0) *s_next = core.start(blockIdx.x);
  }
  // After every thread has read *s_next and before the barrier that
  // publishes the new value.
  __device__ void advance(uint32_t* s_next, int tid) {
    if (tid == 0) *s_next = core.advance();
  }
  __device__ void finish(int tid) {
    if (tid == 0) core.finish();
  }
};

// Host: which slot a launch may use (the rules above).  One table per device.
class TileSlots {
 public:
  // A slot for a launch on `stream` of the current device, or kNoTileSlot.
  uint32_t acquire(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
      (void)hipGetLastError();
      return kNoTileSlot;
    }
    if (st != hipStreamCaptureStatusNone) return kNoTileSlot;
    Dev* d = dev();
    if (!d) return kNoTileSlot;
    std::lock_guard<std::mutex> lock(d->m);
    for (int tries = 0; tries < 4; ++tries) {
      const uint32_t i = d->next++ % kTileSlots;
      if (d->busy[i]) continue;
      if (!d->ev[i] && hipEventCreateWithFlags(&d->ev[i], hipEventDisableTiming) != hipSuccess) {
        d->ev[i] = nullptr;
        (void)hipGetLastError();
        return kNoTileSlot;
      }
      // Relaxed capture mode for the query: another thread's capture in
      // global mode must not see it as an unsafe call.
      hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
      const bool exch = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
      const hipError_t q = hipEventQuery(d->ev[i]);
      if (exch) (void)hipThreadExchangeStreamCaptureMode(&mode);
      if (q == hipSuccess) {
        d->busy[i] = true;
        return i;
      }
      (void)hipGetLastError();  // hipErrorNotReady: the slot's launch is in flight
    }
    return kNoTileSlot;
  }
  // After the launch (launched = it was enqueued): the slot's event is
  // recorded behind it on `stream` and the slot is free to be checked again.
  // A slot whose event cannot be recorded stays busy for good.
  void release(uint32_t slot, hipStream_t stream, bool launched) {
    if (slot == kNoTileSlot) return;
    Dev* d = dev();
    if (!d) return;
    std::lock_guard<std::mutex> lock(d->m);
    if (launched && hipEventRecord(d->ev[slot], stream) != hipSuccess) {
      (void)hipGetLastError();
      return;
    }
    d->busy[slot] = false;
  }

 private:
  struct Dev {
    std::mutex m;
    hipEvent_t ev[kTileSlots] = {};
    bool busy[kTileSlots] = {};
    uint32_t next = 0;
  };
  static constexpr int kMaxDevices = 64;
  Dev devs_[kMaxDevices];
  Dev* dev() {
    int id = 0;
    if (hipGetDevice(&id) != hipSuccess || id < 0 || id >= kMaxDevices) return nullptr;
    return &devs_[id];
  }
};
#endif

}  // namespace thm
