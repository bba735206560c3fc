// Compile-time layout of the two global -> LDS DMA pipelines: the bf16
// chunk_fwd_h kernel (chunk_fwd_h.hip, PCfg) and the fused h + o kernel
// (chunk_fwd_fused.hip, FCfg).  Plain constants, shared by the kernels and by
// the host-side check of their LDS layout, DMA coverage, stores and wait
// counts (tests/csrc/dma_check.cpp).
#pragma once

namespace thm {
namespace pipe {

constexpr int kBT = 64;     // chunk length (tokens)
constexpr int kTileV = 64;  // state columns per workgroup (V-tile)

// ---------------------------------------------------------------------------
// chunk_fwd_h, bf16 DMA kernel: 4 KS wavefronts; wave w = 4 kh + wq owns state
// rows [kh K / KS, (kh + 1) K / KS) and columns 16 wq .. + 15 of the V-tile.
// Per chunk each wave issues its share of the next chunk's k, w, u DMA (wave 0
// also the gates), then its v_new and h stores.
constexpr int kHKSplit = 2;  // K split
constexpr int kHStages = 2;  // DMA ring depth

template <int K, int KS, int NS, bool DELTA, bool HAS_G, bool STORE_VN>
struct PCfg {
  static constexpr int kWaves = 4 * KS;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kRowK = K * 2;                   // bytes per k / w row
  static constexpr int kTileK = kBT * kRowK;            // bytes per k / w tile
  static constexpr int kRowU = kTileV * 2;              // bytes per u row of the V-tile
  static constexpr int kTileU = kBT * kRowU;
  static constexpr int kGBytes = 1024;                  // the chunk's 64 gates (wave 0's DMA), padded
  static constexpr int kStage = kTileK * (DELTA ? 2 : 1) + kTileU + (HAS_G ? kGBytes : 0);
  static constexpr int kXBytes = (DELTA && KS == 2) ? kWaves * 4 * 64 * 16 : 0;  // P1 partials
  static constexpr int kLds = NS * kStage + kXBytes;
  static constexpr int kRows = K / KS;                  // state rows per wave
  static constexpr int KBH = kRows / 16;                // 16-row accumulator tiles per wave
  static constexpr int kKDma = kTileK / 1024 / kWaves;  // 1 KiB DMA instructions per wave per k tile
  static constexpr int kUDma = kTileU / 1024 / kWaves;
  static constexpr int kJbStore = 4 / KS;               // v_new row tiles stored per wave
  // DMA instructions per chunk: every wave's share of the k, w, u tiles, plus
  // the gate load that only wave 0 issues.
  static constexpr int kDma = kKDma * (DELTA ? 2 : 1) + kUDma;
  static constexpr int kDma0 = kDma + (HAS_G ? 1 : 0);
  static constexpr int kStores = KBH + ((DELTA && STORE_VN) ? kJbStore : 0);
  // vmcnt at the top of chunk c: after this wave's DMA of chunk c it has
  // issued NS - 1 chunks of stores and NS - 2 chunks of DMA.
  static constexpr int kWaitFirst = (NS - 2) * kDma;
  static constexpr int kWaitFirst0 = (NS - 2) * kDma0;
  static constexpr int kWaitSteady = (NS - 1) * kStores + (NS - 2) * kDma;
  static constexpr int kWaitSteady0 = (NS - 1) * kStores + (NS - 2) * kDma0;
  static_assert(KS == 1 || KS == 2, "K split");
  static_assert(NS >= 2, "at least double buffering");
  static_assert(kKDma >= 1 && kUDma >= 1, "whole DMA instructions per wave");
  static_assert(kStage % 1024 == 0, "1 KiB aligned stages");
  static_assert(kLds <= 160 * 1024, "LDS budget");
  static_assert(kWaitSteady0 <= 63, "vmcnt range");
};

// ---------------------------------------------------------------------------
// Fused h + o kernel: 8 wavefronts, state waves 0-3 and output waves 4-7, wave
// wq = w % 4 on columns 16 wq .. + 15 of the V-tile.  In chunk c the state
// waves issue the DMA of chunk c + 1's k, q and gates (in parts between P1's
// row blocks), their v_new stores of chunk c and, after the mid-chunk barrier,
// the DMA of chunk c + 2's w and u: only P1 reads w and u, so their slots in
// stage c % 2 are free from that barrier on, and those tiles get one and a half
// chunk periods to arrive.  There is no L2 prefetch: beside the early w / u
// DMA, every prefetch variant measured slower.
// The A form (FROM_A) reads the chunk's WY matrix A (64 fp32 per row) in the w
// slot, v in the u slot and beta after the gates: its P1 forms v_new =
// A (beta (v - e^g k S)), which equals u - w S, so w and u are never formed.
constexpr int kFThreads = 512;     // 4 state + 4 output wavefronts
constexpr int kFStages = 2;

template <int K, bool HAS_G, bool STORE_VN, bool FROM_A = false>
struct FCfg {
  static constexpr int kRowK = K * 2;             // bytes per k / q (/ w) row
  static constexpr int kTileK = kBT * kRowK;
  static constexpr int kRowW = FROM_A ? kBT * 4 : kRowK;  // bytes per w row, or per A row
  static constexpr int kTileW = kBT * kRowW;
  static constexpr int kRowU = kTileV * 2;        // bytes per u (v) row of the V-tile
  static constexpr int kTileU = kBT * kRowU;
  // The gate block: the chunk's 64 gates (+0), the gate factors e^{g_i}
  // (+64 floats) and e^{g_last - g_j} (+128), beta in the A form (+192).
  static constexpr bool kGates = HAS_G || FROM_A;
  static constexpr int kGBytes = 1024;
  static constexpr int kStage = 2 * kTileK + kTileW + kTileU + (kGates ? kGBytes : 0);
  static constexpr int KB = K / 16;               // 16-row state tiles per column group
  static constexpr int kPBytes = kBT * kBT * 2;   // the chunk's scores P, bf16
  static constexpr int kSBytes = 4 * (KB / 2) * 64 * 16;  // S handed over as bf16 B-operand pairs
  static constexpr int kVBytes = 4 * 2 * 64 * 16;         // v_new handed over the same way
  static constexpr int kLds = kFStages * kStage + kPBytes + kSBytes + kVBytes;
  static constexpr int kKDma = kTileK / 1024 / 4; // 1 KiB DMA instructions per state wave per k / q tile
  static constexpr int kWDma = kTileW / 1024 / 4; // ... per w (A) tile
  static constexpr int kUDma = kTileU / 1024 / 4;
  static constexpr int kWuDma = kWDma + kUDma;    // a chunk's w and u (A and v) tiles, per state wave
  static constexpr int kStores = STORE_VN ? 4 : 0;  // v_new row tiles per state wave
  // Issue schedule, in chunks of lead: chunk x's k, q and gates are DMA'd in
  // P1 of chunk x - kKqLead, its w and u after the mid-chunk barrier of chunk
  // x - kWuLead (chunks x < kWuLead in the prologue), each into stage x % 2.
  static constexpr int kKqLead = 1;
  static constexpr int kWuLead = 2;
  // Ops a state wave issues after the k / q DMA of chunk c before it waits for
  // it: from c = 1 on the v_new stores of chunk c - 1, then the w / u DMA of
  // chunk c - 1 + kWuLead (chunk c's own when kWuLead = 1: nothing after it).
  // At c = 0, the prologue's w / u DMA of chunks 1 .. kWuLead - 1.
  static constexpr int kWaitFirst = (kWuLead - 1) * kWuDma;
  static constexpr int kWaitSteady = kWuLead >= 2 ? kStores + kWuDma : 0;
  static_assert(kFStages == 2, "the wait counts assume double buffering");
  static_assert(kStage % 1024 == 0, "1 KiB aligned stages");
  static_assert(kLds <= 160 * 1024, "LDS budget");
  static_assert(kWaitSteady <= 63, "vmcnt range");
};

// ---------------------------------------------------------------------------
// chunk_fwd_h, small-grid kernel (chunk_fwd_h_small.h): NW state waves and
// NW memory waves per workgroup, a V-tile of 16 NW columns; per stage the
// padded k, w (delta form) and u tiles and the chunk's gate factors, then two
// fp32 out buffers each for h and v_new.  EB = bytes per input element: bf16
// (2) stages k and w as they are, fp32 (4) as bf16 hi and lo tiles (the
// register kernel's split), and u in its own type.
template <int K, int NW, bool DELTA, int EB = 2>
struct SCfg {
  static constexpr bool kSplit = EB == 4;
  static constexpr int kThreads = 128 * NW;
  static constexpr int kCols = 16 * NW;                // V-tile width
  static constexpr int kVE = 16 / EB;                  // input elements per 16-byte piece
  static constexpr int kKPitch = K + 8;                // bf16 elements per k / w row (16-byte pad)
  static constexpr int kUPitch = kCols + kVE;          // input elements per u / v row of the V-tile
  static constexpr int kKTileB = 64 * kKPitch * 2;     // bytes of one bf16 k / w tile
  static constexpr int kKPartB = kKTileB * (kSplit ? 2 : 1);  // k (or w): hi[, lo]
  static constexpr int kUTileB = 64 * kUPitch * EB;
  static constexpr int kGateB = 80 * 4;                // 64 factors e^{g_last - g_j}, e^{g_last}, pad
  static constexpr int kStageB = kKPartB * (DELTA ? 2 : 1) + kUTileB + kGateB;
  // Out buffers: fp32, row-major, kOutPitch floats per row.  The state waves
  // write single floats, 16 lanes of a row-quad group 4 rows apart; a pitch of
  // 4 mod 16 floats puts those 4 rows 16 banks apart (conflict-free).
  static constexpr int kOutPitch = kCols + 4;
  static constexpr int kHOutB = K * kOutPitch * 4;
  static constexpr int kVOutB = DELTA ? 64 * kOutPitch * 4 : 0;
  static constexpr int kLds = 2 * kStageB + 2 * (kHOutB + kVOutB);
  static constexpr bool kFits = kLds <= 160 * 1024;    // fp32 with K = 128 in the delta form does not
  // memory-wave loads per lane per chunk (16-byte pieces of kVE elements)
  static constexpr int kML = 64 * NW;                  // memory lanes
  static constexpr int kKCPR = K / kVE;                // pieces per k / w row
  static constexpr int kKLoads = 64 * kKCPR / kML;
  static constexpr int kUCPR = kCols / kVE;            // pieces per u row of the V-tile
  static constexpr int kULoads = 64 * kUCPR / kML;
  static_assert(EB == 2 || EB == 4, "bf16 or fp32 inputs");
  static_assert(NW == 1 || NW == 2 || NW == 4, "state waves");
  static_assert(kStageB % 16 == 0, "16-byte aligned stages");
  static_assert(64 * kKCPR % kML == 0 && kML % kKCPR == 0 && kML % kUCPR == 0, "load split");
};

}  // namespace pipe
}  // namespace thm
