"""Host-side check of the DMA pipelines' addressing (CPU).

The bf16 chunk_fwd_h kernel and the fused h + o kernel copy chunk tiles
global -> LDS with hand-built 32-bit lane offsets, read them back through an
XOR swizzle and wait for them with hand-counted vmcnt values; the small-grid
chunk_fwd_h kernel stages its tiles and hands h and v_new between its waves
through LDS buffers whose layout it shares with the checker; chunk_fwd_o's
pipelined kernel hands out its tiles at run time (dyn_tile) and loads them with
32-bit per-lane offsets.  A slip there
would fault the GPU or race rather than fail a numerical test, so
tests/csrc/dma_check.cpp evaluates the very index functions and layout
constants the kernels use (theorem_amd/csrc/h_layout.h, pipe_cfg.h) on the
host: DMA coverage and global bounds, read/write consistency of the swizzle,
bank conflicts, store coverage and the wait counts.  The tile-load addressing
it checks replaces kernels/chunk_fwd_h/kernel.py:103-114 (Triton block
pointers) and the fused kernel's loads of kernels/chunk_fwd_o/kernel.py:94-136.

The mutation tests plant plausible slips in copies of the headers
and require the checker to fail on each.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "theorem_amd" / "csrc"
SRC = ROOT / "tests" / "csrc" / "dma_check.cpp"

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")


def _build_and_run(tmp: Path, include_first: Path | None = None) -> subprocess.CompletedProcess:
    exe = tmp / "dma_check"
    inc = ([f"-I{include_first}"] if include_first else []) + [f"-I{CSRC}"]
    subprocess.run(["g++", "-std=c++17", "-O0", "-Wall", *inc, str(SRC), "-o", str(exe)], check=True,
                   capture_output=True, text=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)


def test_dma_layout_check_passes(tmp_path):
    r = _build_and_run(tmp_path)
    assert r.returncode == 0 and "dma_check: ok" in r.stdout, r.stdout + r.stderr


# (header, text in it, planted replacement, what the slip is)
MUTATIONS = [
    ("h_layout.h", "return (P % (row_bytes / 16)) ^ swz(P / (row_bytes / 16), row_bytes);",
     "return ((P + 1) % (row_bytes / 16)) ^ swz(P / (row_bytes / 16), row_bytes);",
     "dma_chunk: chunk index off by one"),
    ("h_layout.h", "return (P % (row_bytes / 16)) ^ swz(P / (row_bytes / 16), row_bytes);",
     "return (P % (row_bytes / 16)) ^ swz(P / (row_bytes / 16) + 1, row_bytes);",
     "dma_chunk: swizzle of the next row"),
    ("h_layout.h", "(((e >> 3) ^ swz(r, row_bytes)) << 4)",
     "(((e >> 3) ^ swz(r + 1, row_bytes)) << 4)",
     "tile_off: swizzle of the next row"),
    ("h_layout.h", "return (uint32_t)(r * row_bytes + (((e >> 3) ^ swz(r, row_bytes)) << 4) + ((e & 7) << 1));",
     "return (uint32_t)(r * row_bytes + (((e >> 3) ^ swz(r, row_bytes)) << 4) + (((e + 1) & 7) << 1));",
     "tile_off: element off by one within the chunk"),
    ("h_layout.h", "+ (((e >> 3) ^ (xswz(r, row_bytes) << 1)) << 4) + ((e & 7) << 1));",
     "+ (((e >> 3) ^ (xswz(r, row_bytes) << 1)) << 4) + (((e + 1) & 7) << 1));",
     "xtile_off: element off by one within the chunk"),
    ("h_layout.h", "((((r & 7) ^ ((r >> 3) & 1)) << 1) | ((r >> 3) & 1))",
     "((((r & 7) ^ ((r >> 3) & 1)) << 1) | ((r >> 2) & 1))",
     "swz: wrong row bit (bank conflicts)"),
    ("h_layout.h", "return tile_off(r0 + 4 * (lane >> 4) + ((lane & 15) >> 2), c0 + 4 * (lane & 3), row_bytes);",
     "return tile_off(r0 + 4 * (lane >> 4) + ((lane & 15) >> 2), c0 + 4 * ((lane + 1) & 3), row_bytes);",
     "tr_frag_off: column group of the neighbouring lane"),
    ("h_layout.h", "return (uint32_t)(dma_row(P, row_bytes) * tok_stride + dma_chunk(P, row_bytes) * 16);",
     "return (uint32_t)((dma_row(P, row_bytes) + 1) * tok_stride + dma_chunk(P, row_bytes) * 16);",
     "dma_src_off: next token row"),
    ("h_layout.h", "(c0 + 4 * (lane & 3)) * eb);",
     "(c0 + 4 * (lane & 3) + 1) * eb);",
     "rowquad_off: store column off by one"),
    ("h_layout.h", "return {(slot / nvt) * 8 + xcd, slot % nvt};",
     "return {(slot / nvt) * 8, slot % nvt};",
     "xcd_tile: XCD index dropped"),
    ("h_layout.h", "? ((r & 3) | (((r >> 3) & 1) << 2))",
     "? ((r & 3) | (((r >> 2) & 1) << 2))",
     "xswz: wrong row bit (bank conflicts in recompute_w_u)"),
    ("h_layout.h", ": (((r >> 1) & 1) | (((r >> 3) & 1) << 1));",
     ": (((r >> 1) & 1) | (((r >> 3) & 1) << 2));",
     "xswz: a pair pushed past a 384-byte row"),
    ("h_layout.h", "THM_HD constexpr int tr_pitch(int row_bytes) { return row_bytes + 32; }",
     "THM_HD constexpr int tr_pitch(int row_bytes) { return row_bytes + 16; }",
     "tr_pitch: 16-byte pad (bank conflicts in the transposed reads)"),
    ("h_layout.h", "return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);",
     "return r;",
     "nat_row: natural-order rows not permuted (bank conflicts)"),
    ("h_layout.h", "return (uint32_t)((k0 + 8 * half + nat_row(8 * (lane >> 4) + ((lane & 15) >> 2))) * pitch",
     "return (uint32_t)((k0 + 4 * half + nat_row(8 * (lane >> 4) + ((lane & 15) >> 2))) * pitch",
     "ntr_frag_off: half offset not permuted with the rows"),
    ("pipe_cfg.h", "static constexpr int kWaitSteady = (NS - 1) * kStores + (NS - 2) * kDma;",
     "static constexpr int kWaitSteady = (NS - 1) * kStores + (NS - 2) * kDma + 1;",
     "chunk_fwd_h: steady-state wait one op too loose"),
    ("pipe_cfg.h", "static constexpr int kWaitSteady = kWuLead >= 2 ? kStores + kWuDma : 0;",
     "static constexpr int kWaitSteady = kWuLead >= 2 ? kStores + kWuDma - 1 : 0;",
     "fused: steady-state wait one op too tight"),
    ("pipe_cfg.h", "static constexpr int kWaitFirst = (kWuLead - 1) * kWuDma;",
     "static constexpr int kWaitFirst = (kWuLead - 1) * kWuDma + 1;",
     "fused: first wait one op too loose"),
    ("pipe_cfg.h", "  static constexpr int kWuLead = 2;", "  static constexpr int kWuLead = 3;",
     "fused: w / u DMA three chunks ahead (overwrites a slot still in use)"),
    ("pipe_cfg.h", "  static constexpr int kKqLead = 1;", "  static constexpr int kKqLead = 2;",
     "fused: k / q DMA two chunks ahead (overwrites a slot still in use)"),
    ("h_layout.h", "THM_HD constexpr int spiece_row(int m, int it, int n, int ml, int e = 8) { return m / (n / e) + it * (ml / (n / e)); }",
     "THM_HD constexpr int spiece_row(int m, int it, int n, int ml, int e = 8) { return m / (n / e) + it * (ml / (2 * n / e)); }",
     "small chunk_fwd_h: load pieces at the wrong row stride"),
    ("h_layout.h", "  return (16 * blk + 4 * (lane >> 4) + r) * pitch + 16 * wq + (lane & 15);",
     "  return (16 * blk + 4 * (lane >> 4) + r) * pitch + 16 * wq + (lane & 7);",
     "small chunk_fwd_h: out-buffer column of half the lanes"),
    ("h_layout.h", "THM_HD constexpr int sout_col(int p, int cols) { return 4 * (p % (cols / 4)); }",
     "THM_HD constexpr int sout_col(int p, int cols) { return 4 * (p % (cols / 8)); }",
     "small chunk_fwd_h: out-buffer pieces miss half the columns"),
    ("pipe_cfg.h", "  static constexpr int kOutPitch = kCols + 4;",
     "  static constexpr int kOutPitch = kCols;",
     "small chunk_fwd_h: out-buffer rows unpadded (bank conflicts)"),
    ("h_layout.h", "THM_HD constexpr int wy_tile_pitch(int n) { return tr_pitch(2 * n); }",
     "THM_HD constexpr int wy_tile_pitch(int n) { return 2 * n + 16; }",
     "fused WY tile: 16-byte row pad (conflicts in the transposed reads)"),
    ("h_layout.h", "  return (sq * 8u + (t & 7u)) * h + (slot - sq * h);",
     "  return (sq * 8u + (t & 7u)) * h + (slot - sq * h) / 2;",
     "xcd_tile_order: head index halved (not a bijection)"),
    ("h_layout.h", "const uint32_t bh = B * H, cq = t / bh, r = t - cq * bh, b = r / H;",
     "const uint32_t bh = B * H, cq = t / bh, r = t - cq * bh, b = r / (H + 1);",
     "chunk_fwd_o walk: batch index from the wrong divisor"),
    ("h_layout.h", "THM_HD constexpr uint32_t dyn_tile(uint32_t grid, uint32_t ticket) { return grid + ticket; }",
     "THM_HD constexpr uint32_t dyn_tile(uint32_t grid, uint32_t ticket) { return grid + ticket - 1; }",
     "chunk_fwd_o hand-out: first ticket repeats the last workgroup's own tile"),
    ("h_layout.h", "THM_HD constexpr uint32_t dyn_tile(uint32_t grid, uint32_t ticket) { return grid + ticket; }",
     "THM_HD constexpr uint32_t dyn_tile(uint32_t grid, uint32_t ticket) { return grid + ticket + 1; }",
     "chunk_fwd_o hand-out: a tile skipped"),
    ("handout.h", "if (Ops::add(finished, 1u) == grid - 1) {", "if (Ops::add(finished, 1u) == grid - 2) {",
     "chunk_fwd_o hand-out: slot reset before the last workgroup is done"),
    ("handout.h", "    const uint32_t n = draw(wg);\n    pend = draw(n);", "    const uint32_t n = draw(wg);\n    pend = n;",
     "chunk_fwd_o hand-out: start draws one ticket for two tiles"),
    ("handout.h", ": prev + grid; }", ": prev + grid + 1; }",
     "chunk_fwd_o fixed walk (graph capture): a stride past G skips tiles"),
    ("handout.h", "      Ops::exch(finished, 0u);\n", "",
     "chunk_fwd_o hand-out: finished count not reset for the slot's next launch"),
    ("h_layout.h", "(uint32_t)(tid % (n / 8)) * 8u) * 2u;", "(uint32_t)(tid % (n / 8)) * 4u) * 2u;",
     "chunk_fwd_o: v / k lane offset at half the element stride"),
    ("h_layout.h", "return (int64_t)it * (256 / (V / 4)) * V * 4; }", "return (int64_t)it * (256 / (V / 4)) * V * 2; }",
     "chunk_fwd_o: h load step at half the row stride"),
    ("h_layout.h", "return half_swz && ((t >> 3) & 1); }", "return false; }",
     "recompute_w_u output staging: no half swap (8-byte writes 2-way)"),
    ("h_layout.h", "constexpr int kWyPitch = 20;", "constexpr int kWyPitch = 17;",
     "WY blocks: pitch 17 (2-way accumulator writes)"),
    ("h_layout.h", "constexpr int kWyPitch = 20;", "constexpr int kWyPitch = 16;",
     "WY blocks: pitch 16 (4-way A operand reads)"),
    ("h_layout.h", "return half_swz && ((t >> 3) & 1); }", "return half_swz && ((t >> 2) & 1); }",
     "recompute_w_u output staging: half swap by the wrong token bit"),
    ("h_layout.h", "return (uint32_t)((t * hp + head) * row_bytes + ((q ^ (t & 7)) << 4));",
     "return (uint32_t)((head * 64 + t) * row_bytes + ((q ^ (t & 7)) << 4));",
     "recompute_w_u output staging: head-major rows (16-byte reads 2-way at 128-byte rows)"),
    ("h_layout.h", "return (uint32_t)((t * hp + head) * row_bytes + ((q ^ (t & 7)) << 4));",
     "return (uint32_t)((t * hp + head) * row_bytes + ((q ^ (t & 3)) << 4));",
     "recompute_w_u output staging: chunk swizzle over 4 tokens"),
]


@pytest.mark.parametrize("header,old,new,what", MUTATIONS, ids=[m[3] for m in MUTATIONS])
def test_dma_layout_check_catches_planted_slip(tmp_path, header, old, new, what):
    text = (CSRC / header).read_text()
    assert text.count(old) == 1, f"mutation site not found in {header}: {old}"
    mut = tmp_path / "mut"
    mut.mkdir()
    for h in ("h_layout.h", "pipe_cfg.h", "handout.h"):
        (mut / h).write_text((CSRC / h).read_text())
    (mut / header).write_text(text.replace(old, new))
    r = _build_and_run(tmp_path, include_first=mut)
    assert r.returncode != 0, f"planted slip not caught ({what}):\n{r.stdout}{r.stderr}"
