// Tiling arithmetic shared by the kernels (device) and the launch planner (host).
//
// The kernels and the exported plan/coverage functions call the same inline
// functions, so a CPU test of the coverage function checks the mapping the GPU
// actually runs: every output written by exactly one (workgroup, tile, wave,
// slot), every weight row and K chunk in bounds.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define FTK_HD __host__ __device__ __forceinline__
#else
#define FTK_HD inline
#endif

namespace ftk {

constexpr int kWaves = 4;           // waves per workgroup
constexpr int kThreads = 64 * kWaves;

enum Epilogue : int {
  EPI_STORE = 0,   // y[m, n] = bf16(sum)
  EPI_SWIGLU = 1,  // y[m, j] = swiglu(sum(gate row j), sum(up row I + j))
  EPI_ARGMAX = 2,  // logits (optional) + greedy id per input row
};

// ---- M <= 4: HBM-streaming GEMV (one wave owns whole weight rows) --------

// Outputs one row group produces per tile: RPW rows, or RPW/2 gate/up pairs.
FTK_HD int gemv_per_wave(int epi, int rpw) { return epi == EPI_SWIGLU ? rpw / 2 : rpw; }

// Output columns: N (store / argmax) or I = N / 2 (SwiGLU pairs).
FTK_HD int gemv_outputs(int epi, int n_rows) { return epi == EPI_SWIGLU ? n_rows / 2 : n_rows; }

// Row groups per workgroup: the waves in groups of KW waves that split K (a
// workgroup is 4 waves, or KW waves when KW > 4: one group).
FTK_HD int gemv_groups(int kw) { return kw > kWaves ? 1 : kWaves / kw; }

FTK_HD int gemv_tiles(int epi, int n_rows, int rpw, int kw) {
  const int per_tile = gemv_groups(kw) * gemv_per_wave(epi, rpw);
  return (gemv_outputs(epi, n_rows) + per_tile - 1) / per_tile;
}

// Output column of (tile, row group, slot).
FTK_HD int gemv_output(int tile, int group, int slot, int per_group, int groups) {
  return (tile * groups + group) * per_group + slot;
}

// Weight row feeding output ``col``: the row itself, or for SwiGLU the gate row
// (half 0) or the up row I + col (half 1) of cat(W_gate, W_up) (engine/layers.py:92-95).
FTK_HD int gemv_weight_row(int epi, int col, int half, int n_rows) {
  return epi == EPI_SWIGLU ? col + half * (n_rows / 2) : col;
}

// ---- M <= 4 with K = 512 C KW: the STREAM kind (x slice in registers) ------
// Same tiles, row groups and weight rows as the GEMV kind above. Workgroup b
// walks tiles b, b + grid, ... (at most kStreamMaxTiles of them) and lane l of
// wave kw of a row group owns the K chunks (j KW + kw) 64 + l, j < C.

constexpr int kStreamMaxTiles = 8;  // tiles per workgroup: their wave totals wait in LDS

// 16-byte chunks per lane per weight row (C), or 0 when K is not 512 C KW.
FTK_HD int stream_chunks(int k, int kw) { return (kw < 1 || k % (512 * kw)) ? 0 : k / (512 * kw); }

// Waves per STREAM workgroup: 4, or KW when one row group needs more (KW = 8).
FTK_HD int stream_waves(int kw) { return kw > kWaves ? kw : kWaves; }

// Largest M the STREAM kind takes: M <= 4 run exact-size kernels; 5..8 run the
// 8-row kernel with the missing rows zero.
constexpr int kStreamMaxRows = 8;

// ---- M >= 4: BF16 MFMA skinny GEMM (T subtiles of 16 weight rows per workgroup)

constexpr int kMfmaK = 32;          // K per MFMA step (v_mfma_f32_16x16x32_bf16)

// Outputs one workgroup produces: 16 T rows, or 8 T gate/up pairs.
FTK_HD int mfma_out_per_tile(int epi, int t) { return epi == EPI_SWIGLU ? 8 * t : 16 * t; }

FTK_HD int mfma_tiles(int epi, int n_rows, int t) {
  const int per = mfma_out_per_tile(epi, t);
  return (gemv_outputs(epi, n_rows) + per - 1) / per;
}

// Weight row that lane ``li`` (0..15) of subtile ``sub`` reads in ``tile``, clamped in bounds.
// SwiGLU: subtiles [0, T/2) are gate rows, [T/2, T) the matching up rows (cat(W_gate, W_up)).
FTK_HD int mfma_weight_row(int epi, int tile, int sub, int li, int n_rows, int t) {
  if (epi == EPI_SWIGLU) {
    const int half = n_rows / 2;
    const int up = sub >= t / 2 ? 1 : 0;
    const int col = tile * 8 * t + (sub - up * (t / 2)) * 16 + li;
    return (col < half ? col : half - 1) + up * half;
  }
  const int r = tile * 16 * t + sub * 16 + li;
  return r < n_rows ? r : n_rows - 1;
}

// ---- M = 5..16 with K = 32 S KW: the MFMA_STREAM kind -----------------------
// A workgroup is KW waves that split K; a tile is 16 T weight rows (MFMA
// subtiles, laid out as in the MFMA kind: mfma_weight_row / mfma_tiles). Wave
// kw's step s covers k = 32 (kw S + s) .. + 31; lane l (li = l % 16, g = l / 16)
// holds k = 32 (kw S + s) + 8 g .. + 7 of weight row li and of x row li.
// Workgroup b walks tiles b, b + grid, ... (at most mstream_max_depth(T)).

constexpr int kMstreamMaxRows = 16;
FTK_HD int mstream_steps(int k, int kw) { return (kw < 1 || k % (32 * kw)) ? 0 : k / (32 * kw); }
// Tiles a workgroup may walk: their per-wave partials wait in 64 KiB of LDS.
FTK_HD int mstream_max_depth(int t, int kw) { return (64 * 1024) / (t * kw * 1024); }

// ---- M = 2..16 with K = 128 C KW: the QUAD kind (4x4x4 MFMA blocks) --------
// Same tiles, row groups and weight rows as the GEMV kind, with 4 RS weight
// rows per row group per tile (rows_per_wave = 4 RS). Lane l = 4 b + i of wave
// kw of a row group reads weight row i of each row set at K segment j KW + kw
// (j < C), chunk b: elements 128 (j KW + kw) + 8 b .. + 7; it holds x rows
// 4 q + i at the same elements. Workgroup b walks tiles b, b + grid, ... (at
// most kStreamMaxTiles of them).

constexpr int kQuadMaxRows = 16;
// 128-element segments per lane per weight row (C), or 0 when K is not 128 C KW.
FTK_HD int quad_segments(int k, int kw) { return (kw < 1 || k % (128 * kw)) ? 0 : k / (128 * kw); }
// Groups of 4 x rows a kernel is built for: 1 (M <= 4), 2 (M <= 8), 4 (M <= 16).
FTK_HD int quad_groups(int m) { return m < 1 ? 0 : m <= 4 ? 1 : m <= 8 ? 2 : m <= 16 ? 4 : 0; }
// Whether a QUAD shape keeps its registers without spilling, estimated from the
// gfx950 builds: the x slice (4 MQ C), the weight window (4 RS C), the
// accumulators (4 RS MQ) and, with the prologue, what is live while it runs
// (the residual, the gain and temporaries: 6 MQ C + 4 C) and the gain kept
// through the first tile, where the slice is normalised (4 C + 24). Where the
// prologue and the window would not fit together, the window is issued after
// the prologue. The cap is 248 registers (128 for a 16-wave workgroup); shapes
// over it are not built.
constexpr int quad_cap(int kw) { return kw >= 16 ? 128 : 248; }
constexpr int quad_main_regs(int mq, int rs, int c) { return 4 * mq * c + 4 * rs * c + 4 * rs * mq + 32; }
// With the prologue: issue the first weight window only after it, where the two
// would not fit together.
constexpr bool quad_late(int mq, int rs, int c, int kw, bool pro) {
  return pro && quad_main_regs(mq, rs, c) + 6 * mq * c + 4 * c > quad_cap(kw);
}
constexpr bool quad_fits(int mq, int rs, int c, int kw, bool pro) {
  const int main_loop = quad_main_regs(mq, rs, c);
  if (!pro) return main_loop <= quad_cap(kw);
  // The slice is normalised during the first tile, so the gain stays live there.
  const int first_tile = main_loop + 4 * c + 24;
  const int prologue = quad_late(mq, rs, c, kw, pro) ? 10 * mq * c + 4 * c + 32 : main_loop + 6 * mq * c + 4 * c;
  return (first_tile > prologue ? first_tile : prologue) <= quad_cap(kw);
}

// ---- M = 5..16 with K = 128 C KW: the STAGE kind (16x16x32 MFMA via LDS) -----
// Tiles, subtiles and weight rows as the MFMA kind (mfma_weight_row /
// mfma_tiles), segments as the QUAD kind: wave kw of a workgroup reads the
// 128-wide K segments j KW + kw. Workgroup b walks tiles b, b + grid, ...; the
// per-wave partials of up to stage_max_depth(T, KW) of them wait in 64 KiB of
// LDS before their epilogue runs.
constexpr int kStageMaxRows = 16;
FTK_HD constexpr int stage_max_depth(int t, int kw) { return (64 * 1024) / (t * kw * 1024); }

// ---- M = 1..16 with K = 128 C KW: the RING kind (direct-to-LDS loads) --------
// Segments as the QUAD kind (wave kw reads the 128-wide K segments j KW + kw).
// A tile is RT weight rows: rows RT t .. RT t + RT - 1 (RT = 16, or 24 where 16-row
// tiles would leave a partial round of workgroups, e.g. N = 6144 on 256 CUs), or
// for SwiGLU (RT = 16) the gate rows 8 t .. 8 t + 7 (unit rows 0..7) and the
// matching up rows (unit rows 8..15). Workgroup b walks tiles b, b + grid, ...;
// after every ring_max_depth tiles the workgroup sums their per-wave partials and
// runs their epilogue.
constexpr int kRingMaxRows = 16;
// x rows one unit carries, in loads of 4 rows: 8 rows up to M = 8, else 16.
FTK_HD constexpr int ring_x_loads(int m) { return m <= 8 ? 2 : 4; }
FTK_HD constexpr int ring_out_per_tile(int epi, int rt = 16) { return epi == EPI_SWIGLU ? 8 : rt; }
FTK_HD int ring_tiles(int epi, int n_rows, int rt = 16) {
  const int per = ring_out_per_tile(epi, rt);
  return (gemv_outputs(epi, n_rows) + per - 1) / per;
}
// XOR swizzle of a unit row's 16 chunks (a permutation of 0..15; rows 16..23 as 0..7).
FTK_HD constexpr int ring_swz(int row) { return 4 * (row & 3) + ((row & 15) >> 2); }
// Tile of step i of RING workgroup wg in a grid of G over `tiles` tiles (steps
// i < ceil((tiles - wg) / G)). The dispatcher deals workgroups to the 8 XCDs in
// turn (wg on XCD wg % 8), so in every full round of G tiles each XCD's G / 8
// workgroups take one contiguous run of G / 8 tiles; the round as a whole still
// covers one contiguous range. A partial last round, and a grid that is not a
// multiple of 8, keep tile wg + i G. (Measured on MI355X against wg + i G: O at
// 5..16 rows 0.2-0.5 us faster, gate/up + SwiGLU at 16 rows 0.7 us; for STREAM's
// thousands of short-lived workgroups the plain order is faster.)
FTK_HD int ring_tile(int wg, int i, int G, int tiles) {
  if ((G & 7) != 0 || (i + 1) * G > tiles) return wg + i * G;
  return i * G + (G >> 3) * (wg & 7) + (wg >> 3);
}
// Weight row of unit row r (0..RT-1) in tile t, clamped in bounds.
FTK_HD int ring_weight_row(int epi, int t, int r, int n_rows, int rt = 16) {
  if (epi == EPI_SWIGLU) {
    const int half = n_rows / 2;
    int c = t * 8 + (r & 7);
    c = c < half ? c : half - 1;
    return r < 8 ? c : half + c;
  }
  const int n = t * rt + r;
  return n < n_rows ? n : n_rows - 1;
}
// 16-byte slots of one wave's ring: D units of RT/4 KiB of weights + NX KiB of x.
// With C <= 4 and tiles of at most 16 rows (x kept in registers after the first
// tile) the ring holds the first tile's two units with x, or four weight-only
// units for the later tiles; with fewer than 16 rows, the MFMA's unused rows past
// the last unit read a pad (their outputs are never stored).
FTK_HD constexpr int ring_xreg_slots(int nx, int rt) {
  return (4 * 16 * rt > 2 * (16 * rt + 64 * nx) ? 4 * 16 * rt : 2 * (16 * rt + 64 * nx)) + 16 * (16 - rt);
}
FTK_HD constexpr int ring_wave_slots(int c, int d, int nx, int rt = 16) {
  return (c <= 4 && rt <= 16) ? ring_xreg_slots(nx, rt) : d * (16 * rt + 64 * nx);
}
// LDS of a RING workgroup besides its per-tile partials: the rings, the gain (K
// BF16) with the prologue, the argmax keys and the row scales.
FTK_HD constexpr int ring_lds_fixed(int c, int kw, int d, int nx, bool pro, int rt = 16) {
  return kw * ring_wave_slots(c, d, nx, rt) * 16 + (pro ? 16 * c * kw * 16 : 16) + kw * 16 * 8 + 64;
}
// Tiles whose per-wave partials (KW KiB per 16-row subtile) fit beside it in
// 160 KiB (at most 8).
FTK_HD constexpr int ring_max_depth(int c, int kw, int d, int nx, bool pro, int rt = 16) {
  const int avail = 160 * 1024 - 512 - ring_lds_fixed(c, kw, d, nx, pro, rt);
  const int depth = avail < 0 ? 0 : avail / (kw * 1024 * ((rt + 15) / 16));
  return depth > 8 ? 8 : depth;
}

// ---- workspace layout of one projection call (bytes) -----------------------
// The row scales are written by the prologue pass before they are read. The
// argmax key words are zero between calls: a workspace is zeroed when it is
// allocated, and whichever reads the keys (the finalize launch, or the gathering
// workgroup of the one-launch argmax) zeroes each word it has read.
constexpr int64_t kWsScale = 0;     // [32] f32 RMSNorm row scales (MFMA kind)
constexpr int64_t kWsClaim = 128;   // u32 tail-tile claims of a RING launch (zero between calls)
// RING walks of at least this many tiles per workgroup claim their last tiles (the
// tail) from kWsClaim: lm_head + argmax at 5 rows 185.5 -> 179.2 us per graph node on
// MI355X. Shorter walks keep the static order (gate/up's six tiles: 32.8 -> 34.3 us
// claimed; its claims crowd into the walks' last tile).
constexpr int kRingTailMinTiles = 16;
constexpr int64_t kWsKeys = 256;    // [grid][M] u64 per-workgroup greedy-argmax keys

// Persistent launch: the fewest programs that keep the deepest walk at
// ceil(tiles / units) (the rule of engine/kernels/gemm.py:330-338).
FTK_HD int persistent_programs(int tiles, int units) {
  if (tiles <= 0 || units <= 0) return 0;
  const int depth = (tiles + units - 1) / units;
  return (tiles + depth - 1) / depth;
}

}  // namespace ftk
