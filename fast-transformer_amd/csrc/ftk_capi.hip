// extern "C" entry points of libftk.so (declared in include/ftk.h): argument
// checks, launch planning and dispatch to the gfx950 kernels.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "../../include/ftk.h"
#include "ftk_internal.h"

namespace ftk {

static thread_local int g_last_hip_error = 0;

int hip_status(hipError_t e) {
  if (e == hipSuccess) return FTK_OK;
  g_last_hip_error = (int)e;
  return FTK_ERR_HIP;
}

DeviceInfo device_info() {
  static DeviceInfo cache[64];
  int dev = 0;
  DeviceInfo none = {0, 0, 0};
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return none;
  DeviceInfo& d = cache[dev];
  if (!d.ok) {
    int cus = 0, lds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return none;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) lds = 65536;
    d.cus = cus;
    d.lds_per_group_max = lds;
    d.ok = 1;
  }
  return d;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Planner defaults (from the launch-shape sweeps on MI355X).
constexpr int kDefaultGroupsPerCu = 16;

// GEMV launch shape by problem size, measured at M = 1 on the Qwen3 shapes:
// few outputs want K split across the waves (more workgroups in flight),
// long rows want more 16-byte loads in flight per wave.
struct GemvDefault {
  int rpw, unroll, kw;
};
static GemvDefault gemv_default(int epi, int64_t N, int64_t K) {
  const int64_t outputs = gemv_outputs(epi, (int)N);
  const int64_t kc = K / 8;
  GemvDefault d;
  if (outputs <= 1024)
    d = {1, 1, 4};          // 0.6B O / down
  else if (outputs <= 4096 && K >= 8192)
    d = {2, 4, 2};          // 8B down
  else if (outputs <= 4096)
    d = {1, 2, 2};          // 8B O, 0.6B QKV
  else if (outputs >= 12288)
    d = {2, 2, 4};          // gate/up, lm_head
  else
    d = {2, 4, 1};          // 8B QKV
  // Keep the unrolled batches whole (the pipelined path needs K % (512 U KW) == 0).
  while (d.unroll > 1 && kc % (64 * d.unroll * d.kw)) d.unroll /= 2;
  while (d.kw > 1 && kc % (64 * d.unroll * d.kw)) d.kw /= 2;
  if (epi == FTK_EPI_SWIGLU && d.rpw % 2) d.rpw = 2;
  if (!gemv_supported(1, d.rpw, d.unroll, d.kw, epi)) d = {2, 4, 1};  // always instantiated
  return d;
}
// STREAM launch shape, from the M = 1 sweep of the Qwen3 shapes on MI355X: the
// widest K split whose chunk count is instantiated; 4 rows per group for long
// outputs with short rows (QKV, gate/up, lm_head), else 2.
struct StreamDefault {
  int rpw, kw;
};
static StreamDefault stream_default(int64_t M, int epi, int64_t N, int64_t K) {
  if (M < 1 || M > kStreamMaxRows || K > INT32_MAX || N > INT32_MAX) return {0, 0};
  // One wave per row group (KW = 1: whole rows per wave, no LDS round and no barrier
  // before the stores) for rows of at most 3072 elements at one x row, STORE and
  // SwiGLU. Qwen3-0.6B shapes, graphs of 28-64 distinct weights: 0.6B QKV without
  // the norm 3.52 -> 3.30 us, with it 3.87 -> 3.74, O 3.06 -> 2.96, gate/up + SwiGLU
  // 4.51 -> 4.46, down 3.47 -> 3.28. At the 8B shapes it measured slower (QKV
  // 9.45 -> 9.58 us, O 7.04 -> 7.12, gate/up 29.7 -> 31.0).
  if (M == 1 && K <= 3072 && epi != FTK_EPI_ARGMAX) {
    const int rpw = (K <= 1024 || epi == FTK_EPI_SWIGLU) ? 2 : 1;
    if (stream_supported(1, rpw, (int)K, 1, epi)) return {rpw, 1};
  }
  // Rows longer than 8192 (down, K = 12288) split K over 8 waves (M = 1 down:
  // 16.25 us against 17.0 with 4); otherwise 4 waves first.
  const int order_long[] = {8, 4, 2, 1}, order[] = {4, 2, 1, 8};
  for (int kw : (K > 8192 ? order_long : order)) {
    const int c = stream_chunks((int)K, kw);
    if (c == 0) continue;
    // 4 rows per tile for gate/up's 12288 outputs (29.6 us against 31.3 with 2),
    // else 2 (QKV's 6144: 9.28 us against 9.51 with 4; lm_head + argmax at
    // M = 1: 192.6 us against 194.8 with 4).
    const int want = (c <= 2 && epi != FTK_EPI_ARGMAX && gemv_outputs(epi, (int)N) > 6144) ? 4 : 2;
    for (int rpw : {want, 2, 4, 8})
      if (stream_supported((int)M, rpw, (int)K, kw, epi)) return {rpw, kw};
  }
  return {0, 0};
}
// STREAM grid cap: small projections run best as ~2 workgroups per CU walking
// several tiles (the prologue is paid once per workgroup), mid-size ones one
// tile per workgroup, the largest (lm_head) as deep walks of kStreamMaxTiles.
// Rows of at most 1024 elements (Qwen3-0.6B's QKV and gate/up) take two tiles
// per workgroup when a prologue is paid per workgroup (0.6B gate/up + SwiGLU:
// 4.70 -> 4.45 us), one without it (0.6B QKV without the norm: 3.60 -> 3.48 us,
// graphs of 64 distinct weights).
static int64_t stream_default_cap(int tiles, int cus, int64_t M, int64_t K, bool pro, int kw) {
  // One wave per row group at one x row: one tile per workgroup, two with the
  // prologue (each wave forms its row's norm scale once per workgroup).
  if (kw == 1 && M == 1) return pro ? (tiles + 1) / 2 : tiles;
  if (K <= 1024 && tiles <= 4096) {
    if (!pro) return tiles;
    return tiles / 2 > 2LL * cus ? tiles / 2 : 2LL * cus;
  }
  // Long rows (down, K = 12288): at M = 1 one tile per workgroup; with more x
  // rows one workgroup per CU walking tiles (M = 2..4: 16.9-17.9 us, against
  // 19.6-22.1 with one tile each).
  if (K > 8192 && tiles <= 4096) return M == 1 ? tiles : cus;
  if (tiles <= 4096) return 2LL * cus;
  // One tile per workgroup at M = 1; from two x rows three tiles per workgroup
  // (gate/up + SwiGLU at M = 2: 31.0 us against 32.5 with one).
  if (tiles <= 16384) return M == 1 ? 32LL * cus : 8LL * cus;
  return 0;  // the depth limit sets the grid
}

// MFMA_STREAM launch shape, from the M = 5 / 16 sweep of the Qwen3-8B shapes on
// MI355X: 8 waves split K (16 steps of 32 at K = 4096) with 8 steps in flight
// (16 for lm_head); 16 waves and 4 steps for a small projection with the
// prologue (QKV); two subtiles per tile for SwiGLU (a gate and an up subtile).
// K = 12288 runs without the prologue only, with x streamed: 8 waves, 16 steps
// in flight.
struct MstreamDefault {
  int t, kw, unroll;
};
static MstreamDefault mstream_default(int64_t M, int epi, bool pro, int64_t N, int64_t K) {
  if (M < 1 || M > kMstreamMaxRows || K > INT32_MAX || N > INT32_MAX) return {0, 0, 0};
  const int t = epi == FTK_EPI_SWIGLU ? 2 : 1;
  const bool small_pro = pro && epi == FTK_EPI_STORE && mfma_tiles(epi, (int)N, 1) <= 512;
  // Long K without the prologue streams x beside the weights: 16 steps in flight.
  const bool long_k = !pro && mstream_steps((int)K, 8) > 16;
  const MstreamDefault order[] = {
      long_k ? MstreamDefault{t, 8, 16}
             : small_pro ? MstreamDefault{t, 16, 4} : MstreamDefault{t, 8, epi == FTK_EPI_ARGMAX ? 16 : 8},
      {t, 8, 8}, {t, 8, 4}, {t, 16, 4}, {t, 16, 6}, {t, 16, 2}};
  for (const MstreamDefault& d : order)
    if (mstream_supported((int)M, d.t, (int)K, d.kw, d.unroll, epi, pro)) return d;
  return {0, 0, 0};
}

// QUAD launch shape, from the M = 1..16 sweep of the Qwen3-8B shapes on MI355X:
// 8 waves split K; 16 rows per tile for SwiGLU (two gate and two up row sets),
// 4 for lm_head (many short walks: the fewest registers), 24 for a projection
// with the prologue at up to 4 rows (QKV), 8 otherwise; the first shape that
// fits the registers.
struct QuadDefault {
  int rows, kw;
};
static QuadDefault quad_default(int64_t M, int epi, bool pro, int64_t N, int64_t K) {
  if (M < 1 || M > kQuadMaxRows || K > INT32_MAX || N > INT32_MAX) return {0, 0};
  const int want = epi == FTK_EPI_SWIGLU ? 16 : epi == FTK_EPI_ARGMAX ? 4 : (pro && M <= 4) ? 24 : 8;
  const QuadDefault order[] = {{want, 8}, {8, 8}, {4, 8}, {want, 4}, {8, 4}, {4, 4}, {8, 16}};
  for (const QuadDefault& d : order)
    if (quad_supported((int)M, d.rows, (int)K, d.kw, epi, pro)) return d;
  return {0, 0};
}
// QUAD grid cap: one workgroup per CU walking several tiles (their prologue is
// paid once); lm_head at up to 4 rows as shallow walks of many workgroups.
static int64_t quad_default_cap(int64_t M, int tiles, int cus) {
  return (tiles > 8192 && M <= 4) ? 32LL * cus : (int64_t)cus;
}
// Where QUAD beats the other kinds (MI355X, Qwen3-8B shapes): below 5 rows
// (against STREAM) lm_head from 2 rows, SwiGLU from 3, any projection with the
// prologue at 4; at 5..8 (against STAGE) the prologue projection without an
// epilogue (QKV). Elsewhere from 5 rows STAGE's 16x16x32 tiles, a quarter of the
// MFMA issue per byte, win.
static bool quad_preferred(int64_t M, int epi, bool pro) {
  if (M > 8) return false;
  if (M >= 5) return pro && epi == FTK_EPI_STORE;
  if (epi == FTK_EPI_ARGMAX) return M >= 2;
  if (epi == FTK_EPI_SWIGLU) return M >= 3;
  return pro && M >= 4;
}

// STAGE launch shape, from the M = 5..16 sweep of the Qwen3-8B shapes on MI355X:
// 8 waves split K; two segments in flight (three for the long K, four for
// lm_head); two subtiles per tile for SwiGLU (a gate and an up subtile).
struct StageDefault {
  int t, kw, unroll;
};
static StageDefault stage_default(int64_t M, int epi, bool pro, int64_t N, int64_t K) {
  if (M < 1 || M > kStageMaxRows || K > INT32_MAX || N > INT32_MAX) return {0, 0, 0};
  const int t = epi == FTK_EPI_SWIGLU ? 2 : 1;
  // Segments in flight per wave: 3 for the long K (x streamed beside the
  // weights), else 2 (lm_head + argmax at 5 rows: 208 us against 220 with 4).
  const int u = quad_segments((int)K, 8) > 4 ? 3 : 2;
  const StageDefault order[] = {{t, 8, u}, {t, 8, 2}, {t, 8, 4}, {t, 8, 3}};
  for (const StageDefault& d : order)
    if (stage_supported((int)M, d.t, (int)K, d.kw, d.unroll, epi, pro)) return d;
  return {0, 0, 0};
}

// RING launch shape: 8 waves split K; two units in flight, three for the long K
// (K = 12288) at up to 8 rows, where they fit the LDS.
// lm_head + argmax (thousands of tiles) walks them in one round of workgroups whose
// last eighth of the tiles is claimed (ring_kernel's tail): 179.2 us per graph node
// at 5 rows on MI355X, against 185.5 in the static two rounds used before.
// Rows per tile (STORE): the fewest rows on the busiest CU, 16 first, then 12.
// Where 16-row tiles leave a partial round of workgroups (N = 6144 on 256 CUs:
// 384 tiles, so 192 workgroups walk two each), 12-row tiles fill every CU with
// two, the second run from registers four units deep. QKV 6144 x 4096 on
// MI355X, graphs of 36 distinct weights: with the prologue 10.83 / 10.88 /
// 12.50 us at M = 5 / 8 / 16 against 11.36 / 11.44 / 12.74 with 16 rows; without
// it 9.82 / 9.99 / 10.72 against 10.58 / 10.32 (24 rows) and 11.22 (16 rows).
// 24-row tiles (one per CU there) stay a launch choice.
struct RingDefault {
  int kw, depth, groups_per_cu, rows;
};
static int ring_busiest_rows(int tiles, int rt, int units) {
  const int grid = persistent_programs(tiles, tiles < units ? tiles : units);
  return grid > 0 ? (tiles + grid - 1) / grid * rt : 0;
}
static RingDefault ring_default(int64_t M, int epi, bool pro, int64_t N, int64_t K, int cus) {
  if (M < 1 || M > kRingMaxRows || K > INT32_MAX || N > INT32_MAX) return {0, 0, 0, 0};
  const int c = quad_segments((int)K, 8);
  // One workgroup per CU, all resident: long walks claim their last tiles
  // (ring_kernel), so workgroups that run ahead take more of them.
  const int gpc = 1;
  int rows = 16;
  if (epi == FTK_EPI_STORE && ring_supported((int)M, (int)K, 8, 2, epi, pro, 12) &&
      ring_busiest_rows(ring_tiles(epi, (int)N, 12), 12, gpc * cus) <
          ring_busiest_rows(ring_tiles(epi, (int)N, 16), 16, gpc * cus))
    rows = 12;
  const RingDefault order[] = {{8, c > 4 && M <= 8 ? 3 : 2, gpc, rows}, {8, 2, gpc, 16}};
  for (const RingDefault& d : order)
    if (ring_supported((int)M, (int)K, d.kw, d.depth, epi, pro, d.rows)) return d;
  return {0, 0, 0, 0};
}
// Where RING beats the other kinds (MI355X, Qwen3-8B shapes): at 5..16 rows every
// projection, SwiGLU and lm_head + argmax, with or without the norm prologue; at
// 1..4 rows lm_head + argmax with the prologue where every workgroup walks enough
// tiles for the claimed tail (151936 x 4096, per graph node: 177.7 us at M = 1
// against STREAM's one launch, 184.4; 178.0 at M = 2 against QUAD, 187).
// Not with the prologue's residual add, which RING does not take (project_impl
// plans such calls without it).
static bool ring_preferred(int64_t M, int epi, bool pro, int64_t N, int64_t K, int cus) {
  if (M >= 5) return true;
  return epi == FTK_EPI_ARGMAX && M >= 1 && ring_tail_supported((int)M, (int)K, 8, 2, epi, pro, 16) &&
         ring_tiles(epi, (int)N, 16) >= (int64_t)kRingTailMinTiles * cus;
}

constexpr int kMfmaDefaultUnroll = 4;
constexpr int kMfmaDefaultWaves = 16;

static int64_t argmax_keys_bytes(int grid, int64_t M) { return kWsKeys + (int64_t)grid * M * 8; }

// epi may carry FTK_PLAN_PROLOGUE: plan a call with the RMSNorm prologue.
// epi may carry FTK_PLAN_RESIDUAL: the prologue adds a residual, which the RING kind does not take.
static int plan(int64_t M, int64_t N, int64_t K, int epi, int cus, const ftk_config* cfg, ftk_plan* p) {
  const bool pro = (epi & FTK_PLAN_PROLOGUE) != 0;
  const bool ring_ok = (epi & FTK_PLAN_RESIDUAL) == 0;
  epi &= ~(FTK_PLAN_PROLOGUE | FTK_PLAN_RESIDUAL);
  memset(p, 0, sizeof(*p));
  if (M < 1 || M > FTK_MAX_ROWS || N < 1 || K < 1 || cus < 1) return FTK_ERR_INVALID;
  if (N > INT32_MAX / 2 || K > INT32_MAX / 2) return FTK_ERR_INVALID;
  if (epi < FTK_EPI_STORE || epi > FTK_EPI_ARGMAX) return FTK_ERR_INVALID;
  if (epi == FTK_EPI_SWIGLU && (N % 2)) return FTK_ERR_INVALID;
  int kind = cfg && cfg->kind ? cfg->kind : FTK_KIND_AUTO;
  if (kind == FTK_KIND_AUTO) {
    // Measured on MI355X at the Qwen3-8B shapes: RING (direct-to-LDS 16x16x32
    // tiles) where ring_preferred says so; below that STREAM (v_dot2) at M = 1 and
    // up to M = 4; QUAD (4x4x4 MFMA blocks) where quad_preferred says so; STAGE
    // (16x16x32 via LDS) for the rest of M = 5..16; MFMA_STREAM where neither has
    // the shape.
    const bool quad = quad_default(M, epi, pro, N, K).rows != 0;
    const bool stage = M >= 5 && stage_default(M, epi, pro, N, K).t != 0;
    const RingDefault rd = ring_ok && ring_preferred(M, epi, pro, N, K, cus) ? ring_default(M, epi, pro, N, K, cus)
                                                                             : RingDefault{0, 0, 0, 0};
    // RING holds one workgroup per CU: where its tiles would leave more than half
    // the CUs idle and QUAD is preferred at these rows, QUAD's smaller tiles keep
    // more of them streaming (a Qwen3-8B eight-way tensor-parallel shard's QKV,
    // 768 x 4096 with the norm, at M = 5: 64 RING tiles 7.80 us, QUAD 6.55).
    const bool ring = rd.kw != 0 && (ring_tiles(epi, (int)N, rd.rows) >= cus / 2 || !quad ||
                                     !quad_preferred(M, epi, pro));
    if (K % 8)
      kind = FTK_KIND_GENERIC;
    else if (ring)
      kind = FTK_KIND_RING;
    else if (quad && quad_preferred(M, epi, pro))
      kind = FTK_KIND_QUAD;
    else if (stage)
      kind = FTK_KIND_STAGE;
    else if (M <= 4 && stream_default(M, epi, N, K).rpw)
      kind = FTK_KIND_STREAM;
    else if (M <= 4)
      kind = FTK_KIND_GEMV;
    else {
      const MstreamDefault d = mstream_default(M, epi, pro, N, K);
      // K = 12288 (24 MFMA steps per wave) at M <= 8: 8 waves of v_dot2 (the
      // 8-row STREAM kernel) beat the 16-wave MFMA kernel on MI355X.
      const bool long_k = d.t && mstream_steps((int)K, d.kw) > 16;
      if (d.t && !(long_k && M <= kStreamMaxRows && stream_default(M, epi, N, K).rpw))
        kind = FTK_KIND_MFMA_STREAM;
      else if (M <= kStreamMaxRows && stream_default(M, epi, N, K).rpw)
        kind = FTK_KIND_STREAM;
      else
        kind = FTK_KIND_MFMA;
    }
  }
  p->kind = kind;
  p->threads = kThreads;
  p->splits = 1;
  p->k_slice = (int)K;
  if (kind == FTK_KIND_GENERIC) {
    if (epi != FTK_EPI_STORE) return FTK_ERR_UNSUPPORTED;
    p->tiles = (int)((N + kWaves - 1) / kWaves);
    p->grid = p->tiles;
    p->rows_per_wave = 1;
    p->unroll = 1;
    p->waves = 1;
    return FTK_OK;
  }
  if (K % 8 != 0) return FTK_ERR_UNSUPPORTED;
  if (kind == FTK_KIND_GEMV) {
    if (M > 4) return FTK_ERR_UNSUPPORTED;
    const GemvDefault d = gemv_default(epi, N, K);
    const bool given = cfg && cfg->rows_per_wave;
    const int rpw = given ? cfg->rows_per_wave : d.rpw;
    const int unroll = cfg && cfg->unroll ? cfg->unroll : (given ? 2 : d.unroll);
    const int gpc = cfg && cfg->groups_per_cu ? cfg->groups_per_cu : kDefaultGroupsPerCu;
    const int kw = cfg && cfg->waves ? cfg->waves : (given ? 1 : d.kw);
    if (!gemv_supported((int)M, rpw, unroll, kw, epi)) return FTK_ERR_INVALID;
    p->rows_per_wave = rpw;
    p->unroll = unroll;
    p->waves = kw;
    p->tiles = gemv_tiles(epi, (int)N, rpw, kw);
    const int64_t cap = (int64_t)gpc * cus;
    p->grid = (int)(p->tiles < cap ? p->tiles : cap);
    p->lds_bytes = M * K * 2;  // + K * 2 for the staged gain when the prologue is on
    p->workspace_bytes = epi == FTK_EPI_ARGMAX ? argmax_keys_bytes(p->grid, M) : 0;
    if (p->lds_bytes + K * 2 > 160 * 1024) return FTK_ERR_UNSUPPORTED;
    return FTK_OK;
  }
  if (kind == FTK_KIND_STREAM) {
    if (M > kStreamMaxRows) return FTK_ERR_UNSUPPORTED;
    const StreamDefault d = stream_default(M, epi, N, K);
    const int kw = cfg && cfg->waves ? cfg->waves : d.kw;
    const int rpw = cfg && cfg->rows_per_wave ? cfg->rows_per_wave : d.rpw;
    const int c = stream_chunks((int)K, kw);
    if (c == 0) return FTK_ERR_UNSUPPORTED;  // K is not 512 C KW
    if (!stream_supported((int)M, rpw, (int)K, kw, epi)) return FTK_ERR_INVALID;
    p->rows_per_wave = rpw;
    p->unroll = c;
    p->waves = kw;
    p->threads = 64 * stream_waves(kw);
    p->tiles = gemv_tiles(epi, (int)N, rpw, kw);
    // Fewest workgroups that keep every walk at the same depth, and no deeper than
    // kStreamMaxTiles (each workgroup parks its tiles' wave totals in LDS).
    const int64_t cap = cfg && cfg->groups_per_cu ? (int64_t)cfg->groups_per_cu * cus
                                                  : stream_default_cap(p->tiles, cus, M, K, pro, kw);
    const int64_t floor = (p->tiles + kStreamMaxTiles - 1) / kStreamMaxTiles;
    const int64_t units = cap > floor ? cap : floor;
    p->grid = persistent_programs(p->tiles, (int)(units < p->tiles ? units : p->tiles));
    p->workspace_bytes = epi == FTK_EPI_ARGMAX ? argmax_keys_bytes(p->grid, M) : 0;
    return FTK_OK;
  }
  if (kind == FTK_KIND_QUAD) {
    if (M > kQuadMaxRows) return FTK_ERR_UNSUPPORTED;
    const QuadDefault d = quad_default(M, epi, pro, N, K);
    const int kw = cfg && cfg->waves ? cfg->waves : d.kw;
    int rows = cfg && cfg->rows_per_wave ? cfg->rows_per_wave : d.rows;
    // Four rows per tile where the default would leave more than half the CUs
    // without a tile (the shard's QKV at M = 5: 4-row tiles 6.55 us, 8-row 7.08).
    if (!(cfg && cfg->rows_per_wave) && gemv_tiles(epi, (int)N, rows, kw) < cus / 2 &&
        quad_supported((int)M, 4, (int)K, kw, epi, pro))
      rows = 4;
    const int c = quad_segments((int)K, kw);
    if (c == 0) return FTK_ERR_UNSUPPORTED;  // K is not 128 C KW
    if (!quad_supported((int)M, rows, (int)K, kw, epi, pro)) return FTK_ERR_INVALID;
    p->rows_per_wave = rows;
    p->unroll = c;
    p->waves = kw;
    p->threads = 64 * stream_waves(kw);
    p->tiles = gemv_tiles(epi, (int)N, rows, kw);
    const int64_t cap = cfg && cfg->groups_per_cu ? (int64_t)cfg->groups_per_cu * cus
                                                  : quad_default_cap(M, p->tiles, cus);
    const int64_t floor = (p->tiles + kStreamMaxTiles - 1) / kStreamMaxTiles;
    const int64_t units = cap > floor ? cap : floor;
    p->grid = persistent_programs(p->tiles, (int)(units < p->tiles ? units : p->tiles));
    p->workspace_bytes = epi == FTK_EPI_ARGMAX ? argmax_keys_bytes(p->grid, M) : 0;
    return FTK_OK;
  }
  if (kind == FTK_KIND_STAGE) {
    if (M > kStageMaxRows) return FTK_ERR_UNSUPPORTED;
    const StageDefault d = stage_default(M, epi, pro, N, K);
    const int rows = cfg && cfg->rows_per_wave ? cfg->rows_per_wave : 16 * (d.t ? d.t : 1);
    const int kw = cfg && cfg->waves ? cfg->waves : (d.kw ? d.kw : 8);
    const int unroll = cfg && cfg->unroll ? cfg->unroll : (d.unroll ? d.unroll : 2);
    if (quad_segments((int)K, kw) == 0) return FTK_ERR_UNSUPPORTED;  // K is not 128 C KW
    if (rows % 16 || !stage_supported((int)M, rows / 16, (int)K, kw, unroll, epi, pro)) return FTK_ERR_INVALID;
    const int t = rows / 16;
    p->rows_per_wave = rows;
    p->unroll = unroll;
    p->waves = kw;
    p->threads = 64 * kw;
    p->tiles = mfma_tiles(epi, (int)N, t);
    // One workgroup per CU (the LDS of one fills most of a CU), each walking its
    // share of the tiles: lm_head + argmax at 5 rows no longer runs a partial
    // last round of workgroups.
    const int64_t units = (int64_t)(cfg && cfg->groups_per_cu ? cfg->groups_per_cu : 1) * cus;
    p->grid = persistent_programs(p->tiles, (int)(units < p->tiles ? units : p->tiles));
    p->workspace_bytes = epi == FTK_EPI_ARGMAX ? argmax_keys_bytes(p->grid, M) : 0;
    return FTK_OK;
  }
  if (kind == FTK_KIND_RING) {
    if (M < 1 || M > kRingMaxRows) return FTK_ERR_UNSUPPORTED;
    const RingDefault d = ring_default(M, epi, pro, N, K, cus);
    const int kw = cfg && cfg->waves ? cfg->waves : (d.kw ? d.kw : 8);
    const int depth = cfg && cfg->unroll ? cfg->unroll : (d.depth ? d.depth : 2);
    const int rows = cfg && cfg->rows_per_wave ? cfg->rows_per_wave : (d.rows ? d.rows : 16);
    if (quad_segments((int)K, kw) == 0) return FTK_ERR_UNSUPPORTED;  // K is not 128 C KW
    if ((rows != 12 && rows != 16 && rows != 24) || !ring_supported((int)M, (int)K, kw, depth, epi, pro, rows))
      return FTK_ERR_INVALID;
    p->rows_per_wave = rows;
    p->unroll = depth;
    p->waves = kw;
    p->threads = 64 * kw;
    p->tiles = ring_tiles(epi, (int)N, rows);
    // One workgroup per CU at a time (its LDS fills the CU), each walking its
    // share (the last tiles claimed, with a workspace).
    const int64_t units = (int64_t)(cfg && cfg->groups_per_cu ? cfg->groups_per_cu : (d.groups_per_cu ? d.groups_per_cu : 1)) * cus;
    p->grid = persistent_programs(p->tiles, (int)(units < p->tiles ? units : p->tiles));
    // A grid that is a multiple of 8 lets ring_tile give each XCD one contiguous
    // run of tiles per full round: round up to one (more workgroups never make a
    // walk longer). lm_head + argmax at 5 / 8 / 16 rows: 504 workgroups instead
    // of 500, 1-2 us faster per call on MI355X.
    const int even = (p->grid + 7) / 8 * 8;
    if (even <= p->tiles) p->grid = even;
    p->workspace_bytes = epi == FTK_EPI_ARGMAX ? argmax_keys_bytes(p->grid, M) : 0;
    // The claims of long walks (without a workspace the walk keeps its static order
    // throughout).
    if (p->tiles >= kRingTailMinTiles * p->grid && p->workspace_bytes < kWsClaim + 4)
      p->workspace_bytes = kWsClaim + 4;
    return FTK_OK;
  }
  if (kind == FTK_KIND_MFMA_STREAM) {
    if (M > kMstreamMaxRows) return FTK_ERR_UNSUPPORTED;
    const MstreamDefault d = mstream_default(M, epi, pro, N, K);
    const int rows = cfg && cfg->rows_per_wave ? cfg->rows_per_wave : 16 * d.t;
    const int kw = cfg && cfg->waves ? cfg->waves : d.kw;
    const int unroll = cfg && cfg->unroll ? cfg->unroll : d.unroll;
    if (mstream_steps((int)K, kw) == 0) return FTK_ERR_UNSUPPORTED;  // K is not 32 S KW
    if (rows % 16 || !mstream_supported((int)M, rows / 16, (int)K, kw, unroll, epi, pro)) return FTK_ERR_INVALID;
    const int t = rows / 16;
    p->rows_per_wave = rows;
    p->unroll = unroll;
    p->waves = kw;
    p->threads = 64 * kw;
    p->tiles = mfma_tiles(epi, (int)N, t);
    const int64_t cap = (int64_t)(cfg && cfg->groups_per_cu ? cfg->groups_per_cu : 1) * cus;
    const int depth = mstream_max_depth(t, kw);
    const int64_t floor = (p->tiles + depth - 1) / depth;
    const int64_t units = cap > floor ? cap : floor;
    p->grid = persistent_programs(p->tiles, (int)(units < p->tiles ? units : p->tiles));
    p->workspace_bytes = epi == FTK_EPI_ARGMAX ? argmax_keys_bytes(p->grid, M) : 0;
    return FTK_OK;
  }
  if (kind == FTK_KIND_MFMA) {
    // Defaults from the MI355X sweep: 16 rows (SwiGLU: one gate + one up subtile)
    // per workgroup of 16 waves; 32 rows once M > 16 (two MFMA column blocks).
    const int rows = cfg && cfg->rows_per_wave ? cfg->rows_per_wave : (epi == FTK_EPI_SWIGLU || M > 16 ? 32 : 16);
    if (rows % 16) return FTK_ERR_INVALID;
    const int t = rows / 16;
    const int unroll = cfg && cfg->unroll ? cfg->unroll : (t >= 4 ? 2 : kMfmaDefaultUnroll);
    const int waves = cfg && cfg->waves ? cfg->waves : (epi == FTK_EPI_SWIGLU ? 8 : kMfmaDefaultWaves);
    if (!mfma_supported((int)M, t, unroll, waves, epi)) return FTK_ERR_INVALID;
    p->rows_per_wave = rows;
    p->unroll = unroll;
    p->waves = waves;
    p->threads = 64 * waves;
    p->tiles = mfma_tiles(epi, (int)N, t);
    p->grid = p->tiles;
    p->workspace_bytes = epi == FTK_EPI_ARGMAX ? argmax_keys_bytes(p->grid, M) : kWsKeys;  // row scales
    return FTK_OK;
  }
  return FTK_ERR_INVALID;
}

// Workspace a call needs: argmax keys, and the RMSNorm row scales of the MFMA kind.
static int64_t call_workspace(const ftk_plan& p, int epi, bool pro) {
  if (epi == FTK_EPI_ARGMAX) return p.workspace_bytes;
  if (p.kind == FTK_KIND_MFMA && pro) return kWsKeys;
  return 0;
}

// ---- decode attention: launch planning --------------------------------------

// Workgroups the default split count aims at: one per CU (measured on MI355X:
// 32 intervals per KV head beat 64 at B = 1 from 1K to 32K slots).
constexpr int kAttnGroupsPerCu = 1;

static int attn_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t C, int64_t D, int cus, const ftk_attn_config* cfg,
                     ftk_attn_plan* p, AttnShape* shape) {
  if (B < 1 || Hq < 1 || Hkv < 1 || C < 1 || Hq % Hkv || cus < 1) return FTK_ERR_INVALID;
  const int64_t G = Hq / Hkv;
  if ((D != 64 && D != 128) || G > kAttnMaxGroup) return FTK_ERR_UNSUPPORTED;
  if (C > INT32_MAX / 2 || B * Hkv > INT32_MAX / 2) return FTK_ERR_INVALID;
  const int groups = (int)(B * Hkv);
  // QUAD addresses a (row, KV head) cache with 32-bit byte offsets, reaching
  // up to 9 x 32 slots past its end (the ragged last unit and the next step's loads).
  const bool quad_fits = (C + 512) * D * 2 <= (int64_t)UINT32_MAX;
  int kind = cfg && cfg->kind ? cfg->kind : (D == 128 && G <= 4 && quad_fits ? FTK_ATTN_QUAD : FTK_ATTN_ROWS);
  if (kind == FTK_ATTN_QUAD && !quad_fits) return FTK_ERR_UNSUPPORTED;
  const int waves = cfg && cfg->waves ? cfg->waves : 4;
  int unroll = cfg && cfg->unroll ? cfg->unroll : (kind == FTK_ATTN_QUAD ? 1 : 4);
  if (kind == FTK_ATTN_ROWS && !(cfg && cfg->unroll) && !attn_supported(kind, (int)D, (int)G, waves, unroll))
    unroll = 2;
  if (!attn_supported(kind, (int)D, (int)G, waves, unroll)) return FTK_ERR_INVALID;
  const int64_t unit = kind == FTK_ATTN_QUAD ? 16 * unroll : (64 / (D / 8)) * unroll;  // slots per wave step
  int64_t splits;
  if (cfg && cfg->splits) {
    if (cfg->splits < 1) return FTK_ERR_INVALID;
    splits = cfg->splits < C ? cfg->splits : C;
    if (splits > kAttnMaxSplits) return FTK_ERR_INVALID;
  } else {
    const int64_t want = ((int64_t)kAttnGroupsPerCu * cus + groups - 1) / groups;
    const int64_t most = (C + waves * unit - 1) / (waves * unit);  // at least one step per wave
    splits = want < most ? want : most;
    if (splits > kAttnMaxSplits) splits = kAttnMaxSplits;
    if (splits < 1) splits = 1;
  }
  const int64_t chunk = (C + splits - 1) / splits;
  splits = (C + chunk - 1) / chunk;  // no interval lies wholly past the cache
  if ((int64_t)groups * splits > INT32_MAX) return FTK_ERR_INVALID;
  p->kind = kind;
  p->splits = (int)splits;
  p->chunk = (int)chunk;
  p->waves = waves;
  p->unroll = unroll;
  p->grid = (int)(groups * splits);
  p->workspace_bytes = splits > 1 ? (int64_t)groups * splits * G * (D + 2) * 4 : 0;
  if (shape) *shape = AttnShape{kind, (int)D, (int)G, groups, (int)splits, (int)chunk, waves, unroll};
  return FTK_OK;
}

// ---- static scratch of the entry point that allocates nothing ----------------
// File-scope device array: every GPU the library runs on holds its own copy,
// at its own address, until the process ends. Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol):
// it passes the device address hipGetSymbolAddress returned for the current
// device, looked up once per device and kept here. It starts zeroed (a device
// variable without an initializer), as the argmax key words must be at a call's
// start; every call leaves them zero.
static __device__ __align__(256) unsigned char scratch[FTK_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_lock;

// The current device's address of `scratch` (looked up on the first call on that device).
static int static_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e);
  if (dev < 0 || dev >= kMaxDevices) return FTK_ERR_INVALID;
  std::lock_guard<std::mutex> lock(g_scratch_lock);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e);
    if (ptr == nullptr) return hip_status(hipErrorInvalidSymbol);
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FTK_OK;
}

}  // namespace ftk

using namespace ftk;

extern "C" {

const char* ftk_version(void) { return "ftk 0.1 gfx950"; }

const char* ftk_status_string(int status) {
  switch (status) {
    case FTK_OK: return "ok";
    case FTK_ERR_INVALID: return "invalid argument";
    case FTK_ERR_UNSUPPORTED: return "shape or alignment not supported by this entry point";
    case FTK_ERR_WORKSPACE: return "workspace missing or too small";
    case FTK_ERR_HIP: return "HIP launch failed";
    case FTK_ERR_TOO_LARGE: return "the call needs more scratch than the static array holds (FTK_STATIC_SCRATCH_BYTES)";
  }
  return "unknown status";
}

int ftk_last_hip_error(void) { return g_last_hip_error; }

int ftk_persistent_programs(int tiles, int units) { return persistent_programs(tiles, units); }
int ftk_ring_tile(int wg, int step, int grid, int tiles) {
  if (grid <= 0 || tiles <= 0 || wg < 0 || wg >= grid || step < 0 || wg + step * grid >= tiles) return -1;
  return ring_tile(wg, step, grid, tiles);
}

int ftk_device_compute_units(void) {
  DeviceInfo d = device_info();
  return d.ok ? d.cus : -1;
}

int64_t ftk_argmax_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows < 1 || vocab < 1 || vocab > INT32_MAX) return 0;
  return 8 * rows * argmax_blocks((int)vocab);
}

int ftk_plan_project(int64_t M, int64_t N, int64_t K, int epilogue, int compute_units, const ftk_config* cfg,
                     ftk_plan* p) {
  if (p == nullptr) return FTK_ERR_INVALID;
  return plan(M, N, K, epilogue, compute_units, cfg, p);
}

int64_t ftk_project_workspace_bytes(int64_t M, int64_t N, int64_t K, int epilogue, const ftk_config* cfg) {
  DeviceInfo d = device_info();
  ftk_plan p;
  if (plan(M, N, K, epilogue, d.ok ? d.cus : 256, cfg, &p) != FTK_OK) return 0;
  return p.workspace_bytes;
}

int ftk_plan_coverage(const ftk_plan* p, int64_t N, int epilogue, int32_t* counts, int64_t outputs,
                      int64_t* max_row) {
  if (p == nullptr || counts == nullptr || max_row == nullptr) return FTK_ERR_INVALID;
  if (outputs != gemv_outputs(epilogue, (int)N)) return FTK_ERR_INVALID;
  memset(counts, 0, sizeof(int32_t) * outputs);
  *max_row = -1;
  if (p->kind == FTK_KIND_GENERIC) {
    for (int b = 0; b < p->grid; ++b)
      for (int w = 0; w < kWaves; ++w) {
        const int64_t row = (int64_t)b * kWaves + w;
        if (row < N) {
          counts[row] += 1;
          if (row > *max_row) *max_row = row;
        }
      }
    return FTK_OK;
  }
  if (p->kind == FTK_KIND_MFMA) {
    // Workgroup b owns tile b: T subtiles of 16 weight rows over all of K.
    const int t = p->rows_per_wave / 16;
    if (t < 1 || p->grid != p->tiles) return FTK_ERR_INVALID;
    const int per = mfma_out_per_tile(epilogue, t);
    for (int b = 0; b < p->grid; ++b) {
      for (int sub = 0; sub < t; ++sub)
        for (int li = 0; li < 16; ++li) {
          const int64_t row = mfma_weight_row(epilogue, b, sub, li, (int)N, t);
          if (row > *max_row) *max_row = row;
        }
      for (int r = 0; r < per; ++r) {
        const int64_t col = (int64_t)b * per + r;
        if (col < outputs) counts[col] += 1;
      }
    }
    return FTK_OK;
  }
  if (p->kind == FTK_KIND_MFMA_STREAM || p->kind == FTK_KIND_STAGE) {
    // Workgroup b walks tiles b + i grid; a tile is T subtiles of 16 weight rows.
    const int t = p->rows_per_wave / 16;
    if (t < 1 || p->grid < 1 || p->grid > p->tiles) return FTK_ERR_INVALID;
    if (p->kind == FTK_KIND_MFMA_STREAM && (p->tiles + p->grid - 1) / p->grid > mstream_max_depth(t, p->waves))
      return FTK_ERR_INVALID;
    const int per = mfma_out_per_tile(epilogue, t);
    for (int b = 0; b < p->grid; ++b)
      for (int tile = b; tile < p->tiles; tile += p->grid) {
        for (int sub = 0; sub < t; ++sub)
          for (int li = 0; li < 16; ++li) {
            const int64_t row = mfma_weight_row(epilogue, tile, sub, li, (int)N, t);
            if (row > *max_row) *max_row = row;
          }
        for (int r = 0; r < per; ++r) {
          const int64_t col = (int64_t)tile * per + r;
          if (col < outputs) counts[col] += 1;
        }
      }
    return FTK_OK;
  }
  if (p->kind == FTK_KIND_RING) {
    // Workgroup b takes tile ring_tile(b, i, grid, tiles) at step i (as the kernel
    // does); unit rows 0..RT-1 of a tile.
    if (p->grid < 1 || p->grid > p->tiles) return FTK_ERR_INVALID;
    const int rt = p->rows_per_wave;
    const int per = ring_out_per_tile(epilogue, rt);
    for (int b = 0; b < p->grid; ++b)
      for (int i = 0; b + i * p->grid < p->tiles; ++i) {
        const int tile = ring_tile(b, i, p->grid, p->tiles);
        for (int r = 0; r < rt; ++r) {
          const int64_t row = ring_weight_row(epilogue, tile, r, (int)N, rt);
          if (row > *max_row) *max_row = row;
        }
        for (int r = 0; r < per; ++r) {
          const int64_t col = (int64_t)tile * per + r;
          if (col < outputs) counts[col] += 1;
        }
      }
    return FTK_OK;
  }
  if (p->kind != FTK_KIND_GEMV && p->kind != FTK_KIND_STREAM && p->kind != FTK_KIND_QUAD) return FTK_ERR_UNSUPPORTED;
  if (p->grid < 1 || p->grid > p->tiles) return FTK_ERR_INVALID;
  if ((p->kind == FTK_KIND_STREAM || p->kind == FTK_KIND_QUAD) && (p->tiles + p->grid - 1) / p->grid > kStreamMaxTiles)
    return FTK_ERR_INVALID;
  const int pw = gemv_per_wave(epilogue, p->rows_per_wave);
  const int groups = gemv_groups(p->waves);
  const int halves = epilogue == FTK_EPI_SWIGLU ? 2 : 1;
  for (int b = 0; b < p->grid; ++b)
    for (int tile = b; tile < p->tiles; tile += p->grid)
      for (int w = 0; w < groups; ++w)
        for (int s = 0; s < pw; ++s) {
          const int col = gemv_output(tile, w, s, pw, groups);
          const int clamped = col < outputs ? col : (int)outputs - 1;
          for (int h = 0; h < halves; ++h) {
            const int64_t row = gemv_weight_row(epilogue, clamped, h, (int)N);
            if (row > *max_row) *max_row = row;
          }
          if (col < outputs) counts[col] += 1;
        }
  return FTK_OK;
}

// The one-launch greedy argmax is on unless FTK_ARGMAX_GATHER=0 (read once per process): the
// switch keeps the two-launch form measurable beside it.
static bool argmax_gather_on() {
  static const bool on = [] {
    const char* v = getenv("FTK_ARGMAX_GATHER");
    return v == nullptr || strcmp(v, "0") != 0;
  }();
  return on;
}

static bool overlaps(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes) {
  if (a == nullptr || b == nullptr) return false;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + (uintptr_t)b_bytes && pb < pa + (uintptr_t)a_bytes;
}

// Every projection entry point lands here; `out_add` (STORE only) is the residual
// stream the rounded outputs are added to, or null.
static int project_impl(const void* x, const ftk_rows* rows, const void* gamma, float eps, const void* w, void* y,
                        int64_t M, int64_t N, int64_t K, int epilogue, void* ids, int ids_bytes, float* top,
                        void* workspace, int64_t workspace_bytes, const ftk_config* cfg, const void* out_add,
                        void* stream) {
  if (x == nullptr || w == nullptr) return FTK_ERR_INVALID;
  if (epilogue != FTK_EPI_ARGMAX && y == nullptr) return FTK_ERR_INVALID;
  if (epilogue == FTK_EPI_ARGMAX) {
    if (ids == nullptr || (ids_bytes != 4 && ids_bytes != 8)) return FTK_ERR_INVALID;
    if (workspace == nullptr) return FTK_ERR_WORKSPACE;
  }
  ftk_rows r = {nullptr, nullptr, nullptr, 0, 0, nullptr, nullptr};
  if (rows != nullptr) r = *rows;
  const bool extra = r.residual != nullptr || r.sum != nullptr || r.x_ids != nullptr;
  if (r.sumsq != nullptr) {  // the norm's sums of x's rows, in place of the rows
    if (gamma == nullptr || extra) return FTK_ERR_INVALID;
    if (K % 16 || !aligned16(r.sumsq)) return FTK_ERR_UNSUPPORTED;
  }
  if (r.sumsq_out != nullptr) {
    if (epilogue != FTK_EPI_STORE) return FTK_ERR_UNSUPPORTED;
    if ((reinterpret_cast<uintptr_t>(r.sumsq_out) & 3) != 0) return FTK_ERR_INVALID;
    const int64_t sq_bytes = M * ((N + 15) / 16) * 4;
    if (overlaps(r.sumsq_out, sq_bytes, y, M * N * 2) || overlaps(r.sumsq_out, sq_bytes, x, M * K * 2) ||
        overlaps(r.sumsq_out, sq_bytes, out_add, M * N * 2) || overlaps(r.sumsq_out, sq_bytes, r.sumsq, M * (K / 16) * 4))
      return FTK_ERR_INVALID;
  }
  if (extra) {
    if (gamma == nullptr) return FTK_ERR_INVALID;  // the rows feed the norm
    if (r.x_ids != nullptr && ((r.x_ids_bytes != 4 && r.x_ids_bytes != 8) || r.x_rows < 1)) return FTK_ERR_INVALID;
    if (M < 1 || K < 1 || M > FTK_MAX_ROWS || K > INT32_MAX) return FTK_ERR_INVALID;
    // Workgroup 0 writes sum while every workgroup reads x and the residual.
    const int64_t rows_bytes = M * K * 2;
    const int64_t out_cols = epilogue == FTK_EPI_SWIGLU ? N / 2 : N;
    if ((r.x_ids == nullptr && overlaps(r.sum, rows_bytes, x, rows_bytes)) ||
        overlaps(r.sum, rows_bytes, r.residual, rows_bytes) || overlaps(r.sum, rows_bytes, y, M * out_cols * 2))
      return FTK_ERR_INVALID;
    if ((r.residual && !aligned16(r.residual)) || (r.sum && !aligned16(r.sum))) return FTK_ERR_UNSUPPORTED;
  }
  DeviceInfo d = device_info();
  if (!d.ok) return hip_status(hipErrorNoDevice);
  ftk_plan p;
  int st = plan(M, N, K,
                epilogue | (gamma != nullptr ? FTK_PLAN_PROLOGUE : 0) | (r.residual != nullptr ? FTK_PLAN_RESIDUAL : 0),
                d.cus, cfg, &p);
  if (st != FTK_OK) return st;
  const int64_t need = call_workspace(p, epilogue, gamma != nullptr);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return FTK_ERR_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (p.kind == FTK_KIND_GENERIC) {
    if (gamma != nullptr) return FTK_ERR_UNSUPPORTED;
    return hip_status(launch_gemm_generic((const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y,
                                          (const uint16_t*)out_add, (int)M, (int)N,
                                          (int)K, s));
  }
  if (!aligned16(x) || !aligned16(w) || (gamma && !aligned16(gamma))) return FTK_ERR_UNSUPPORTED;
  ProjArgs a;
  memset(&a, 0, sizeof(a));
  a.x = (const uint16_t*)x;
  a.w = (const uint16_t*)w;
  a.gamma = (const uint16_t*)gamma;
  a.y = (uint16_t*)y;
  a.eps = eps;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.ids = ids;
  a.ids_bytes = ids_bytes;
  a.top = top;
  a.residual = (const uint16_t*)r.residual;
  a.sum = (uint16_t*)r.sum;
  a.x_ids = r.x_ids;
  a.x_ids_bytes = r.x_ids_bytes;
  a.x_rows = r.x_rows;
  a.out_add = (const uint16_t*)out_add;
  // The MFMA kind's projection reads the pre-pass's stored rows: it needs sum.
  if (p.kind == FTK_KIND_MFMA && (r.residual != nullptr || r.x_ids != nullptr) && r.sum == nullptr)
    return FTK_ERR_UNSUPPORTED;
  // The RING kind loads x rows as they are: no residual add in its prologue.
  if (p.kind == FTK_KIND_RING && r.residual != nullptr) return FTK_ERR_UNSUPPORTED;
  // Row sums of squares travel between RING launches only (16-row STORE tiles write them).
  if (r.sumsq != nullptr && p.kind != FTK_KIND_RING) return FTK_ERR_UNSUPPORTED;
  if (r.sumsq_out != nullptr && (p.kind != FTK_KIND_RING || p.rows_per_wave != 16)) return FTK_ERR_UNSUPPORTED;
  a.sumsq = r.sumsq;
  a.sumsq_out = r.sumsq_out;
  // Long RING walks claim their last tiles from the workspace's counter.
  if (p.kind == FTK_KIND_RING && p.tiles >= kRingTailMinTiles * p.grid && workspace != nullptr &&
      workspace_bytes >= kWsClaim + 4)
    a.claim = reinterpret_cast<unsigned*>(static_cast<char*>(workspace) + kWsClaim);
  char* ws = (char*)workspace;
  if (epilogue == FTK_EPI_ARGMAX) a.keys = (unsigned long long*)(ws + kWsKeys);
  // Greedy argmax in one launch (argmax_gather) for the STREAM kind: one row, or at most one key
  // word per gathering lane. (M = 1 lm_head: 184.7-185.1 us per graph node against 189.0-190.8 with
  // the second launch, same box. The RING kind at M = 5 measured the other way, 189.8-190.0 against
  // 186.5-187.0, so its keys go to the second launch.)
  a.fused = epilogue == FTK_EPI_ARGMAX && argmax_gather_on() && p.kind == FTK_KIND_STREAM &&
            (M == 1 || p.grid <= p.threads);
  hipError_t e;
  if (p.kind == FTK_KIND_STREAM) {
    StreamShape g = {p.rows_per_wave, p.waves, p.grid, p.tiles};
    e = launch_stream(a, epilogue, g, s);
  } else if (p.kind == FTK_KIND_MFMA_STREAM) {
    MstreamShape g = {p.rows_per_wave / 16, p.unroll, p.waves, p.grid, p.tiles};
    e = launch_mstream(a, epilogue, g, s);
  } else if (p.kind == FTK_KIND_QUAD) {
    QuadShape g = {p.rows_per_wave, p.waves, p.grid, p.tiles};
    e = launch_quad(a, epilogue, g, s);
  } else if (p.kind == FTK_KIND_STAGE) {
    StageShape g = {p.rows_per_wave / 16, p.unroll, p.waves, p.grid, p.tiles};
    e = launch_stage(a, epilogue, g, s);
  } else if (p.kind == FTK_KIND_RING) {
    RingShape g = {p.unroll, p.waves, p.grid, p.tiles, p.rows_per_wave};
    e = launch_ring(a, epilogue, g, s);
  } else if (p.kind == FTK_KIND_GEMV) {
    GemvShape g = {p.rows_per_wave, p.unroll, p.waves, p.grid, p.tiles, (size_t)p.lds_bytes};
    e = launch_gemv(a, epilogue, g, s);
  } else {
    MfmaShape shape = {p.rows_per_wave / 16, p.unroll, p.waves, p.grid};
    MfmaArgs m;
    m.row_scale = gamma != nullptr ? (const float*)(ws + kWsScale) : nullptr;
    e = launch_mfma(a, epilogue, shape, m, s);
  }
  if (e == hipSuccess && epilogue == FTK_EPI_ARGMAX && !a.fused)
    e = launch_argmax_finalize(a.keys, p.grid, (int)M, ids, ids_bytes, top, s);
  return hip_status(e);
}

int ftk_project_rows_bf16(const void* x, const ftk_rows* rows, const void* gamma, float eps, const void* w, void* y,
                          int64_t M, int64_t N, int64_t K, int epilogue, void* ids, int ids_bytes, float* top,
                          void* workspace, int64_t workspace_bytes, const ftk_config* cfg, void* stream) {
  return project_impl(x, rows, gamma, eps, w, y, M, N, K, epilogue, ids, ids_bytes, top, workspace, workspace_bytes,
                      cfg, nullptr, stream);
}

int ftk_project_bf16(const void* x, const void* gamma, float eps, const void* w, void* y, int64_t M, int64_t N,
                     int64_t K, int epilogue, void* ids, int ids_bytes, float* top, void* workspace,
                     int64_t workspace_bytes, const ftk_config* cfg, void* stream) {
  return project_impl(x, nullptr, gamma, eps, w, y, M, N, K, epilogue, ids, ids_bytes, top, workspace,
                      workspace_bytes, cfg, nullptr, stream);
}

int ftk_project_add_rows_bf16(const void* x, const ftk_rows* rows, const void* w, const void* residual, void* y,
                              int64_t M, int64_t N, int64_t K, const ftk_config* cfg, void* stream) {
  if (residual == nullptr || y == nullptr) return FTK_ERR_INVALID;
  // Only the sums of the stored outputs: the prologue's fields describe a norm, which this call has not.
  if (rows != nullptr && (rows->residual || rows->sum || rows->x_ids || rows->sumsq)) return FTK_ERR_INVALID;
  // y may be the residual itself (each output reads its own residual element,
  // then writes it), but no other overlap with the inputs.
  const int64_t out_bytes = M * N * 2;
  if (y != residual && overlaps(y, out_bytes, residual, out_bytes)) return FTK_ERR_INVALID;
  if (overlaps(y, out_bytes, x, M * K * 2) || overlaps(y, out_bytes, w, N * K * 2)) return FTK_ERR_INVALID;
  int st = project_impl(x, rows, nullptr, 0.f, w, y, M, N, K, FTK_EPI_STORE, nullptr, 0, nullptr, nullptr, 0, cfg,
                        residual, stream);
  // An unaligned pointer or an unsplit MFMA x slice: the generic kind, which writes no sums.
  if (st == FTK_ERR_UNSUPPORTED && cfg == nullptr && (rows == nullptr || rows->sumsq_out == nullptr)) {
    const ftk_config c = {FTK_KIND_GENERIC, 0, 0, 0, 0};
    st = project_impl(x, nullptr, nullptr, 0.f, w, y, M, N, K, FTK_EPI_STORE, nullptr, 0, nullptr, nullptr, 0, &c,
                      residual, stream);
  }
  return st;
}

int ftk_project_add_bf16(const void* x, const void* w, const void* residual, void* y, int64_t M, int64_t N,
                         int64_t K, const ftk_config* cfg, void* stream) {
  return ftk_project_add_rows_bf16(x, nullptr, w, residual, y, M, N, K, cfg, stream);
}

int ftk_linear_bf16(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K, void* stream) {
  if (x && w && (!aligned16(x) || !aligned16(w))) {
    ftk_config c = {FTK_KIND_GENERIC, 0, 0, 0, 0};
    return ftk_project_bf16(x, nullptr, 0.f, w, y, M, N, K, FTK_EPI_STORE, nullptr, 0, nullptr, nullptr, 0, &c,
                            stream);
  }
  const int st = ftk_project_bf16(x, nullptr, 0.f, w, y, M, N, K, FTK_EPI_STORE, nullptr, 0, nullptr, nullptr, 0,
                                 nullptr, stream);
  if (st == FTK_ERR_UNSUPPORTED) {  // e.g. an unsplit MFMA x slice larger than LDS: no workspace here
    ftk_config c = {FTK_KIND_GENERIC, 0, 0, 0, 0};
    return ftk_project_bf16(x, nullptr, 0.f, w, y, M, N, K, FTK_EPI_STORE, nullptr, 0, nullptr, nullptr, 0, &c,
                            stream);
  }
  return st;
}

int ftk_rms_norm_linear_bf16(const void* x, const void* gamma, float eps, const void* w, void* y, int64_t M,
                             int64_t N, int64_t K, void* stream) {
  if (gamma == nullptr) return FTK_ERR_INVALID;
  if (K % 8) return FTK_ERR_UNSUPPORTED;
  return ftk_project_bf16(x, gamma, eps, w, y, M, N, K, FTK_EPI_STORE, nullptr, 0, nullptr, nullptr, 0, nullptr,
                          stream);
}

int ftk_gate_up_swiglu_bf16(const void* x, const void* gamma, float eps, const void* w, void* y, int64_t M,
                            int64_t I, int64_t K, void* stream) {
  if (K % 8) return FTK_ERR_UNSUPPORTED;
  return ftk_project_bf16(x, gamma, eps, w, y, M, 2 * I, K, FTK_EPI_SWIGLU, nullptr, 0, nullptr, nullptr, 0,
                          nullptr, stream);
}

int ftk_lm_head_argmax_bf16(const void* x, const void* gamma, float eps, const void* w, void* logits, void* ids,
                            int ids_bytes, float* top, int64_t M, int64_t V, int64_t K, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  if (K % 8) return FTK_ERR_UNSUPPORTED;
  return ftk_project_bf16(x, gamma, eps, w, logits, M, V, K, FTK_EPI_ARGMAX, ids, ids_bytes, top, workspace,
                          workspace_bytes, nullptr, stream);
}

int ftk_lm_head_argmax_static_bf16(const void* x, const void* gamma, float eps, const void* w, void* logits,
                                   void* ids, int ids_bytes, float* top, int64_t M, int64_t V, int64_t K,
                                   void* stream) {
  if (K % 8) return FTK_ERR_UNSUPPORTED;
  if (x == nullptr || w == nullptr || ids == nullptr || (ids_bytes != 4 && ids_bytes != 8)) return FTK_ERR_INVALID;
  DeviceInfo d = device_info();
  if (!d.ok) return hip_status(hipErrorNoDevice);
  ftk_plan p;
  const int st = plan(M, V, K, FTK_EPI_ARGMAX | (gamma != nullptr ? FTK_PLAN_PROLOGUE : 0), d.cus, nullptr, &p);
  if (st != FTK_OK) return st;
  // Every key slot the finalize pass reads is written earlier in the same call,
  // so the array needs no clearing between calls.
  if (call_workspace(p, FTK_EPI_ARGMAX, gamma != nullptr) > FTK_STATIC_SCRATCH_BYTES) return FTK_ERR_TOO_LARGE;
  void* ws = nullptr;
  const int got = static_scratch(&ws);
  if (got != FTK_OK) return got;
  return project_impl(x, nullptr, gamma, eps, w, logits, M, V, K, FTK_EPI_ARGMAX, ids, ids_bytes, top, ws,
                      FTK_STATIC_SCRATCH_BYTES, nullptr, nullptr, stream);
}

int ftk_rms_norm_bf16(const void* x, int64_t row_stride, const void* gamma, void* y, int64_t rows, int64_t cols,
                      float eps, void* stream) {
  if (!x || !gamma || !y || rows < 1 || cols < 1 || row_stride < cols || rows > INT32_MAX || cols > INT32_MAX)
    return FTK_ERR_INVALID;
  return hip_status(launch_rms_norm((const uint16_t*)x, row_stride, (const uint16_t*)gamma, (uint16_t*)y, (int)rows,
                                    (int)cols, eps, reinterpret_cast<hipStream_t>(stream)));
}

int ftk_add_rms_norm_bf16(const void* x, int x_splits, int64_t x_split_stride, const void* residual,
                          const void* gamma, void* y, void* sum, int64_t rows, int64_t cols, float eps, void* stream) {
  if (!x || !residual || !gamma || !y || !sum || rows < 1 || cols < 1 || x_splits < 0 || rows > INT32_MAX ||
      cols > INT32_MAX)
    return FTK_ERR_INVALID;
  if (x_splits > 0 && x_split_stride < rows * cols) return FTK_ERR_INVALID;
  return hip_status(launch_add_rms_norm(x, x_splits, x_split_stride, (const uint16_t*)residual,
                                        (const uint16_t*)gamma, (uint16_t*)y, (uint16_t*)sum, (int)rows, (int)cols,
                                        eps, reinterpret_cast<hipStream_t>(stream)));
}

int ftk_embed_rms_norm_bf16(const void* ids, int ids_bytes, const void* table, const void* gamma, void* y,
                            void* hidden, int64_t rows, int64_t cols, float eps, void* stream) {
  if (!ids || !table || !gamma || !y || !hidden || (ids_bytes != 4 && ids_bytes != 8) || rows < 1 || cols < 1 ||
      rows > INT32_MAX || cols > INT32_MAX)
    return FTK_ERR_INVALID;
  return hip_status(launch_embed_rms_norm(ids, ids_bytes, (const uint16_t*)table, (const uint16_t*)gamma,
                                          (uint16_t*)y, (uint16_t*)hidden, (int)rows, (int)cols, eps,
                                          reinterpret_cast<hipStream_t>(stream)));
}

int ftk_swiglu_bf16(const void* packed, int splits, int64_t split_stride, void* out, int64_t rows, int64_t width,
                    void* stream) {
  if (!packed || !out || rows < 1 || width < 1 || splits < 0 || rows > INT32_MAX || width > INT32_MAX)
    return FTK_ERR_INVALID;
  if (splits > 0 && split_stride < 2 * rows * width) return FTK_ERR_INVALID;
  if (rows * width > (int64_t)UINT32_MAX * kThreads) return FTK_ERR_INVALID;
  return hip_status(launch_swiglu(packed, splits, split_stride, (uint16_t*)out, (int)rows, (int)width,
                                  reinterpret_cast<hipStream_t>(stream)));
}

int ftk_argmax_bf16(const void* logits, int64_t rows, int64_t vocab, void* ids, int ids_bytes, float* top,
                    void* workspace, int64_t workspace_bytes, void* stream) {
  if (!logits || !ids || rows < 1 || vocab < 1 || (ids_bytes != 4 && ids_bytes != 8)) return FTK_ERR_INVALID;
  if (rows > 65535 || vocab > INT32_MAX) return FTK_ERR_INVALID;
  if (workspace == nullptr || workspace_bytes < ftk_argmax_workspace_bytes(rows, vocab)) return FTK_ERR_WORKSPACE;
  return hip_status(launch_argmax((const uint16_t*)logits, (int)rows, (int)vocab, ids, ids_bytes, top,
                                  (unsigned long long*)workspace, reinterpret_cast<hipStream_t>(stream)));
}

int ftk_plan_decode_attention(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t capacity, int64_t dim,
                              int compute_units, const ftk_attn_config* cfg, ftk_attn_plan* plan) {
  if (!plan) return FTK_ERR_INVALID;
  return attn_plan(batch, q_heads, kv_heads, capacity, dim, compute_units, cfg, plan, nullptr);
}

int64_t ftk_decode_attention_workspace_bytes(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t capacity,
                                             int64_t dim, const ftk_attn_config* cfg) {
  DeviceInfo d = device_info();
  ftk_attn_plan p;
  if (!d.ok || attn_plan(batch, q_heads, kv_heads, capacity, dim, d.cus, cfg, &p, nullptr) != FTK_OK) return -1;
  return p.workspace_bytes;
}

// Plans the launch, checks the workspace and fills the fields both attention
// entry points share; `a` holds the rest (q, or the RoPE prologue's inputs).
static int run_attention(AttnArgs& a, const void* k, const void* v, const int64_t* position, int positions,
                         void* out, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t capacity, int64_t dim,
                         double scale, void* workspace, int64_t workspace_bytes, const ftk_attn_config* cfg,
                         bool rope, void* stream) {
  if (!k || !v || !position || !out) return FTK_ERR_INVALID;
  if (positions != 1 && positions != batch) return FTK_ERR_INVALID;
  if (!aligned16(k) || !aligned16(v) || !aligned16(out)) return FTK_ERR_UNSUPPORTED;
  if (rope && cfg && cfg->kind && cfg->kind != FTK_ATTN_QUAD) return FTK_ERR_UNSUPPORTED;
  DeviceInfo d = device_info();
  if (!d.ok) return FTK_ERR_INVALID;
  ftk_attn_plan p;
  AttnShape shape;
  const int st = attn_plan(batch, q_heads, kv_heads, capacity, dim, d.cus, cfg, &p, &shape);
  if (st != FTK_OK) return st;
  if (rope && p.kind != FTK_ATTN_QUAD) return FTK_ERR_UNSUPPORTED;
  float* partial = nullptr;
  float* stats = nullptr;
  if (p.splits > 1) {
    if (!workspace || workspace_bytes < p.workspace_bytes || !aligned16(workspace)) return FTK_ERR_WORKSPACE;
    partial = (float*)workspace;
    stats = partial + (size_t)shape.groups * p.splits * shape.group_size * dim;
  }
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.position = position;
  a.pos_stride = (positions == 1 && batch > 1) ? 0 : 1;
  a.out = (uint16_t*)out;
  a.partial = partial;
  a.stats = stats;
  a.kv_heads = (int)kv_heads;
  a.q_heads = (int)q_heads;
  a.capacity = (int)capacity;
  a.splits = p.splits;
  a.chunk = p.chunk;
  a.scale_log2 = (float)(scale * 1.4426950408889634);
  return hip_status(launch_attention(a, shape, reinterpret_cast<hipStream_t>(stream)));
}

int ftk_decode_attention_bf16(const void* q, const void* k, const void* v, const int64_t* position,
                              int positions, void* out, int64_t batch, int64_t q_heads, int64_t kv_heads,
                              int64_t capacity, int64_t dim, double scale, void* workspace, int64_t workspace_bytes,
                              const ftk_attn_config* cfg, void* stream) {
  if (!q) return FTK_ERR_INVALID;
  if (!aligned16(q)) return FTK_ERR_UNSUPPORTED;
  AttnArgs a{};
  a.q = (const uint16_t*)q;
  return run_attention(a, k, v, position, positions, out, batch, q_heads, kv_heads, capacity, dim, scale, workspace,
                       workspace_bytes, cfg, false, stream);
}

int ftk_rope_decode_attention_bf16(const void* packed, const void* q_gain, const void* k_gain, float q_eps,
                                   float k_eps, const void* cos, const void* sin, int64_t table_rows,
                                   const int64_t* position, int positions, const int64_t* phases, void* keys,
                                   void* values, void* out, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                   int64_t capacity, int64_t dim, double scale, void* workspace,
                                   int64_t workspace_bytes, const ftk_attn_config* cfg, void* stream) {
  if (!packed || !q_gain || !k_gain || !cos || !sin || table_rows < 1) return FTK_ERR_INVALID;
  if (!aligned16(packed) || !aligned16(q_gain) || !aligned16(k_gain) || !aligned16(cos) || !aligned16(sin))
    return FTK_ERR_UNSUPPORTED;
  if (dim != 128) return FTK_ERR_UNSUPPORTED;
  AttnArgs a{};
  a.packed = (const uint16_t*)packed;
  a.q_gain = (const uint16_t*)q_gain;
  a.k_gain = (const uint16_t*)k_gain;
  a.q_eps = q_eps;
  a.k_eps = k_eps;
  a.cos = (const uint16_t*)cos;
  a.sin = (const uint16_t*)sin;
  a.table_rows = table_rows;
  a.phases = phases;
  a.k_store = (uint16_t*)keys;
  a.v_store = (uint16_t*)values;
  return run_attention(a, keys, values, position, positions, out, batch, q_heads, kv_heads, capacity, dim, scale,
                       workspace, workspace_bytes, cfg, true, stream);
}

int ftk_qk_rope_cache_bf16(const void* packed, int splits, int64_t split_stride, const void* q_gain,
                           const void* k_gain, float q_eps, float k_eps, const void* cos, const void* sin,
                           int64_t table_rows, const int64_t* position, const int64_t* phases, void* query,
                           void* keys, void* values, int64_t batch, int64_t tokens, int64_t q_heads,
                           int64_t kv_heads, int64_t capacity, int64_t dim, int mode, void* stream) {
  if (!packed || !q_gain || !k_gain || !cos || !sin || !query || !keys || !values) return FTK_ERR_INVALID;
  if (batch < 1 || tokens < 1 || q_heads < 1 || kv_heads < 1 || capacity < 1 || table_rows < 1 || splits < 1)
    return FTK_ERR_INVALID;
  if (mode & ~(FTK_ROPE_PREFILL | FTK_ROPE_ROWS | FTK_ROPE_TABLE)) return FTK_ERR_INVALID;
  if ((mode & FTK_ROPE_PREFILL) && (mode & FTK_ROPE_ROWS)) return FTK_ERR_INVALID;
  if ((mode & FTK_ROPE_TABLE) && (!(mode & FTK_ROPE_ROWS) || !phases)) return FTK_ERR_INVALID;
  if (!(mode & FTK_ROPE_PREFILL) && !position) return FTK_ERR_INVALID;
  if (tokens > capacity || (splits > 1 && split_stride < batch * tokens * (q_heads + 2 * kv_heads) * dim))
    return FTK_ERR_INVALID;
  if (!(mode & FTK_ROPE_TABLE) && table_rows < ((mode & FTK_ROPE_ROWS) ? batch * tokens : tokens))
    return FTK_ERR_INVALID;  // shared [1, T, D] or per-row [B, T, D] rows must cover every phase
  if (dim != 64 && dim != 128) return FTK_ERR_UNSUPPORTED;
  if (batch * tokens > INT32_MAX / 2 || q_heads + kv_heads > 65535 * 4 || capacity > INT32_MAX) return FTK_ERR_INVALID;
  const void* ptrs[] = {packed, q_gain, k_gain, cos, sin, query, keys, values};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) & 3u) return FTK_ERR_UNSUPPORTED;
  RopeArgs a;
  a.packed = packed;
  a.splits = splits;
  a.split_stride = split_stride;
  a.q_gain = (const uint16_t*)q_gain;
  a.k_gain = (const uint16_t*)k_gain;
  a.q_eps = q_eps;
  a.k_eps = k_eps;
  a.cos = (const uint16_t*)cos;
  a.sin = (const uint16_t*)sin;
  a.table_rows = table_rows;
  a.position = position;
  a.phases = phases;
  a.query = (uint16_t*)query;
  a.keys = (uint16_t*)keys;
  a.values = (uint16_t*)values;
  a.tokens = (int)tokens;
  a.q_heads = (int)q_heads;
  a.kv_heads = (int)kv_heads;
  a.capacity = (int)capacity;
  a.dim = (int)dim;
  a.mode = mode;
  return hip_status(launch_qk_rope(a, (int)(batch * tokens), reinterpret_cast<hipStream_t>(stream)));
}

int ftk_stream_read(const void* src, int64_t bytes, void* sink, int grid, int loads, void* stream) {
  if (!src || !sink || bytes < 16 || bytes % 16 != 0 || grid < 0 || !aligned16(src)) return FTK_ERR_INVALID;
  if (loads != 2 && loads != 4 && loads != 8 && loads != 16) return FTK_ERR_INVALID;
  if (grid == 0 && stream_read_once_grid(bytes, loads) > INT32_MAX) return FTK_ERR_INVALID;
  return hip_status(launch_stream_read(src, bytes, (uint32_t*)sink, grid, loads,
                                       reinterpret_cast<hipStream_t>(stream)));
}

int ftk_merge_splits_bf16(const float* partial, int64_t splits, int64_t count, void* out, void* stream) {
  if (!partial || !out || splits < 1 || count < 1 || splits > INT32_MAX) return FTK_ERR_INVALID;
  if (count > (int64_t)UINT32_MAX * kThreads) return FTK_ERR_INVALID;
  return hip_status(launch_merge_splits(partial, (int)splits, count, (uint16_t*)out,
                                        reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"
