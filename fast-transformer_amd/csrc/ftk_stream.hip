// M = 1..8 skinny BF16 projection, STREAM kind: an HBM-streaming GEMV whose
// x slice lives in registers, for K = 512 C KW (every model shape of the path).
//
// Same sums, roundings and fused extras as the GEMV kind (engine/kernels/linear.py:27-47
// _gemv; RMSNorm prologue engine/kernels/rmsnorm.py:21-46; SwiGLU epilogue
// engine/kernels/swiglu.py:13-24; greedy-argmax epilogue engine/kernels/argmax.py:19-48),
// and for the same (rows per group, KW) the same FP32 sums bit for bit: lane l of
// wave kw accumulates chunks (j KW + kw) 64 + l in j order, the DPP tree sums the
// lanes, the KW wave totals are added in wave order.
//
// What differs is the schedule, built to keep HBM busy from the first cycle to
// the last:
//   * Lane l only ever multiplies its own C chunks of K, so it loads those chunks
//     of x (normalised in registers when the prologue is on) once, and never
//     touches LDS in the main loop.
//   * Rolling prefetch: as each weight chunk of tile i is consumed, the load of
//     the same chunk of tile i + 1 is issued into the register it frees, so a
//     wave keeps RPW x C 16-byte loads in flight through its whole life.
//   * Every load of the prologue (x, the residual, the gain) and the first
//     tile's weights are issued before any of them is waited for; a load under
//     a condition would compile to a branch whose join waits for it.
//   * No barrier inside the tile loop: each wave's per-tile totals wait in LDS,
//     and one barrier at the end lets all threads combine the KW totals and run
//     the epilogue for every output of the workgroup (the argmax keeps one wave
//     when every output fits it).
//   * One wave per row group (KW = 1): a wave holds its rows' whole sums, so it
//     stores its outputs as soon as a tile is summed, with no LDS round and no
//     barrier, and forms its rows' norm scale itself.
//   * lm_head + argmax can finish in the same launch: the walkers publish their
//     keys and one extra workgroup, dispatched last, gathers them
//     (argmax_gather).
#include "ftk_device.h"
#include "ftk_internal.h"

namespace ftk {

// MR: rows the kernel is built for; a.M <= MR rows are real (the rest are zero
// and never stored). W: waves per workgroup (4, or 8 when KW = 8).
template <int MR, int RPW, int C, int KW, int W, bool PRO, int EPI>
__global__ __launch_bounds__(64 * W) void stream_kernel(ProjArgs a, int tiles) {
  constexpr int T = 64 * W;
  constexpr int GROUPS = W / KW;
  constexpr int PW = (EPI == EPI_SWIGLU) ? RPW / 2 : RPW;  // outputs per row group per tile
  constexpr size_t kStep = (size_t)KW * 512;                // elements between a lane's chunks
  __shared__ float part[kStreamMaxTiles][W][RPW][MR];       // wave totals per tile
  __shared__ float red[MR][kWaves];
  __shared__ unsigned long long best_lds[W][MR];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = wave / KW, kw = wave - grp * KW;
  const int K = a.K;  // == 512 C KW (checked by the planner)
  const int M = a.M;  // <= MR
  const int outputs = gemv_outputs(EPI, a.N);
  const size_t first = (size_t)(kw * 64 + lane) * 8;  // this lane's chunk j = 0
  int walkers = (int)gridDim.x;  // workgroups walking tiles
  if constexpr (EPI == EPI_ARGMAX) {
    if (a.fused) {
      walkers -= kGatherExtra;
      if ((int)blockIdx.x >= walkers) {  // the extra workgroups walk no tiles; the last gathers
        if ((int)blockIdx.x == walkers + kGatherExtra - 1) argmax_gather<T, MR>(a, walkers, &best_lds[0][0]);
        return;
      }
    }
  }

  auto row_ptrs = [&](int tile, const uint16_t* (&wr)[RPW]) {
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int col = gemv_output(tile, grp, p, PW, GROUPS);
      const int c = col < outputs ? col : outputs - 1;  // clamp: loads stay in bounds
      wr[p] = a.w + (size_t)gemv_weight_row(EPI, c, 0, a.N) * K + first;
      if constexpr (EPI == EPI_SWIGLU) wr[PW + p] = a.w + (size_t)gemv_weight_row(EPI, c, 1, a.N) * K + first;
    }
  };

  // ---- this lane's slice of x (and of the residual and the gain) ------------
  // Small, mostly cache hits, issued first: loads complete in issue order, so
  // the prologue below waits for these and not for the weight batch issued
  // after them. Nothing is computed from a load before the weights are in
  // flight: the residual add waits until then (an add at the load would be a
  // join behind a runtime branch, and the join waits for the load). With the
  // prologue, row m is x[m] or the gathered x[x_ids[m]], plus the residual.
  const uint16_t* xrow[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) xrow[m] = (PRO && m < M) ? x_row(a, m) : a.x + (size_t)m * K;
  auto x_in = [&](int m, size_t k) { return PRO ? prologue_in(a, xrow[m], m, k) : load16(xrow[m] + k); };
  u32x4_t xr[MR][C];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int j = 0; j < C; ++j)  // row 0 is always real (M >= 1): no branch around its loads
      xr[m][j] = (m == 0 || m < M) ? load16(xrow[m] + first + j * kStep) : u32x4_t{0u, 0u, 0u, 0u};
  const bool residual = PRO && a.residual != nullptr;
  u32x4_t rr[PRO ? MR : 1][PRO ? C : 1];
  if constexpr (PRO) {
    if (residual) {
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int j = 0; j < C; ++j)
          if (m == 0 || m < M) rr[m][j] = load16(a.residual + (size_t)m * K + first + j * kStep);
    }
  }
  u32x4_t g[PRO ? C : 1];
  if constexpr (PRO) {
#pragma unroll
    for (int j = 0; j < C; ++j) g[j] = load16(a.gamma + first + j * kStep);
  }

  // ---- first tile's weights in flight before the prologue -------------------
  const int wg = blockIdx.x;  // tiles wg, wg + grid, ... (grid <= tiles)
  int tile = wg;
  const uint16_t* wr[RPW];
  row_ptrs(tile, wr);
  u32x4_t wv[C][RPW];
#pragma unroll
  for (int j = 0; j < C; ++j)
#pragma unroll
    for (int r = 0; r < RPW; ++r) wv[j][r] = load_stream16(wr[r] + j * kStep);
  if constexpr (PRO) {
    if (residual) {  // s = bf16(x + residual), as prologue_in forms it
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int j = 0; j < C; ++j)
          if (m == 0 || m < M) xr[m][j] = add8(xr[m][j], rr[m][j]);
    }
  }

  // ---- RMSNorm prologue: normalise the slice in registers -------------------
  if constexpr (PRO && KW == 1) {
    // One wave per row group holds every chunk of the row: lane l's chunk j is
    // j 64 + l. The other kinds' thread t < 256 sums chunks t, t + 256, ..., i.e.
    // wave w's lane l sums chunks j = w, w + 4, ... of this lane. So each wave
    // forms those four per-wave sums itself, in that order, reduces each with the
    // same DPP tree and adds them in wave order: the same scale bits, no barrier.
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float parts[kWaves];
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        float ss = 0.f;
#pragma unroll
        for (int j = w; j < C; j += kWaves) ss = sum_squares8(xr[m][j], ss);
        parts[w] = wave_sum(ss);
      }
      if (a.sum != nullptr && blockIdx.x == 0 && wave == 0 && m < M) {
#pragma unroll
        for (int j = 0; j < C; ++j) store16(a.sum + (size_t)m * K + first + j * kStep, xr[m][j]);
      }
      const float scale = rms_scale(parts, K, a.eps);
#pragma unroll
      for (int j = 0; j < C; ++j) xr[m][j] = norm8(xr[m][j], g[j], scale);
    }
  } else if constexpr (PRO) {
    // Sum of squares in the thread order of the other kinds' prologues
    // (thread t < 256: chunks t, t + 256, ...), so every kind scales a row
    // alike. With KW = W = 4 thread t's own chunks (4 j + wave) 64 + lane are
    // exactly those, in that order. With one chunk per lane (C = 1) and
    // KW <= 4, the first row group's thread t holds chunk t and every chunk
    // is below 64 KW, so the other threads add nothing. Otherwise the first
    // 4 waves re-read x (after the weight window: those loads wait for it).
    constexpr bool kOwnChunks = (KW == kWaves && W == kWaves) || (C == 1 && KW <= kWaves);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float ss = 0.f;
      if constexpr (kOwnChunks) {
        if (grp == 0) {
#pragma unroll
          for (int j = 0; j < C; ++j) ss = sum_squares8(xr[m][j], ss);
        }
      } else {
        const int KC = K >> 3;
        if (m < M && tid < kThreads)
          for (int c = tid; c < KC; c += kThreads) ss = sum_squares8(x_in(m, (size_t)c * 8), ss);
      }
      const float s = wave_sum(ss);
      if (lane == 0 && wave < kWaves) red[m][wave] = s;
    }
    // The normalised rows themselves (x + residual) go out once, from workgroup 0
    // (its first row group covers all of K).
    if (a.sum != nullptr && blockIdx.x == 0 && grp == 0) {
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M)
#pragma unroll
          for (int j = 0; j < C; ++j) store16(a.sum + (size_t)m * K + first + j * kStep, xr[m][j]);
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float scale = rms_scale(red[m], K, a.eps);
#pragma unroll
      for (int j = 0; j < C; ++j) xr[m][j] = norm8(xr[m][j], g[j], scale);
    }
  }

  // ---- tiles: consume, prefetch the next tile chunk by chunk, park the totals
  int count = 0;
  for (;;) {
    const int next = tile + walkers;
    float acc[RPW][MR];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[r][m] = 0.f;
    if (next < tiles) {
      const uint16_t* wn[RPW];
      row_ptrs(next, wn);
#pragma unroll
      for (int j = 0; j < C; ++j)
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          // Consume, then reload the same register: the new load never has to
          // live beside the old value, so it needs no copy at the loop edge.
#pragma unroll
          for (int m = 0; m < MR; ++m) acc[r][m] = dot8(wv[j][r], xr[m][j], acc[r][m]);
          wv[j][r] = load_stream16(wn[r] + j * kStep);
        }
    } else {
#pragma unroll
      for (int j = 0; j < C; ++j)
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
          for (int m = 0; m < MR; ++m) acc[r][m] = dot8(wv[j][r], xr[m][j], acc[r][m]);
    }
    if constexpr (KW == 1 && EPI != EPI_ARGMAX) {
      // The wave holds its rows' whole sums: it finishes its outputs now, with no
      // LDS round and no barrier (lane 0 stores; the sums are wave-uniform).
#pragma unroll
      for (int p = 0; p < PW; ++p) {
        const int col = gemv_output(tile, grp, p, PW, GROUPS);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const float s = wave_sum(acc[p][m]);
          if constexpr (EPI == EPI_STORE) {
            if (lane == 0 && m < M && col < outputs) a.y[(size_t)m * a.N + col] = (uint16_t)store_bits(a, s, m, col);
          } else {
            const float u = wave_sum(acc[PW + p][m]);
            if (lane == 0 && m < M && col < outputs) a.y[(size_t)m * (a.N / 2) + col] = (uint16_t)swiglu_bf16(s, u);
          }
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const float t = wave_sum(acc[r][m]);
          if (lane == 0) part[count][wave][r][m] = t;
        }
    }
    ++count;
    if (next >= tiles) break;
    tile = next;
  }
  if constexpr (KW == 1 && EPI != EPI_ARGMAX) return;  // every output is stored
  __syncthreads();

  // ---- epilogue: every thread takes outputs (tile i, group, slot) ------------
  // The argmax keeps one wave when every output of the walk fits it: that wave
  // alone reduces the keys, so no second barrier (the others leave now).
  constexpr bool kOneWave = EPI == EPI_ARGMAX && kStreamMaxTiles * GROUPS * PW <= 64;
  if (kOneWave && wave != 0) return;
  unsigned long long best[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) best[m] = 0ull;
  const int entries = count * GROUPS * PW;  // count is the same in every wave of the workgroup
  for (int e = kOneWave ? lane : tid; e < entries; e += kOneWave ? 64 : T) {
    const int p = e % PW;
    const int g = (e / PW) % GROUPS;
    const int i = e / (PW * GROUPS);
    const int col = gemv_output(wg + i * walkers, g, p, PW, GROUPS);
    if (col >= outputs) continue;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= M) break;
      float s = part[i][g * KW][p][m];
#pragma unroll
      for (int k = 1; k < KW; ++k) s += part[i][g * KW + k][p][m];
      if constexpr (EPI == EPI_STORE) {
        a.y[(size_t)m * a.N + col] = (uint16_t)store_bits(a, s, m, col);
      } else if constexpr (EPI == EPI_SWIGLU) {
        float u = part[i][g * KW][PW + p][m];
#pragma unroll
        for (int k = 1; k < KW; ++k) u += part[i][g * KW + k][PW + p][m];
        a.y[(size_t)m * (a.N / 2) + col] = (uint16_t)swiglu_bf16(s, u);
      } else {
        const uint32_t bits = f32_to_bf16(s);
        if (a.y != nullptr) a.y[(size_t)m * a.N + col] = (uint16_t)bits;
        best[m] = key_max(best[m], argmax_key(bf16_to_f32(bits), (uint32_t)col));
      }
    }
  }

  if constexpr (kOneWave) {
    // This workgroup's best key per input row (lane m publishes row m); the
    // finalize pass (or the gathering workgroup) reduces the workgroups.
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      best[m] = wave_max_key(best[m]);
      if (lane == m && m < M) publish_key(a, (size_t)blockIdx.x * M + m, best[m]);
    }
  } else if constexpr (EPI == EPI_ARGMAX) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      best[m] = wave_max_key(best[m]);
      if (lane == 0) best_lds[wave][m] = best[m];
    }
    __syncthreads();
    if (tid < M) {
      unsigned long long k = best_lds[0][tid];
      for (int w = 1; w < W; ++w) k = key_max(k, best_lds[w][tid]);
      publish_key(a, (size_t)blockIdx.x * M + tid, k);
    }
  }
}

// ---- dispatch -------------------------------------------------------------------

typedef void (*StreamKernel)(ProjArgs, int);

// Instantiated (rows per group, C, KW): the K of each model shape of the path
// (1024, 2048, 3072, 4096, 12288) with two or three row-group sizes each; the
// 8-row kernel (M = 5..8) for the 8B model's K (4096, 12288).
#define FTK_STREAM_SHAPES(MR, PRO, EPI)   \
  FTK_STREAM_SHAPE(MR, 2, 1, 2, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 4, 1, 2, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 8, 1, 2, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 2, 1, 4, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 4, 1, 4, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 2, 3, 2, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 4, 3, 2, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 2, 2, 4, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 4, 2, 4, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 8, 2, 4, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 2, 6, 4, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 4, 6, 4, PRO, EPI) \
  FTK_STREAM_SHAPE(MR, 2, 3, 8, PRO, EPI)

#define FTK_STREAM_SHAPES_8(PRO, EPI)    \
  FTK_STREAM_SHAPE(8, 2, 2, 4, PRO, EPI) \
  FTK_STREAM_SHAPE(8, 4, 2, 4, PRO, EPI) \
  FTK_STREAM_SHAPE(8, 2, 3, 8, PRO, EPI) \
  FTK_STREAM_SHAPE(8, 4, 3, 8, PRO, EPI)

// One wave per row group (KW = 1, whole rows per wave, no barrier in the
// epilogue) at one x row: the K of the Qwen3 shapes up to 4096, and 512 / 1536
// (the O and down rows of a Qwen3-8B eight-way tensor-parallel shard). One row
// per wave only where there is no SwiGLU (which pairs a gate and an up row).
#define FTK_STREAM_SHAPES_KW1(PRO, EPI) \
  FTK_STREAM_SHAPE(1, 2, 1, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 2, 2, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 2, 3, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 2, 4, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 2, 6, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 2, 8, 1, PRO, EPI)
#define FTK_STREAM_SHAPES_KW1_ROW(PRO, EPI) \
  FTK_STREAM_SHAPE(1, 1, 1, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 1, 2, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 1, 3, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 1, 4, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 1, 6, 1, PRO, EPI) \
  FTK_STREAM_SHAPE(1, 1, 8, 1, PRO, EPI)

#define FTK_STREAM_SHAPE(MR, R, CC, KW, PRO, EPI) \
  if (rpw == R && c == CC && kw == KW) return stream_kernel<MR, R, CC, KW, (KW > kWaves ? KW : kWaves), PRO, EPI>;

template <int MR, bool PRO, int EPI>
static StreamKernel pick_stream_shape(int rpw, int c, int kw) {
  if constexpr (MR == kStreamMaxRows) {
    FTK_STREAM_SHAPES_8(PRO, EPI)
  } else {
    FTK_STREAM_SHAPES(MR, PRO, EPI)
  }
  if constexpr (MR == 1) {
    FTK_STREAM_SHAPES_KW1(PRO, EPI)
    if constexpr (EPI != EPI_SWIGLU) {
      FTK_STREAM_SHAPES_KW1_ROW(PRO, EPI)
    }
  }
  return nullptr;
}
#undef FTK_STREAM_SHAPE

template <int MR>
static StreamKernel pick_stream_mr(int rpw, int c, int kw, bool pro, int epi) {
  switch (epi) {
    case EPI_STORE: return pro ? pick_stream_shape<MR, true, EPI_STORE>(rpw, c, kw)
                               : pick_stream_shape<MR, false, EPI_STORE>(rpw, c, kw);
    case EPI_SWIGLU: return pro ? pick_stream_shape<MR, true, EPI_SWIGLU>(rpw, c, kw)
                                : pick_stream_shape<MR, false, EPI_SWIGLU>(rpw, c, kw);
    case EPI_ARGMAX: return pro ? pick_stream_shape<MR, true, EPI_ARGMAX>(rpw, c, kw)
                                : pick_stream_shape<MR, false, EPI_ARGMAX>(rpw, c, kw);
  }
  return nullptr;
}

static StreamKernel pick_stream(int M, int rpw, int c, int kw, bool pro, int epi) {
  switch (M) {
    case 1: return pick_stream_mr<1>(rpw, c, kw, pro, epi);
    case 2: return pick_stream_mr<2>(rpw, c, kw, pro, epi);
    case 3: return pick_stream_mr<3>(rpw, c, kw, pro, epi);
    case 4: return pick_stream_mr<4>(rpw, c, kw, pro, epi);
    case 5:
    case 6:
    case 7:
    case 8: return pick_stream_mr<kStreamMaxRows>(rpw, c, kw, pro, epi);
  }
  return nullptr;
}

bool stream_supported(int M, int rpw, int K, int kw, int epi) {
  const int c = stream_chunks(K, kw);
  return c > 0 && pick_stream(M, rpw, c, kw, false, epi) != nullptr;
}

hipError_t launch_stream(const ProjArgs& a, int epi, const StreamShape& s, hipStream_t stream) {
  const int c = stream_chunks(a.K, s.kw);
  StreamKernel k = c > 0 ? pick_stream(a.M, s.rpw, c, s.kw, a.gamma != nullptr, epi) : nullptr;
  if (k == nullptr) return hipErrorInvalidValue;
  // Every workgroup walks at most kStreamMaxTiles tiles (their totals wait in LDS).
  if (s.grid < 1 || s.grid > s.tiles || (s.tiles + s.grid - 1) / s.grid > kStreamMaxTiles)
    return hipErrorInvalidValue;
  // With the one-launch argmax, kGatherExtra more workgroups than the walkers: the last gathers the keys.
  const int grid = s.grid + (epi == EPI_ARGMAX && a.fused ? kGatherExtra : 0);
  hipLaunchKernelGGL(k, dim3(grid), dim3(64 * stream_waves(s.kw)), 0, stream, a, s.tiles);
  return hipGetLastError();
}

}  // namespace ftk
