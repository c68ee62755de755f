// M = 5..16 skinny BF16 projection, STAGE kind: the weight stream of the QUAD
// kind (4 rows x 256 contiguous bytes per wave load) feeding 16x16x32 BF16
// MFMAs (v_mfma_f32_16x16x32_bf16) through a per-wave LDS staging buffer.
//
// Same sums, roundings and fused extras as the other kinds
// (engine/kernels/linear.py:50-78 _skinny_gemm; RMSNorm prologue
// engine/kernels/rmsnorm.py:21-46; SwiGLU engine/kernels/swiglu.py:13-24;
// greedy argmax engine/kernels/argmax.py:19-48), FP32 accumulation, one rounding.
//
// Why: a 16x16x32 MFMA needs 16 weight rows x 8 k per wave in its A operand, so
// loaded directly every wave load covers 16 rows x 64 bytes, the slowest
// pattern measured on MI355X; the 4x4x4 MFMA of the QUAD kind takes the fast
// 4 rows x 256 bytes directly but needs four times the MFMA issue per byte at
// 16 x rows. Here the fast loads go to LDS and come back in MFMA layout: one
// MFMA per KiB of weights, one LDS write and one LDS read.
//
// Layout and schedule:
//   * A workgroup is KW waves splitting K; wave kw owns the 128-wide K segments
//     j KW + kw (j < C, K = 128 C KW). A tile is T subtiles of 16 weight rows.
//   * A unit of work is one segment of one tile: per subtile four loads (row set
//     r: lane 4 b + i gets row 4 r + i, chunk b), 4 T KiB per wave. The loads
//     of the next U units are in flight at all times, across tile boundaries.
//   * Per unit and subtile, the wave writes its four loads to its own 4 KiB of
//     LDS and reads back the A operand of four MFMA steps (lane l: row l % 16,
//     chunk 4 s + l / 16). Only this wave touches that memory, so no barrier:
//     a wave's LDS instructions execute in order.
//   * The x slice (B operand, lane l: x row l % 16 at the same k) is resident in
//     registers, or, for the long K without the prologue, streamed beside the
//     weights with the same lookahead. With the prologue the row scales are found
//     first (sums of squares, one barrier), and each K segment of the slice is
//     normalised in the first tile right before its MFMAs, with the gain read
//     from LDS: that VALU work overlaps the weight stream instead of delaying it.
//   * Per-tile 16 x 16 partials wait in LDS. After every DMAX tiles of the walk
//     (and after the last) a barrier lets the workgroup sum the KW partials in
//     wave order (deterministic) and run the epilogue on those tiles' outputs;
//     the next tiles' loads are in flight meanwhile. So a workgroup may walk any
//     number of tiles, and the grid can match the CUs exactly (no partial last
//     round of workgroups).
#include "ftk_device.h"
#include "ftk_internal.h"

namespace ftk {

template <int T, int C, int KW, int U, bool PRO, int EPI>
__global__ __launch_bounds__(64 * KW) void stage_kernel(ProjArgs a, int tiles) {
  static_assert(C % U == 0, "the window must tile the segments of a tile");
  static_assert(EPI != EPI_SWIGLU || T % 2 == 0, "SwiGLU pairs gate and up subtiles");
  constexpr int DMAX = stage_max_depth(T, KW);
  constexpr bool XS = !PRO && C > 4;          // long K without the prologue: x streamed
  constexpr size_t kStep = (size_t)KW * 128;  // elements between a wave's segments
  __shared__ f32x4_t part[DMAX][KW][T][64];
  __shared__ u32x4_t stage[KW][256];          // one subtile's 16 rows x 16 chunks per wave
  __shared__ float red[KW][16];
  __shared__ unsigned long long best_lds[KW][16];
  constexpr int GCH = PRO ? 16 * C * KW : 1;  // 16-byte chunks of the RMSNorm gain (K / 8)
  __shared__ u32x4_t gain[GCH];

  const int tid = threadIdx.x, lane = tid & 63, kw = tid >> 6;
  const int i4 = lane & 3, cb = lane >> 2;   // load layout: row i4 of a row set, chunk cb
  const int li = lane & 15, g = lane >> 4;   // MFMA layout: weight / x row li, k quarter g
  const int M = a.M, K = a.K;                // K == 128 C KW (checked by the planner)
  const bool mine = li < M;                  // this lane's x row is real
  const size_t seg0 = (size_t)kw * 128;
  // Element of x (and the gain) that lane l feeds to MFMA step s of segment j.
  auto xoff = [&](int j, int s) { return seg0 + (size_t)j * kStep + 32 * s + 8 * g; };
  // Staging slot of (row, chunk), XOR-swizzled: the loads' writes (rows 4 r + i,
  // chunks 0..3 per 16 lanes) and the MFMA reads (rows 0..15, one chunk per 16
  // lanes) each fall in 16 distinct 16-byte bank groups.
  auto slot_of = [](int row, int chunk) { return row * 16 + (chunk ^ (4 * (row & 3) + (row >> 2))); };
  u32x4_t* st = stage[kw];

  // ---- the gain first (for LDS), then the x slice (normalised in place with the
  // prologue) -----------------------------------------------------------------------
  constexpr int GPT = (GCH + 64 * KW - 1) / (64 * KW);  // gain chunks per thread
  u32x4_t gload[PRO ? GPT : 1];
  if constexpr (PRO) {
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int c = tid + i * 64 * KW;
      if (c < GCH) gload[i] = load16(a.gamma + (size_t)c * 8);
    }
  }
  // With the prologue, row li is x[li] or the gathered x[x_ids[li]], plus the residual.
  const uint16_t* xrow = (PRO && mine) ? x_row(a, li) : a.x + (size_t)(mine ? li : 0) * K;
  auto x_frag = [&](int j, int s) { return mine ? load16(xrow + xoff(j, s)) : u32x4_t{0u, 0u, 0u, 0u}; };
  // x streamed beside the weights: lanes past the last row read row M - 1 again
  // (in bounds). Unconditional loads keep branches out of the main loop (their
  // joins would wait for each load); those lanes feed only MFMA output columns
  // li >= M, which are never stored.
  const uint16_t* xs_row = a.x + (size_t)(mine ? li : M - 1) * K;
  auto x_stream = [&](int j, int s) { return load16(xs_row + xoff(j, s)); };
  u32x4_t xr[XS ? 1 : C][4];
  u32x4_t xv[XS ? U : 1][4];
  if constexpr (!XS) {
#pragma unroll
    for (int j = 0; j < C; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        xr[j][s] = !mine ? u32x4_t{0u, 0u, 0u, 0u} : PRO ? prologue_in(a, xrow, li, xoff(j, s)) : x_frag(j, s);
  }

  // ---- the first U units of the first tile ---------------------------------------
  const int wg = blockIdx.x;
  int tile = wg;  // grid <= tiles
  auto rows_of = [&](int tl, const uint16_t* (&p)[T][4]) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        p[t][r] = a.w + (size_t)mfma_weight_row(EPI, tl, t, 4 * r + i4, a.N, T) * K + seg0 + 8 * cb;
  };
  const uint16_t* wp[T][4];
  rows_of(tile, wp);
  u32x4_t wv[U][T][4];
#pragma unroll
  for (int q = 0; q < U; ++q) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) wv[q][t][r] = load_stream16(wp[t][r] + q * kStep);
    if constexpr (XS) {
#pragma unroll
      for (int s = 0; s < 4; ++s) xv[q][s] = x_stream(q, s);
    }
  }

  // ---- RMSNorm prologue: row sums of squares over (wave, quarter, step) in order.
  // Only the scale is found here; each K segment is normalised in the first tile,
  // right before its MFMAs, so that work overlaps the weight stream. -------------
  float scale = 0.f;
  if constexpr (PRO) {
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int c = tid + i * 64 * KW;
      if (c < GCH) gain[c] = gload[i];
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < C; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s) ss = sum_squares8(xr[j][s], ss);
    ss += __shfl_xor(ss, 16);  // the four lane quarters holding row li, pairwise:
    ss += __shfl_xor(ss, 32);  // (g0 + g1) + (g2 + g3) in every one of them
    if (g == 0) red[kw][li] = ss;
    // The rows the norm reads (x + residual) go out once, from workgroup 0.
    if (a.sum != nullptr && blockIdx.x == 0 && mine) {
#pragma unroll
      for (int j = 0; j < C; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s) store16(a.sum + (size_t)li * K + xoff(j, s), xr[j][s]);
    }
    __syncthreads();
    float total = red[0][li];
#pragma unroll
    for (int w = 1; w < KW; ++w) total += red[w][li];
    scale = 1.0f / sqrtf(total / (float)K + a.eps);
  }

  // ---- epilogue of parked tiles: thread e takes (tile i, subtile t, lane position ln)
  // D[4 gg + r][ll] of subtile t: weight row 16 t + 4 gg + r of the tile, x row ll.
  // part[0 .. n) holds the walk's tiles done .. done + n - 1 (tile wg + i grid).
  constexpr int TO = (EPI == EPI_SWIGLU) ? T / 2 : T;  // output subtiles
  const int outputs = gemv_outputs(EPI, a.N);
  unsigned long long best = 0ull;
  auto flush = [&](int n, int done) {
    const int entries = n * TO * 64;
    for (int e = tid; e < entries; e += 64 * KW) {
      const int ln = e & 63, t = (e >> 6) % TO, i = e / (64 * TO);
      const int ll = ln & 15, gg = ln >> 4;
      if (ll >= M) continue;
      const int tl = wg + (done + i) * (int)gridDim.x;
      f32x4_t s = part[i][0][t][ln];
#pragma unroll
      for (int w = 1; w < KW; ++w) s += part[i][w][t][ln];
      if constexpr (EPI == EPI_SWIGLU) {
        f32x4_t u = part[i][0][t + T / 2][ln];
#pragma unroll
        for (int w = 1; w < KW; ++w) u += part[i][w][t + T / 2][ln];
        const int c0 = tl * 8 * T + t * 16 + 4 * gg;
        uint16_t* yr = a.y + (size_t)ll * outputs;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (c0 + r < outputs) yr[c0 + r] = (uint16_t)swiglu_bf16(s[r], u[r]);
      } else {
        const int n0 = tl * 16 * T + t * 16 + 4 * gg;
        uint32_t bits[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (EPI == EPI_STORE)
            bits[r] = n0 + r < a.N ? store_bits(a, s[r], ll, n0 + r) : 0u;
          else
            bits[r] = f32_to_bf16(s[r]);
        }
        if (a.y != nullptr) {
          uint16_t* yr = a.y + (size_t)ll * a.N;
          if (n0 + 3 < a.N && (a.N & 3) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 7) == 0) {
            *reinterpret_cast<u32x2_t*>(yr + n0) = u32x2_t{bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n0 + r < a.N) yr[n0 + r] = (uint16_t)bits[r];
          }
        }
        if constexpr (EPI == EPI_ARGMAX) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n0 + r < a.N) best = key_max(best, argmax_key(bf16_to_f32(bits[r]), (uint32_t)(n0 + r)));
        }
      }
    }
  };

  // ---- tiles: stage each unit through LDS into the MFMAs, refill the window.
  // Every DMAX tiles (and after the last) the parked partials are summed and
  // stored; the next tiles' loads stay in flight across those two barriers. ----
  int count = 0, done = 0;
  for (;;) {
    const int next = tile + (int)gridDim.x;
    const bool more = next < tiles;
    const uint16_t* wn[T][4];
    if (more) rows_of(next, wn);
    f32x4_t acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const int q = j % U;
      if constexpr (PRO) {
        if (count == 0 && done == 0) {  // first tile: normalise this segment of the slice in place
#pragma unroll
          for (int s = 0; s < 4; ++s) xr[j][s] = norm8(xr[j][s], gain[xoff(j, s) >> 3], scale);
        }
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) st[slot_of(4 * r + i4, cb)] = wv[q][t][r];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const u32x4_t w = st[slot_of(li, 4 * s + g)];
          acc[t] = mfma16x16x32(w, XS ? xv[q][s] : xr[XS ? 0 : j][s], acc[t]);
        }
        __builtin_amdgcn_wave_barrier();
      }
      // refill the freed slot: segment j + U of this tile, or of the next
      if (j + U < C) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) wv[q][t][r] = load_stream16(wp[t][r] + (j + U) * kStep);
        if constexpr (XS) {
#pragma unroll
          for (int s = 0; s < 4; ++s) xv[q][s] = x_stream(j + U, s);
        }
      } else if (more) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) wv[q][t][r] = load_stream16(wn[t][r] + (j + U - C) * kStep);
        if constexpr (XS) {
#pragma unroll
          for (int s = 0; s < 4; ++s) xv[q][s] = x_stream(j + U - C, s);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) part[count][kw][t][lane] = acc[t];
    ++count;
    if (count == DMAX || !more) {  // workgroup-uniform: every wave walks the same tiles
      __syncthreads();
      flush(count, done);
      done += count;
      count = 0;
      if (!more) break;
      __syncthreads();  // the next tiles park in the same slots
    }
    tile = next;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) wp[t][r] = wn[t][r];
  }

  if constexpr (EPI == EPI_ARGMAX) {
    // Lanes ll, ll + 16, ll + 32, ll + 48 of every wave hold keys of x row ll.
    best = key_max(best, __shfl_xor(best, 16));
    best = key_max(best, __shfl_xor(best, 32));
    if (g == 0) best_lds[kw][li] = best;
    __syncthreads();
    if (tid < M) {
      unsigned long long k = best_lds[0][tid];
      for (int w = 1; w < KW; ++w) k = key_max(k, best_lds[w][tid]);
      a.keys[(size_t)blockIdx.x * M + tid] = k;
    }
  }
}

// ---- dispatch -------------------------------------------------------------------

typedef void (*StageKernel)(ProjArgs, int);

// Instantiated (T, C, KW, U): K = 4096 (C = 4 at KW = 8) with two or four
// segments in flight; without the prologue, K = 12288 (C = 12 at KW = 8, x
// streamed).
#define FTK_STAGE_SHAPES_EVEN(PRO, EPI) \
  FTK_STAGE_SHAPE(2, 4, 8, 2, PRO, EPI) \
  FTK_STAGE_SHAPE(2, 4, 8, 4, PRO, EPI)

#define FTK_STAGE_SHAPES_ONE(PRO, EPI)  \
  FTK_STAGE_SHAPE(1, 4, 8, 2, PRO, EPI) \
  FTK_STAGE_SHAPE(1, 4, 8, 4, PRO, EPI)

#define FTK_STAGE_SHAPES_LONG(EPI)        \
  FTK_STAGE_SHAPE(1, 12, 8, 3, false, EPI) \
  FTK_STAGE_SHAPE(1, 12, 8, 4, false, EPI)

#define FTK_STAGE_SHAPE(T_, C_, KW_, U_, PRO, EPI) \
  if (t == T_ && c == C_ && kw == KW_ && u == U_) return stage_kernel<T_, C_, KW_, U_, PRO, EPI>;

template <bool PRO, int EPI>
static StageKernel pick_stage_shape(int t, int c, int kw, int u) {
  FTK_STAGE_SHAPES_EVEN(PRO, EPI)
  if constexpr (EPI != EPI_SWIGLU) {
    FTK_STAGE_SHAPES_ONE(PRO, EPI)
    if constexpr (!PRO) {
      FTK_STAGE_SHAPES_LONG(EPI)
    }
  }
  return nullptr;
}
#undef FTK_STAGE_SHAPE

static StageKernel pick_stage(int t, int c, int kw, int u, bool pro, int epi) {
  switch (epi) {
    case EPI_STORE: return pro ? pick_stage_shape<true, EPI_STORE>(t, c, kw, u)
                               : pick_stage_shape<false, EPI_STORE>(t, c, kw, u);
    case EPI_SWIGLU: return pro ? pick_stage_shape<true, EPI_SWIGLU>(t, c, kw, u)
                                : pick_stage_shape<false, EPI_SWIGLU>(t, c, kw, u);
    case EPI_ARGMAX: return pro ? pick_stage_shape<true, EPI_ARGMAX>(t, c, kw, u)
                                : pick_stage_shape<false, EPI_ARGMAX>(t, c, kw, u);
  }
  return nullptr;
}

bool stage_supported(int M, int t, int K, int kw, int unroll, int epi, bool pro) {
  const int c = quad_segments(K, kw);
  return M >= 1 && M <= kStageMaxRows && c > 0 && pick_stage(t, c, kw, unroll, pro, epi) != nullptr;
}

hipError_t launch_stage(const ProjArgs& a, int epi, const StageShape& sh, hipStream_t stream) {
  const int c = quad_segments(a.K, sh.kw);
  StageKernel k = c > 0 ? pick_stage(sh.subtiles, c, sh.kw, sh.unroll, a.gamma != nullptr, epi) : nullptr;
  if (k == nullptr || a.M < 1 || a.M > kStageMaxRows) return hipErrorInvalidValue;
  if (sh.grid < 1 || sh.grid > sh.tiles) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(sh.grid), dim3(64 * sh.kw), 0, stream, a, sh.tiles);
  return hipGetLastError();
}

}  // namespace ftk
