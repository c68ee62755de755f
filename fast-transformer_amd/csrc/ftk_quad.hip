// M = 2..16 skinny BF16 projection, QUAD kind: the STREAM schedule with the
// 16-block 4x4x4 BF16 MFMA (v_mfma_f32_4x4x4_16b_bf16) doing the products.
//
// Same sums, roundings and fused extras as the other kinds
// (engine/kernels/linear.py:50-78 _skinny_gemm; RMSNorm prologue
// engine/kernels/rmsnorm.py:21-46; SwiGLU engine/kernels/swiglu.py:13-24;
// greedy argmax engine/kernels/argmax.py:19-48), FP32 accumulation, one rounding.
//
// Why this MFMA: its A operand is what one 16-byte-per-lane load of "4 weight
// rows x 256 contiguous bytes" already holds. Lane l = 4 b + i loads 8 BF16 of
// weight row i at K chunk b of a 128-wide K segment, which is A_b[i][0..3] and
// A_b[i][4..7] of two MFMAs (block b = chunk b). So the weights stream in wide
// row-contiguous pieces, straight from HBM into MFMA operands, with no LDS
// staging. The matching B operand (lane 4 b + j: x row 4 q + j at chunk b)
// is this lane's own slice of x, loaded once into registers.
//
// Layout and schedule:
//   * A workgroup is W waves in row groups of KW waves; a row group owns 4 RS
//     weight rows per tile (SwiGLU: 2 RS gate rows and the matching up rows of
//     cat(W_gate, W_up)), wave kw of the group reads the K segments j KW + kw,
//     j < C (K = 128 C KW).
//   * D_b[i][j] of each 4x4 block accumulates over the lane's segments; at the
//     end of a tile the 16 blocks (lane bits 2..5) are summed by a transposing
//     reduction: two shuffle steps halve the four items per lane, two DPP row
//     rotations finish, and each lane holds one (row, x row) total.
//   * Rolling prefetch: as each weight load of tile i is consumed, the same
//     load of tile i + 1 is issued into the register it frees.
//   * Per-tile wave totals wait in LDS; one barrier at the end, then the
//     workgroup adds the KW totals in wave order (deterministic, independent of
//     the grid) and runs the epilogue for every output of its tiles.
#include "ftk_device.h"
#include "ftk_internal.h"

namespace ftk {

// Sum of a 16-block accumulator over its blocks (lane bits 2..5). Lane l
// returns the total of element (l >> 4) & 3 for x column l & 3; lanes that
// differ only in bits 2 and 3 return the same bits.
__device__ __forceinline__ float quad_block_sum(f32x4_t v, int lane) {
  const bool h5 = (lane & 32) != 0, h4 = (lane & 16) != 0;
  // bit 5: keep elements {2 h5, 2 h5 + 1}, hand the other two to lane ^ 32
  const float a0 = h5 ? v[2] : v[0], a1 = h5 ? v[3] : v[1];
  const float s0 = h5 ? v[0] : v[2], s1 = h5 ? v[1] : v[3];
  const float u0 = a0 + __shfl_xor(s0, 32), u1 = a1 + __shfl_xor(s1, 32);
  // bit 4: keep element 2 h5 + h4
  float w = (h4 ? u1 : u0) + __shfl_xor(h4 ? u0 : u1, 16);
  // bits 3 and 2, inside each row of 16 lanes
  w += dpp<0x128, 0xF>(w);  // row_ror:8
  w += dpp<0x124, 0xF>(w);  // row_ror:4
  return w;
}

// MQ: groups of 4 x rows the kernel is built for (a.M <= 4 MQ are real; the
// rest are zero and never stored). W: waves per workgroup (4, or KW when KW > 4).
template <int MQ, int RS, int C, int KW, int W, bool PRO, int EPI>
__global__ __launch_bounds__(64 * W) void quad_kernel(ProjArgs a, int tiles) {
  static_assert(EPI != EPI_SWIGLU || RS % 2 == 0, "SwiGLU pairs gate and up row sets");
  constexpr int T = 64 * W;
  constexpr int GROUPS = W / KW;
  constexpr int R = 4 * RS;                            // weight rows per row group per tile
  constexpr int PW = (EPI == EPI_SWIGLU) ? R / 2 : R;  // outputs per row group per tile
  constexpr int MX = 4 * MQ;
  constexpr size_t kStep = (size_t)KW * 128;  // elements between a lane's segments
  __shared__ float part[kStreamMaxTiles][W][R][MX];
  __shared__ float red[W][MX];
  __shared__ unsigned long long best_lds[W][MX];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave / KW, kw = wave - grp * KW;
  const int i4 = lane & 3;  // weight row in a row set; x row in a group of 4
  const int K = a.K;        // == 128 C KW (checked by the planner)
  const int M = a.M;        // <= 4 MQ
  const int outputs = gemv_outputs(EPI, a.N);
  const size_t first = (size_t)kw * 128 + (size_t)(lane >> 2) * 8;  // segment j = 0, chunk b

  auto row_ptrs = [&](int tile, const uint16_t* (&wr)[RS]) {
#pragma unroll
    for (int r = 0; r < RS; ++r) {
      const int half = (EPI == EPI_SWIGLU && r >= RS / 2) ? 1 : 0;
      const int col = gemv_output(tile, grp, 4 * (r - half * (RS / 2)) + i4, PW, GROUPS);
      const int c = col < outputs ? col : outputs - 1;  // clamp: loads stay in bounds
      wr[r] = a.w + (size_t)gemv_weight_row(EPI, c, half, a.N) * K + first;
    }
  };

  // ---- this lane's slice of x: rows 4 q + i4 at its segments ------------------
  // With the prologue, row m is x[m] or the gathered x[x_ids[m]], plus the residual.
  u32x4_t xr[MQ][C];
#pragma unroll
  for (int q = 0; q < MQ; ++q) {
    const int m = 4 * q + i4;
    const bool real = m < M;
    const uint16_t* xrow = (PRO && real) ? x_row(a, m) : a.x + (size_t)(real ? m : 0) * K;
#pragma unroll
    for (int j = 0; j < C; ++j)
      xr[q][j] = !real ? u32x4_t{0u, 0u, 0u, 0u}
                       : PRO ? prologue_in(a, xrow, m, first + j * kStep) : load16(xrow + first + j * kStep);
  }
  // The gain too, before the weights: loads complete in issue order, so the
  // prologue then waits for x and the gain only, never for the weight window.
  u32x4_t gv[PRO ? C : 1];
  if constexpr (PRO) {
#pragma unroll
    for (int j = 0; j < C; ++j) gv[j] = load16(a.gamma + first + j * kStep);
  }

  // ---- the first tile's weight window: in flight during the prologue, except
  // where the prologue's raw rows, residual and gain would not fit in the
  // registers beside it (then issued right after the prologue) -----------------
  constexpr bool LATE = quad_late(MQ, RS, C, KW, PRO);
  const int wg = blockIdx.x;  // tiles wg, wg + grid, ... (grid <= tiles)
  int tile = wg;
  u32x4_t wv[C][RS];
  auto first_window = [&]() {
    const uint16_t* wr[RS];
    row_ptrs(tile, wr);
#pragma unroll
    for (int j = 0; j < C; ++j)
#pragma unroll
      for (int r = 0; r < RS; ++r) wv[j][r] = load_stream16(wr[r] + j * kStep);
  };
  if constexpr (!LATE) first_window();

  // ---- RMSNorm prologue: the row scales ----------------------------------------
  float scale[MQ];
  if constexpr (PRO) {
    // Row m's sum of squares: each lane over its segments in order, the 16
    // lanes of the row, then the KW waves of the row group in wave order.
#pragma unroll
    for (int q = 0; q < MQ; ++q) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < C; ++j) ss = sum_squares8(xr[q][j], ss);
      ss = quad_lane_sum(ss);
      if (lane < 4) red[wave][4 * q + lane] = ss;
    }
    // The rows the norm reads (x + residual) go out once, from workgroup 0's
    // first row group (its KW waves cover all of K).
    if (a.sum != nullptr && blockIdx.x == 0 && grp == 0) {
#pragma unroll
      for (int q = 0; q < MQ; ++q)
        if (4 * q + i4 < M)
#pragma unroll
          for (int j = 0; j < C; ++j) store16(a.sum + (size_t)(4 * q + i4) * K + first + j * kStep, xr[q][j]);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < MQ; ++q) {
      float total = red[grp * KW][4 * q + i4];
#pragma unroll
      for (int w = 1; w < KW; ++w) total += red[grp * KW + w][4 * q + i4];
      scale[q] = 1.0f / sqrtf(total / (float)K + a.eps);
    }
    // Only the scales are found here: each K segment of the slice is normalised
    // in the first tile right before its MFMAs, so that VALU work overlaps the
    // weight stream instead of delaying it.
  }
  if constexpr (LATE) first_window();

  // ---- tiles: consume, prefetch the next tile load by load, park the totals ----
  int count = 0;
  for (;;) {
    const int next = tile + (int)gridDim.x;
    const bool more = next < tiles;
    const uint16_t* wn[RS];
    if (more) row_ptrs(next, wn);
    f32x4_t acc[RS][MQ];
#pragma unroll
    for (int r = 0; r < RS; ++r)
#pragma unroll
      for (int q = 0; q < MQ; ++q) acc[r][q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < C; ++j) {
      if constexpr (PRO) {
        if (count == 0) {  // first tile: normalise this segment of the slice in place
          float gf[8];
          widen8(gv[j], gf);  // the gain of a chunk, widened once for the MQ rows that use it
#pragma unroll
          for (int q = 0; q < MQ; ++q) xr[q][j] = norm8w(xr[q][j], gf, scale[q]);
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < RS; ++r) {
          const u32x4_t wvr = wv[j][r];
          const uint32_t w0 = wvr[2 * h], w1 = wvr[2 * h + 1];
#pragma unroll
          for (int q = 0; q < MQ; ++q) {
            const u32x4_t xq = xr[q][j];
            acc[r][q] = mfma4x4x4(w0, w1, xq[2 * h], xq[2 * h + 1], acc[r][q]);
          }
        }
      // Both halves consumed: reload the same registers with the next tile's load.
      if (more) {
#pragma unroll
        for (int r = 0; r < RS; ++r) wv[j][r] = load_stream16(wn[r] + j * kStep);
      }
    }
#pragma unroll
    for (int r = 0; r < RS; ++r)
#pragma unroll
      for (int q = 0; q < MQ; ++q) {
        const float t = quad_block_sum(acc[r][q], lane);
        if ((lane & 12) == 0) part[count][wave][4 * r + ((lane >> 4) & 3)][4 * q + i4] = t;
      }
    ++count;
    if (!more) break;
    tile = next;
  }
  __syncthreads();

  // ---- epilogue: every thread takes outputs (tile i, group, slot) --------------
  unsigned long long best[MX];
#pragma unroll
  for (int m = 0; m < MX; ++m) best[m] = 0ull;
  const int entries = count * GROUPS * PW;  // count is the same in every wave of the workgroup
  for (int e = tid; e < entries; e += T) {
    const int p = e % PW;
    const int g = (e / PW) % GROUPS;
    const int i = e / (PW * GROUPS);
    const int col = gemv_output(wg + i * (int)gridDim.x, g, p, PW, GROUPS);
    if (col >= outputs) continue;
#pragma unroll
    for (int m = 0; m < MX; ++m) {
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

  if constexpr (EPI == EPI_ARGMAX) {
    // This workgroup's best key per input row; the finalize pass reduces the workgroups.
#pragma unroll
    for (int m = 0; m < MX; ++m) {
      best[m] = wave_max_key(best[m]);
      if (lane == 0) best_lds[wave][m] = best[m];
    }
    __syncthreads();
    if (tid < M) {
      unsigned long long k = best_lds[0][tid];
      for (int w = 1; w < W; ++w) k = key_max(k, best_lds[w][tid]);
      a.keys[(size_t)blockIdx.x * M + tid] = k;
    }
  }
}

// ---- dispatch -------------------------------------------------------------------

typedef void (*QuadKernel)(ProjArgs, int);

// Instantiated (row sets RS, segments per lane C, KW), where they fit the
// registers (quad_fits): K = 4096 (the 8B model's QKV, O, gate/up, lm_head)
// with 4 or 8 waves splitting K and up to 24 rows per tile; K = 12288 (down)
// with 8 or 16; K = 1024 / 2048 / 3072 (the 0.6B model) with 4.
#define FTK_QUAD_SHAPES(MQ, PRO, EPI)   \
  FTK_QUAD_SHAPE(MQ, 2, 8, 4, PRO, EPI)  \
  FTK_QUAD_SHAPE(MQ, 4, 8, 4, PRO, EPI)  \
  FTK_QUAD_SHAPE(MQ, 2, 4, 8, PRO, EPI)  \
  FTK_QUAD_SHAPE(MQ, 4, 4, 8, PRO, EPI)  \
  FTK_QUAD_SHAPE(MQ, 6, 4, 8, PRO, EPI)  \
  FTK_QUAD_SHAPE(MQ, 2, 12, 8, PRO, EPI) \
  FTK_QUAD_SHAPE(MQ, 2, 6, 16, PRO, EPI) \
  FTK_QUAD_SHAPE(MQ, 2, 2, 4, PRO, EPI)  \
  FTK_QUAD_SHAPE(MQ, 2, 4, 4, PRO, EPI)  \
  FTK_QUAD_SHAPE(MQ, 2, 6, 4, PRO, EPI)

// Single row sets (store / argmax only; SwiGLU needs a gate and an up set).
#define FTK_QUAD_SHAPES_ONE(MQ, PRO, EPI) \
  FTK_QUAD_SHAPE(MQ, 1, 8, 4, PRO, EPI)   \
  FTK_QUAD_SHAPE(MQ, 1, 4, 8, PRO, EPI)   \
  FTK_QUAD_SHAPE(MQ, 1, 12, 8, PRO, EPI)

#define FTK_QUAD_SHAPE(MQ, RS_, CC, KW_, PRO, EPI)                                                  \
  if constexpr (quad_fits(MQ, RS_, CC, KW_, PRO)) {                                                 \
    if (rs == RS_ && c == CC && kw == KW_) return quad_kernel<MQ, RS_, CC, KW_, (KW_ > kWaves ? KW_ : kWaves), PRO, EPI>; \
  }

template <int MQ, bool PRO, int EPI>
static QuadKernel pick_quad_shape(int rs, int c, int kw) {
  FTK_QUAD_SHAPES(MQ, PRO, EPI)
  if constexpr (EPI != EPI_SWIGLU) {
    FTK_QUAD_SHAPES_ONE(MQ, PRO, EPI)
  }
  return nullptr;
}
#undef FTK_QUAD_SHAPE

template <int MQ>
static QuadKernel pick_quad_mq(int rs, int c, int kw, bool pro, int epi) {
  switch (epi) {
    case EPI_STORE: return pro ? pick_quad_shape<MQ, true, EPI_STORE>(rs, c, kw)
                               : pick_quad_shape<MQ, false, EPI_STORE>(rs, c, kw);
    case EPI_SWIGLU: return pro ? pick_quad_shape<MQ, true, EPI_SWIGLU>(rs, c, kw)
                                : pick_quad_shape<MQ, false, EPI_SWIGLU>(rs, c, kw);
    case EPI_ARGMAX: return pro ? pick_quad_shape<MQ, true, EPI_ARGMAX>(rs, c, kw)
                                : pick_quad_shape<MQ, false, EPI_ARGMAX>(rs, c, kw);
  }
  return nullptr;
}

static QuadKernel pick_quad(int M, int rs, int c, int kw, bool pro, int epi) {
  switch (quad_groups(M)) {
    case 1: return pick_quad_mq<1>(rs, c, kw, pro, epi);
    case 2: return pick_quad_mq<2>(rs, c, kw, pro, epi);
    case 4: return pick_quad_mq<4>(rs, c, kw, pro, epi);
  }
  return nullptr;
}

bool quad_supported(int M, int rows, int K, int kw, int epi, bool pro) {
  const int c = quad_segments(K, kw);
  return c > 0 && rows % 4 == 0 && pick_quad(M, rows / 4, c, kw, pro, epi) != nullptr;
}

hipError_t launch_quad(const ProjArgs& a, int epi, const QuadShape& s, hipStream_t stream) {
  const int c = quad_segments(a.K, s.kw);
  QuadKernel k = (c > 0 && s.rows % 4 == 0) ? pick_quad(a.M, s.rows / 4, c, s.kw, a.gamma != nullptr, epi) : nullptr;
  if (k == nullptr || a.M < 1 || a.M > kQuadMaxRows) return hipErrorInvalidValue;
  // Every workgroup walks at most kStreamMaxTiles tiles (their totals wait in LDS).
  if (s.grid < 1 || s.grid > s.tiles || (s.tiles + s.grid - 1) / s.grid > kStreamMaxTiles)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(s.grid), dim3(64 * stream_waves(s.kw)), 0, stream, a, s.tiles);
  return hipGetLastError();
}

}  // namespace ftk
