// M = 1..4 skinny BF16 projection as an HBM-streaming GEMV for gfx950.
//
// Computes the sums of engine/kernels/linear.py:27-47 (_gemv): y[m, n] =
// bf16(sum_k f32(x[m, k]) * f32(W[n, k])), FP32 accumulation, one rounding,
// with three fused extras the reference runs as separate launches:
//   * RMSNorm prologue (engine/kernels/rmsnorm.py:21-46 cast order),
//   * SwiGLU epilogue over cat(W_gate, W_up) (engine/kernels/swiglu.py:13-24),
//   * greedy-argmax epilogue (engine/kernels/argmax.py:19-48, :73-106).
//
// Layout and schedule:
//   * A workgroup is 4 waves. It stages x (normalised when the prologue is on)
//     in LDS once, then walks row tiles grid-stride.
//   * The 4 waves form 4 / KW row groups; a group owns RPW whole weight rows
//     per tile and its KW waves split K by interleaved 1 KiB chunk blocks
//     (KW > 1 gives small-N shapes enough workgroups). Lane l of a wave reads
//     16-byte chunks l, l + 64, ... of its blocks, so every wave-wide load is
//     1 KiB of contiguous HBM; loads are non-temporal (weights are read once).
//   * The first batch of weight loads is issued before x is staged.
//   * Products use v_dot2_f32_bf16 (two exact BF16 products + FP32 add per
//     instruction, no unpacking), accumulating per lane in FP32.
//   * Each row's lane partials are summed with a DPP tree, the KW wave totals
//     in LDS in wave order; the result is rounded to BF16 once.
//   * Argmax: per-row keys (orderable BF16 value, inverted index) reduced by
//     max within the workgroup and stored per workgroup; a second small kernel
//     reduces the workgroups (the two stages of engine/kernels/argmax.py:19-48).
//     max is order-independent, so the result is deterministic and equals
//     torch.argmax's lowest-index rule. No workgroup ever waits on another.
#include "ftk_device.h"
#include "ftk_internal.h"

namespace ftk {

template <int MR, int RPW, int U, int KW, bool PRO, int EPI>
__global__ __launch_bounds__(kThreads) void gemv_kernel(ProjArgs a, int tiles) {
  extern __shared__ u32x4_t xs[];  // x as [MR][K/8] chunks of 8 BF16 (+ the gain when PRO)
  __shared__ float red[MR][kWaves];
  __shared__ float part[kWaves][RPW][MR];
  __shared__ unsigned long long best_lds[kWaves][MR];

  constexpr int GROUPS = kWaves / KW;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = wave / KW, kw = wave - grp * KW;
  const int K = a.K;
  const int KC = K >> 3;  // 16-byte chunks per row

  // ---- the weight rows this wave streams -------------------------------------
  constexpr int PW = (EPI == EPI_SWIGLU) ? RPW / 2 : RPW;  // outputs per row group per tile
  const int outputs = gemv_outputs(EPI, a.N);
  unsigned long long best[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) best[m] = 0ull;

  // This lane's first chunk (block kw) of every weight row the group reads for ``tile``.
  auto row_ptrs = [&](int tile, const uint16_t* (&wr)[RPW]) {
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int col = gemv_output(tile, grp, p, PW, GROUPS);
      const int c = col < outputs ? col : outputs - 1;  // clamp: loads stay in bounds
      const size_t first = (size_t)(kw * 64 + lane) * 8;
      wr[p] = a.w + (size_t)gemv_weight_row(EPI, c, 0, a.N) * K + first;
      if constexpr (EPI == EPI_SWIGLU) wr[PW + p] = a.w + (size_t)gemv_weight_row(EPI, c, 1, a.N) * K + first;
    }
  };

  const uint16_t* wr[RPW];
  const bool full = KC % (64 * U * KW) == 0;
  constexpr size_t kStep = (size_t)KW * 512;  // elements between this wave's consecutive chunk blocks
  u32x4_t pre[U][RPW];
  if (full) {
    // The first batch of weight loads goes out before x is staged, so its HBM
    // latency overlaps the staging instead of following it (grid <= tiles).
    row_ptrs(blockIdx.x, wr);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < RPW; ++r) pre[u][r] = load_stream16(wr[r] + u * kStep);
  }

  // ---- stage x (and the RMSNorm gain) into LDS, then the prologue ----------
  // The gain is staged in the same pass as x, so the prologue pays one load
  // latency (hidden behind the weight prefetch above), not two in sequence.
  u32x4_t* gs = xs + MR * KC;  // [K/8] gain chunks, prologue only
  if constexpr (PRO) {
    for (int c = tid; c < KC; c += kThreads) gs[c] = load16(a.gamma + (size_t)c * 8);
  }
  float ss[MR];
  const bool keep = PRO && a.sum != nullptr && blockIdx.x == 0;  // workgroup 0 stores x + residual
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    ss[m] = 0.f;
    const uint16_t* xr = PRO ? x_row(a, m) : a.x + (size_t)m * K;
    for (int c = tid; c < KC; c += kThreads) {
      const u32x4_t v = PRO ? prologue_in(a, xr, m, (size_t)c * 8) : load16(xr + (size_t)c * 8);
      xs[m * KC + c] = v;
      if constexpr (PRO) {
        ss[m] = sum_squares8(v, ss[m]);
        if (keep) store16(a.sum + (size_t)m * K + (size_t)c * 8, v);
      }
    }
  }
  if constexpr (PRO) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float s = wave_sum(ss[m]);
      if (lane == 0) red[m][wave] = s;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      // Same fixed order in every workgroup: every workgroup normalises identically.
      const float scale = rms_scale(red[m], K, a.eps);
      for (int c = tid; c < KC; c += kThreads) xs[m * KC + c] = norm8(xs[m * KC + c], gs[c], scale);
    }
  }
  __syncthreads();

  // Reduce the partials of ``tile`` (lanes, then the group's KW waves in wave
  // order), run the epilogue on the group's first wave, clear the accumulators.
  auto finish = [&](int tile, float (&acc)[RPW][MR]) {
    float tot[RPW][MR];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        tot[r][m] = wave_sum(acc[r][m]);
        acc[r][m] = 0.f;
      }
    if constexpr (KW > 1) {
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
          for (int m = 0; m < MR; ++m) part[wave][r][m] = tot[r][m];
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          float t = part[grp * KW][r][m];
#pragma unroll
          for (int j = 1; j < KW; ++j) t += part[grp * KW + j][r][m];
          tot[r][m] = t;
        }
      __syncthreads();  // part[] is rewritten by the next tile
    }
    if (kw != 0) return;
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int col = gemv_output(tile, grp, p, PW, GROUPS);
      if (col >= outputs) continue;
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if constexpr (EPI == EPI_STORE) {
          if (lane == 0) a.y[(size_t)m * a.N + col] = (uint16_t)store_bits(a, tot[p][m], m, col);
        } else if constexpr (EPI == EPI_SWIGLU) {
          if (lane == 0) a.y[(size_t)m * (a.N / 2) + col] = (uint16_t)swiglu_bf16(tot[p][m], tot[PW + p][m]);
        } else {
          const uint32_t bits = f32_to_bf16(tot[p][m]);
          if (a.y != nullptr && lane == 0) a.y[(size_t)m * a.N + col] = (uint16_t)bits;
          best[m] = key_max(best[m], argmax_key(bf16_to_f32(bits), (uint32_t)col));
        }
      }
    }
  };

  float acc[RPW][MR];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[r][m] = 0.f;

  if (full) {
    // Every lane's chunks are in range: batches of U x RPW 16-byte loads, all
    // issued before the first is consumed. Memory parallelism comes from the
    // batch size and from the other waves resident on the SIMD.
    const int NB = KC / (64 * U * KW);
    bool first = true;
    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
      if (!first) row_ptrs(tile, wr);
      for (int b = 0; b < NB; ++b) {
        u32x4_t wv[U][RPW];
        if (first) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int r = 0; r < RPW; ++r) wv[u][r] = pre[u][r];
          first = false;
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int r = 0; r < RPW; ++r) wv[u][r] = load_stream16(wr[r] + (size_t)(b * U + u) * kStep);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = ((b * U + u) * KW + kw) * 64 + lane;
#pragma unroll
          for (int m = 0; m < MR; ++m) {
            const u32x4_t xv = xs[m * KC + c];
#pragma unroll
            for (int r = 0; r < RPW; ++r) acc[r][m] = dot8(wv[u][r], xv, acc[r][m]);
          }
        }
      }
      finish(tile, acc);
    }
  } else {
    // Ragged chunk count: per-lane bounds checks.
    const int C = (KC + 63) >> 6;  // chunk blocks per row
    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
      row_ptrs(tile, wr);
      for (int j = kw; j < C; j += KW) {
        const int c = j * 64 + lane;
        if (c < KC) {
          u32x4_t wv[RPW];
#pragma unroll
          for (int r = 0; r < RPW; ++r) wv[r] = load_stream16(wr[r] + (size_t)(j - kw) * 512);
#pragma unroll
          for (int m = 0; m < MR; ++m) {
            const u32x4_t xv = xs[m * KC + c];
#pragma unroll
            for (int r = 0; r < RPW; ++r) acc[r][m] = dot8(wv[r], xv, acc[r][m]);
          }
        }
      }
      finish(tile, acc);
    }
  }

  if constexpr (EPI == EPI_ARGMAX) {
    // This workgroup's best key per input row; the finalize pass reduces the workgroups.
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MR; ++m) best_lds[wave][m] = best[m];
    }
    __syncthreads();
    if (tid < MR) {
      unsigned long long k = best_lds[0][tid];
      for (int w = 1; w < kWaves; ++w) k = key_max(k, best_lds[w][tid]);
      a.keys[(size_t)blockIdx.x * MR + tid] = k;
    }
  }
}

// ---- ragged / unaligned fallback: one wave per weight row, scalar loads --------
template <int MAXM>
__global__ __launch_bounds__(kThreads) void gemm_generic_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ w,
                                                                uint16_t* y, const uint16_t* add, int M, int N,
                                                                int K) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= N) return;  // whole wave leaves together; no barrier below
  float acc[MAXM];
#pragma unroll
  for (int m = 0; m < MAXM; ++m) acc[m] = 0.f;
  const uint16_t* wr = w + (size_t)row * K;
  for (int k = lane; k < K; k += 64) {
    const float wk = bf16_to_f32(wr[k]);
#pragma unroll
    for (int m = 0; m < MAXM; ++m)
      if (m < M) acc[m] += bf16_to_f32(x[(size_t)m * K + k]) * wk;
  }
#pragma unroll
  for (int m = 0; m < MAXM; ++m) {
    if (m < M) {
      const float s = wave_sum(acc[m]);
      if (lane == 0) {
        const uint32_t b = f32_to_bf16(s);
        y[(size_t)m * N + row] =
            (uint16_t)(add == nullptr ? b : f32_to_bf16(bf16_to_f32(b) + bf16_to_f32(add[(size_t)m * N + row])));
      }
    }
  }
}

// ---- dispatch -------------------------------------------------------------------

typedef void (*GemvKernel)(ProjArgs, int);

// Instantiated launch shapes: (rows per group, unroll, waves per group).
#define FTK_GEMV_SHAPES(MR, PRO, EPI)   \
  FTK_GEMV_SHAPE(MR, 2, 4, 1, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 4, 2, 1, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 4, 4, 1, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 8, 1, 1, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 8, 2, 1, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 1, 1, 2, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 2, 1, 2, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 1, 2, 2, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 2, 2, 2, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 2, 4, 2, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 1, 1, 4, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 2, 1, 4, PRO, EPI) \
  FTK_GEMV_SHAPE(MR, 2, 2, 4, PRO, EPI)

#define FTK_GEMV_SHAPE(MR, R, U, KW, PRO, EPI) \
  if (rpw == R && unroll == U && kw == KW) return gemv_kernel<MR, R, U, KW, PRO, EPI>;

template <int MR, bool PRO, int EPI>
static GemvKernel pick_shape(int rpw, int unroll, int kw) {
  if constexpr (EPI == EPI_SWIGLU) {
    // A SwiGLU row group needs a gate row and its up row: even RPW only.
    if (rpw % 2) return nullptr;
    if (rpw == 2 && unroll == 4 && kw == 1) return gemv_kernel<MR, 2, 4, 1, PRO, EPI>;
    if (rpw == 4 && unroll == 2 && kw == 1) return gemv_kernel<MR, 4, 2, 1, PRO, EPI>;
    if (rpw == 4 && unroll == 4 && kw == 1) return gemv_kernel<MR, 4, 4, 1, PRO, EPI>;
    if (rpw == 8 && unroll == 1 && kw == 1) return gemv_kernel<MR, 8, 1, 1, PRO, EPI>;
    if (rpw == 8 && unroll == 2 && kw == 1) return gemv_kernel<MR, 8, 2, 1, PRO, EPI>;
    if (rpw == 2 && unroll == 1 && kw == 2) return gemv_kernel<MR, 2, 1, 2, PRO, EPI>;
    if (rpw == 2 && unroll == 2 && kw == 2) return gemv_kernel<MR, 2, 2, 2, PRO, EPI>;
    if (rpw == 2 && unroll == 4 && kw == 2) return gemv_kernel<MR, 2, 4, 2, PRO, EPI>;
    if (rpw == 2 && unroll == 1 && kw == 4) return gemv_kernel<MR, 2, 1, 4, PRO, EPI>;
    if (rpw == 2 && unroll == 2 && kw == 4) return gemv_kernel<MR, 2, 2, 4, PRO, EPI>;
    return nullptr;
  } else {
    FTK_GEMV_SHAPES(MR, PRO, EPI)
    return nullptr;
  }
}
#undef FTK_GEMV_SHAPE

template <int MR>
static GemvKernel pick_mr(int rpw, int unroll, int kw, bool pro, int epi) {
  switch (epi) {
    case EPI_STORE: return pro ? pick_shape<MR, true, EPI_STORE>(rpw, unroll, kw)
                               : pick_shape<MR, false, EPI_STORE>(rpw, unroll, kw);
    case EPI_SWIGLU: return pro ? pick_shape<MR, true, EPI_SWIGLU>(rpw, unroll, kw)
                                : pick_shape<MR, false, EPI_SWIGLU>(rpw, unroll, kw);
    case EPI_ARGMAX: return pro ? pick_shape<MR, true, EPI_ARGMAX>(rpw, unroll, kw)
                                : pick_shape<MR, false, EPI_ARGMAX>(rpw, unroll, kw);
  }
  return nullptr;
}

static GemvKernel pick_gemv(int M, int rpw, int unroll, int kw, bool pro, int epi) {
  switch (M) {
    case 1: return pick_mr<1>(rpw, unroll, kw, pro, epi);
    case 2: return pick_mr<2>(rpw, unroll, kw, pro, epi);
    case 3: return pick_mr<3>(rpw, unroll, kw, pro, epi);
    case 4: return pick_mr<4>(rpw, unroll, kw, pro, epi);
  }
  return nullptr;
}

bool gemv_supported(int M, int rpw, int unroll, int kw, int epi) {
  return pick_gemv(M, rpw, unroll, kw, false, epi) != nullptr;
}

hipError_t launch_gemv(const ProjArgs& a, int epi, const GemvShape& s, hipStream_t stream) {
  GemvKernel k = pick_gemv(a.M, s.rpw, s.unroll, s.kw, a.gamma != nullptr, epi);
  if (k == nullptr) return hipErrorInvalidValue;
  const size_t lds = s.lds + (a.gamma != nullptr ? (size_t)a.K * 2 : 0);  // + the staged gain
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k, dim3(s.grid), dim3(kThreads), lds, stream, a, s.tiles);
  return hipGetLastError();
}

hipError_t launch_gemm_generic(const uint16_t* x, const uint16_t* w, uint16_t* y, const uint16_t* add, int M, int N,
                               int K, hipStream_t stream) {
  const int grid = (N + kWaves - 1) / kWaves;
  if (M <= 4)
    hipLaunchKernelGGL(gemm_generic_kernel<4>, dim3(grid), dim3(kThreads), 0, stream, x, w, y, add, M, N, K);
  else if (M <= 16)
    hipLaunchKernelGGL(gemm_generic_kernel<16>, dim3(grid), dim3(kThreads), 0, stream, x, w, y, add, M, N, K);
  else
    hipLaunchKernelGGL(gemm_generic_kernel<32>, dim3(grid), dim3(kThreads), 0, stream, x, w, y, add, M, N, K);
  return hipGetLastError();
}

}  // namespace ftk
