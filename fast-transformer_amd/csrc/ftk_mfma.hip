// M = 4..32 skinny BF16 projection on gfx950 MFMA (v_mfma_f32_16x16x32_bf16).
//
// The same sums as the GEMV kind and as the reference's tile kinds
// (engine/kernels/linear.py:50-78 _skinny_gemm, engine/kernels/gemm.py:51-116):
// y[m, n] = bf16(sum_k f32(x[m, k]) * f32(W[n, k])), FP32 accumulation, one rounding.
//
// Layout and schedule:
//   * A workgroup (W = 4, 8 or 16 waves) owns 16 T weight rows (T MFMA row subtiles; for
//     SwiGLU half of them are gate rows and half the matching up rows) over the
//     whole of K. No workgroup ever waits for another: there is no split-K
//     across workgroups and no device-scope fence, so N = 4096 still gives 256+
//     workgroups and nothing stalls the weight stream.
//   * The W waves split K by interleaved 32-wide MFMA steps (wave w takes
//     steps w, w + W, ...), so at any moment the workgroup reads 64 W contiguous
//     bytes of every row it owns, with U steps per wave in flight.
//   * Per step, lane l loads 16 bytes of row (l % 16) at k = 8 (l / 16): the A
//     operand of the MFMA (A[i][k] in lane i + 16 (k / 8)). x[m][k] is the B
//     operand (B[k][j] in lane j + 16 (k / 8)), read straight from L2 (x is a
//     few KB and shared by every workgroup) and normalised in registers when
//     the RMSNorm prologue is on (row scales from row_scale_kernel, cast order of
//     engine/kernels/rmsnorm.py:35-46). D[i][j] lands in lane j + 16 (i / 4), element i % 4.
//   * The waves' accumulators are summed in LDS in wave order (deterministic);
//     wave 0 runs the epilogue: BF16 store, SwiGLU, or per-row greedy-argmax keys.
#include "ftk_device.h"
#include "ftk_internal.h"

namespace ftk {

// rsqrt(mean(x[m]^2) + eps) per row: the arithmetic (per-thread order, wave
// tree, fixed wave order) of the GEMV kind's prologue, so both kinds scale alike.
// With a residual or gathered rows it also stores the rows it normalises
// (x + residual) into a.sum, which the projection kernel then reads as its x.
__global__ __launch_bounds__(kThreads) void row_scale_kernel(ProjArgs a, float* __restrict__ scale) {
  __shared__ float red[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m = blockIdx.x, K = a.K, KC = K >> 3;
  const uint16_t* xr = x_row(a, m);
  float ss = 0.f;
  for (int c = tid; c < KC; c += kThreads) {
    const u32x4_t v = prologue_in(a, xr, m, (size_t)c * 8);
    ss = sum_squares8(v, ss);
    if (a.sum != nullptr) store16(a.sum + (size_t)m * K + (size_t)c * 8, v);
  }
  const float s = wave_sum(ss);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (tid == 0) scale[m] = rms_scale(red, K, a.eps);
}

template <int MB, int T, int U, int W, int EPI, bool PRO>
__global__ __launch_bounds__(64 * W) void mfma_kernel(ProjArgs a, MfmaArgs p) {
  __shared__ f32x4_t red[W - 1][T][MB][64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const int tile = blockIdx.x;
  const int K = a.K, M = a.M;
  const int steps = (K + 31) >> 5;

  // This lane's weight row in each subtile (A-operand row l % 16), clamped in bounds.
  const uint16_t* wp[T];
#pragma unroll
  for (int t = 0; t < T; ++t)
    wp[t] = a.w + (size_t)mfma_weight_row(EPI, tile, t, li, a.N, T) * K + 8 * g;

  // This lane's x rows (B-operand column l % 16 of each column block) and their scales.
  bool mok[MB];
  const uint16_t* xp[MB];
  float sc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = li + 16 * mb;
    mok[mb] = m < M;
    xp[mb] = a.x + (size_t)(mok[mb] ? m : 0) * K + 8 * g;
    if constexpr (PRO) sc[mb] = mok[mb] ? p.row_scale[m] : 0.f;
  }

  f32x4_t acc[T][MB];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[t][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int j0 = wave; j0 < steps; j0 += W * U) {
    u32x4_t xv[U][MB];
    u32x4_t gv[U];
    u32x4_t wv[U][T];
    // x (and gamma) first: L2 hits that arrive while the weight loads are in flight.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (j0 + W * u) * 32 + 8 * g;
      const bool in = (j0 + kWaves * u < steps) && k < K;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        xv[u][mb] = (in && mok[mb]) ? load16(xp[mb] + (size_t)(j0 + W * u) * 32) : u32x4_t{0u, 0u, 0u, 0u};
      if constexpr (PRO) gv[u] = in ? load16(a.gamma + k) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (j0 + W * u) * 32 + 8 * g;
      const bool in = (j0 + kWaves * u < steps) && k < K;
#pragma unroll
      for (int t = 0; t < T; ++t)
        wv[u][t] = in ? load_stream16(wp[t] + (size_t)(j0 + W * u) * 32) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j0 + kWaves * u < steps) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          u32x4_t b = xv[u][mb];
          if constexpr (PRO) {
            // bf16(x * rsqrt) first, then the gain multiply, rounded again.
            b = norm8(b, gv[u], sc[mb]);
          }
#pragma unroll
          for (int t = 0; t < T; ++t) acc[t][mb] = mfma16x16x32(wv[u][t], b, acc[t][mb]);
        }
      }
    }
  }

  // ---- fixed-order sum of the four waves' partial products ----------------------
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) red[wave - 1][t][mb][lane] = acc[t][mb];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < W - 1; ++w)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[t][mb] += red[w][t][mb][lane];

  // ---- epilogue (wave 0): lane (li, g) holds rows 4g..4g+3 of each subtile, column li + 16 mb
  if constexpr (EPI == EPI_STORE) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int n0 = tile * 16 * T + t * 16 + 4 * g;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        if (!mok[mb]) continue;
        uint16_t* yr = a.y + (size_t)(li + 16 * mb) * a.N;
        if (a.out_add == nullptr && n0 + 3 < a.N && (a.N & 3) == 0 &&
            (reinterpret_cast<uintptr_t>(a.y) & 7) == 0) {
          *reinterpret_cast<u32x2_t*>(yr + n0) =
              u32x2_t{pack_bf16(acc[t][mb][0], acc[t][mb][1]), pack_bf16(acc[t][mb][2], acc[t][mb][3])};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n0 + r < a.N) yr[n0 + r] = (uint16_t)store_bits(a, acc[t][mb][r], li + 16 * mb, n0 + r);
        }
      }
    }
  } else if constexpr (EPI == EPI_SWIGLU) {
    const int I = a.N / 2;
#pragma unroll
    for (int t = 0; t < T / 2; ++t) {
      const int c0 = tile * 8 * T + t * 16 + 4 * g;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        if (!mok[mb]) continue;
        uint16_t* yr = a.y + (size_t)(li + 16 * mb) * I;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (c0 + r < I) yr[c0 + r] = (uint16_t)swiglu_bf16(acc[t][mb][r], acc[t + T / 2][mb][r]);
      }
    }
  } else {  // EPI_ARGMAX: per input row, the best (BF16 value, lowest index) key of this tile
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      unsigned long long best = 0ull;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int n0 = tile * 16 * T + t * 16 + 4 * g;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (n0 + r < a.N) {
            const uint32_t bits = f32_to_bf16(acc[t][mb][r]);
            if (a.y != nullptr && mok[mb]) a.y[(size_t)(li + 16 * mb) * a.N + n0 + r] = (uint16_t)bits;
            best = key_max(best, argmax_key(bf16_to_f32(bits), (uint32_t)(n0 + r)));
          }
        }
      }
      // lanes li, li + 16, li + 32, li + 48 hold the same input row
      best = key_max(best, __shfl_xor(best, 16, 64));
      best = key_max(best, __shfl_xor(best, 32, 64));
      if (g == 0 && mok[mb]) a.keys[(size_t)tile * M + li + 16 * mb] = best;
    }
  }
}

typedef void (*MfmaKernel)(ProjArgs, MfmaArgs);

template <int MB, int T, int U, int W>
static MfmaKernel pick_mfma_mtuw(int epi, bool pro) {
  switch (epi) {
    case EPI_STORE:
      return pro ? mfma_kernel<MB, T, U, W, EPI_STORE, true> : mfma_kernel<MB, T, U, W, EPI_STORE, false>;
    case EPI_SWIGLU:
      if constexpr (T % 2 == 0)
        return pro ? mfma_kernel<MB, T, U, W, EPI_SWIGLU, true> : mfma_kernel<MB, T, U, W, EPI_SWIGLU, false>;
      return nullptr;
    case EPI_ARGMAX:
      return pro ? mfma_kernel<MB, T, U, W, EPI_ARGMAX, true> : mfma_kernel<MB, T, U, W, EPI_ARGMAX, false>;
  }
  return nullptr;
}

// Instantiated launch shapes (T subtiles, U steps in flight, W waves).
template <int MB>
static MfmaKernel pick_mfma_m(int t, int unroll, int waves, int epi, bool pro) {
#define FTK_MFMA_SHAPE(T_, U_, W_) \
  if (t == T_ && unroll == U_ && waves == W_) return pick_mfma_mtuw<MB, T_, U_, W_>(epi, pro);
  FTK_MFMA_SHAPE(1, 4, 4)
  FTK_MFMA_SHAPE(1, 8, 4)
  FTK_MFMA_SHAPE(1, 4, 8)
  FTK_MFMA_SHAPE(1, 8, 8)
  FTK_MFMA_SHAPE(1, 4, 16)
  FTK_MFMA_SHAPE(2, 4, 4)
  FTK_MFMA_SHAPE(2, 8, 4)
  FTK_MFMA_SHAPE(2, 4, 8)
  FTK_MFMA_SHAPE(2, 8, 8)
  FTK_MFMA_SHAPE(2, 4, 16)
  FTK_MFMA_SHAPE(4, 2, 4)
  FTK_MFMA_SHAPE(4, 4, 4)
  FTK_MFMA_SHAPE(4, 2, 8)
#undef FTK_MFMA_SHAPE
  return nullptr;
}

static MfmaKernel pick_mfma(int M, int t, int unroll, int waves, int epi, bool pro) {
  switch ((M + 15) / 16) {
    case 1: return pick_mfma_m<1>(t, unroll, waves, epi, pro);
    case 2: return pick_mfma_m<2>(t, unroll, waves, epi, pro);
  }
  return nullptr;
}

bool mfma_supported(int M, int t, int unroll, int waves, int epi) {
  return pick_mfma(M, t, unroll, waves, epi, false) != nullptr;
}

hipError_t launch_mfma(const ProjArgs& a, int epi, const MfmaShape& s, const MfmaArgs& p, hipStream_t stream) {
  MfmaKernel k = pick_mfma(a.M, s.subtiles, s.unroll, s.waves, epi, a.gamma != nullptr);
  if (k == nullptr) return hipErrorInvalidValue;
  ProjArgs main = a;
  if (a.gamma != nullptr) {
    hipLaunchKernelGGL(row_scale_kernel, dim3(a.M), dim3(kThreads), 0, stream, a, const_cast<float*>(p.row_scale));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (a.residual != nullptr || a.x_ids != nullptr) {
      // the projection reads the rows the pre-pass stored (x + residual, or the gathered rows)
      if (a.sum == nullptr) return hipErrorInvalidValue;
      main.x = a.sum;
      main.residual = nullptr;
      main.x_ids = nullptr;
    }
    main.sum = nullptr;
  }
  hipLaunchKernelGGL(k, dim3(s.grid), dim3(64 * s.waves), 0, stream, main, p);
  return hipGetLastError();
}

}  // namespace ftk
