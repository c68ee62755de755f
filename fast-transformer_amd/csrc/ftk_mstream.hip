// M = 5..16 skinny BF16 projection, MFMA_STREAM kind: the STREAM kind's
// schedule with v_mfma_f32_16x16x32_bf16 doing the products.
//
// Same sums, roundings and fused extras as the other kinds
// (engine/kernels/linear.py:50-78 _skinny_gemm; RMSNorm prologue
// engine/kernels/rmsnorm.py:21-46; SwiGLU engine/kernels/swiglu.py:13-24;
// greedy argmax engine/kernels/argmax.py:19-48), FP32 accumulation, one rounding.
//
// Layout and schedule:
//   * A workgroup is KW waves splitting K into contiguous ranges; a tile is T
//     subtiles of 16 weight rows. Per 32-wide K step a wave runs one MFMA per subtile: A = 16 weight
//     rows (lane l: row l % 16, 8 k at 8 (l / 16)), B = x (lane l: x row l % 16,
//     same 8 k). x rows >= M are zero.
//   * Lane l only ever needs x at its own k, so its S steps of x are loaded once
//     into registers (and normalised there when the prologue is on: one
//     barrier to combine the row sums of squares), never re-read per tile.
//     For the long K without the prologue (K = 12288) x instead streams beside
//     the weights with the same lookahead (L2 hits), which leaves the registers
//     to a deeper weight window; the sums are the same either way.
//   * Rolling window: the weight loads of the next U steps are in flight at all
//     times, across tile boundaries (step s of tile i is consumed, then step
//     s + U, possibly of tile i + 1, is loaded into the registers it freed).
//   * Each wave parks its 16 x 16 partial per tile in LDS; one barrier at the
//     end, then the workgroup sums the KW partials in wave order (deterministic)
//     and runs the epilogue on every output of its tiles.
#include "ftk_device.h"
#include "ftk_internal.h"

namespace ftk {

template <int T, int S, int KW, int U, bool PRO, int EPI>
__global__ __launch_bounds__(64 * KW) void mstream_kernel(ProjArgs a, int tiles) {
  static_assert(S % U == 0, "the weight window must tile the steps of a tile");
  static_assert(EPI != EPI_SWIGLU || T % 2 == 0, "SwiGLU pairs gate and up subtiles");
  constexpr int DMAX = (64 * 1024) / (T * KW * 1024);
  __shared__ f32x4_t part[DMAX][KW][T][64];
  __shared__ float red[KW][16];
  __shared__ unsigned long long best_lds[KW][16];

  const int tid = threadIdx.x, lane = tid & 63, kw = tid >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int M = a.M, K = a.K;  // K == 32 S KW (checked by the planner)
  const bool mine = li < M;    // this lane's x row is real
  // Wave kw owns the contiguous K range [32 S kw, 32 S (kw + 1)): over its steps each
  // row is read front to back in 64-byte pieces (measured on MI355X: ~10 % more HBM
  // throughput than interleaving the waves' steps).
  auto koff = [&](int s) { return (size_t)(32 * (kw * S + s) + 8 * g); };

  // The x slice: with the prologue (row li is x[li] or the gathered x[x_ids[li]],
  // plus the residual) and for K up to 16 steps per wave, all S steps stay in
  // registers. For the long K without the prologue (XS) a resident slice would
  // leave no registers for the weight window, so x streams beside the weights:
  // step s's x is loaded with step s's weights (waiting for one never waits for
  // later-issued loads) and hits in L2. The sums are the same either way.
  constexpr bool XS = !PRO && S > 16;
  const uint16_t* xrow = (PRO && mine) ? x_row(a, li) : a.x + (size_t)(mine ? li : 0) * K;
  auto x_step = [&](int s) { return mine ? load16(xrow + koff(s)) : u32x4_t{0u, 0u, 0u, 0u}; };
  u32x4_t xr[XS ? 1 : S];
  u32x4_t xv[XS ? U : 1];
  if constexpr (!XS) {
#pragma unroll
    for (int s = 0; s < S; ++s) xr[s] = !mine ? u32x4_t{0u, 0u, 0u, 0u} : PRO ? prologue_in(a, xrow, li, koff(s)) : x_step(s);
  }

  const int wg = blockIdx.x;
  int tile = wg;  // grid <= tiles
  const uint16_t* wp[T];
  auto rows_of = [&](int tl, const uint16_t* (&p)[T]) {
#pragma unroll
    for (int t = 0; t < T; ++t) p[t] = a.w + (size_t)mfma_weight_row(EPI, tl, t, li, a.N, T) * K;
  };
  rows_of(tile, wp);
  u32x4_t wv[U][T];
#pragma unroll
  for (int q = 0; q < U; ++q) {
#pragma unroll
    for (int t = 0; t < T; ++t) wv[q][t] = load_stream16(wp[t] + koff(q));
    if constexpr (XS) xv[q] = x_step(q);
  }

  // ---- RMSNorm prologue: row sums of squares over (wave, group, step) in order
  if constexpr (PRO) {
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) ss = sum_squares8(xr[s], ss);
    ss += __shfl_xor(ss, 16);  // the four lane groups holding row li, pairwise:
    ss += __shfl_xor(ss, 32);  // (g0 + g1) + (g2 + g3) in every one of them
    if (g == 0) red[kw][li] = ss;
    // The normalised rows themselves (x + residual) go out once, from workgroup 0.
    if (a.sum != nullptr && blockIdx.x == 0 && mine) {
#pragma unroll
      for (int s = 0; s < S; ++s) store16(a.sum + (size_t)li * K + koff(s), xr[s]);
    }
    __syncthreads();
    float total = red[0][li];
#pragma unroll
    for (int w = 1; w < KW; ++w) total += red[w][li];
    const float scale = 1.0f / sqrtf(total / (float)K + a.eps);
    // The gain is loaded only now (cache hits behind the weight window), so its
    // S registers are never live beside the window's (measured faster here than
    // loading it before the window).
#pragma unroll
    for (int s = 0; s < S; ++s) xr[s] = norm8(xr[s], load16(a.gamma + koff(s)), scale);
  }

  // ---- tiles -------------------------------------------------------------------
  int count = 0;
  for (;;) {
    const int next = tile + (int)gridDim.x;
    const bool more = next < tiles;
    const uint16_t* wn[T];
    if (more) rows_of(next, wn);
    f32x4_t acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const u32x4_t xs = XS ? xv[s % U] : xr[XS ? 0 : s];
#pragma unroll
      for (int t = 0; t < T; ++t) acc[t] = mfma16x16x32(wv[s % U][t], xs, acc[t]);
      // refill the freed window slot: step s + U of this tile, or of the next
      if (s + U < S) {
#pragma unroll
        for (int t = 0; t < T; ++t) wv[s % U][t] = load_stream16(wp[t] + koff(s + U));
        if constexpr (XS) xv[s % U] = x_step(s + U);
      } else if (more) {
#pragma unroll
        for (int t = 0; t < T; ++t) wv[s % U][t] = load_stream16(wn[t] + koff(s + U - S));
        if constexpr (XS) xv[s % U] = x_step(s + U - S);
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) part[count][kw][t][lane] = acc[t];
    ++count;
    if (!more) break;
    tile = next;
    for (int t = 0; t < T; ++t) wp[t] = wn[t];
  }
  __syncthreads();

  // ---- epilogue: thread e takes (tile i, subtile t, lane position ln) ----------
  // D[4 gg + r][ll] of subtile t: weight row 16 t + 4 gg + r of the tile, x row ll.
  constexpr int TO = (EPI == EPI_SWIGLU) ? T / 2 : T;  // output subtiles
  const int outputs = gemv_outputs(EPI, a.N);
  unsigned long long best = 0ull;
  const int entries = count * TO * 64;
  for (int e = tid; e < entries; e += 64 * KW) {
    const int ln = e & 63, t = (e >> 6) % TO, i = e / (64 * TO);
    const int ll = ln & 15, gg = ln >> 4;
    if (ll >= M) continue;
    const int tl = wg + i * (int)gridDim.x;
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

typedef void (*MstreamKernel)(ProjArgs, int);

// Instantiated (T, S, KW, U): K = 4096 (S = 8 at KW = 16, S = 16 at KW = 8) and,
// without the prologue (x streamed), deeper windows and K = 12288 (S = 24 at
// KW = 16, S = 48 at KW = 8; the 8B down projection).
#define FTK_MSTREAM_SHAPES_EVEN(PRO, EPI)  \
  FTK_MSTREAM_SHAPE(2, 8, 16, 4, PRO, EPI) \
  FTK_MSTREAM_SHAPE(2, 16, 8, 4, PRO, EPI) \
  FTK_MSTREAM_SHAPE(2, 16, 8, 8, PRO, EPI)

#define FTK_MSTREAM_SHAPES_ONE(PRO, EPI)   \
  FTK_MSTREAM_SHAPE(1, 8, 16, 4, PRO, EPI) \
  FTK_MSTREAM_SHAPE(1, 8, 16, 8, PRO, EPI) \
  FTK_MSTREAM_SHAPE(1, 16, 8, 4, PRO, EPI) \
  FTK_MSTREAM_SHAPE(1, 16, 8, 8, PRO, EPI) \
  FTK_MSTREAM_SHAPE(1, 16, 8, 16, PRO, EPI)

#define FTK_MSTREAM_SHAPES_LONG(EPI)         \
  FTK_MSTREAM_SHAPE(1, 24, 16, 2, false, EPI) \
  FTK_MSTREAM_SHAPE(1, 24, 16, 6, false, EPI) \
  FTK_MSTREAM_SHAPE(1, 48, 8, 16, false, EPI)

#define FTK_MSTREAM_SHAPE(T_, S_, KW_, U_, PRO, EPI) \
  if (t == T_ && s == S_ && kw == KW_ && u == U_) return mstream_kernel<T_, S_, KW_, U_, PRO, EPI>;

template <bool PRO, int EPI>
static MstreamKernel pick_mstream_shape(int t, int s, int kw, int u) {
  FTK_MSTREAM_SHAPES_EVEN(PRO, EPI)
  if constexpr (!PRO) {
    FTK_MSTREAM_SHAPE(2, 8, 16, 8, PRO, EPI)
    FTK_MSTREAM_SHAPE(2, 16, 8, 16, PRO, EPI)
  }
  if constexpr (EPI != EPI_SWIGLU) {
    FTK_MSTREAM_SHAPES_ONE(PRO, EPI)
    if constexpr (!PRO) {
      FTK_MSTREAM_SHAPES_LONG(EPI)
    }
  }
  return nullptr;
}
#undef FTK_MSTREAM_SHAPE

static MstreamKernel pick_mstream(int t, int s, int kw, int u, bool pro, int epi) {
  switch (epi) {
    case EPI_STORE: return pro ? pick_mstream_shape<true, EPI_STORE>(t, s, kw, u)
                               : pick_mstream_shape<false, EPI_STORE>(t, s, kw, u);
    case EPI_SWIGLU: return pro ? pick_mstream_shape<true, EPI_SWIGLU>(t, s, kw, u)
                                : pick_mstream_shape<false, EPI_SWIGLU>(t, s, kw, u);
    case EPI_ARGMAX: return pro ? pick_mstream_shape<true, EPI_ARGMAX>(t, s, kw, u)
                                : pick_mstream_shape<false, EPI_ARGMAX>(t, s, kw, u);
  }
  return nullptr;
}

bool mstream_supported(int M, int t, int K, int kw, int unroll, int epi, bool pro) {
  const int s = mstream_steps(K, kw);
  return M >= 1 && M <= kMstreamMaxRows && s > 0 && pick_mstream(t, s, kw, unroll, pro, epi) != nullptr;
}

hipError_t launch_mstream(const ProjArgs& a, int epi, const MstreamShape& sh, hipStream_t stream) {
  const int s = mstream_steps(a.K, sh.kw);
  MstreamKernel k = s > 0 ? pick_mstream(sh.subtiles, s, sh.kw, sh.unroll, a.gamma != nullptr, epi) : nullptr;
  if (k == nullptr || a.M < 1 || a.M > kMstreamMaxRows) return hipErrorInvalidValue;
  if (sh.grid < 1 || sh.grid > sh.tiles ||
      (sh.tiles + sh.grid - 1) / sh.grid > mstream_max_depth(sh.subtiles, sh.kw))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(sh.grid), dim3(64 * sh.kw), 0, stream, a, sh.tiles);
  return hipGetLastError();
}

}  // namespace ftk
