// Projection chain: a list of dependent M = 1 projections (a decode layer's QKV, O,
// gate/up + SwiGLU and down, for as many layers as the list holds) run by ONE
// cooperative launch, one 16-wave workgroup per CU.
//
// Arithmetic per stage is that of the STREAM kind (engine/kernels/linear.py:27-47
// _gemv; RMSNorm prologue engine/kernels/rmsnorm.py:21-46; SwiGLU epilogue
// engine/kernels/swiglu.py:13-24; the residual add of engine/kernels/rmsnorm.py:86-95
// in the epilogue): FP32 dot products of BF16 weights and the (normalised) BF16
// input row, one rounding to BF16.
//
// What the chain removes is the kernel boundary between dependent projections:
//   * A workgroup issues its first weight window of stage s before it waits for
//     stage s's input, so HBM streams while the previous stage's last outputs land.
//   * Outputs travel as tagged words: bf16 value | tag << 16 in one 32-bit word,
//     stored with agent-scope stores. A consumer polls the words it needs with
//     agent-scope (sc1) loads until every tag is this launch's tag. Value and
//     tag arrive together, so no fence and no separate flag is needed.
//   * Every wait is bounded (kChainWaitTicks of the 100 MHz real-time clock). A
//     workgroup that times out writes an error word and the whole launch stops;
//     every later launch of the chain exits at once until the host prepares it
//     again. Every wave always reaches the end of the kernel.
//
// Tags: tag = epoch % 65535 + 1 (never 0, the value of cleared memory). Each
// launch reads the epoch word at its start; workgroup 0 advances it after every
// workgroup has finished the last stage (so all of them have read it). Each
// stage has its own tagged buffer, written in full by every launch, so a word
// always holds either this launch's value or an older launch's tag.
#include <string.h>

#include <mutex>
#include <vector>

#include "../../include/ftk.h"
#include "ftk_internal.h"

namespace ftk {

constexpr int kChainWaves = 16;
constexpr int kChainThreads = 64 * kChainWaves;
constexpr int kChainMaxK = 12288;              // x staged in LDS as BF16 (24 KiB)
constexpr int kChainMaxTiles = 8;  // tiles per workgroup per stage (their totals wait in LDS)
constexpr int kChainMaxRpw = 4;
constexpr long long kChainWaitTicks = 2000000;  // 20 ms at 100 MHz: a wait that long is a failure
constexpr int kChainCtlBytes = 256;

// Device-side stage descriptor (written by ftk_chain_prepare).
struct ChainStage {
  const uint16_t* w;        // [N, K] BF16
  const uint16_t* gamma;    // [K] RMSNorm gain, or null
  const uint16_t* x;        // external BF16 input [K] (when src is null)
  const uint16_t* add;      // external BF16 residual [N_out] added in the epilogue, or null
  uint16_t* y;              // plain BF16 output [N_out], or null
  uint32_t* tagged;         // this stage's tagged output [N_out]
  uint32_t* done;           // this stage's per-workgroup done words [grid]
  const uint32_t* src;      // tagged input (an earlier stage's output), or null
  const uint32_t* add_src;  // tagged residual (an earlier stage's output), or null
  const uint32_t* after;    // done words of a stage that must finish first, or null
  int N, K, epi, shape, tiles, index;
  int pad[2];
};
static_assert(sizeof(ChainStage) == 112, "descriptor layout");

struct ChainArgs {
  int n_stages;
  uint32_t* ctl;            // [0] epoch, [1] error (0 = none, else 1 + stage)
  long long* stamps;        // [3 n_stages + 1][grid] real-time clock: per stage start, input ready, end; kernel start
  float eps;
};

struct ChainLds {
  uint16_t xs[kChainMaxK];
  float part[kChainMaxTiles][kChainWaves][kChainMaxRpw];  // per-wave totals of each tile walked
  float red[kChainWaves];
  int abort;
};

__device__ __forceinline__ uint32_t load_word(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_word(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes (4 tagged words) at agent scope: the cache policy of an agent-scope atomic load.
__device__ __forceinline__ u32x4_t load_words4(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 16));
}
__device__ __forceinline__ bool tagged4(u32x4_t v, uint32_t tag) {
  return (v[0] >> 16) == tag && (v[1] >> 16) == tag && (v[2] >> 16) == tag && (v[3] >> 16) == tag;
}

// Records a failed wait: the first failure's stage goes to the error word.
__device__ void chain_fail(uint32_t* ctl, int stage) {
  uint32_t none = 0u;
  __hip_atomic_compare_exchange_strong(ctl + 1, &none, (uint32_t)(1 + stage), __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
}

// The input row of a stage (K elements) is read in two steps around the issue
// of the stage's weight window. Loads return in issue order within a wave, so
// the input's first loads go out before the window (they come back without
// waiting for it); only re-polls of words not yet published queue behind it.
template <int K>
struct ChainInput {
  static constexpr int kTagged = (K / 4 + kChainThreads - 1) / kChainThreads;  // 16-byte groups of tagged words
  static constexpr int kPlain = (K / 8 + kChainThreads - 1) / kChainThreads;   // 16-byte chunks of BF16
  u32x4_t v[kTagged];  // tagged words (input from an earlier stage)
  u32x4_t p[kPlain];   // BF16 chunks (external input)
  uint32_t fence;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t words_rsrc(const uint32_t* p, int words) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(p), 0, words * 4, kBufferFlags);
}

// First round: the tagged words (or the external BF16 row) and the fence word.
// Both kinds of load are issued without a branch: the resource of the absent
// input has no records, so its loads return zeros without touching memory (and
// past the row's end a load returns zeros too); those registers are never used.
template <int K>
__device__ __forceinline__ void chain_input_issue(const ChainStage& st, ChainInput<K>& in) {
  const int t = threadIdx.x;
  const __amdgpu_buffer_rsrc_t rt = words_rsrc(st.src, st.src != nullptr ? K : 0);
  const __amdgpu_buffer_rsrc_t rp =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(st.x), 0, st.src == nullptr ? K * 2 : 0, kBufferFlags);
#pragma unroll
  for (int i = 0; i < ChainInput<K>::kTagged; ++i)  // group q holds words 4 q .. 4 q + 3
    in.v[i] = load_words4(rt, (uint32_t)(t + i * kChainThreads) * 16);
#pragma unroll
  for (int i = 0; i < ChainInput<K>::kPlain; ++i)  // chunk c holds elements 8 c .. 8 c + 7
    in.p[i] = __builtin_bit_cast(u32x4_t,
                                 __builtin_amdgcn_raw_buffer_load_b128(rp, (uint32_t)(t + i * kChainThreads) * 16, 0, 0));
  if (st.after != nullptr && t < (int)gridDim.x) in.fence = load_word(st.after + t);
}

// Second round: wait until every word carries this launch's tag (re-polling the
// ones that do not, within the deadline), stage the row into LDS as BF16, and
// with the prologue return the RMSNorm scale. Returns false when the launch must stop.
template <int K>
__device__ __forceinline__ bool chain_input_finish(const ChainStage& st, ChainInput<K>& in, uint32_t tag,
                                                   uint32_t* ctl, float eps, ChainLds& lds, float* scale) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const long long deadline = wall_clock64() + kChainWaitTicks;
  bool failed = false;
  float ss = 0.f;
  if (st.src != nullptr) {
    constexpr int kPer = ChainInput<K>::kTagged;
    const __amdgpu_buffer_rsrc_t r = words_rsrc(st.src, K);
    int spins = 0;
    for (;;) {
      // A word's tag only ever moves forward to this launch's, so a group once
      // seen complete stays complete: every group is simply re-read until all are.
      bool all = true;
#pragma unroll
      for (int i = 0; i < kPer; ++i) all = all && ((t + i * kChainThreads) * 4 >= K || tagged4(in.v[i], tag));
      if (all) break;
      if (wall_clock64() > deadline || ((++spins & 63) == 0 && load_word(ctl + 1) != 0)) {
        failed = true;
        break;
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) in.v[i] = load_words4(r, (uint32_t)(t + i * kChainThreads) * 16);
    }
    if (!failed) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int q = t + i * kChainThreads;
        if (q * 4 < K) {
          const uint32_t p0 = (in.v[i][0] & 0xFFFFu) | (in.v[i][1] << 16);
          const uint32_t p1 = (in.v[i][2] & 0xFFFFu) | (in.v[i][3] << 16);
          *reinterpret_cast<u32x2_t*>(lds.xs + q * 4) = u32x2_t{p0, p1};
          if (st.gamma != nullptr) {
            const float a = lo_f32(p0), b = hi_f32(p0), c = lo_f32(p1), d = hi_f32(p1);
            ss = fmaf(a, a, ss);
            ss = fmaf(b, b, ss);
            ss = fmaf(c, c, ss);
            ss = fmaf(d, d, ss);
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < ChainInput<K>::kPlain; ++i) {
      const int c = t + i * kChainThreads;
      if (c * 8 < K) {
        store16(lds.xs + c * 8, in.p[i]);
        if (st.gamma != nullptr) ss = sum_squares8(in.p[i], ss);
      }
    }
  }
  if (st.after != nullptr && t < (int)gridDim.x && !failed) {
    int spins = 0;
    while (in.fence != tag) {
      if (wall_clock64() > deadline || ((++spins & 63) == 0 && load_word(ctl + 1) != 0)) {
        failed = true;
        break;
      }
      in.fence = load_word(st.after + t);
    }
  }
  if (failed) {
    chain_fail(ctl, st.index);
    lds.abort = 1;
  }
  if (st.gamma != nullptr) {
    ss = wave_sum(ss);
    if (lane == 0) lds.red[wave] = ss;
  }
  __syncthreads();
  if (lds.abort) return false;
  if (st.gamma != nullptr) {
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kChainWaves; ++w) total += lds.red[w];
    *scale = 1.0f / sqrtf(total / (float)K + eps);
  }
  return true;
}

// One stage on shape (C chunks per lane per row, KW waves per row group, RPW
// weight rows per group per tile). K = 512 C KW. Weights are read through a
// buffer resource: the lane's part of the offset is one VGPR, the row's part is
// wave-uniform (an SGPR), so a wider window costs only its data registers.
template <int C, int KW, int RPW, int EPI>
__device__ __forceinline__ bool chain_stage(const ChainStage* __restrict__ sp, uint32_t tag, uint32_t* ctl, float eps,
                                            ChainLds& lds, long long* stamp) {
  const ChainStage& st = *sp;
  constexpr int GROUPS = kChainWaves / KW;
  constexpr int PW = EPI == EPI_SWIGLU ? RPW / 2 : RPW;
  constexpr int K = 512 * C * KW;
  constexpr uint32_t kStepBytes = (uint32_t)KW * 1024;  // bytes between a lane's chunks
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int grp = wave / KW, kw = wave - grp * KW;
  const int G = gridDim.x, wg = blockIdx.x;
  const int outputs = gemv_outputs(EPI, st.N);
  const uint32_t first = (uint32_t)(kw * 64 + lane) * 8;  // this lane's element of chunk 0
  const __amdgpu_buffer_rsrc_t wres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(st.w), 0, (int)((size_t)st.N * K * 2), kBufferFlags);

  // Byte offsets of the tile's weight rows (wave-uniform; rows past the end clamp in bounds).
  auto row_offsets = [&](int tile, uint32_t (&ro)[RPW]) {
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int col = gemv_output(tile, grp, p, PW, GROUPS);
      const int c = col < outputs ? col : outputs - 1;
      ro[p] = (uint32_t)gemv_weight_row(EPI, c, 0, st.N) * (uint32_t)(K * 2);
      if constexpr (EPI == EPI_SWIGLU) ro[PW + p] = (uint32_t)gemv_weight_row(EPI, c, 1, st.N) * (uint32_t)(K * 2);
    }
  };
  auto wload = [&](uint32_t row_off, int j) {
    return __builtin_bit_cast(
        u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wres, first * 2 + (uint32_t)j * kStepBytes, row_off, 2));
  };

  // ---- the first tile's weights, then the gain and the input's first loads ------
  int tile = wg;
  const bool busy = tile < st.tiles;
  // The whole first tile goes out before the wait, then the gain and the input's
  // first round. (Measured on MI355X: issuing the input first, or only part of the
  // window before the wait, made the Qwen3-8B layer slower, 64-68 us against 62.)
  ChainInput<K> in;
  in.fence = 0;
  u32x4_t gv[C];
  u32x4_t wv[C][RPW];
  if (busy) {
    uint32_t ro[RPW];
    row_offsets(tile, ro);
#pragma unroll
    for (int j = 0; j < C; ++j)
#pragma unroll
      for (int r = 0; r < RPW; ++r) wv[j][r] = wload(ro[r], j);
    if (st.gamma != nullptr) {
#pragma unroll
      for (int j = 0; j < C; ++j) gv[j] = load16(st.gamma + first + (uint32_t)j * (kStepBytes / 2));
    }
    chain_input_issue<K>(st, in);
  }

  // ---- the input row (waits for the producer), the norm's scale ----------------
  // (A workgroup without a tile in this stage needs no input: `busy` is uniform.)
  float scale = 1.f;
  if (busy && !chain_input_finish<K>(st, in, tag, ctl, eps, lds, &scale)) return false;
  if (t == 0) stamp[(size_t)gridDim.x] = busy ? wall_clock64() : 0;  // input ready

  int count = 0;
  if (busy) {
    u32x4_t xr[C];
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const uint32_t e = first + (uint32_t)j * (kStepBytes / 2);
      xr[j] = *reinterpret_cast<const u32x4_t*>(lds.xs + e);
      if (st.gamma != nullptr) xr[j] = norm8(xr[j], gv[j], scale);
    }
    // ---- tiles wg, wg + G, ...: consume, refill the registers with the next tile ----
    for (;;) {
      const int next = tile + G;
      float acc[RPW];
#pragma unroll
      for (int r = 0; r < RPW; ++r) acc[r] = 0.f;
      if (next < st.tiles) {
        uint32_t rn[RPW];
        row_offsets(next, rn);
#pragma unroll
        for (int j = 0; j < C; ++j)
#pragma unroll
          for (int r = 0; r < RPW; ++r) {
            acc[r] = dot8(wv[j][r], xr[j], acc[r]);
            wv[j][r] = wload(rn[r], j);
          }
      } else {
#pragma unroll
        for (int j = 0; j < C; ++j)
#pragma unroll
          for (int r = 0; r < RPW; ++r) acc[r] = dot8(wv[j][r], xr[j], acc[r]);
      }
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const float sum = wave_sum(acc[r]);
        if (lane == 0) lds.part[count][wave][r] = sum;
      }
      ++count;
      if (next >= st.tiles) break;
      tile = next;
    }
  }
  __syncthreads();

  // ---- epilogue: outputs (tile i, group, slot), KW wave totals in wave order ----
  bool failed = false;
  const int entries = count * GROUPS * PW;
  for (int e = t; e < entries; e += kChainThreads) {
    const int p = e % PW;
    const int g = (e / PW) % GROUPS;
    const int i = e / (PW * GROUPS);
    const int col = gemv_output(wg + i * G, g, p, PW, GROUPS);
    if (col >= outputs) continue;
    float s = lds.part[i][g * KW][p];
#pragma unroll
    for (int q = 1; q < KW; ++q) s += lds.part[i][g * KW + q][p];
    uint32_t bits;
    if constexpr (EPI == EPI_SWIGLU) {
      float u = lds.part[i][g * KW][PW + p];
#pragma unroll
      for (int q = 1; q < KW; ++q) u += lds.part[i][g * KW + q][PW + p];
      bits = swiglu_bf16(s, u);
    } else {
      bits = f32_to_bf16(s);
      uint32_t add = 0xFFFFFFFFu;
      if (st.add_src != nullptr) {
        const long long deadline = wall_clock64() + kChainWaitTicks;
        uint32_t word = load_word(st.add_src + col);
        while ((word >> 16) != tag) {
          if (wall_clock64() > deadline) {
            failed = true;
            break;
          }
          word = load_word(st.add_src + col);
        }
        add = word & 0xFFFFu;
      } else if (st.add != nullptr) {
        add = st.add[col];
      }
      if (add != 0xFFFFFFFFu) bits = f32_to_bf16(bf16_to_f32(bits) + bf16_to_f32(add));
    }
    if (st.y != nullptr) st.y[col] = (uint16_t)bits;
    store_word(st.tagged + col, bits | (tag << 16));
  }
  if (failed) {
    chain_fail(ctl, st.index);
    lds.abort = 1;
  }
  __syncthreads();
  if (lds.abort) return false;
  if (t == 0) store_word(st.done + wg, tag);
  return true;
}

// The (C, KW, RPW, epilogue) shapes built, by id (the planner picks one per stage).
#define FTK_CHAIN_SHAPES(X)       \
  X(0, 1, 2, 2, EPI_STORE)        \
  X(1, 1, 2, 4, EPI_STORE)        \
  X(2, 1, 2, 2, EPI_SWIGLU)       \
  X(3, 1, 2, 4, EPI_SWIGLU)       \
  X(4, 1, 4, 1, EPI_STORE)        \
  X(5, 1, 4, 2, EPI_STORE)        \
  X(6, 1, 4, 4, EPI_STORE)        \
  X(7, 1, 4, 2, EPI_SWIGLU)       \
  X(8, 3, 2, 1, EPI_STORE)        \
  X(9, 3, 2, 2, EPI_STORE)        \
  X(10, 3, 2, 2, EPI_SWIGLU)      \
  X(11, 2, 4, 2, EPI_STORE)       \
  X(12, 2, 4, 4, EPI_STORE)       \
  X(13, 2, 4, 2, EPI_SWIGLU)      \
  X(14, 2, 4, 4, EPI_SWIGLU)      \
  X(15, 1, 8, 2, EPI_STORE)       \
  X(16, 1, 8, 4, EPI_STORE)       \
  X(17, 1, 8, 4, EPI_SWIGLU)      \
  X(18, 3, 8, 2, EPI_STORE)       \
  X(19, 3, 8, 4, EPI_STORE)       \
  X(20, 3, 8, 2, EPI_SWIGLU)      \
  X(21, 3, 8, 4, EPI_SWIGLU)

struct ChainShape {
  int c, kw, rpw, epi;
};
static const ChainShape kChainShapes[] = {
#define FTK_CHAIN_ROW(ID, C, KW, RPW, EPI) {C, KW, RPW, EPI},
    FTK_CHAIN_SHAPES(FTK_CHAIN_ROW)
#undef FTK_CHAIN_ROW
};
constexpr int kChainShapeCount = sizeof(kChainShapes) / sizeof(kChainShapes[0]);

// `stages` is a parameter of its own, __restrict__ and never written by the
// kernel, so descriptor fields are uniform scalar loads.
__global__ __launch_bounds__(kChainThreads) void chain_kernel(const ChainStage* __restrict__ stages, ChainArgs a) {
  __shared__ ChainLds lds;
  __shared__ uint32_t head[2];
  const int t = threadIdx.x, wg = blockIdx.x, G = gridDim.x;
  if (t == 0) {
    head[0] = load_word(a.ctl);
    head[1] = load_word(a.ctl + 1);
    lds.abort = 0;
    a.stamps[(size_t)3 * a.n_stages * G + wg] = wall_clock64();
  }
  __syncthreads();
  const uint32_t epoch = head[0];
  if (head[1] != 0) return;  // a failed launch stops the chain until it is prepared again
  const uint32_t tag = epoch % 65535u + 1u;
  for (int s = 0; s < a.n_stages; ++s) {
    const ChainStage* sp = stages + s;
    long long* stamp = a.stamps + (size_t)3 * s * G + wg;  // [3 s][wg]: start, [3 s + 1]: input, [3 s + 2]: end
    if (t == 0) stamp[0] = wall_clock64();
    bool ok = false;
    switch (sp->shape) {
#define FTK_CHAIN_CASE(ID, C, KW, RPW, EPI) \
  case ID: ok = chain_stage<C, KW, RPW, EPI>(sp, tag, a.ctl, a.eps, lds, stamp); break;
      FTK_CHAIN_SHAPES(FTK_CHAIN_CASE)
#undef FTK_CHAIN_CASE
    }
    if (!ok) return;
    if (t == 0) stamp[(size_t)2 * G] = wall_clock64();
  }
  // Workgroup 0 advances the epoch once every workgroup has finished the last
  // stage: by then every workgroup has read this launch's epoch.
  if (wg == 0) {
    const uint32_t* last = stages[a.n_stages - 1].done;
    bool failed = false;
    if (t < G) {
      const long long deadline = wall_clock64() + kChainWaitTicks;
      while (load_word(last + t) != tag) {
        if (wall_clock64() > deadline) {
          failed = true;
          break;
        }
      }
    }
    if (failed) {
      chain_fail(a.ctl, a.n_stages - 1);
      lds.abort = 1;
    }
    __syncthreads();
    if (t == 0 && !lds.abort) store_word(a.ctl, epoch + 1);
  }
}

// ---- host side --------------------------------------------------------------------

// The shape for one stage: K = 512 C KW; the fewest outputs on the busiest
// workgroup, then the widest weight window (RPW C), then the most rows per tile.
static int chain_pick_shape(int64_t N, int64_t K, int epi, int grid, int* tiles_out) {
  const int64_t outputs = epi == FTK_EPI_SWIGLU ? N / 2 : N;
  int best = -1, best_tiles = 0;
  int64_t best_load = 0;
  int best_window = 0, best_rows = 0;
  for (int id = 0; id < kChainShapeCount; ++id) {
    const ChainShape& s = kChainShapes[id];
    if (s.epi != epi || K != (int64_t)512 * s.c * s.kw) continue;
    const int groups = kChainWaves / s.kw;
    const int per_tile = groups * (epi == FTK_EPI_SWIGLU ? s.rpw / 2 : s.rpw);
    const int64_t tiles = (outputs + per_tile - 1) / per_tile;
    const int64_t depth = (tiles + grid - 1) / grid;
    if (depth > kChainMaxTiles) continue;
    const int64_t load = depth * per_tile;
    const int window = s.rpw * s.c;
    if (best < 0 || load < best_load || (load == best_load && window > best_window) ||
        (load == best_load && window == best_window && per_tile > best_rows)) {
      best = id;
      best_tiles = (int)tiles;
      best_load = load;
      best_window = window;
      best_rows = per_tile;
    }
  }
  if (best >= 0) *tiles_out = best_tiles;
  return best;
}

struct ChainLayout {
  int64_t stages_off, done_off, tagged_off, stamps_off, total;
  std::vector<int64_t> tagged;  // offset of each stage's tagged buffer
};

static int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

static ChainLayout chain_layout(const ftk_chain_stage* st, int n, int grid) {
  ChainLayout l;
  l.stages_off = kChainCtlBytes;
  l.done_off = align256(l.stages_off + (int64_t)n * (int64_t)sizeof(ChainStage));
  int64_t off = align256(l.done_off + (int64_t)n * grid * 4);
  l.tagged_off = off;
  l.tagged.resize(n);
  for (int i = 0; i < n; ++i) {
    l.tagged[i] = off;
    const int64_t outs = st[i].epilogue == FTK_EPI_SWIGLU ? st[i].N / 2 : st[i].N;
    off = align256(off + outs * 4);
  }
  l.stamps_off = off;
  l.total = off + (int64_t)(3 * n + 1) * grid * 8;
  return l;
}

static int chain_hip(hipError_t e) { return hip_status(e); }


static int chain_grid(int* grid) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return chain_hip(e);
  if (cus < 1 || cus > kChainThreads) return FTK_ERR_UNSUPPORTED;
  *grid = cus;
  return FTK_OK;
}

// Validation shared by the size query and prepare.
static int chain_check(const ftk_chain_stage* st, int n, int grid, int* shapes, int* tiles) {
  if (st == nullptr || n < 1 || n > FTK_CHAIN_MAX_STAGES) return FTK_ERR_INVALID;
  for (int i = 0; i < n; ++i) {
    const ftk_chain_stage& s = st[i];
    if (s.w == nullptr || s.N < 1 || s.K < 1 || s.N > INT32_MAX) return FTK_ERR_INVALID;
    if (s.epilogue != FTK_EPI_STORE && s.epilogue != FTK_EPI_SWIGLU) return FTK_ERR_INVALID;
    if (s.epilogue == FTK_EPI_SWIGLU && s.N % 2) return FTK_ERR_INVALID;
    if (s.source >= i || s.add_source >= i || s.after >= i) return FTK_ERR_INVALID;  // earlier stages only
    if ((s.source < 0) == (s.x == nullptr)) return FTK_ERR_INVALID;                  // exactly one input
    if (s.add_source >= 0 && s.add != nullptr) return FTK_ERR_INVALID;
    if ((s.add_source >= 0 || s.add != nullptr) && s.epilogue != FTK_EPI_STORE) return FTK_ERR_INVALID;
    const int64_t outs = s.epilogue == FTK_EPI_SWIGLU ? s.N / 2 : s.N;
    if (s.source >= 0) {
      const ftk_chain_stage& p = st[s.source];
      if ((p.epilogue == FTK_EPI_SWIGLU ? p.N / 2 : p.N) != s.K) return FTK_ERR_INVALID;
    }
    if (s.add_source >= 0) {
      const ftk_chain_stage& p = st[s.add_source];
      if ((p.epilogue == FTK_EPI_SWIGLU ? p.N / 2 : p.N) != outs) return FTK_ERR_INVALID;
    }
    if (s.K > kChainMaxK || s.K % 8) return FTK_ERR_UNSUPPORTED;
    if (s.N * s.K * 2 > (int64_t)INT32_MAX) return FTK_ERR_UNSUPPORTED;  // one buffer resource spans W
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!a16(s.w) || (s.x && !a16(s.x)) || (s.gamma && !a16(s.gamma))) return FTK_ERR_UNSUPPORTED;
    if ((s.add && (reinterpret_cast<uintptr_t>(s.add) & 1u)) || (s.y && (reinterpret_cast<uintptr_t>(s.y) & 1u)))
      return FTK_ERR_INVALID;
    int t = 0;
    const int shape = chain_pick_shape(s.N, s.K, s.epilogue, grid, &t);
    if (shape < 0) return FTK_ERR_UNSUPPORTED;
    if (shapes) shapes[i] = shape;
    if (tiles) tiles[i] = t;
  }
  return FTK_OK;
}

}  // namespace ftk

using namespace ftk;

extern "C" {

int64_t ftk_chain_workspace_bytes(const ftk_chain_stage* stages, int n_stages) {
  int grid = 0;
  if (chain_grid(&grid) != FTK_OK) return -1;
  if (chain_check(stages, n_stages, grid, nullptr, nullptr) != FTK_OK) return -1;
  return chain_layout(stages, n_stages, grid).total;
}

int ftk_chain_prepare(const ftk_chain_stage* stages, int n_stages, float eps, void* workspace,
                      int64_t workspace_bytes, ftk_chain* chain) {
  if (chain == nullptr || workspace == nullptr) return FTK_ERR_INVALID;
  int grid = 0;
  int st = chain_grid(&grid);
  if (st != FTK_OK) return st;
  std::vector<int> shapes(n_stages > 0 ? n_stages : 1), tiles(n_stages > 0 ? n_stages : 1);
  st = chain_check(stages, n_stages, grid, shapes.data(), tiles.data());
  if (st != FTK_OK) return st;
  const ChainLayout l = chain_layout(stages, n_stages, grid);
  if (workspace_bytes < l.total) return FTK_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) & 255u) return FTK_ERR_UNSUPPORTED;
  // One workgroup of 1024 threads per CU must fit, all resident at once.
  int per_cu = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)chain_kernel, kChainThreads, 0);
  if (e != hipSuccess) return chain_hip(e);
  if (per_cu < 1) return FTK_ERR_UNSUPPORTED;
  char* ws = (char*)workspace;
  std::vector<ChainStage> dev(n_stages);
  for (int i = 0; i < n_stages; ++i) {
    const ftk_chain_stage& s = stages[i];
    ChainStage& d = dev[i];
    memset(&d, 0, sizeof(d));
    d.w = (const uint16_t*)s.w;
    d.gamma = (const uint16_t*)s.gamma;
    d.x = s.source < 0 ? (const uint16_t*)s.x : nullptr;
    d.add = (const uint16_t*)s.add;
    d.y = (uint16_t*)s.y;
    d.tagged = (uint32_t*)(ws + l.tagged[i]);
    d.done = (uint32_t*)(ws + l.done_off + (int64_t)i * grid * 4);
    d.src = s.source >= 0 ? (const uint32_t*)(ws + l.tagged[s.source]) : nullptr;
    d.add_src = s.add_source >= 0 ? (const uint32_t*)(ws + l.tagged[s.add_source]) : nullptr;
    d.after = s.after >= 0 ? (const uint32_t*)(ws + l.done_off + (int64_t)s.after * grid * 4) : nullptr;
    d.N = (int)s.N;
    d.K = (int)s.K;
    d.epi = s.epilogue;
    d.shape = shapes[i];
    d.tiles = tiles[i];
    d.index = i;
  }
  // Cleared control words, done words and tagged buffers (tag 0 never matches).
  e = hipMemset(workspace, 0, (size_t)l.stamps_off);
  if (e == hipSuccess) e = hipMemcpy(ws + l.stages_off, dev.data(), dev.size() * sizeof(ChainStage),
                                     hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) return chain_hip(e);
  chain->workspace = workspace;
  chain->stages = n_stages;
  chain->grid = grid;
  chain->eps = eps;
  chain->stamps_offset = l.stamps_off;
  return FTK_OK;
}

int ftk_chain_launch(const ftk_chain* chain, void* stream) {
  if (chain == nullptr || chain->workspace == nullptr || chain->stages < 1 || chain->grid < 1) return FTK_ERR_INVALID;
  char* ws = (char*)chain->workspace;
  const ChainStage* stages = (const ChainStage*)(ws + kChainCtlBytes);
  ChainArgs a;
  a.n_stages = chain->stages;
  a.ctl = (uint32_t*)ws;
  a.stamps = (long long*)(ws + chain->stamps_offset);
  a.eps = chain->eps;
  void* args[] = {&stages, &a};
  return chain_hip(hipLaunchCooperativeKernel((const void*)chain_kernel, dim3(chain->grid), dim3(kChainThreads), args,
                                              0, reinterpret_cast<hipStream_t>(stream)));
}

int ftk_chain_status(const ftk_chain* chain) {
  if (chain == nullptr || chain->workspace == nullptr) return -1;
  uint32_t ctl[2] = {0, 0};
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(ctl, chain->workspace, sizeof(ctl), hipMemcpyDeviceToHost);
  if (e != hipSuccess) {
    chain_hip(e);
    return -1;
  }
  return (int)ctl[1];
}

int ftk_chain_stamps(const ftk_chain* chain, int64_t* out) {
  if (chain == nullptr || chain->workspace == nullptr || out == nullptr) return FTK_ERR_INVALID;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess)
    e = hipMemcpy(out, (char*)chain->workspace + chain->stamps_offset,
                  (size_t)(3 * chain->stages + 1) * chain->grid * 8, hipMemcpyDeviceToHost);
  return chain_hip(e);
}

int ftk_chain_plan(const ftk_chain_stage* stages, int n_stages, int compute_units, int* shapes, int* tiles) {
  if (compute_units < 1 || compute_units > kChainThreads) return FTK_ERR_INVALID;
  return chain_check(stages, n_stages, compute_units, shapes, tiles);
}

int ftk_chain_shape(int shape, int* c, int* kw, int* rows_per_group, int* epilogue) {
  if (shape < 0 || shape >= kChainShapeCount) return FTK_ERR_INVALID;
  if (c) *c = kChainShapes[shape].c;
  if (kw) *kw = kChainShapes[shape].kw;
  if (rows_per_group) *rows_per_group = kChainShapes[shape].rpw;
  if (epilogue) *epilogue = kChainShapes[shape].epi;
  return FTK_OK;
}

}  // extern "C"
