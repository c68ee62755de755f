// M = 1..16 skinny BF16 projection, RING kind: weight and x segments land in a
// per-wave LDS ring by direct-to-LDS loads (global_load_lds_dwordx4) and feed
// 16x16x32 BF16 MFMAs (v_mfma_f32_16x16x32_bf16).
//
// Same sums, roundings and fused extras as the other kinds
// (engine/kernels/linear.py:50-78 _skinny_gemm; RMSNorm prologue
// engine/kernels/rmsnorm.py:21-46; SwiGLU engine/kernels/swiglu.py:13-24;
// greedy argmax engine/kernels/argmax.py:19-48), FP32 accumulation, one rounding.
//
// Why: at 5..16 rows the kernels that hold x in registers spend as many L2
// requests on x as on the weights. An MFMA B operand needs x row l % 16 in lane
// l, so a register load of it touches 16 rows x 64 bytes per wave instruction.
// Here x travels like the weights, 4 rows x 256 contiguous bytes per wave
// instruction, straight into LDS, and is read back in MFMA layout. The weight
// window lives in LDS too, so it costs no registers. (Below 5 rows the planner
// takes this kind for lm_head + argmax only, whose long walks end in the
// claimed tail.)
//
// Layout and schedule:
//   * A tile is 16 weight rows (SwiGLU: 8 gate rows and the matching 8 up rows)
//     over all of K, or 12 or 24 (one subtile with four pad rows, or two MFMA
//     subtiles with the second half used) where 16-row tiles would leave a
//     partial round of workgroups. A workgroup is KW waves splitting K; wave kw
//     owns the 128-wide K segments j KW + kw (j < C, K = 128 C KW). A unit is one
//     segment of one tile: RT / 4 KiB of weights (RT / 4 loads of 4 rows x 256
//     bytes) and, while the B operand is not held in registers, 4 NX rows of x
//     (NX loads).
//   * Workgroup wg takes tile ring_tile(wg, i, G, tiles) at step i: in a full
//     round the workgroups of one XCD take one contiguous run of tiles.
//   * Lane l of load q brings row 4 q + l / 16, chunk (l % 16) ^ h(row), into
//     slot row * 16 + l % 16 of the unit's LDS: the XOR-swizzled layout whose
//     MFMA reads (lane l: row l % 16, chunk 4 s + l / 16) hit 16 distinct
//     16-byte bank groups per 16 lanes.
//   * Each wave keeps D units in flight in its own D slots; it waits for the
//     oldest with an exact vmcnt (direct-to-LDS loads count there and return in
//     order), reads it into registers, refills the slot, then runs the unit's
//     arithmetic. No other wave touches those slots, so the main loop has no
//     barrier.
//   * x rows past M re-read row M - 1 (in bounds); rows past 4 NX are not loaded:
//     their lanes read the unit's first x slot. Either way they feed only MFMA
//     output columns >= M, which are never stored (nor summed, nor compared).
//   * With C <= 4 the first tile's B operands (normalised, with the prologue)
//     stay in registers and later tiles load weights only, into 4 KiB slots:
//     a wave's 16 KiB then hold all four units of the next tile in flight
//     while it reads the current one. Otherwise x is loaded with every unit.
//   * RMSNorm prologue: a pre-pass reads the x rows (or the gathered rows)
//     row-contiguously for their sums of squares (wave w: rows w, w + KW, ...;
//     lanes in chunk order, the DPP tree, one barrier) and workgroup 0 stores
//     them when asked; the gain waits in LDS; each B operand chunk is
//     normalised as it is read. The pre-pass loads go out before the first
//     units, so the scales are ready while those units stream. The prologue's
//     residual add is not a RING form.
//   * Per-tile 16 x 16 partials wait in LDS; after every DMAX tiles (and after
//     the last) a barrier lets the workgroup sum them in wave order and run the
//     epilogue, with the next units in flight.
#include <type_traits>

#include "ftk_device.h"
#include "ftk_internal.h"

namespace ftk {

namespace {

typedef __attribute__((address_space(1))) const void global_void_t;
typedef __attribute__((address_space(3))) void lds_void_t;

// 16 bytes per lane from `src` into LDS at dst + 16 lane (dst is wave-uniform).
// AUX 2: non-temporal (the weights, read once per call); 0: cached (x).
template <int AUX>
__device__ __forceinline__ void dma16(const void* src, void* dst) {
  __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)dst, 16, 0, AUX);
}

// Wait until at most N vector memory instructions of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// LDS reads of the ring and the gain. The compiler cannot tell which ring slot
// a direct-to-LDS load writes, so before a plain LDS read it would wait for
// every such load in flight (vmcnt(0)), emptying the ring. These reads are
// ordered by the explicit vmcnt waits instead; lds_ready() waits for them, and
// ties their registers so that no use is scheduled before the wait.
__device__ __forceinline__ u32x4_t lds_read16(const u32x4_t* p) {
  u32x4_t v;
  const uint32_t at = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const u32x4_t*)p;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(at) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void lds_ready(u32x4_t (&v)[N]) {
  static_assert(N == 4 || N == 8 || N == 12 || N == 16, "operand sets of one unit");
  if constexpr (N == 4)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3])::"memory");
  else if constexpr (N == 8)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])::"memory");
  else if constexpr (N == 12)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]),
                   "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11])::"memory");
  else
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]),
                   "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]), "+v"(v[12]), "+v"(v[13]), "+v"(v[14]),
                   "+v"(v[15])::"memory");
}

// Global loads and LDS accesses of the prologue, issued as inline assembly. The
// compiler counts plain loads and direct-to-LDS loads in flight together as
// possibly out of order, so before the first use of a plain load's result it
// would wait for every load (vmcnt(0)), the first units included. These are
// ordered by explicit waits instead: after the wait, tie() marks the registers
// as produced there, so no use is scheduled before it.
__device__ __forceinline__ u32x4_t asm_load16(const void* p) {
  u32x4_t v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ void tie(u32x4_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void lds_write16(u32x4_t* p, u32x4_t v) {
  const uint32_t at = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4_t*)p;
  asm volatile("ds_write_b128 %0, %1" ::"v"(at), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_write_f32(float* p, float v) {
  const uint32_t at = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)p;
  asm volatile("ds_write_b32 %0, %1" ::"v"(at), "v"(v) : "memory");
}
__device__ __forceinline__ float lds_read_f32(const float* p) {
  float v;
  const uint32_t at = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const float*)p;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(at) : "memory");
  return v;
}

__device__ __forceinline__ void lds_write_u32(uint32_t* p, uint32_t v) {
  const uint32_t at = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)p;
  asm volatile("ds_write_b32 %0, %1" ::"v"(at), "v"(v) : "memory");
}
__device__ __forceinline__ uint32_t lds_read_u32(const uint32_t* p) {
  uint32_t v;
  const uint32_t at = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint32_t*)p;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(at) : "memory");
  return v;
}
// An agent-scope atomic add returning the old value, as assembly: the compiler does
// not count it, so it adds no wait of its own; the walk's exact waits return it.
// Like every load written as assembly, the compiler takes its destination as
// written at issue, so nothing may copy or reuse that register before the wait:
// the claim's one value (claim_v) must stay in place across the walk's loop. The
// claimed-tail builds' assembly holds it in one register throughout (checked when
// this was written); a change that makes the compiler move it would read the claim
// before it returns.
__device__ __forceinline__ uint32_t claim_add(unsigned* p) {
  uint32_t old;
  asm volatile("global_atomic_add %0, %1, %2, off sc0" : "=v"(old) : "v"(p), "v"(1u) : "memory");
  return old;
}

// Workgroup barrier for LDS traffic only. __syncthreads() also waits for every
// vector memory operation (vmcnt(0)), which would empty the ring mid-walk.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

}  // namespace

template <int C, int KW, int D, int NX, bool PRO, int EPI, int RT, bool TAIL = false>
__global__ __launch_bounds__(64 * KW) void ring_kernel(ProjArgs a, int tiles) {
  static_assert(C % D == 0, "a tile's units must fill the ring exactly");
  static_assert(NX == 2 || NX == 4, "x rows per unit: 8 or 16");
  static_assert(RT == 16 || ((RT == 24 || RT == 12) && EPI == EPI_STORE), "12- and 24-row tiles: the STORE epilogue");
  constexpr int SUB = (RT + 15) / 16;               // 16-row MFMA subtiles per tile
  constexpr int WL = RT / 4;                        // weight loads per unit (4 rows each)
  constexpr bool XREG = C <= 4 && RT <= 16;         // B operands kept after the first tile
  constexpr int XS = 64 * NX;                       // x slots (16 bytes) per unit
  constexpr int WS = 16 * RT;                       // weight slots (16 bytes) per unit
  constexpr int SLOT = WS + XS;                     // 16-byte slots per unit with x
  constexpr int RW = ring_wave_slots(C, D, NX, RT);  // 16-byte slots of one wave's ring
  static_assert(!XREG || (C == 4 && D == 2 && RW >= 4 * WS && RW >= 2 * SLOT), "the walk below is written for C = 4, D = 2");
  constexpr int DMAX = ring_max_depth(C, KW, D, NX, PRO, RT);
  static_assert(DMAX >= 1, "the ring leaves no LDS for the partials");
  constexpr int GCH = PRO ? 16 * C * KW : 1;        // 16-byte chunks of the gain (K / 8)
  __shared__ u32x4_t ring[KW][RW];
  __shared__ f32x4_t part[DMAX][KW][SUB][64];
  __shared__ u32x4_t gain[GCH];
  __shared__ float red[16];
  __shared__ unsigned long long best_lds[KW][16];

  const int tid = threadIdx.x, lane = tid & 63, kw = tid >> 6;
  const int li = lane & 15, g = lane >> 4;  // MFMA layout: row li, k quarter g
  const int M = a.M, K = a.K;               // K == 128 C KW (checked by the planner)
  const int wg = blockIdx.x, G = gridDim.x;
  // Claimed tail (TAIL builds, given a.claim; register-held B operands and
  // kRingTailMinTiles or more tiles per workgroup): the first `rounds` positions of workgroup wg's walk are its static
  // tiles (ring_tile over rounds * G tiles); the rest of the tiles, the tail, are
  // claimed from *a.claim (the c-th claim of the launch is tile rounds * G + c; a
  // claim past the tail ends the walk), so the workgroups that run ahead take more of
  // them. Wave 0 claims position k + 2 at the top of position k, before it issues the
  // units of position k + 1: loads complete in order, so the wait for position
  // k + 1's first unit returns the claim too. It publishes each claimed tile in
  // seq_lds (slot k % 16, tagged with the position); the other waves read it there,
  // waiting for the tag while wave 0 is behind (no barrier lies between, so wave 0
  // never waits for them on the way). Every walk ends with exactly one claim past
  // the tail, so the launch's last claim finds the counter at tail + G - 1 and puts
  // it back to zero.
  const int per = tiles / G;
  const bool dyn = TAIL && XREG && per >= kRingTailMinTiles;  // uniform
  const int rounds = dyn ? per - per / 8 : 0;  // the tail: about an eighth of the tiles
  const int static_tiles = dyn ? rounds * G : tiles, tail = tiles - static_tiles;
  const int my_tiles = (static_tiles - wg + G - 1) / G;  // static steps of this workgroup (grid <= tiles)
  auto tile_at = [&](int i) { return ring_tile(wg, i, G, static_tiles); };
  __shared__ uint32_t seq_lds[16];
  uint32_t claim_v = 0;  // wave 0, lane 0: the claim in flight
  auto seq_word = [](int k, int tile) { return ((uint32_t)(k & 0xFFF) << 20) | (uint32_t)(tile + 1); };
  // Tile of position k (-1 past the walk's end), once published.
  auto walk_tile = [&](int k) {
    if (!dyn) return k < my_tiles ? tile_at(k) : -1;
    if (k < rounds) return tile_at(k);
    const uint32_t want = (uint32_t)(k & 0xFFF) << 20;
    uint32_t v = lds_read_u32(&seq_lds[k & 15]);
    while ((v & 0xFFF00000u) != want) {
      __builtin_amdgcn_s_sleep(1);
      v = lds_read_u32(&seq_lds[k & 15]);
    }
    return (int)(v & 0xFFFFFu) - 1;
  };
  // At the top of position k (its first unit's wait done): publish position k + 1
  // if it was claimed (the wait returned its claim), claim position k + 2 if it lies
  // in the tail and the walk goes on. Returns the tile of position k + 1.
  auto advance = [&](int k) {
    if (dyn && kw == 0 && k + 2 >= rounds) {
      if (k + 1 >= rounds) asm volatile("" : "+v"(claim_v));  // returned by the wait before this
      if (lane == 0) {
        bool go = true;
        if (k + 1 >= rounds) {
          const int c = (int)claim_v;
          const int next = c < tail ? static_tiles + c : -1;
          lds_write_u32(&seq_lds[(k + 1) & 15], seq_word(k + 1, next));
          go = next >= 0;
          if (!go && c == tail + G - 1) __hip_atomic_store(a.claim, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (go) claim_v = claim_add(a.claim);
      }
    }
    return walk_tile(k + 1);
  };
  // The tile of a parked position (static builds: the static order).
  auto flush_tile = [&](int k) {
    if constexpr (TAIL) return walk_tile(k);
    else return tile_at(k);
  };
  if constexpr (TAIL) {
    // Slot s starts with the tag of position s - 16 (never read: each slot is written
    // before its position is read); the barrier before the walk (the prologue's, or
    // the one after the first units) orders these writes first.
    if (dyn && kw == 0 && lane < 16) lds_write_u32(&seq_lds[lane], seq_word(lane - 16, -1));
  }
  const int outputs = gemv_outputs(EPI, a.N);

  // ---- where this lane's loads go -------------------------------------------
  // Load q brings unit row 4 q + lane / 16; its chunk within the segment is
  // swizzled so that it lands in slot row * 16 + lane % 16.
  int w_chunk[WL];  // element offset of this lane's swizzled chunk in unit row 4 q + lane / 16
  int x_off[NX];
  const size_t seg0 = (size_t)kw * 128;
#pragma unroll
  for (int q = 0; q < WL; ++q) w_chunk[q] = 8 * ((lane & 15) ^ ring_swz(4 * q + (lane >> 4)));
  const uint16_t* xrow[NX];
#pragma unroll
  for (int q = 0; q < NX; ++q) {
    const int row = 4 * q + (lane >> 4);
    const int r = row < M ? row : M - 1;
    xrow[q] = PRO ? x_row(a, r) : a.x + (size_t)r * K;
    x_off[q] = 8 * ((lane & 15) ^ ring_swz(row));
  }
  auto issue = [&](int t, int j, u32x4_t* dst, bool with_x) {
    const size_t k0 = seg0 + (size_t)j * KW * 128;
    if (with_x) {
#pragma unroll
      for (int q = 0; q < NX; ++q) dma16<0>(xrow[q] + k0 + x_off[q], dst + WS + 64 * q);
    }
#pragma unroll
    for (int q = 0; q < WL; ++q) {
      const int row = ring_weight_row(EPI, t, 4 * q + (lane >> 4), a.N, RT);
      dma16<2>(a.w + (size_t)row * K + k0 + w_chunk[q], dst + 64 * q);
    }
  };

  // ---- RMSNorm prologue, part 1: the gain and the x rows (row-contiguous), issued
  // before the first units so that they return first (loads complete in order) --
  constexpr int GPT = PRO ? (GCH + 64 * KW - 1) / (64 * KW) : 1;
  constexpr int RPW = (16 + KW - 1) / KW;  // rows per wave at most
  constexpr int CPL = C * KW / 4;          // chunks per lane per row: K / 512
  constexpr int SPL = (CPL + 7) / 8;       // 4-part chunks per lane per row of sumsq: K / 16 / 256
  const int parts = K / 16;                // parts per row of sumsq
  const bool from_sums = PRO && a.sumsq != nullptr;  // uniform
  u32x4_t gl[GPT];
  u32x4_t xv[PRO ? RPW : 1][PRO ? CPL : 1];
  if constexpr (PRO) {
    static_assert(CPL * 512 == 128 * C * KW, "K must be a multiple of 512 for the prologue");
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int c = tid + i * 64 * KW;
      gl[i] = asm_load16(a.gamma + (size_t)(c < GCH ? c : 0) * 8);
    }
    // Rows kw + i KW (their parts of sumsq, or the rows themselves); waves past the
    // last row load nothing (the wait below counts only the units issued after
    // these loads). Lanes past the last part read the row's last four (discarded).
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int m = kw + i * KW;
      if (m < M && from_sums) {  // wave-uniform
#pragma unroll
        for (int c = 0; c < SPL; ++c) {
          const int at = (lane + 64 * c) * 4;
          xv[i][c] = asm_load16(a.sumsq + (size_t)m * parts + (at < parts ? at : parts - 4));
        }
#pragma unroll
        for (int c = SPL; c < CPL; ++c) xv[i][c] = u32x4_t{0u, 0u, 0u, 0u};
      } else if (m < M) {  // wave-uniform
        const uint16_t* xr = x_row(a, m);
#pragma unroll
        for (int c = 0; c < CPL; ++c) xv[i][c] = asm_load16(xr + (size_t)(lane + 64 * c) * 8);
      } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) xv[i][c] = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
  }

  // ---- the first D units (all of the first tile: D <= C) ----------------------
  asm volatile("" ::: "memory");  // keep the prologue's loads ahead of the units (the count below)
  const int tile0 = tile_at(0);
#pragma unroll
  for (int d = 0; d < D; ++d) issue(tile0, d, ring[kw] + d * SLOT, true);
  if constexpr (TAIL && !PRO) {
    if (dyn) lds_barrier();  // the tail's slots are written
  }

  // ---- RMSNorm prologue, part 2: row scales while the first units stream -------
  float scale = 0.f;
  if constexpr (PRO) {
    wait_vm<D * (WL + NX)>();  // the gain and x rows are in; the D units may still be in flight
#pragma unroll
    for (int i = 0; i < GPT; ++i) tie(gl[i]);
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
      for (int c = 0; c < CPL; ++c) tie(xv[i][c]);
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int c = tid + i * 64 * KW;
      if (c < GCH) lds_write16(gain + c, gl[i]);
    }
    // The rows the norm reads (the gathered rows) go out once, from workgroup 0.
    if (a.sum != nullptr && wg == 0) {
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        const int m = kw + i * KW;
        if (m < M) {
#pragma unroll
          for (int c = 0; c < CPL; ++c) store16(a.sum + (size_t)m * K + (size_t)(lane + 64 * c) * 8, xv[i][c]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      float ss = 0.f;
      if (from_sums) {
#pragma unroll
        for (int c = 0; c < SPL; ++c) {
          const f32x4_t v = __builtin_bit_cast(f32x4_t, xv[i][c]);
          if ((lane + 64 * c) * 4 < parts) ss += (v[0] + v[1]) + (v[2] + v[3]);
        }
      } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) ss = sum_squares8(xv[i][c], ss);
      }
      const float total = wave_sum(ss);
      const int m = kw + i * KW;
      if (lane == 0 && m < 16) lds_write_f32(red + m, total);
    }
    lds_barrier();
    scale = li < M ? 1.0f / sqrtf(lds_read_f32(red + li) / (float)K + a.eps) : 0.f;
  }

  // ---- epilogue of parked tiles: thread e takes (tile i, lane position ln);
  // D[4 gg + r][ll] of a tile is unit row 4 gg + r, x row ll ------------------
  unsigned long long best = 0ull;
  auto flush = [&](int n, int done) {
    if constexpr (EPI == EPI_SWIGLU) {
      // Gate rows 4 h + r sit at gg = h, the matching up rows at gg = 2 + h.
      const int entries = n * 32;
      for (int e = tid; e < entries; e += 64 * KW) {
        const int ll = e & 15, h = (e >> 4) & 1, i = e >> 5;
        if (ll >= M) continue;
        const int tl = flush_tile(done + i);
        f32x4_t s = part[i][0][0][h * 16 + ll];
        f32x4_t u = part[i][0][0][(2 + h) * 16 + ll];
#pragma unroll
        for (int w = 1; w < KW; ++w) {
          s += part[i][w][0][h * 16 + ll];
          u += part[i][w][0][(2 + h) * 16 + ll];
        }
        const int c0 = tl * 8 + 4 * h;
        uint16_t* yr = a.y + (size_t)ll * outputs;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (c0 + r < outputs) yr[c0 + r] = (uint16_t)swiglu_bf16(s[r], u[r]);
      }
    } else {
      // Subtile sub holds unit rows 16 sub + 4 gg + r; with 24-row tiles the second
      // subtile's rows past 23 are not the tile's.
      const int entries = n * 64 * SUB;
      for (int e = tid; e < entries; e += 64 * KW) {
        const int ln = e & 63, sub = (e >> 6) % SUB, i = e / (64 * SUB);
        const int ll = ln & 15, gg = ln >> 4;
        if (ll >= M || 16 * sub + 4 * gg >= RT) continue;
        const int tl = flush_tile(done + i);
        f32x4_t s = part[i][0][sub][ln];
#pragma unroll
        for (int w = 1; w < KW; ++w) s += part[i][w][sub][ln];
        const int n0 = tl * RT + 16 * sub + 4 * gg;
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
        if constexpr (EPI == EPI_STORE && RT == 16) {
          if (a.sumsq_out != nullptr) {  // the entry's sum of squares waits in the slot it came from
            const float v0 = bf16_to_f32(bits[0]), v1 = bf16_to_f32(bits[1]);
            const float v2 = bf16_to_f32(bits[2]), v3 = bf16_to_f32(bits[3]);
            part[i][0][0][ln][0] = (v0 * v0 + v1 * v1) + (v2 * v2 + v3 * v3);
          }
        }
        if constexpr (EPI == EPI_ARGMAX) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n0 + r < a.N) best = key_max(best, argmax_key(bf16_to_f32(bits[r]), (uint32_t)(n0 + r)));
        }
      }
      // The stored rows' sums of squares by tile (16 outputs), when asked: each entry's
      // four squares (left in its parked slot above, by the same lane) summed over the
      // wave's lanes ln, ln + 16, ln + 32, ln + 48 by two lane-half swaps, in the order
      // (0 + 1) + (2 + 3). Every lane of a wave takes the same entries here (64 per tile).
      if constexpr (EPI == EPI_STORE && RT == 16) {
        if (a.sumsq_out != nullptr) {
          for (int e = tid; e < entries; e += 64 * KW) {
            const int ln = e & 63, i = e >> 6;
            const int ll = ln & 15, gg = ln >> 4;
            const uint32_t sq = __float_as_uint(ll < M ? part[i][0][0][ln][0] : 0.f);
            const auto r16 = __builtin_amdgcn_permlane16_swap(sq, sq, false, false);
            const uint32_t pair = __float_as_uint(__uint_as_float(r16[0]) + __uint_as_float(r16[1]));
            const auto r32 = __builtin_amdgcn_permlane32_swap(pair, pair, false, false);
            const float total = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
            if (gg == 0 && ll < M) a.sumsq_out[(size_t)ll * ((a.N + 15) / 16) + flush_tile(done + i)] = total;
          }
        }
      }
    }
  };

  // ---- the walk --------------------------------------------------------------
  const int rd = li * 16, hs = ring_swz(li);
  const bool x_real = li < 4 * NX;
  u32x4_t xr[XREG ? C : 1][4];
  int count = 0, done = 0;
  // One unit at u (segment J of the current tile): read it into registers, refill
  // (the slot's contents are in registers, so the next load is not held back by
  // the normalisation and the MFMAs), then the four MFMAs. `fresh`: the B
  // operands come from this unit's x (normalised with the prologue) and, with
  // XREG, are kept for the later tiles.
  auto unit = [&](const u32x4_t* u, auto J, bool fresh, f32x4_t (&acc)[SUB], auto&& refill) {
    constexpr int j = decltype(J)::value;
    const size_t kseg = seg0 + (size_t)j * KW * 128;
    // Operands: the weights of each subtile [4 sub, 4 sub + 4), x [XO, XO + 4), the gain after.
    constexpr int XO = 4 * SUB;
    constexpr int NOPS = XO + 4 + (PRO ? 4 : 0);
    u32x4_t op[NOPS];
    // The second subtile of a 24-row tile reads unit rows 16 + (li & 7); its
    // output rows past 23 are discarded.
    const int r1 = 16 + (li & 7), rd1 = r1 * 16, hs1 = ring_swz(r1);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int at = rd + ((4 * s + g) ^ hs);
      op[s] = lds_read16(u + at);
      if constexpr (SUB == 2) op[4 + s] = lds_read16(u + rd1 + ((4 * s + g) ^ hs1));
      if (fresh) {
        op[XO + s] = lds_read16(u + WS + (x_real ? at : 0));
        if constexpr (PRO) op[XO + 4 + s] = lds_read16(gain + ((kseg + 32 * s + 8 * g) >> 3));
      }
    }
    lds_ready(op);
    refill();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4_t b;
      if (fresh) {
        b = op[XO + s];
        if constexpr (PRO) b = norm8(b, op[XO + 4 + s], scale);
        if constexpr (XREG) xr[j][s] = b;
      } else {
        b = xr[XREG ? j : 0][s];
      }
#pragma unroll
      for (int t = 0; t < SUB; ++t) acc[t] = mfma16x16x32(op[4 * t + s], b, acc[t]);
    }
  };
  // Park a finished tile's partials; every DMAX tiles (and after the last) the
  // workgroup sums them and runs their epilogue. Returns false after the last.
  auto park = [&](const f32x4_t (&acc)[SUB], bool more) {
#pragma unroll
    for (int t = 0; t < SUB; ++t) part[count][kw][t][lane] = acc[t];
    ++count;
    if (count == DMAX || !more) {  // workgroup-uniform: every wave walks the same tiles
      lds_barrier();
      flush(count, done);
      done += count;
      count = 0;
      if (!more) return false;
      lds_barrier();  // the next tiles park in the same slots
    }
    return true;
  };

  if constexpr (XREG) {
    // First tile: units of x and weights, two in flight, in the two x-sized slots
    // at 0 and SLOT. From its third unit on, the wave's ring holds four weight-only
    // slots q0..q3 (RT / 4 KiB each) and the next tile's units go there, all four
    // in flight: those wholly inside slot 0 (q0, and q1 too with 16 x rows) once
    // slot 0 is free, the rest once slot 1 is.
    if constexpr (TAIL) {
      int tile1 = dyn ? -1 : walk_tile(1);
      bool more0 = tile1 >= 0;
      f32x4_t acc[SUB] = {};
      static_for<0, C>([&](auto J) {
        constexpr int j = decltype(J)::value;
        constexpr int early = SLOT / WS;  // next-tile units issued after unit C - 2
        if constexpr (j < C - 1) {
          wait_vm<WL + NX>();
        } else {
          if (more0) wait_vm<WL * early>(); else wait_vm<0>();
        }
        if constexpr (j == 0) {
          if (dyn) {
            tile1 = advance(0);
            more0 = tile1 >= 0;
          }
        }
        unit(ring[kw] + (j % 2) * SLOT, J, true, acc, [&] {
          if constexpr (j + 2 < C) {
            issue(tile0, j + 2, ring[kw] + (j % 2) * SLOT, true);
          } else if constexpr (j == C - 2) {
            if (more0) {
  #pragma unroll
              for (int q = 0; q < early; ++q) issue(tile1, q, ring[kw] + WS * q, false);
            }
          } else {
            if (more0) {
  #pragma unroll
              for (int q = early; q < 4; ++q) issue(tile1, q, ring[kw] + WS * q, false);
            }
          }
        });
      });
      if (park(acc, more0)) {
        // Later tiles: unit j of tile i sits in q_j; after reading it, unit j of
        // tile i + 1 takes its place, so the next tile is in flight in full.
        for (int i = 1; dyn || i < my_tiles; ++i) {
          int tile_next = dyn ? -1 : walk_tile(i + 1);
          bool more = dyn || tile_next >= 0;
          f32x4_t acc2[SUB] = {};
          static_for<0, C>([&](auto J) {
            constexpr int j = decltype(J)::value;
            // issued after unit j: units j+1..3 of this tile and units 0..j-1 of the next
            if (more) wait_vm<WL * (C - 1)>(); else wait_vm<WL * (C - 1 - j)>();
            if constexpr (j == 0) {
              if (dyn) {
                tile_next = advance(i);
                more = tile_next >= 0;
              }
            }
            unit(ring[kw] + WS * j, J, false, acc2, [&] {
              if (more) issue(tile_next, j, ring[kw] + WS * j, false);
            });
          });
          if (!park(acc2, more)) break;
        }
      }
    } else {
      const bool more0 = my_tiles > 1;
      f32x4_t acc[SUB] = {};
      static_for<0, C>([&](auto J) {
        constexpr int j = decltype(J)::value;
        constexpr int early = SLOT / WS;  // next-tile units issued after unit C - 2
        if constexpr (j < C - 1) {
          wait_vm<WL + NX>();
        } else {
          if (more0) wait_vm<WL * early>(); else wait_vm<0>();
        }
        unit(ring[kw] + (j % 2) * SLOT, J, true, acc, [&] {
          if constexpr (j + 2 < C) {
            issue(tile_at(0), j + 2, ring[kw] + (j % 2) * SLOT, true);
          } else if constexpr (j == C - 2) {
            if (more0) {
  #pragma unroll
              for (int q = 0; q < early; ++q) issue(tile_at(1), q, ring[kw] + WS * q, false);
            }
          } else {
            if (more0) {
  #pragma unroll
              for (int q = early; q < 4; ++q) issue(tile_at(1), q, ring[kw] + WS * q, false);
            }
          }
        });
      });
      if (park(acc, more0)) {
        // Later tiles: unit j of tile i sits in q_j; after reading it, unit j of
        // tile i + 1 takes its place, so the next tile is in flight in full.
        for (int i = 1; i < my_tiles; ++i) {
          const int tile_next = tile_at(i + 1);
          const bool more = i + 1 < my_tiles;
          f32x4_t acc2[SUB] = {};
          static_for<0, C>([&](auto J) {
            constexpr int j = decltype(J)::value;
            // issued after unit j: units j+1..3 of this tile and units 0..j-1 of the next
            if (more) wait_vm<WL * (C - 1)>(); else wait_vm<WL * (C - 1 - j)>();
            unit(ring[kw] + WS * j, J, false, acc2, [&] {
              if (more) issue(tile_next, j, ring[kw] + WS * j, false);
            });
          });
          if (!park(acc2, more)) break;
        }
      }
    }
  } else {
    // x travels with every unit: D units in flight in D slots of SLOT.
    for (int i = 0; i < my_tiles; ++i) {
      const int tile = tile_at(i), tile_next = tile_at(i + 1);
      const bool more = i + 1 < my_tiles;
      f32x4_t acc[SUB] = {};
      static_for<0, C>([&](auto J) {
        constexpr int j = decltype(J)::value;
        constexpr int slot = j % D;
        // Units issued after this one: the rest of the ring in this tile, then
        // (with more tiles) the first units of the next one; WL + NX loads each.
        constexpr int n_same = (D - 1) < (C - 1 - j) ? (D - 1) : (C - 1 - j);
        constexpr int n_next = (D - 1) - n_same;
        if (more) wait_vm<(n_same + n_next) * (WL + NX)>(); else wait_vm<n_same * (WL + NX)>();
        unit(ring[kw] + slot * SLOT, J, true, acc, [&] {
          if constexpr (j + D < C) {
            issue(tile, j + D, ring[kw] + slot * SLOT, true);
          } else {
            if (more) issue(tile_next, j + D - C, ring[kw] + slot * SLOT, true);
          }
        });
      });
      if (!park(acc, more)) break;
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
      a.keys[(size_t)wg * M + tid] = k;
    }
  }
}

// ---- dispatch -------------------------------------------------------------------

typedef void (*RingKernel)(ProjArgs, int);

// Claimed-tail builds: lm_head + argmax with the norm (the walks long enough, at
// kRingTailMinTiles tiles per workgroup, are the vocabulary's).
static RingKernel pick_ring_tail(int c, int kw, int d, int nx, int rt, bool pro, int epi) {
  if (epi != EPI_ARGMAX || !pro || c != 4 || kw != 8 || d != 2 || rt != 16) return nullptr;
  if (nx == 2) return ring_kernel<4, 8, 2, 2, true, EPI_ARGMAX, 16, true>;
  if (nx == 4) return ring_kernel<4, 8, 2, 4, true, EPI_ARGMAX, 16, true>;
  return nullptr;
}

// Instantiated (C, KW, D, NX, RT): K = 4096 (C = 4 at 8 waves, with or without the
// prologue, every epilogue) with two units in flight, and 24-row tiles for the
// STORE epilogue at up to 8 rows; K = 12288 (C = 12, no prologue, STORE) with two
// or three (three only for 8 x rows: 16 would not fit the LDS). NX = 2 serves
// 2..8 rows, NX = 4 9..16.
#define FTK_RING_SHAPE(C_, KW_, D_, NX_, RT_, PRO, EPI) \
  if (c == C_ && kw == KW_ && d == D_ && nx == NX_ && rt == RT_) return ring_kernel<C_, KW_, D_, NX_, PRO, EPI, RT_>;

template <bool PRO, int EPI>
static RingKernel pick_ring_shape(int c, int kw, int d, int nx, int rt) {
  FTK_RING_SHAPE(4, 8, 2, 2, 16, PRO, EPI)
  FTK_RING_SHAPE(4, 8, 2, 4, 16, PRO, EPI)
  if constexpr (EPI == EPI_STORE) {
    FTK_RING_SHAPE(4, 8, 2, 2, 24, PRO, EPI)
    FTK_RING_SHAPE(4, 8, 2, 2, 12, PRO, EPI)
    FTK_RING_SHAPE(4, 8, 2, 4, 12, PRO, EPI)
  }
  if constexpr (!PRO && EPI == EPI_STORE) {
    FTK_RING_SHAPE(12, 8, 2, 2, 16, PRO, EPI)
    FTK_RING_SHAPE(12, 8, 3, 2, 16, PRO, EPI)
    FTK_RING_SHAPE(12, 8, 2, 4, 16, PRO, EPI)
  }
  return nullptr;
}
#undef FTK_RING_SHAPE

static RingKernel pick_ring(int c, int kw, int d, int nx, int rt, bool pro, int epi) {
  switch (epi) {
    case EPI_STORE: return pro ? pick_ring_shape<true, EPI_STORE>(c, kw, d, nx, rt)
                               : pick_ring_shape<false, EPI_STORE>(c, kw, d, nx, rt);
    case EPI_SWIGLU: return pro ? pick_ring_shape<true, EPI_SWIGLU>(c, kw, d, nx, rt)
                                : pick_ring_shape<false, EPI_SWIGLU>(c, kw, d, nx, rt);
    case EPI_ARGMAX: return pro ? pick_ring_shape<true, EPI_ARGMAX>(c, kw, d, nx, rt)
                                : pick_ring_shape<false, EPI_ARGMAX>(c, kw, d, nx, rt);
  }
  return nullptr;
}

bool ring_supported(int M, int K, int kw, int depth, int epi, bool pro, int rows) {
  const int c = quad_segments(K, kw);
  return M >= 1 && M <= kRingMaxRows && c > 0 &&
         pick_ring(c, kw, depth, ring_x_loads(M), rows, pro, epi) != nullptr;
}

bool ring_tail_supported(int M, int K, int kw, int depth, int epi, bool pro, int rows) {
  const int c = quad_segments(K, kw);
  return M >= 1 && M <= kRingMaxRows && c > 0 &&
         pick_ring_tail(c, kw, depth, ring_x_loads(M), rows, pro, epi) != nullptr;
}

hipError_t launch_ring(const ProjArgs& a, int epi, const RingShape& sh, hipStream_t stream) {
  const int c = quad_segments(a.K, sh.kw);
  RingKernel k = nullptr;
  if (c > 0 && a.claim != nullptr)
    k = pick_ring_tail(c, sh.kw, sh.depth, ring_x_loads(a.M), sh.rows, a.gamma != nullptr, epi);
  if (k == nullptr && c > 0) k = pick_ring(c, sh.kw, sh.depth, ring_x_loads(a.M), sh.rows, a.gamma != nullptr, epi);
  if (k == nullptr || a.M < 1 || a.M > kRingMaxRows) return hipErrorInvalidValue;
  if (sh.grid < 1 || sh.grid > sh.tiles) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(sh.grid), dim3(64 * sh.kw), 0, stream, a, sh.tiles);
  return hipGetLastError();
}

}  // namespace ftk
