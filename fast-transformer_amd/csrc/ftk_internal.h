// Internal launch interface between the C-ABI layer (ftk_capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ftk_device.h"
#include "ftk_plan.h"

namespace ftk {

// FTK_OK for hipSuccess; otherwise records e as this thread's last HIP error
// (ftk_last_hip_error) and returns FTK_ERR_HIP.
int hip_status(hipError_t e);

// Arguments of one skinny projection launch (GEMV or MFMA kind).
struct ProjArgs {
  const uint16_t* x;      // [M, K] BF16, row-major, 16-byte aligned
  const uint16_t* w;      // [N, K] BF16 (PyTorch Linear layout), 16-byte aligned
  const uint16_t* gamma;  // [K] RMSNorm gain, or null (no prologue)
  uint16_t* y;            // STORE: [M, N]; SWIGLU: [M, N/2]; ARGMAX: logits [M, N] or null
  float eps;
  int M, N, K;
  // EPI_ARGMAX only
  void* ids;              // [M] int32 or int64
  int ids_bytes;
  float* top;             // [M] winning logit as FP32, or null
  unsigned long long* keys;  // [grid][M] per-workgroup best keys (workspace; zero between calls)
  int fused;              // 1: one extra workgroup, the grid's last, gathers the keys (argmax_gather)
  // Prologue inputs beyond x (gamma != null only): the rows the norm reads are
  //   s[m] = bf16(xrow(m) + residual[m])   (or xrow(m) without a residual),
  // xrow(m) = x[x_ids[m]] (an embedding gather) or x[m]. Workgroup 0 stores s
  // into sum when sum != null.
  const uint16_t* residual;  // [M, K] or null
  uint16_t* sum;             // [M, K] or null
  const void* x_ids;         // [M] int32 / int64 row indices into x, or null
  int x_ids_bytes;
  int64_t x_rows;            // rows of the table x_ids index (>= 1 with x_ids)
  // EPI_STORE only: the residual stream the outputs are added to, or null. The
  // stored value is then bf16(bf16(y) + out_add[m, n]) (the add of add_rms_norm
  // moved into the producer; it may alias y).
  const uint16_t* out_add;   // [M, N] or null
  // The norm's statistics handed from one projection to the next (RING kind only):
  // sumsq_out (STORE, 16-row tiles) receives, for each output row m and 16-column
  // part t, the FP32 sum of the squares of the stored BF16 outputs, at
  // [m][ceil(N / 16)] + t; a prologue given sumsq ([M][K / 16], written that way for
  // its x) sums those parts instead of reading the rows of x.
  const float* sumsq;
  float* sumsq_out;
  // Long RING walks (kRingTailMinTiles or more tiles per workgroup): the counter their
  // last tiles are claimed from (zero between calls; the launch's last claim resets
  // it), or null for the static order throughout.
  unsigned* claim;
};

// The BF16 bits a STORE epilogue writes for output (m, n) with FP32 sum s.
__device__ __forceinline__ uint32_t store_bits(const ProjArgs& a, float s, int m, int n) {
  const uint32_t b = f32_to_bf16(s);
  if (a.out_add == nullptr) return b;
  return f32_to_bf16(bf16_to_f32(b) + bf16_to_f32(a.out_add[(size_t)m * a.N + n]));
}

// ---- greedy argmax in one launch ------------------------------------------------
// With a.fused, every tile workgroup publishes its best key per row, keys[wg M + m],
// as an agent-scope store (coherent across the XCDs' L2s) of a non-zero word, and
// one extra workgroup -- the grid's last, which walks no tiles -- gathers them: it
// polls the words until each is non-zero, reduces them to the ids (and the top
// values), and zeroes every word once it has read it. The key region is zero
// before every call (zeroed at allocation; the two-launch finalize zeroes what it
// reads too), so a non-zero word is a key of this call. A key is never zero: its
// low half is ~index, and a workgroup without outputs publishes 1, below every
// real key (whose high half is at least orderable(-inf) > 0).
// Only the gatherer waits on other workgroups, so its wait ends in whatever order
// the workgroups run (it holds one workgroup slot; the others need no more). The
// wait is bounded all the same: past kGatherTicks of the 100 MHz clock the gather
// stops and writes id -1 (top NaN) for the row.
constexpr uint64_t kGatherTicks = 100000000ull;  // 1 s
// Workgroups added to the walkers' grid: one per XCD, so that a grid that is a
// multiple of 8 stays one (the hardware deals workgroups to the 8 XCDs in turn,
// which the RING kind's per-XCD tile order relies on). The last gathers; the
// others return at once.
constexpr int kGatherExtra = 8;

__device__ __forceinline__ void publish_key(const ProjArgs& a, size_t slot, unsigned long long k) {
  if (a.fused)
    __hip_atomic_store(a.keys + slot, k ? k : 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    a.keys[slot] = k;
}

__device__ __forceinline__ unsigned long long take_key(unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void clear_key(unsigned long long* p) {
  __hip_atomic_store(p, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void write_id(const ProjArgs& a, int m, unsigned long long k, bool late) {
  const int64_t id = late ? -1 : (int64_t)key_index(k);
  if (a.ids_bytes == 8)
    reinterpret_cast<int64_t*>(a.ids)[m] = id;
  else
    reinterpret_cast<int32_t*>(a.ids)[m] = (int32_t)id;
  if (a.top != nullptr) a.top[m] = late ? __uint_as_float(0x7FC00000u) : from_orderable((uint32_t)(k >> 32));
}

// The gathering workgroup (T threads) of a grid of `walkers` tile workgroups,
// dispatched after every walker. Every word is read in one of two layouts:
// - one row: thread t reads words t, t + T, ..., eight at a time, in walker
//   order; the early batches are ready when it starts, so it consumes them
//   while the last walkers stream;
// - at most T walkers (M > 1): thread t reads the M <= MR words of walker t,
//   each thread on its own, from the gatherer's start.
// Loads are issued together and then checked; a word that is still zero is read
// again after a short sleep, so the handoff leaves about one round of reads
// after the last walker's store. `red` is the kernel's own LDS, T / 64 * MR
// words (the workgroup walks no tiles, so nothing else uses it).
template <int T, int MR>
__device__ void argmax_gather(const ProjArgs& a, int walkers, unsigned long long* red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = a.M;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  bool late = false;
  unsigned long long best[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) best[m] = 0ull;
  if (M == 1) {
    for (int base = tid; base < walkers && !late; base += 8 * T) {
      uint32_t need = 0;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (base + u * T < walkers) need |= 1u << u;
      while (need) {
        unsigned long long k[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) k[u] = take_key(a.keys + min(base + u * T, walkers - 1));
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (((need >> u) & 1u) && k[u] != 0ull) {
            best[0] = key_max(best[0], k[u]);
            need &= ~(1u << u);
            clear_key(a.keys + base + u * T);
          }
        if (need) {
          if (__builtin_amdgcn_s_memrealtime() - t0 > kGatherTicks) {
            late = true;
            break;
          }
          __builtin_amdgcn_s_sleep(4);
        }
      }
    }
  } else if (tid < walkers) {
    uint32_t need = (1u << M) - 1u;  // M <= MR <= 16
    while (need) {
      unsigned long long k[MR];
#pragma unroll
      // Every load is issued (rows past M re-read row M - 1, never used): a load under
      // a condition compiles to a branch whose join waits for it, one round trip each.
      for (int m = 0; m < MR; ++m) k[m] = take_key(a.keys + (size_t)tid * M + (m < M ? m : M - 1));
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (((need >> m) & 1u) && k[m] != 0ull) {
          best[m] = key_max(best[m], k[m]);
          need &= ~(1u << m);
          clear_key(a.keys + (size_t)tid * M + m);
        }
      if (need) {
        if (__builtin_amdgcn_s_memrealtime() - t0 > kGatherTicks) {
          late = true;
          break;
        }
        __builtin_amdgcn_s_sleep(4);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) best[m] = wave_max_key(best[m]);
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[wave * MR + m] = best[m];
  }
  const bool any_late = __syncthreads_or(late) != 0;
  if (tid < M) {
    unsigned long long k = red[tid];
    for (int w = 1; w < T / 64; ++w) k = key_max(k, red[w * MR + tid]);
    write_id(a, tid, k, any_late);
  }
}

// Row m of the prologue's x: x[x_ids[m]] (embedding gather) or x[m]. The host
// cannot see device-side ids, so an id outside [0, x_rows) is clamped into the
// table (below 0 reads row 0, past the end the last row): reads stay in bounds.
__device__ __forceinline__ const uint16_t* x_row(const ProjArgs& a, int m) {
  if (a.x_ids == nullptr) return a.x + (size_t)m * a.K;
  int64_t id = a.x_ids_bytes == 8 ? reinterpret_cast<const int64_t*>(a.x_ids)[m]
                                  : (int64_t) reinterpret_cast<const int32_t*>(a.x_ids)[m];
  id = id < 0 ? 0 : id >= a.x_rows ? a.x_rows - 1 : id;
  return a.x + (size_t)id * a.K;
}

// 8 BF16 values of the prologue's input row m at element k: x (+ residual).
__device__ __forceinline__ u32x4_t prologue_in(const ProjArgs& a, const uint16_t* xr, int m, size_t k) {
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xr + k);
  if (a.residual == nullptr) return v;
  return add8(v, *reinterpret_cast<const u32x4_t*>(a.residual + (size_t)m * a.K + k));
}

// Launch shape of the GEMV kind.
struct GemvShape {
  int rpw;       // weight rows per row group per tile (even for SwiGLU)
  int unroll;    // 16-byte chunks per lane issued per batch of loads
  int kw;        // waves per row group, splitting K (1, 2, 4)
  int grid;      // workgroups (grid-stride over tiles)
  int tiles;
  size_t lds;    // dynamic LDS bytes (x staged as BF16)
};

// Device properties the planner needs (cached per device).
struct DeviceInfo {
  int cus;
  int lds_per_group_max;
  int ok;
};
DeviceInfo device_info();

bool gemv_supported(int M, int rpw, int unroll, int kw, int epi);
hipError_t launch_gemv(const ProjArgs& a, int epi, const GemvShape& shape, hipStream_t stream);

// Launch shape of the STREAM kind (K = 512 C KW, C chunks per lane per row).
struct StreamShape {
  int rpw;       // weight rows per row group per tile (even for SwiGLU)
  int kw;        // waves per row group, splitting K (1, 2, 4)
  int grid;      // workgroups; each walks ceil(tiles / grid) <= kStreamMaxTiles tiles
  int tiles;
};
bool stream_supported(int M, int rpw, int K, int kw, int epi);
hipError_t launch_stream(const ProjArgs& a, int epi, const StreamShape& shape, hipStream_t stream);

// Launch shape of the MFMA_STREAM kind (K = 32 S KW).
struct MstreamShape {
  int subtiles;  // T: 16-row MFMA subtiles per tile
  int unroll;    // U: K steps of weight loads in flight per wave
  int kw;        // waves per workgroup, splitting K (8 or 16)
  int grid;      // workgroups; each walks <= mstream_max_depth(T, KW) tiles
  int tiles;
};
bool mstream_supported(int M, int t, int K, int kw, int unroll, int epi, bool pro);
hipError_t launch_mstream(const ProjArgs& a, int epi, const MstreamShape& shape, hipStream_t stream);

// Launch shape of the QUAD kind (K = 128 C KW, 4x4x4 MFMA blocks).
struct QuadShape {
  int rows;      // weight rows per row group per tile (4 RS; a multiple of 8 for SwiGLU)
  int kw;        // waves per row group, splitting K (4, 8, 16)
  int grid;      // workgroups; each walks ceil(tiles / grid) <= kStreamMaxTiles tiles
  int tiles;
};
bool quad_supported(int M, int rows, int K, int kw, int epi, bool pro);
hipError_t launch_quad(const ProjArgs& a, int epi, const QuadShape& shape, hipStream_t stream);

// Launch shape of the STAGE kind (K = 128 C KW; weights staged through LDS into 16x16x32 MFMAs).
struct StageShape {
  int subtiles;  // T: 16-row MFMA subtiles per tile
  int unroll;    // U: K segments of weight loads in flight per wave
  int kw;        // waves per workgroup, splitting K
  int grid;      // workgroups; each walks tiles wg, wg + grid, ...
  int tiles;
};
bool stage_supported(int M, int t, int K, int kw, int unroll, int epi, bool pro);
hipError_t launch_stage(const ProjArgs& a, int epi, const StageShape& shape, hipStream_t stream);

// Launch shape of the RING kind (K = 128 C KW; weights and x loaded straight into LDS).
struct RingShape {
  int depth;     // D: units (K segments of one tile) in flight per wave
  int kw;        // waves per workgroup, splitting K
  int grid;      // workgroups; workgroup wg takes tile ring_tile(wg, i, grid, tiles) at step i
  int tiles;
  int rows;      // RT: weight rows per tile (12, 16 or 24)
};
bool ring_supported(int M, int K, int kw, int depth, int epi, bool pro, int rows = 16);
// A build with the claimed tail exists for this shape (long walks of lm_head + argmax).
bool ring_tail_supported(int M, int K, int kw, int depth, int epi, bool pro, int rows);
hipError_t launch_ring(const ProjArgs& a, int epi, const RingShape& shape, hipStream_t stream);

// Launch shape of the MFMA kind.
struct MfmaShape {
  int subtiles;  // T: 16-row MFMA subtiles per workgroup
  int unroll;    // MFMA K steps of weight loads in flight per wave
  int waves;     // W: waves per workgroup, splitting K
  int grid;      // workgroups (one per 16 T rows)
};
struct MfmaArgs {
  const float* row_scale;     // [M] RMSNorm scales, written by the prologue pass
};
bool mfma_supported(int M, int t, int unroll, int waves, int epi);
hipError_t launch_mfma(const ProjArgs& a, int epi, const MfmaShape& shape, const MfmaArgs& p, hipStream_t stream);

// Arguments of one split-KV decode-attention launch (engine/kernels/decode_attention.py:31-149).
// A group is one (row, KV head) pair: group = row * kv_heads + kv_head.
struct AttnArgs {
  const uint16_t* q;        // [groups * G, D] BF16: the G query heads of each group, head-major
  const uint16_t* k;        // [groups, capacity, D] BF16 (the [B, Hkv, C, D] cache)
  const uint16_t* v;        // same layout as k
  const int64_t* position;  // newest cache slot: position[pos_stride * row]
  int pos_stride;           // 0: one position for every row; 1: one per row
  uint16_t* out;            // [groups * G, D] BF16
  float* partial;           // [groups, splits, G, D] FP32 numerators (splits > 1 only)
  float* stats;             // [groups, splits, G, 2] FP32 (max, denominator) (splits > 1 only)
  int kv_heads;
  int capacity;             // cache slots per group
  int splits, chunk;        // slot intervals per group and slots per interval
  float scale_log2;         // scale * log2(e), formed in double
  // Q/K head norm + RoPE in the QUAD kind's prologue (rope_attention): q is
  // unused; query, key and value heads come from the packed QKV rows, and the
  // split holding the row's own slot writes its key and value to k_store / v_store.
  const uint16_t* packed;   // [rows, (Hq + 2 Hkv) D] BF16
  const uint16_t* q_gain;   // [D]
  const uint16_t* k_gain;   // [D]
  const uint16_t* cos;      // [table_rows, D] BF16
  const uint16_t* sin;
  const int64_t* phases;    // [rows] RoPE phase added to the position, or null
  uint16_t* k_store;        // the caches k, v as written
  uint16_t* v_store;
  int64_t table_rows;
  int q_heads;
  float q_eps, k_eps;
};

// Launch shape of the decode attention.
struct AttnShape {
  int kind;        // FTK_ATTN_ROWS or FTK_ATTN_QUAD
  int dim;         // D: 64 or 128
  int group_size;  // G: query heads per KV head (1..kAttnMaxGroup)
  int groups;      // rows * KV heads
  int splits;      // slot intervals per group (1: the partials kernel writes the output)
  int chunk;       // slots per interval
  int waves;       // W: waves per workgroup (4, 8)
  int unroll;      // U: cache-row loads of K (and of V) in flight per lane (2, 4, 8)
};
constexpr int kAttnMaxGroup = 8;
constexpr int kAttnMaxSplits = 1024;  // slot intervals per group the merge kernel takes
bool attn_supported(int kind, int dim, int group_size, int waves, int unroll);
hipError_t launch_attention(const AttnArgs& a, const AttnShape& s, hipStream_t stream);

// Arguments of one Q/K head RMSNorm + RoPE + KV-cache update (engine/kernels/qk_rope.py:13-94).
struct RopeArgs {
  const void* packed;        // BF16 [rows, (Hq + 2 Hkv) D], or FP32 partials [splits][rows * (Hq + 2 Hkv) D]
  int splits;                // 1: BF16 input
  int64_t split_stride;      // elements between partial planes (splits > 1)
  const uint16_t* q_gain;    // [D] q_norm weight
  const uint16_t* k_gain;    // [D] k_norm weight
  float q_eps, k_eps;
  const uint16_t* cos;       // [table_rows, D] BF16
  const uint16_t* sin;
  int64_t table_rows;
  const int64_t* position;   // [1], [B] (rows) or the prefill positions (unused)
  const int64_t* phases;     // [rows] with FTK_ROPE_TABLE, else null
  uint16_t* query;           // [rows, Hq, D]
  uint16_t* keys;            // [B, Hkv, C, D]
  uint16_t* values;
  int tokens, q_heads, kv_heads, capacity, dim, mode;
};
hipError_t launch_qk_rope(const RopeArgs& a, int rows, hipStream_t stream);

// Greedy-argmax second stage: ids[m] (and top[m]) from keys[slot * M + m], slot < slots.
hipError_t launch_argmax_finalize(unsigned long long* keys, int slots, int M, void* ids, int ids_bytes,
                                  float* top, hipStream_t stream);

// Ragged or unaligned shapes: one wave per weight row, scalar loads, no prologue/epilogue.
hipError_t launch_gemm_generic(const uint16_t* x, const uint16_t* w, uint16_t* y, const uint16_t* add, int M, int N,
                               int K, hipStream_t stream);

// Standalone operators (the reference's separate kernels).
hipError_t launch_rms_norm(const uint16_t* x, int64_t row_stride, const uint16_t* gamma, uint16_t* y, int rows,
                           int cols, float eps, hipStream_t stream);
hipError_t launch_embed_rms_norm(const void* ids, int ids_bytes, const uint16_t* table, const uint16_t* gamma,
                                 uint16_t* y, uint16_t* hidden, int rows, int cols, float eps, hipStream_t stream);
hipError_t launch_add_rms_norm(const void* x, int splits, int64_t split_stride, const uint16_t* residual,
                               const uint16_t* gamma, uint16_t* y, uint16_t* sum, int rows, int cols, float eps,
                               hipStream_t stream);
hipError_t launch_swiglu(const void* packed, int splits, int64_t split_stride, uint16_t* out, int rows, int width,
                         hipStream_t stream);
hipError_t launch_argmax(const uint16_t* logits, int rows, int vocab, void* ids, int ids_bytes, float* top,
                         unsigned long long* keys, hipStream_t stream);
int argmax_blocks(int vocab);
hipError_t launch_merge_splits(const float* partial, int splits, int64_t count, uint16_t* out, hipStream_t stream);
// Pure streaming read of `bytes` (the bandwidth reference of the projections): `grid`
// persistent workgroups, or with grid 0 one-shot workgroups of `loads` chunks per lane;
// `loads` (2, 4, 8 or 16) 16-byte loads in flight per lane.
hipError_t launch_stream_read(const void* src, int64_t bytes, uint32_t* sink, int grid, int loads,
                              hipStream_t stream);
int64_t stream_read_once_grid(int64_t bytes, int loads);

}  // namespace ftk
