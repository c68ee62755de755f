// Standalone operators of the path, for callers that keep them separate:
//   rms_norm       engine/kernels/rmsnorm.py:21-72
//   add_rms_norm   engine/kernels/rmsnorm.py:75-125 (BF16 input or FP32 split partials)
//   swiglu         engine/kernels/swiglu.py:13-40   (BF16 input or FP32 split partials)
//   argmax         engine/kernels/argmax.py:19-70   (lowest index on ties; two stages)
//   merge_splits   engine/kernels/linear.py:81-93, engine/kernels/merged.py:37-45
// These are small, launch-bound kernels; the projections fold the norm, SwiGLU
// and argmax into themselves and do not need them.
#include "ftk_device.h"
#include "ftk_internal.h"

namespace ftk {

// Sum over the workgroup in a fixed order (wave DPP tree, then waves 0..3).
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const float total = ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();
  return total;
}

// Value of element ``off`` of a BF16 tensor, or bf16(sum of FP32 partials in split order).
__device__ __forceinline__ float merged_value(const void* src, int splits, int64_t stride, int64_t off) {
  if (splits == 0) return bf16_to_f32(reinterpret_cast<const uint16_t*>(src)[off]);
  const float* p = reinterpret_cast<const float*>(src);
  float total = p[off];
  for (int s = 1; s < splits; ++s) total += p[(int64_t)s * stride + off];
  return round_bf16(total);
}

__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const uint16_t* __restrict__ x, int64_t row_stride,
                                                            const uint16_t* __restrict__ gamma,
                                                            uint16_t* __restrict__ y, int cols, float eps) {
  __shared__ float red[kWaves];
  const uint16_t* xr = x + (int64_t)blockIdx.x * row_stride;
  uint16_t* yr = y + (int64_t)blockIdx.x * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float v = bf16_to_f32(xr[c]);
    ss += v * v;
  }
  const float scale = 1.0f / sqrtf(block_sum(ss, red) / (float)cols + eps);
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float n = round_bf16(bf16_to_f32(xr[c]) * scale);
    yr[c] = (uint16_t)f32_to_bf16(n * bf16_to_f32(gamma[c]));
  }
}

// embed_rms_norm (engine/kernels/rmsnorm.py:128-162): row r is table[ids[r]],
// copied out as the residual stream and normalised like rms_norm.
__global__ __launch_bounds__(kThreads) void embed_rms_norm_kernel(const void* __restrict__ ids, int ids_bytes,
                                                                  const uint16_t* __restrict__ table,
                                                                  const uint16_t* __restrict__ gamma,
                                                                  uint16_t* __restrict__ y,
                                                                  uint16_t* __restrict__ hidden, int cols, float eps) {
  __shared__ float red[kWaves];
  const int r = blockIdx.x;
  const int64_t id = ids_bytes == 8 ? reinterpret_cast<const int64_t*>(ids)[r]
                                    : (int64_t) reinterpret_cast<const int32_t*>(ids)[r];
  const uint16_t* xr = table + id * cols;
  uint16_t* hr = hidden + (int64_t)r * cols;
  uint16_t* yr = y + (int64_t)r * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const uint16_t v = xr[c];
    hr[c] = v;
    const float f = bf16_to_f32(v);
    ss += f * f;
  }
  const float scale = 1.0f / sqrtf(block_sum(ss, red) / (float)cols + eps);
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float n = round_bf16(bf16_to_f32(xr[c]) * scale);
    yr[c] = (uint16_t)f32_to_bf16(n * bf16_to_f32(gamma[c]));
  }
}

__global__ __launch_bounds__(kThreads) void add_rms_norm_kernel(const void* __restrict__ x, int splits,
                                                                int64_t split_stride,
                                                                const uint16_t* __restrict__ residual,
                                                                const uint16_t* __restrict__ gamma,
                                                                uint16_t* __restrict__ y, uint16_t* __restrict__ sum,
                                                                int cols, float eps) {
  __shared__ float red[kWaves];
  const int64_t base = (int64_t)blockIdx.x * cols;
  float ss = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    // The residual addition is a BF16 tensor operation: round the sum first.
    const float s = round_bf16(merged_value(x, splits, split_stride, base + c) + bf16_to_f32(residual[base + c]));
    sum[base + c] = (uint16_t)f32_to_bf16(s);
    ss += s * s;
  }
  const float scale = 1.0f / sqrtf(block_sum(ss, red) / (float)cols + eps);
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float s = round_bf16(merged_value(x, splits, split_stride, base + c) + bf16_to_f32(residual[base + c]));
    const float n = round_bf16(s * scale);
    y[base + c] = (uint16_t)f32_to_bf16(n * bf16_to_f32(gamma[c]));
  }
}

__global__ __launch_bounds__(kThreads) void swiglu_kernel(const void* __restrict__ packed, int splits,
                                                          int64_t split_stride, uint16_t* __restrict__ out,
                                                          int width, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= total) return;
  const int64_t row = i / width, j = i - row * width;
  const int64_t g_off = row * 2 * width + j;
  const float g = merged_value(packed, splits, split_stride, g_off);
  const float u = merged_value(packed, splits, split_stride, g_off + width);
  out[i] = (uint16_t)swiglu_bf16(g, u);
}

// ---- Row-resident forms ------------------------------------------------------
// For rows of cols % 8 == 0 elements, at most 8 kThreads R of them, on 16-byte
// aligned pointers. Thread t holds chunks t, t + kThreads, ... (8 elements each)
// of its row in registers, so every load of a row goes out at once: one round
// trip instead of one per loop step. The squares are summed through
// sum_squares8 in that chunk order and the wave totals in wave order, as the
// STREAM kind's prologue sums them (thread t: chunks t, t + 256, ...), so
// rms_norm followed by an M = 1 projection scales each row exactly as the
// fused default does at M = 1. The output pass reads nothing but registers
// (the gain is loaded beside the row).
// Loads are unconditional (a chunk index past the row re-reads the last chunk,
// whose value is then replaced by zero), so no branch joins wait on them.

// bf16(bf16(v * scale) * gain) for 8 values, as stored (every NaN as 0x7FC0):
// the cast order of engine/kernels/rmsnorm.py:35-46.
__device__ __forceinline__ u32x4_t norm8_store(u32x4_t v, u32x4_t g, float scale) {
  const uint32_t e[4] = {v[0], v[1], v[2], v[3]};
  const uint32_t ge[4] = {g[0], g[1], g[2], g[3]};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t n = rne_pair(lo_f32(e[i]) * scale, hi_f32(e[i]) * scale);
    o[i] = pack_bf16(lo_f32(n) * lo_f32(ge[i]), hi_f32(n) * hi_f32(ge[i]));
  }
  return u32x4_t{o[0], o[1], o[2], o[3]};
}

// 4 FP32 values from a 16-byte chunk (elements copied to scalars first, as widen8 does).
__device__ __forceinline__ void widen4f(u32x4_t v, float* out) {
  const uint32_t e[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(e[i]);
}

// Chunk j of this thread, clamped into the row for an unconditional load.
__device__ __forceinline__ int row_chunk(int j, int chunks) {
  const int c = (int)threadIdx.x + j * kThreads;
  return c < chunks ? c : chunks - 1;
}
__device__ __forceinline__ bool own_chunk(int j, int chunks) { return (int)threadIdx.x + j * kThreads < chunks; }

// Sum of squares of R chunks (zero chunks add nothing) and the row's scale.
template <int R>
__device__ __forceinline__ float rows_scale(const u32x4_t (&v)[R], int cols, float eps, float* red) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < R; ++j) ss = sum_squares8(v[j], ss);
  return 1.0f / sqrtf(block_sum(ss, red) / (float)cols + eps);
}

template <int R>
__global__ __launch_bounds__(kThreads) void rms_norm_rows_kernel(const uint16_t* __restrict__ x, int64_t row_stride,
                                                                 const uint16_t* __restrict__ gamma,
                                                                 uint16_t* __restrict__ y, int cols, float eps) {
  __shared__ float red[kWaves];
  const int chunks = cols >> 3;
  const uint16_t* xr = x + (int64_t)blockIdx.x * row_stride;
  uint16_t* yr = y + (int64_t)blockIdx.x * cols;
  u32x4_t v[R], g[R];
#pragma unroll
  for (int j = 0; j < R; ++j) v[j] = load16(xr + 8 * row_chunk(j, chunks));
#pragma unroll
  for (int j = 0; j < R; ++j) g[j] = load16(gamma + 8 * row_chunk(j, chunks));
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (!own_chunk(j, chunks)) v[j] = u32x4_t{0u, 0u, 0u, 0u};
  const float scale = rows_scale(v, cols, eps, red);
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (own_chunk(j, chunks)) store16(yr + 8 * ((int)threadIdx.x + j * kThreads), norm8_store(v[j], g[j], scale));
}

template <int R>
__global__ __launch_bounds__(kThreads) void embed_rms_norm_rows_kernel(const void* __restrict__ ids, int ids_bytes,
                                                                       const uint16_t* __restrict__ table,
                                                                       const uint16_t* __restrict__ gamma,
                                                                       uint16_t* __restrict__ y,
                                                                       uint16_t* __restrict__ hidden, int cols,
                                                                       float eps) {
  __shared__ float red[kWaves];
  const int chunks = cols >> 3;
  const int r = blockIdx.x;
  const int64_t id = ids_bytes == 8 ? reinterpret_cast<const int64_t*>(ids)[r]
                                    : (int64_t) reinterpret_cast<const int32_t*>(ids)[r];
  const uint16_t* xr = table + id * cols;
  u32x4_t v[R], g[R];
#pragma unroll
  for (int j = 0; j < R; ++j) g[j] = load16(gamma + 8 * row_chunk(j, chunks));
#pragma unroll
  for (int j = 0; j < R; ++j) v[j] = load16(xr + 8 * row_chunk(j, chunks));
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (!own_chunk(j, chunks)) v[j] = u32x4_t{0u, 0u, 0u, 0u};
  const float scale = rows_scale(v, cols, eps, red);
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (own_chunk(j, chunks)) {
      const int64_t at = (int64_t)r * cols + 8 * ((int)threadIdx.x + j * kThreads);
      store16(hidden + at, v[j]);
      store16(y + at, norm8_store(v[j], g[j], scale));
    }
}

// S == 0: x is BF16. S = 1..4: x is S FP32 partial planes, summed in split
// order and rounded once (engine/kernels/merged.py:37-45), then added to the
// residual as a BF16 tensor operation (rmsnorm.py:86-88).
template <int R, int S>
__global__ __launch_bounds__(kThreads) void add_rms_norm_rows_kernel(const void* __restrict__ x, int64_t split_stride,
                                                                     const uint16_t* __restrict__ residual,
                                                                     const uint16_t* __restrict__ gamma,
                                                                     uint16_t* __restrict__ y,
                                                                     uint16_t* __restrict__ sum, int cols,
                                                                     float eps) {
  __shared__ float red[kWaves];
  const int chunks = cols >> 3;
  const int64_t base = (int64_t)blockIdx.x * cols;
  u32x4_t v[R], g[R], r[R];
  if constexpr (S == 0) {
    const uint16_t* xr = reinterpret_cast<const uint16_t*>(x) + base;
#pragma unroll
    for (int j = 0; j < R; ++j) v[j] = load16(xr + 8 * row_chunk(j, chunks));
#pragma unroll
    for (int j = 0; j < R; ++j) r[j] = load16(residual + base + 8 * row_chunk(j, chunks));
#pragma unroll
    for (int j = 0; j < R; ++j) g[j] = load16(gamma + 8 * row_chunk(j, chunks));
#pragma unroll
    for (int j = 0; j < R; ++j) v[j] = add8(v[j], r[j]);
  } else {
    const float* xr = reinterpret_cast<const float*>(x) + base;
    u32x4_t p[S][R][2];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const float* at = xr + s * split_stride + 8 * row_chunk(j, chunks);
        p[s][j][0] = load16(at);
        p[s][j][1] = load16(at + 4);
      }
#pragma unroll
    for (int j = 0; j < R; ++j) r[j] = load16(residual + base + 8 * row_chunk(j, chunks));
#pragma unroll
    for (int j = 0; j < R; ++j) g[j] = load16(gamma + 8 * row_chunk(j, chunks));
#pragma unroll
    for (int j = 0; j < R; ++j) {
      float t[8];
      widen4f(p[0][j][0], t);
      widen4f(p[0][j][1], t + 4);
#pragma unroll
      for (int s = 1; s < S; ++s) {
        float q[8];
        widen4f(p[s][j][0], q);
        widen4f(p[s][j][1], q + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) t[e] += q[e];
      }
      const uint32_t re[4] = {r[j][0], r[j][1], r[j][2], r[j][3]};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] = pack_bf16(round_bf16(t[2 * i]) + lo_f32(re[i]), round_bf16(t[2 * i + 1]) + hi_f32(re[i]));
      v[j] = u32x4_t{o[0], o[1], o[2], o[3]};
    }
  }
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (!own_chunk(j, chunks)) v[j] = u32x4_t{0u, 0u, 0u, 0u};
  const float scale = rows_scale(v, cols, eps, red);
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (own_chunk(j, chunks)) {
      const int64_t at = base + 8 * ((int)threadIdx.x + j * kThreads);
      store16(sum + at, v[j]);
      store16(y + at, norm8_store(v[j], g[j], scale));
    }
}

// SwiGLU on V outputs per thread (width % 8 == 0, 16-byte aligned), the gate and
// up values loaded together: V = 8 from BF16 (two 16-byte loads), V = 4 from S
// FP32 partial planes (two 16-byte loads per plane, so twice the threads).
template <int S>
__global__ __launch_bounds__(kThreads) void swiglu_rows_kernel(const void* __restrict__ packed, int64_t split_stride,
                                                               uint16_t* __restrict__ out, int width,
                                                               int64_t groups) {
  constexpr int V = S == 0 ? 8 : 4;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= groups) return;
  const int64_t per_row = width / V;
  const int64_t row = i / per_row, j = i - row * per_row;
  const int64_t g_off = row * 2 * width + V * j;
  float g[V], u[V];
  if constexpr (S == 0) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(packed);
    widen8(load16(p + g_off), g);
    widen8(load16(p + g_off + width), u);
  } else {
    const float* p = reinterpret_cast<const float*>(packed);
    u32x4_t q[S][2];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      q[s][0] = load16(p + s * split_stride + g_off);
      q[s][1] = load16(p + s * split_stride + g_off + width);
    }
    widen4f(q[0][0], g);
    widen4f(q[0][1], u);
#pragma unroll
    for (int s = 1; s < S; ++s) {
      float a[4], b[4];
      widen4f(q[s][0], a);
      widen4f(q[s][1], b);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        g[e] += a[e];
        u[e] += b[e];
      }
    }
  }
  uint32_t o[V / 2];
#pragma unroll
  for (int k = 0; k < V / 2; ++k)
    o[k] = swiglu_bf16(g[2 * k], u[2 * k]) | (swiglu_bf16(g[2 * k + 1], u[2 * k + 1]) << 16);
  uint16_t* dst = out + row * width + V * j;
  if constexpr (V == 8)
    store16(dst, u32x4_t{o[0], o[1], o[2], o[3]});
  else
    *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{o[0], o[1]};
}

// Stage one: one workgroup per (row, column block of 8192) reduces its block to
// a key (orderable BF16 value, inverted index) and stores it (argmax.py:19-31).
constexpr int kArgmaxBlock = 8192;

int argmax_blocks(int vocab) { return (vocab + kArgmaxBlock - 1) / kArgmaxBlock; }

// Largest key of a kThreads workgroup (valid in thread 0).
__device__ __forceinline__ unsigned long long block_max_key(unsigned long long v, unsigned long long* red) {
  v = wave_max_key(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  for (int w = 1; w < kWaves; ++w) v = key_max(v, red[w]);
  return key_max(v, red[0]);
}

__global__ __launch_bounds__(kThreads) void argmax_block_kernel(const uint16_t* __restrict__ logits, int vocab,
                                                                unsigned long long* __restrict__ keys, int rows) {
  __shared__ unsigned long long red[kWaves];
  const int row = blockIdx.y;
  const int begin = blockIdx.x * kArgmaxBlock;
  const int end = min(begin + kArgmaxBlock, vocab);
  const uint16_t* lr = logits + (int64_t)row * vocab;
  unsigned long long best = 0ull;
  for (int c = begin + threadIdx.x; c < end; c += kThreads)
    best = key_max(best, argmax_key(bf16_to_f32(lr[c]), (uint32_t)c));
  best = block_max_key(best, red);
  if (threadIdx.x == 0) keys[(size_t)blockIdx.x * rows + row] = best;  // [slot][row]
}

// Stage one for rows of vocab % 8 == 0 on 16-byte aligned logits: each thread
// loads its four 8-logit chunks of the block (t, t + 256, ...) at once, so the
// block costs one round trip. Same keys as argmax_block_kernel.
__global__ __launch_bounds__(kThreads) void argmax_block_rows_kernel(const uint16_t* __restrict__ logits, int vocab,
                                                                     unsigned long long* __restrict__ keys,
                                                                     int rows) {
  constexpr int kChunks = kArgmaxBlock / 8 / kThreads;  // 16-byte chunks per thread
  __shared__ unsigned long long red[kWaves];
  const int row = blockIdx.y;
  const int begin = blockIdx.x * kArgmaxBlock;
  const int n = (min(begin + kArgmaxBlock, vocab) - begin) >> 3;  // chunks in this block
  const uint16_t* lr = logits + (int64_t)row * vocab + begin;
  u32x4_t v[kChunks];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) v[j] = load16(lr + 8 * row_chunk(j, n));
  unsigned long long best = 0ull;
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    if (!own_chunk(j, n)) continue;
    const int c0 = begin + 8 * ((int)threadIdx.x + j * kThreads);
    float f[8];
    widen8(v[j], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) best = key_max(best, argmax_key(f[e], (uint32_t)(c0 + e)));
  }
  best = block_max_key(best, red);
  if (threadIdx.x == 0) keys[(size_t)blockIdx.x * rows + row] = best;  // [slot][row]
}

// Stage two: one workgroup per row picks the best of ``slots`` keys and writes
// the id (and the winning logit) (argmax.py:34-48 _first_best). The keys were
// just written by other CUs, so every load is a long trip: each thread issues
// its kFinalizeLoads loads together (unconditionally, slots past the end
// re-reading the last one: a load under a condition compiles to a branch whose
// join waits for it). The workgroup is as small as covers the slots in one round
// (one wave for up to 512 slots), up to 1024 threads (8192 slots a round). Every
// key is zeroed once read: the key region is zero between calls, which the
// one-launch argmax (argmax_gather) relies on when it shares the workspace.
constexpr int kFinalizeLoads = 8;
template <int T>
__global__ __launch_bounds__(T) void argmax_finalize_kernel(unsigned long long* __restrict__ keys, int slots,
                                                            int rows, void* ids, int ids_bytes, float* top) {
  __shared__ unsigned long long red[T / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  unsigned long long best = 0ull;
  for (int base = 0; base < slots; base += kFinalizeLoads * T) {
    unsigned long long k[kFinalizeLoads];
#pragma unroll
    for (int u = 0; u < kFinalizeLoads; ++u) {
      const int s = base + u * T + tid;
      k[u] = keys[(size_t)(s < slots ? s : slots - 1) * rows + row];
    }
#pragma unroll
    for (int u = 0; u < kFinalizeLoads; ++u) {
      const int s = base + u * T + tid;
      if (s < slots) keys[(size_t)s * rows + row] = 0ull;
    }
#pragma unroll
    for (int u = 0; u < kFinalizeLoads; ++u) best = key_max(best, k[u]);
  }
  best = wave_max_key(best);
  if constexpr (T > 64) {
    if ((tid & 63) == 0) red[tid >> 6] = best;
    __syncthreads();
    for (int w = 0; w < T / 64; ++w) best = key_max(best, red[w]);
  }
  if (tid == 0) {
    const uint32_t idx = key_index(best);
    if (ids_bytes == 8)
      reinterpret_cast<int64_t*>(ids)[row] = (int64_t)idx;
    else
      reinterpret_cast<int32_t*>(ids)[row] = (int32_t)idx;
    if (top != nullptr) top[row] = from_orderable((uint32_t)(best >> 32));
  }
}

__global__ __launch_bounds__(kThreads) void merge_splits_kernel(const float* __restrict__ partial, int splits,
                                                                int64_t count, uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= count) return;
  float total = partial[i];
  for (int s = 1; s < splits; ++s) total += partial[(int64_t)s * count + i];
  out[i] = (uint16_t)f32_to_bf16(total);
}

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// 16-byte chunks per thread of the row-resident forms for a row of `cols`
// elements, or 0 where only the element loop applies (ragged or long rows).
int rows_chunks(int64_t cols) {
  if (cols % 8 != 0 || cols > 8 * kThreads * 4) return 0;
  const int64_t per = (cols / 8 + kThreads - 1) / kThreads;
  return per <= 1 ? 1 : per <= 2 ? 2 : 4;
}

}  // namespace

hipError_t launch_rms_norm(const uint16_t* x, int64_t row_stride, const uint16_t* gamma, uint16_t* y, int rows,
                           int cols, float eps, hipStream_t stream) {
  const int r = rows_chunks(cols);
  if (r && row_stride % 8 == 0 && aligned16(x) && aligned16(gamma) && aligned16(y)) {
    auto kernel = r == 1 ? rms_norm_rows_kernel<1> : r == 2 ? rms_norm_rows_kernel<2> : rms_norm_rows_kernel<4>;
    hipLaunchKernelGGL(kernel, dim3(rows), dim3(kThreads), 0, stream, x, row_stride, gamma, y, cols, eps);
  } else {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, row_stride, gamma, y, cols, eps);
  }
  return hipGetLastError();
}

hipError_t launch_embed_rms_norm(const void* ids, int ids_bytes, const uint16_t* table, const uint16_t* gamma,
                                 uint16_t* y, uint16_t* hidden, int rows, int cols, float eps, hipStream_t stream) {
  const int r = rows_chunks(cols);
  if (r && aligned16(table) && aligned16(gamma) && aligned16(y) && aligned16(hidden)) {
    auto kernel = r == 1   ? embed_rms_norm_rows_kernel<1>
                  : r == 2 ? embed_rms_norm_rows_kernel<2>
                           : embed_rms_norm_rows_kernel<4>;
    hipLaunchKernelGGL(kernel, dim3(rows), dim3(kThreads), 0, stream, ids, ids_bytes, table, gamma, y, hidden, cols,
                       eps);
  } else {
    hipLaunchKernelGGL(embed_rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, ids, ids_bytes, table, gamma, y,
                       hidden, cols, eps);
  }
  return hipGetLastError();
}

hipError_t launch_add_rms_norm(const void* x, int splits, int64_t split_stride, const uint16_t* residual,
                               const uint16_t* gamma, uint16_t* y, uint16_t* sum, int rows, int cols, float eps,
                               hipStream_t stream) {
  const int r = rows_chunks(cols);
  if (r && splits <= 4 && (splits == 0 || split_stride % 4 == 0) && aligned16(x) && aligned16(residual) &&
      aligned16(gamma) && aligned16(y) && aligned16(sum)) {
    typedef void (*Kernel)(const void*, int64_t, const uint16_t*, const uint16_t*, uint16_t*, uint16_t*, int, float);
    static const Kernel table[3][5] = {
        {add_rms_norm_rows_kernel<1, 0>, add_rms_norm_rows_kernel<1, 1>, add_rms_norm_rows_kernel<1, 2>,
         add_rms_norm_rows_kernel<1, 3>, add_rms_norm_rows_kernel<1, 4>},
        {add_rms_norm_rows_kernel<2, 0>, add_rms_norm_rows_kernel<2, 1>, add_rms_norm_rows_kernel<2, 2>,
         add_rms_norm_rows_kernel<2, 3>, add_rms_norm_rows_kernel<2, 4>},
        {add_rms_norm_rows_kernel<4, 0>, add_rms_norm_rows_kernel<4, 1>, add_rms_norm_rows_kernel<4, 2>,
         add_rms_norm_rows_kernel<4, 3>, add_rms_norm_rows_kernel<4, 4>},
    };
    hipLaunchKernelGGL(table[r == 1 ? 0 : r == 2 ? 1 : 2][splits], dim3(rows), dim3(kThreads), 0, stream, x,
                       split_stride, residual, gamma, y, sum, cols, eps);
  } else {
    hipLaunchKernelGGL(add_rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, splits, split_stride, residual,
                       gamma, y, sum, cols, eps);
  }
  return hipGetLastError();
}

hipError_t launch_swiglu(const void* packed, int splits, int64_t split_stride, uint16_t* out, int rows, int width,
                         hipStream_t stream) {
  const int64_t total = (int64_t)rows * width;
  if (width % 8 == 0 && splits <= 4 && (splits == 0 || split_stride % 4 == 0) && aligned16(packed) &&
      aligned16(out)) {
    typedef void (*Kernel)(const void*, int64_t, uint16_t*, int, int64_t);
    static const Kernel table[5] = {swiglu_rows_kernel<0>, swiglu_rows_kernel<1>, swiglu_rows_kernel<2>,
                                    swiglu_rows_kernel<3>, swiglu_rows_kernel<4>};
    const int64_t groups = total / (splits == 0 ? 8 : 4);
    const int64_t grid = (groups + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(table[splits], dim3((unsigned)grid), dim3(kThreads), 0, stream, packed, split_stride, out,
                       width, groups);
  } else {
    const int64_t grid = (total + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, packed, splits, split_stride,
                       out, width, total);
  }
  return hipGetLastError();
}

hipError_t launch_argmax(const uint16_t* logits, int rows, int vocab, void* ids, int ids_bytes, float* top,
                         unsigned long long* keys, hipStream_t stream) {
  const int blocks = argmax_blocks(vocab);
  if (vocab % 8 == 0 && aligned16(logits))
    hipLaunchKernelGGL(argmax_block_rows_kernel, dim3(blocks, rows), dim3(kThreads), 0, stream, logits, vocab, keys,
                       rows);
  else
    hipLaunchKernelGGL(argmax_block_kernel, dim3(blocks, rows), dim3(kThreads), 0, stream, logits, vocab, keys,
                       rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_argmax_finalize(keys, blocks, rows, ids, ids_bytes, top, stream);
}

hipError_t launch_argmax_finalize(unsigned long long* keys, int slots, int M, void* ids, int ids_bytes,
                                  float* top, hipStream_t stream) {
  if (slots <= 64 * kFinalizeLoads)
    hipLaunchKernelGGL(argmax_finalize_kernel<64>, dim3(M), dim3(64), 0, stream, keys, slots, M, ids, ids_bytes, top);
  else if (slots <= 256 * kFinalizeLoads)
    hipLaunchKernelGGL(argmax_finalize_kernel<256>, dim3(M), dim3(256), 0, stream, keys, slots, M, ids, ids_bytes,
                       top);
  else
    hipLaunchKernelGGL(argmax_finalize_kernel<1024>, dim3(M), dim3(1024), 0, stream, keys, slots, M, ids, ids_bytes,
                       top);
  return hipGetLastError();
}

hipError_t launch_merge_splits(const float* partial, int splits, int64_t count, uint16_t* out, hipStream_t stream) {
  const int64_t grid = (count + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(merge_splits_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, partial, splits, count,
                     out);
  return hipGetLastError();
}

}  // namespace ftk
