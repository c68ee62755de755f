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

// Stage two: one workgroup per row picks the best of ``slots`` keys and writes
// the id (and the winning logit) (argmax.py:34-48 _first_best). The keys were
// just written by other CUs, so every load is a long trip: each thread issues
// its kFinalizeLoads loads together, and 1024 threads cover 8192 slots a round.
constexpr int kFinalizeThreads = 1024;
constexpr int kFinalizeLoads = 8;
__global__ __launch_bounds__(kFinalizeThreads) void argmax_finalize_kernel(const unsigned long long* __restrict__ keys,
                                                                           int slots, int rows, void* ids,
                                                                           int ids_bytes, float* top) {
  __shared__ unsigned long long red[kFinalizeThreads / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  unsigned long long best = 0ull;
  for (int base = 0; base < slots; base += kFinalizeLoads * kFinalizeThreads) {
    unsigned long long k[kFinalizeLoads];
#pragma unroll
    for (int u = 0; u < kFinalizeLoads; ++u) {
      const int s = base + u * kFinalizeThreads + tid;
      k[u] = s < slots ? keys[(size_t)s * rows + row] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < kFinalizeLoads; ++u) best = key_max(best, k[u]);
  }
  best = wave_max_key(best);
  if ((tid & 63) == 0) red[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    for (int w = 0; w < kFinalizeThreads / 64; ++w) best = key_max(best, red[w]);
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

hipError_t launch_rms_norm(const uint16_t* x, int64_t row_stride, const uint16_t* gamma, uint16_t* y, int rows,
                           int cols, float eps, hipStream_t stream) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, row_stride, gamma, y, cols, eps);
  return hipGetLastError();
}

hipError_t launch_embed_rms_norm(const void* ids, int ids_bytes, const uint16_t* table, const uint16_t* gamma,
                                 uint16_t* y, uint16_t* hidden, int rows, int cols, float eps, hipStream_t stream) {
  hipLaunchKernelGGL(embed_rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, ids, ids_bytes, table, gamma, y,
                     hidden, cols, eps);
  return hipGetLastError();
}

hipError_t launch_add_rms_norm(const void* x, int splits, int64_t split_stride, const uint16_t* residual,
                               const uint16_t* gamma, uint16_t* y, uint16_t* sum, int rows, int cols, float eps,
                               hipStream_t stream) {
  hipLaunchKernelGGL(add_rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, splits, split_stride, residual,
                     gamma, y, sum, cols, eps);
  return hipGetLastError();
}

hipError_t launch_swiglu(const void* packed, int splits, int64_t split_stride, uint16_t* out, int rows, int width,
                         hipStream_t stream) {
  const int64_t total = (int64_t)rows * width;
  const int64_t grid = (total + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, packed, splits, split_stride,
                     out, width, total);
  return hipGetLastError();
}

hipError_t launch_argmax(const uint16_t* logits, int rows, int vocab, void* ids, int ids_bytes, float* top,
                         unsigned long long* keys, hipStream_t stream) {
  const int blocks = argmax_blocks(vocab);
  hipLaunchKernelGGL(argmax_block_kernel, dim3(blocks, rows), dim3(kThreads), 0, stream, logits, vocab, keys, rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_argmax_finalize(keys, blocks, rows, ids, ids_bytes, top, stream);
}

hipError_t launch_argmax_finalize(const unsigned long long* keys, int slots, int M, void* ids, int ids_bytes,
                                  float* top, hipStream_t stream) {
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(M), dim3(kFinalizeThreads), 0, stream, keys, slots, M, ids,
                     ids_bytes, top);
  return hipGetLastError();
}

hipError_t launch_merge_splits(const float* partial, int splits, int64_t count, uint16_t* out, hipStream_t stream) {
  const int64_t grid = (count + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(merge_splits_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, partial, splits, count,
                     out);
  return hipGetLastError();
}

}  // namespace ftk
