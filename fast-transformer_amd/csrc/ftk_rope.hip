// Q/K head RMSNorm, RoPE and the KV-cache update of one decode (or prefill)
// step on gfx950: engine/kernels/qk_rope.py:13-94 (_qk_rope_cache).
//
// One wave per (row, head); a workgroup holds W heads of one row. Lane l holds
// the D / 64 consecutive elements starting at l D / 64, so the RoPE partner of
// each element (D / 2 away) sits in lane l ^ 32: one shuffle. Arithmetic is
// FP32 with the reference's roundings: n = bf16(x inv_std), w = bf16(n gain),
// out = bf16(bf16(w cos) + bf16(rot sin)). Query heads go to the token-major
// query [rows, Hq, D]; key heads and the copied value heads to the caches
// [B, Hkv, C, D] at the step's slot. Slots outside the cache and table phases
// outside the cos/sin tables (device-side values the host cannot check) are
// skipped: nothing is read or written out of bounds.
#include "../../include/ftk.h"
#include "ftk_internal.h"

namespace ftk {

template <int E>
__device__ __forceinline__ void load_merged(const RopeArgs& a, int64_t at, float (&v)[E]) {
  if (a.splits == 1) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(a.packed) + at;
    if constexpr (E == 2) {
      const uint32_t pair = *reinterpret_cast<const uint32_t*>(p);
      v[0] = lo_f32(pair);
      v[1] = hi_f32(pair);
    } else {
      v[0] = bf16_to_f32(*p);
    }
    return;
  }
  const float* p = reinterpret_cast<const float*>(a.packed) + at;
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = p[e];
  for (int s = 1; s < a.splits; ++s)
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] += p[(size_t)s * a.split_stride + e];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = round_bf16(v[e]);
}

template <int E>
__device__ __forceinline__ void store_bf16(uint16_t* p, const float (&v)[E]) {
  if constexpr (E == 2) {
    *reinterpret_cast<uint32_t*>(p) = pack_bf16(v[0], v[1]);
  } else {
    *p = (uint16_t)f32_to_bf16(v[0]);
  }
}

template <int E>
__device__ __forceinline__ void load_table(const uint16_t* p, float (&v)[E]) {
  if constexpr (E == 2) {
    const uint32_t pair = *reinterpret_cast<const uint32_t*>(p);
    v[0] = lo_f32(pair);
    v[1] = hi_f32(pair);
  } else {
    v[0] = bf16_to_f32(*p);
  }
}

template <int D, int W>
__global__ __launch_bounds__(64 * W) void qk_rope_kernel(RopeArgs a) {
  constexpr int E = D / 64;
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.y * W + (threadIdx.x >> 6);
  const int heads = a.q_heads + a.kv_heads;
  if (head >= heads) return;  // no barrier in this kernel
  const int r = blockIdx.x;  // row = b * tokens + t
  const int b = r / a.tokens, t = r - b * a.tokens;
  const int col = lane * E;
  const int64_t np = (int64_t)(a.q_heads + 2 * a.kv_heads) * D;
  const bool is_q = head < a.q_heads;

  // Every load that does not depend on the device-side position goes out first
  // (one memory round trip); with shared or per-row cos/sin rows the phase is
  // the token or the row, checked against the tables on the host.
  const bool table = (a.mode & FTK_ROPE_TABLE) != 0;
  const int64_t vat = r * np + (int64_t)(a.q_heads + a.kv_heads + (head - a.q_heads)) * D + col;
  float x[E], g[E], c[E], s[E];
  uint32_t vbits = 0;
  load_merged<E>(a, r * np + (int64_t)head * D + col, x);
  load_table<E>((is_q ? a.q_gain : a.k_gain) + col, g);
  if (!is_q && a.splits == 1) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(a.packed) + vat;
    vbits = E == 2 ? *reinterpret_cast<const uint32_t*>(src) : (uint32_t)*src;
  }
  int64_t phase = (a.mode & FTK_ROPE_ROWS) ? r : t;
  if (!table) {
    load_table<E>(a.cos + phase * D + col, c);
    load_table<E>(a.sin + phase * D + col, s);
  }
  int64_t slot = 0;
  if (!is_q) slot = (a.mode & FTK_ROPE_PREFILL) ? t : a.position[(a.mode & FTK_ROPE_ROWS) ? b : 0] + t;
  if (table) {
    phase = a.position[b] + a.phases[r];
    if (phase < 0 || phase >= a.table_rows) return;  // wave-uniform; no barrier in this kernel
    load_table<E>(a.cos + phase * D + col, c);
    load_table<E>(a.sin + phase * D + col, s);
  }

  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss += x[e] * x[e];
  ss = wave_sum(ss);
  const float inv_std = 1.0f / sqrtf(ss / (float)D + (is_q ? a.q_eps : a.k_eps));
  float w[E], out[E];
#pragma unroll
  for (int e = 0; e < E; ++e) w[e] = round_bf16(round_bf16(x[e] * inv_std) * g[e]);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float partner = __shfl_xor(w[e], 32);  // element col + D/2 (mod D)
    const float rot = lane < 32 ? -partner : partner;
    out[e] = round_bf16(w[e] * c[e]) + round_bf16(rot * s[e]);
  }
  if (is_q) {
    store_bf16<E>(a.query + ((int64_t)r * a.q_heads + head) * D + col, out);
    return;
  }
  if (slot < 0 || slot >= a.capacity) return;
  const int kv = head - a.q_heads;
  const int64_t at = (((int64_t)b * a.kv_heads + kv) * a.capacity + slot) * D + col;
  store_bf16<E>(a.keys + at, out);
  if (a.splits == 1) {  // the value head as it is, bit for bit
    if constexpr (E == 2) {
      *reinterpret_cast<uint32_t*>(a.values + at) = vbits;
    } else {
      a.values[at] = (uint16_t)vbits;
    }
  } else {
    float v[E];
    load_merged<E>(a, vat, v);
    store_bf16<E>(a.values + at, v);
  }
}

hipError_t launch_qk_rope(const RopeArgs& a, int rows, hipStream_t stream) {
  constexpr int W = 4;
  const dim3 grid((unsigned)rows, (unsigned)((a.q_heads + a.kv_heads + W - 1) / W));
  if (a.dim == 128)
    hipLaunchKernelGGL((qk_rope_kernel<128, W>), grid, dim3(64 * W), 0, stream, a);
  else
    hipLaunchKernelGGL((qk_rope_kernel<64, W>), grid, dim3(64 * W), 0, stream, a);
  return hipGetLastError();
}

}  // namespace ftk
