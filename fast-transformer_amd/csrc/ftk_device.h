// Device helpers shared by every gfx950 kernel of the skinny BF16 projection path.
//
// BF16 travels as raw 16-bit patterns (uint16_t); arithmetic is FP32. The
// rounding rule is round-to-nearest-even with every NaN mapped to 0x7FC0, the
// rule torch and the reference's Triton casts use (engine/kernels/linear.py:1-6).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ftk {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Low / high BF16 of a packed pair, widened exactly to FP32.
__device__ __forceinline__ float lo_f32(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float hi_f32(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }

__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two FP32 values rounded to nearest-even BF16, packed (lo in the low half),
// by the compiler's float -> bfloat conversion (one v_cvt_pk_bf16_f32 on
// gfx950). Finite values and infinities round exactly as f32_to_bf16; a NaN
// stays a NaN with an unspecified payload, so this is only for values that
// feed further arithmetic: stored results go through f32_to_bf16.
__device__ __forceinline__ uint32_t rne_pair(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// FP32 -> nearest BF16 value, kept in FP32 (one rounding; an intermediate).
__device__ __forceinline__ float round_bf16(float f) { return lo_f32(rne_pair(f, 0.f)); }

// A stored BF16 pair: round-to-nearest-even, every NaN as 0x7FC0.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
}

__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2_t, v); }

// acc + sum over 8 BF16 products. The products are exact in FP32; v_dot2 adds
// them with FP32 accumulation, so this is an FP32-accumulated dot in some order.
// (Elements are copied to scalars first: bit-casting a vector element
// expression directly made this clang read element 0 for every element.)
__device__ __forceinline__ float dot8(u32x4_t w, u32x4_t x, float acc) {
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3];
  const uint32_t x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w0), as_bf16x2(x0), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w1), as_bf16x2(x1), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w2), as_bf16x2(x2), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(w3), as_bf16x2(x3), acc, false);
  return acc;
}

// ss + the squares of 8 BF16 values, a pair at a time (v_dot2_f32_bf16: the
// squares are exact in FP32, accumulated in FP32). Every fused RMSNorm prologue
// accumulates through this function, so the kinds that sum a row's chunks in
// the same order scale it identically.
__device__ __forceinline__ float sum_squares8(u32x4_t v, float ss) {
  const uint32_t e[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
  for (int i = 0; i < 4; ++i) ss = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(e[i]), as_bf16x2(e[i]), ss, false);
  return ss;
}

// The 8 BF16 values of a 16-byte chunk, widened exactly to FP32.
__device__ __forceinline__ void widen8(u32x4_t v, float (&out)[8]) {
  const uint32_t e[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = lo_f32(e[i]);
    out[2 * i + 1] = hi_f32(e[i]);
  }
}

// norm8 with the gain already widened (shared by the x rows of one K chunk).
__device__ __forceinline__ u32x4_t norm8w(u32x4_t v, const float (&g)[8], float scale) {
  const uint32_t e[4] = {v[0], v[1], v[2], v[3]};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t n = rne_pair(lo_f32(e[i]) * scale, hi_f32(e[i]) * scale);
    o[i] = rne_pair(lo_f32(n) * g[2 * i], hi_f32(n) * g[2 * i + 1]);
  }
  return u32x4_t{o[0], o[1], o[2], o[3]};
}

// RMSNorm of 8 BF16 values: bf16(bf16(x * scale) * gain), the cast order of
// engine/kernels/rmsnorm.py:35-46. The result feeds the projection only.
__device__ __forceinline__ u32x4_t norm8(u32x4_t v, u32x4_t g, float scale) {
  const uint32_t e[4] = {v[0], v[1], v[2], v[3]};
  const uint32_t ge[4] = {g[0], g[1], g[2], g[3]};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t n = rne_pair(lo_f32(e[i]) * scale, hi_f32(e[i]) * scale);
    o[i] = rne_pair(lo_f32(n) * lo_f32(ge[i]), hi_f32(n) * hi_f32(ge[i]));
  }
  return u32x4_t{o[0], o[1], o[2], o[3]};
}

// The residual add of the prologue: bf16(f32(x) + f32(r)) for 8 BF16 values
// (engine/kernels/rmsnorm.py:86-88, a BF16 tensor addition).
__device__ __forceinline__ u32x4_t add8(u32x4_t x, u32x4_t r) {
  const uint32_t e[4] = {x[0], x[1], x[2], x[3]};
  const uint32_t f[4] = {r[0], r[1], r[2], r[3]};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = pack_bf16(lo_f32(e[i]) + lo_f32(f[i]), hi_f32(e[i]) + hi_f32(f[i]));
  return u32x4_t{o[0], o[1], o[2], o[3]};
}

__device__ __forceinline__ void store16(void* p, u32x4_t v) { *reinterpret_cast<u32x4_t*>(p) = v; }

// rsqrt(mean + eps) from the four wave totals of a workgroup, summed in wave order.
__device__ __forceinline__ float rms_scale(const float (&red)[4], int K, float eps) {
  const float total = ((red[0] + red[1]) + red[2]) + red[3];
  return 1.0f / sqrtf(total / (float)K + eps);
}

// D += A B on one 16x16x32 BF16 MFMA. Lane l holds A[l % 16][8 (l / 16) + e] and
// B[8 (l / 16) + e][l % 16] (e = 0..7) and receives D[4 (l / 16) + r][l % 16] (r = 0..3).
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

typedef short s16x4_t __attribute__((ext_vector_type(4)));

// D += A B on the 16-block 4x4x4 BF16 MFMA. Lane 4 b + i holds A_b[i][0..3]
// (four BF16 in two dwords), lane 4 b + j holds B_b[0..3][j], and lane 4 b + j
// receives D_b[r][j] in element r.
__device__ __forceinline__ f32x4_t mfma4x4x4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4_t c) {
  const u32x2_t a = {a0, a1}, b = {b0, b1};
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b), c,
                                                0, 0, 0);
}

// Every pointer these loads take is global memory (a kernel argument plus an
// offset). Saying so keeps them global_load: through a generic pointer that the
// compiler cannot trace to an argument (one carried across loop iterations) it
// emits flat_load, which also counts in lgkmcnt, so every LDS wait after it
// would wait for the memory load too and empty the load window.
typedef __attribute__((address_space(1))) const u32x4_t global_u32x4_t;

// Streaming 16-byte load: weights are read exactly once per call.
__device__ __forceinline__ u32x4_t load_stream16(const void* p) {
  return __builtin_nontemporal_load((global_u32x4_t*)p);
}

// Raw buffer loads: dword 3 of a gfx9 buffer descriptor for untyped 32-bit data.
constexpr int kBufferFlags = 0x00020000;

// 16 bytes at byte `offset` of a buffer, streamed (non-temporal). Past the
// descriptor's range the load returns zeros and does not touch memory.
__device__ __forceinline__ u32x4_t buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 2));
}

__device__ __forceinline__ u32x4_t load16(const void* p) {
  return *(global_u32x4_t*)p;
}

// DPP lane exchange: lanes whose row is masked off read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes of a wave; the total lands in lane 63.
__device__ __forceinline__ float wave_sum_to_last(float v) {
  v += dpp<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141, 0xF>(v);  // row_half_mirror
  v += dpp<0x140, 0xF>(v);  // row_mirror
  v += dpp<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Wave total, made uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v = wave_sum_to_last(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum over lane bits 2..5 of one value per lane (a column of the 16-block MFMA
// layout), the same bits in every lane of the column.
__device__ __forceinline__ float quad_lane_sum(float v) {
  v += dpp<0x128, 0xF>(v);
  v += dpp<0x124, 0xF>(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Greedy-argmax key: larger key = larger BF16 value, then lower index.
// NaN counts as the maximum (torch.argmax), and -0 equals +0.
__device__ __forceinline__ uint32_t orderable(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) u = 0x7FC00000u;
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_orderable(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(u);
}

__device__ __forceinline__ unsigned long long argmax_key(float value, uint32_t index) {
  return (static_cast<unsigned long long>(orderable(value)) << 32) | (0xFFFFFFFFu - index);
}

__device__ __forceinline__ uint32_t key_index(unsigned long long key) {
  return 0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFull);
}

__device__ __forceinline__ unsigned long long key_max(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

// Largest 32-bit word of the wave, in every lane: the wave_sum lane pattern with
// max (a masked-off row reads 0, the identity).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1, 0xF>(v));
  v = max(v, dpp_u32<0x4E, 0xF>(v));
  v = max(v, dpp_u32<0x141, 0xF>(v));
  v = max(v, dpp_u32<0x140, 0xF>(v));
  v = max(v, dpp_u32<0x142, 0xA>(v));
  v = max(v, dpp_u32<0x143, 0xC>(v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Largest key of the wave, in every lane: the largest high word, then the largest
// low word among the lanes that hold it (two DPP reductions instead of six
// 64-bit lane shuffles through LDS).
__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long k) {
  const uint32_t hi = wave_max_u32((uint32_t)(k >> 32));
  const uint32_t lo = wave_max_u32((uint32_t)(k >> 32) == hi ? (uint32_t)k : 0u);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

__device__ __forceinline__ float silu_f32(float g) {
  return g / (1.0f + expf(-g));
}

// SwiGLU on FP32 sums: gate and up are rounded to BF16 first, SiLU's output is
// rounded to BF16, and the product is rounded once more (engine/kernels/swiglu.py:20-24).
__device__ __forceinline__ uint32_t swiglu_bf16(float gate_sum, float up_sum) {
  const float g = round_bf16(gate_sum);
  const float u = round_bf16(up_sum);
  const float a = round_bf16(silu_f32(g));
  return f32_to_bf16(a * u);
}

}  // namespace ftk
