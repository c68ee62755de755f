// Split-KV GQA decode attention on gfx950: engine/kernels/decode_attention.py:31-149
// (_decode_partials, _decode_merge, _attend) and :229-258 (decode_attention).
//
// One workgroup per (row, KV head, split). The G query heads of a KV head
// share every cache row the workgroup reads. A wave load covers 64 / (D / 8)
// whole cache rows (4 rows x 256 bytes at D = 128): lane (r, c) holds the
// 16-byte chunk c of row r, for K and for V. Per lane:
//   - the G query slices of chunk c stay in registers;
//   - each row's G scores are v_dot2 partial dots summed over the row's lanes
//     by a DPP butterfly, so every lane of the row holds the same bits;
//   - an online softmax runs over the rows the lane sees (max, denominator,
//     and the numerator's 8 dimensions of chunk c per query head), with
//     p rounded to BF16 before it multiplies V, as the reference's
//     tl.dot(p.to(bf16), v) does; the denominator sums the FP32 p.
// The rows of a wave, then the waves (through LDS), merge their softmax
// states. One split writes the output; several write FP32 partials and
// (max, denominator) pairs for the merge kernel. Slots at or past
// min(position + 1, capacity) are never used: their scores are -inf and
// their values are replaced by zero before any arithmetic (they may hold NaN).
#include "../../include/ftk.h"
#include "ftk_internal.h"

namespace ftk {

// Sum over aligned groups of CH lanes (CH = 8 or 16). Every step adds a lane
// pair in both orders, so all lanes of a group end with the same bits.
template <int CH>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  v += dpp<0x141, 0xF>(v);  // row_half_mirror: lane ^ 7 within 8
  if constexpr (CH == 16) v += dpp<0x140, 0xF>(v);  // row_mirror: lane ^ 15 within 16
  return v;
}

__device__ __forceinline__ float exp2_f32(float x) { return __builtin_amdgcn_exp2f(x); }

// Softmax state (max m, denominator l, numerator a) of one query head over 8 dimensions.
template <int E>
__device__ __forceinline__ void merge_state(float& m, float& l, float (&a)[E], float m2, float l2,
                                            const float (&a2)[E]) {
  const float top = fmaxf(m, m2);
  const float pivot = top == -INFINITY ? 0.f : top;  // nothing seen on either side: keep zeros
  const float c1 = exp2_f32(m - pivot), c2 = exp2_f32(m2 - pivot);
  l = l * c1 + l2 * c2;
#pragma unroll
  for (int e = 0; e < E; ++e) a[e] = a[e] * c1 + a2[e] * c2;
  m = top;
}

// A workgroup's merged state of query head h, dimensions 8 cc .. 8 cc + 7: the
// output itself (one interval) or the interval's FP32 partial and (max, denominator).
__device__ __forceinline__ void store_state(const AttnArgs& a, int group, int split, int h, int cc, int G, int D,
                                            float m, float l, const float (&acc)[8]) {
  if (a.splits == 1) {
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack_bf16(acc[2 * i] / l, acc[2 * i + 1] / l);
    store16(a.out + ((size_t)group * G + h) * D + cc * 8, u32x4_t{o[0], o[1], o[2], o[3]});
  } else {
    const size_t slot = ((size_t)group * a.splits + split) * G + h;
    float* dst = a.partial + slot * D + cc * 8;
    *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4_t*>(dst + 4) = f32x4_t{acc[4], acc[5], acc[6], acc[7]};
    if (cc == 0) *reinterpret_cast<f32x2_t*>(a.stats + slot * 2) = f32x2_t{m, l};
  }
}

template <int D, int G, int W, int U>
__global__ __launch_bounds__(64 * W) void attn_partials_kernel(AttnArgs a) {
  constexpr int CH = D / 8;     // 16-byte chunks per cache row
  constexpr int RPL = 64 / CH;  // cache rows per wave load
  constexpr int SLOTS = RPL * U;
  __shared__ float acc_lds[W][G][D];
  __shared__ float m_lds[W][G], l_lds[W][G];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane / CH, c = lane - (lane / CH) * CH;
  const int group = blockIdx.x / a.splits, split = blockIdx.x - group * a.splits;
  const int row = group / a.kv_heads;
  const int64_t newest = a.position[a.pos_stride * row];
  const int64_t visible = newest + 1 < (int64_t)a.capacity ? newest + 1 : (int64_t)a.capacity;
  const int begin = split * a.chunk;
  const int end = (int)(begin + a.chunk < visible ? begin + a.chunk : visible);
  const int units = end > begin ? (end - begin + SLOTS - 1) / SLOTS : 0;

  const size_t cache = (size_t)group * a.capacity * D + c * 8;
  const uint16_t* kb = a.k + cache;
  const uint16_t* vb = a.v + cache;
  u32x4_t qv[G];
#pragma unroll
  for (int h = 0; h < G; ++h) qv[h] = load16(a.q + ((size_t)group * G + h) * D + c * 8);

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }

  // Unit i covers slots begin + i SLOTS + [0, SLOTS); wave w takes units w, w + W, ...
  // Rows past `end` load row end - 1 (inside the cache) and are masked below.
  auto load_unit = [&](int unit, u32x4_t (&kr)[U], u32x4_t (&vr)[U]) {
    const int first = begin + unit * SLOTS + r;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = first + u * RPL < end ? first + u * RPL : end - 1;
      kr[u] = load_stream16(kb + (size_t)t * D);
      vr[u] = load_stream16(vb + (size_t)t * D);
    }
  };

  u32x4_t kr[U], vr[U];
  int unit = wave;
  if (unit < units) load_unit(unit, kr, vr);
  for (; unit < units; unit += W) {
    u32x4_t kn[U], vn[U];
    if (unit + W < units) load_unit(unit + W, kn, vn);

    const int first = begin + unit * SLOTS + r;
    float s[G][U];
    float vf[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = first + u * RPL < end;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float dot = group_sum<CH>(dot8(kr[u], qv[h], 0.f));
        s[h][u] = live ? dot * a.scale_log2 : -INFINITY;
      }
      const u32x4_t zero = {0u, 0u, 0u, 0u};
      widen8(live ? vr[u] : zero, vf[u]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float top = m[h];
#pragma unroll
      for (int u = 0; u < U; ++u) top = fmaxf(top, s[h][u]);
      const float pivot = top == -INFINITY ? 0.f : top;
      const float corr = exp2_f32(m[h] - pivot);
      float psum = 0.f;
      float pb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = exp2_f32(s[h][u] - pivot);
        psum += p;
        pb[u] = round_bf16(p);
      }
      l[h] = l[h] * corr + psum;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = acc[h][e] * corr;
#pragma unroll
        for (int u = 0; u < U; ++u) v += pb[u] * vf[u][e];
        acc[h][e] = v;
      }
      m[h] = top;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      kr[u] = kn[u];
      vr[u] = vn[u];
    }
  }

  // The RPL rows of the wave (lanes c, c + CH, ...), then the waves in order.
#pragma unroll
  for (int off = CH; off < 64; off <<= 1) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float a2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a2[e] = __shfl_xor(acc[h][e], off);
      merge_state(m[h], l[h], acc[h], __shfl_xor(m[h], off), __shfl_xor(l[h], off), a2);
    }
  }
  if (r == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc_lds[wave][h][c * 8 + e] = acc[h][e];
      if (c == 0) {
        m_lds[wave][h] = m[h];
        l_lds[wave][h] = l[h];
      }
    }
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < G * CH) {
    const int h = t / CH, cc = t - (t / CH) * CH;
    float mm = m_lds[0][h], ll = l_lds[0][h], aa[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) aa[e] = acc_lds[0][h][cc * 8 + e];
#pragma unroll
    for (int w = 1; w < W; ++w) {
      float a2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a2[e] = acc_lds[w][h][cc * 8 + e];
      merge_state(mm, ll, aa, m_lds[w][h], l_lds[w][h], a2);
    }
    store_state(a, group, split, h, cc, G, D, mm, ll, aa);
  }
}

// ---- QUAD kind: D = 128, up to 4 query heads per KV head --------------------
//
// Q K^T on the 16-block 4x4x4 BF16 MFMA. Lane 4 b + i loads chunk b of cache
// row i of a 4-row group (one wave load = 4 rows x 256 contiguous bytes): that
// is A_b[i][0..7] of two MFMAs; the B operand is chunk b of query head j
// (lane 4 b + j). A unit is 4 such loads, 16 cache rows. The 16 blocks'
// partial scores are summed by a transposing reduction that leaves lane l with
// the score of unit row 4 ((l >> 2) & 3) + ((l >> 4) & 3) for head l & 3, so
// the softmax runs once per (row, head): max and sum over the 16 lanes of a
// head. The BF16 weights pass through LDS to the lanes holding V in the same
// 4-row layout, which accumulate p V on the VALU for their chunk's 8
// dimensions; the softmax state is the same in every lane of a head, so the
// rows of a wave combine by plain sums at the end.

// Score of this lane's (row, head) from the four loads' 16-block accumulators.
__device__ __forceinline__ float quad_transpose_sum(const f32x4_t (&sc)[4], int lane) {
  const bool h5 = (lane & 32) != 0, h4 = (lane & 16) != 0, h3 = (lane & 8) != 0, h2 = (lane & 4) != 0;
  float w[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    // bit 5: keep elements {2 h5, 2 h5 + 1}; bit 4: keep element 2 h5 + h4
    const float a0 = h5 ? sc[u][2] : sc[u][0], a1 = h5 ? sc[u][3] : sc[u][1];
    const float s0 = h5 ? sc[u][0] : sc[u][2], s1 = h5 ? sc[u][1] : sc[u][3];
    const float u0 = a0 + __shfl_xor(s0, 32), u1 = a1 + __shfl_xor(s1, 32);
    w[u] = (h4 ? u1 : u0) + __shfl_xor(h4 ? u0 : u1, 16);
  }
  // bit 3 (lane ^ 8 is row_ror:8 inside a row of 16): keep loads {2 h3, 2 h3 + 1}
  const float x0 = (h3 ? w[2] : w[0]) + dpp<0x128, 0xF>(h3 ? w[0] : w[2]);
  const float x1 = (h3 ? w[3] : w[1]) + dpp<0x128, 0xF>(h3 ? w[1] : w[3]);
  // bit 2: keep load 2 h3 + h2
  return (h2 ? x1 : x0) + __shfl_xor(h2 ? x0 : x1, 4);
}

// Max over the 16 lanes of a head (lane bits 2..5), in every one of them.
__device__ __forceinline__ float head_max(float v) {
  v = fmaxf(v, dpp<0x128, 0xF>(v));  // row_ror:8
  v = fmaxf(v, dpp<0x124, 0xF>(v));  // row_ror:4
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}

// Lane l ^ 32's value: v_permlane32_swap trades lanes 32..63 of its first
// operand with lanes 0..31 of its second; with both = v, the second comes
// back holding v[l + 32] in lanes 0..31 and the first v[l - 32] in lanes 32..63.
__device__ __forceinline__ float lane_xor32(float v, int lane) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, lane < 32 ? p[1] : p[0]);
}

// Lane l ^ 16's value: v_permlane16_swap trades the odd 16-lane rows of its
// first operand with the even rows of its second.
__device__ __forceinline__ float lane_xor16(float v, int lane) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (lane & 16) ? p[0] : p[1]);
}

// Sum over the 16 lanes that share lane bits 0..1, the same bits in all of
// them, on the VALU. row_ror:8 is lane ^ 8 inside a row of 16; its sum is the
// same under ^ 8, so row_ror:4 (which reaches l ^ 4 or l ^ 12) adds lane ^ 4's
// value. Every step adds a lane pair in both orders.
__device__ __forceinline__ float quad_group_sum(float v, int lane) {
  v += dpp<0x128, 0xF>(v);  // row_ror:8
  v += dpp<0x124, 0xF>(v);  // row_ror:4
  v += lane_xor16(v, lane);
  return v + lane_xor32(v, lane);
}

// Head RMSNorm, gain and RoPE of one D = 128 head in the QUAD layout: lane
// 4 c + i holds elements 8 c .. 8 c + 7 (c = 0..15), the 16 lanes of one i the
// whole head; element j + 64 of element j's rotation is in chunk c ^ 8, lane ^ 32.
// n = bf16(x / sqrt(mean(x^2) + eps)), w = bf16(n g),
// out = bf16(bf16(w cos) + bf16(rotate_half(w) sin)) (engine/kernels/qk_rope.py:48-76).
__device__ __forceinline__ u32x4_t quad_head_rope(u32x4_t x, u32x4_t g, u32x4_t c, u32x4_t s, float eps,
                                                  int lane) {
  float xf[8], gf[8], cf[8], sf[8];
  widen8(x, xf);
  widen8(g, gf);
  widen8(c, cf);
  widen8(s, sf);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += xf[e] * xf[e];
  ss = quad_group_sum(ss, lane);
  const float inv_std = 1.0f / sqrtf(ss / 128.f + eps);
  float w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e] = round_bf16(round_bf16(xf[e] * inv_std) * gf[e]);
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float r[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = 2 * i + j;
      const float partner = lane_xor32(w[e], lane);
      const float rot = lane < 32 ? -partner : partner;  // chunk < 8: the first half of the head
      r[j] = round_bf16(w[e] * cf[e]) + round_bf16(rot * sf[e]);
    }
    o[i] = pack_bf16(r[0], r[1]);
  }
  return u32x4_t{o[0], o[1], o[2], o[3]};
}

// ROPE: the query heads are normalised and rotated here from the packed QKV
// row, and the split whose interval holds the row's own slot (the position,
// when it lies inside the cache) takes that slot's key and value from the
// packed row too: it writes them to the cache, reads only the slots before
// it from memory, and starts wave 0's softmax state with the new slot
// (score s, p = 1). No other workgroup of the launch reads that slot.
// FENCE (with ROPE): the head arithmetic is kept behind the first cache loads,
// so it waits for the head loads only. That shortens a short split (the prologue
// is most of it); in a long one the new slot's stores, then in flight ahead of
// the loop, make the loop's waits drain more, so long splits go without.
template <int G, int W, int NG, bool ROPE, bool FENCE = false>
__global__ __launch_bounds__(64 * W) void attn_quad_kernel(AttnArgs a) {
  constexpr int D = 128, SLOTS = 16 * NG;  // a unit: NG groups of 16 cache rows
  __shared__ float p_lds[W][64];
  __shared__ float acc_lds[W][G][D];
  __shared__ float m_lds[W][G], l_lds[W][G];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: loop tests stay scalar
  const int i4 = lane & 3, chunk = lane >> 2;
  const int group = blockIdx.x / a.splits, split = blockIdx.x - group * a.splits;
  const int row = group / a.kv_heads;
  const int64_t newest = a.position[a.pos_stride * row];
  int64_t shift = 0;  // RoPE phase - position
  if constexpr (ROPE) {
    // One load either way (the position again without phases), in flight beside the position's.
    const int64_t loaded = *(a.phases != nullptr ? a.phases + row : a.position + a.pos_stride * row);
    shift = a.phases != nullptr ? loaded : 0;
  }
  const int64_t visible = newest + 1 < (int64_t)a.capacity ? newest + 1 : (int64_t)a.capacity;
  const int begin = split * a.chunk;
  int end = (int)(begin + a.chunk < visible ? begin + a.chunk : visible);
  bool own = ROPE && newest >= begin && newest < (int64_t)begin + a.chunk && newest < (int64_t)a.capacity;
  if (own) end = (int)newest;
  const int units = end > begin ? (end - begin + SLOTS - 1) / SLOTS : 0;
  const u32x4_t zero = {0u, 0u, 0u, 0u};

  // ROPE: every load of the new token's heads goes out before the cache loads.
  u32x4_t xq = zero, xk = zero, vnew = zero, gq = zero, gk = zero, cs = zero, sn = zero;
  if constexpr (ROPE) {
    const int kvh = group - row * a.kv_heads;
    const uint16_t* src = a.packed + (size_t)row * (a.q_heads + 2 * a.kv_heads) * D + chunk * 8;
    if (i4 < G) xq = load16(src + (size_t)(kvh * G + i4) * D);
    xk = load16(src + (size_t)(a.q_heads + kvh) * D);
    vnew = load16(src + (size_t)(a.q_heads + a.kv_heads + kvh) * D);
    gq = load16(a.q_gain + chunk * 8);
    gk = load16(a.k_gain + chunk * 8);
    // A phase outside the tables reads row 0 instead and writes no slot (the row's output is unspecified).
    const int64_t phase = newest + shift;
    const int64_t at = phase >= 0 && phase < a.table_rows ? phase : 0;
    if (at != phase) own = false;
    cs = load16(a.cos + at * D + chunk * 8);
    sn = load16(a.sin + at * D + chunk * 8);
  }

  // K and V through buffer descriptors whose range ends at row `end`: a load
  // of a later row returns zeros without touching memory. So the ragged last
  // unit needs no value masking (and never reads the NaN a stale slot may
  // hold), and the next-unit loads of the last step cost nothing.
  const size_t cache = (size_t)group * a.capacity * D;
  const uint32_t limit = end > 0 ? (uint32_t)end * (D * 2) : 0u;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)(a.k + cache), 0, limit, kBufferFlags);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)(a.v + cache), 0, limit, kBufferFlags);
  u32x4_t qv = zero;
  if constexpr (!ROPE) {
    if (i4 < G) qv = load16(a.q + ((size_t)group * G + i4) * D + chunk * 8);
  }
  const int srow = 4 * ((lane >> 2) & 3) + ((lane >> 4) & 3);  // row of this lane's score in a group

  float m = -INFINITY, l = 0.f;  // head (lane & 3)'s softmax state, the same in its 16 lanes
  float acc[G][8];               // numerators of this chunk's 8 dimensions, over rows i4 of each load
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;

  // Byte offset of this lane's chunk in load u of group g of a unit. Each load
  // goes into the register its predecessor just freed.
  auto at = [&](int unit, int g, int u) {
    return (uint32_t)(begin + unit * SLOTS + 16 * g + 4 * u + i4) * (D * 2) + chunk * 16;
  };

  u32x4_t kr[NG][4], vr[NG][4];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      kr[g][u] = buffer_load16(krs, at(wave, g, u));
      vr[g][u] = buffer_load16(vrs, at(wave, g, u));
    }
  if constexpr (ROPE) {
    if constexpr (FENCE) __builtin_amdgcn_sched_barrier(0);
    qv = quad_head_rope(xq, gq, cs, sn, a.q_eps, lane);
    if (i4 >= G) qv = zero;
    if (own) {
      const u32x4_t knew = quad_head_rope(xk, gk, cs, sn, a.k_eps, lane);
      if (wave == 0) {
        if (i4 == 0) {
          store16(a.k_store + cache + (size_t)newest * D + chunk * 8, knew);
          store16(a.v_store + cache + (size_t)newest * D + chunk * 8, vnew);
        }
        // The new slot's score for head i4, in the head's 16 lanes; p = exp2(s - s) = 1.
        m = quad_group_sum(dot8(knew, qv, 0.f), lane) * a.scale_log2;
        l = 1.f;
        if (i4 == 0) {
          float vf[8];
          widen8(vnew, vf);
#pragma unroll
          for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] = vf[e];
        }
      }
    }
  }
  for (int unit = wave; unit < units; unit += W) {
    const int next = unit + W;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int base = begin + unit * SLOTS + 16 * g;
      f32x4_t sc[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
        sc[u] = mfma4x4x4(kr[g][u][0], kr[g][u][1], qv[0], qv[1], z);
        sc[u] = mfma4x4x4(kr[g][u][2], kr[g][u][3], qv[2], qv[3], sc[u]);
        kr[g][u] = buffer_load16(krs, at(next, g, u));
      }
      const float dot = quad_transpose_sum(sc, lane);
      const float s = base + srow < end ? dot * a.scale_log2 : -INFINITY;
      const float top = fmaxf(m, head_max(s));
      const float pivot = top == -INFINITY ? 0.f : top;
      const float corr = exp2_f32(m - pivot);
      const float p = exp2_f32(s - pivot);
      l = l * corr + quad_lane_sum(p);
      m = top;

      // The BF16 weights to the V lanes: lane 4 b + i needs rows 4 u + i, every head.
      p_lds[wave][lane] = round_bf16(p);
      __builtin_amdgcn_wave_barrier();
      float pb[4][G];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(&p_lds[wave][16 * i4 + 4 * u]);
#pragma unroll
        for (int h = 0; h < G; ++h) pb[u][h] = v4[h];
      }
      __builtin_amdgcn_wave_barrier();

      float cs[G];
      bool rescale = false;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        cs[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), h));
        rescale |= cs[h] != 1.f;
      }
      if (rescale) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] *= cs[h];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float vf[8];
        widen8(vr[g][u], vf);
        vr[g][u] = buffer_load16(vrs, at(next, g, u));
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] += pb[u][h] * vf[e];
      }
    }
  }

  // The four rows of a chunk (lanes 4 b .. 4 b + 3) share the softmax state: plain sums.
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[h][e];
      v += dpp<0xB1, 0xF>(v);  // quad_perm [1,0,3,2]
      v += dpp<0x4E, 0xF>(v);  // quad_perm [2,3,0,1]
      acc[h][e] = v;
    }
  if (i4 == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc_lds[wave][h][chunk * 8 + e] = acc[h][e];
  }
  if (lane < G) {
    m_lds[wave][lane] = m;
    l_lds[wave][lane] = l;
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < G * 16) {
    const int h = t >> 4, cc = t & 15;
    float mm = m_lds[0][h], ll = l_lds[0][h], aa[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) aa[e] = acc_lds[0][h][cc * 8 + e];
#pragma unroll
    for (int w = 1; w < W; ++w) {
      float a2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a2[e] = acc_lds[w][h][cc * 8 + e];
      merge_state(mm, ll, aa, m_lds[w][h], l_lds[w][h], a2);
    }
    store_state(a, group, split, h, cc, G, D, mm, ll, aa);
  }
}

// out[q] = bf16( sum_s acc_s exp2(m_s - M) / sum_s l_s exp2(m_s - M) ), M = max_s m_s,
// for one query head q = group * G + h per workgroup (engine/kernels/decode_attention.py:102-128).
// One memory round trip for up to kMergeWaves * kMergePre splits: each thread
// loads one split's (max, denominator) and each wave the numerators of its
// first kMergePre splits (s = wave + kMergeWaves i) before anything waits.
// The weights are then formed in parallel into LDS, and the wave totals are
// added in wave order.
constexpr int kMergeWaves = 4;
constexpr int kMergePre = 8;

template <int D>
__global__ __launch_bounds__(64 * kMergeWaves) void attn_merge_kernel(const float* partial, const float* stats,
                                                                      uint16_t* out, int splits, int groups_per_kv) {
  constexpr int E = D / 64;  // dimensions per lane
  constexpr int T = 64 * kMergeWaves;
  __shared__ float weight[kAttnMaxSplits];
  __shared__ float red[kMergeWaves];
  __shared__ float num_lds[kMergeWaves][D];
  const int q = blockIdx.x;
  const int group = q / groups_per_kv, h = q - group * groups_per_kv;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  auto slot = [&](int s) { return ((size_t)group * splits + s) * groups_per_kv + h; };

  f32x2_t st = {-INFINITY, 0.f};
  if (t < splits) st = *reinterpret_cast<const f32x2_t*>(stats + slot(t) * 2);
  float pre[kMergePre][E];
#pragma unroll
  for (int i = 0; i < kMergePre; ++i) {
    const int s = wave + kMergeWaves * i;
#pragma unroll
    for (int e = 0; e < E; ++e) pre[i][e] = s < splits ? partial[slot(s) * D + lane * E + e] : 0.f;
  }

  float top = st[0];
  for (int s = t + T; s < splits; s += T) top = fmaxf(top, stats[slot(s) * 2]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) top = fmaxf(top, __shfl_xor(top, off));
  if (lane == 0) red[wave] = top;
  __syncthreads();
  top = red[0];
#pragma unroll
  for (int w = 1; w < kMergeWaves; ++w) top = fmaxf(top, red[w]);
  __syncthreads();

  float den = 0.f;
  if (t < splits) {
    const float c = st[0] == -INFINITY ? 0.f : exp2_f32(st[0] - top);
    weight[t] = c;
    den = st[1] * c;
  }
  for (int s = t + T; s < splits; s += T) {
    const float ms = stats[slot(s) * 2];
    const float c = ms == -INFINITY ? 0.f : exp2_f32(ms - top);
    weight[s] = c;
    den += stats[slot(s) * 2 + 1] * c;
  }
  den = wave_sum(den);
  if (lane == 0) red[wave] = den;
  __syncthreads();
  den = ((red[0] + red[1]) + red[2]) + red[3];

  float num[E];
#pragma unroll
  for (int e = 0; e < E; ++e) num[e] = 0.f;
#pragma unroll
  for (int i = 0; i < kMergePre; ++i) {
    const int s = wave + kMergeWaves * i;
    const float c = s < splits ? weight[s] : 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) num[e] += pre[i][e] * c;
  }
#pragma unroll 4
  for (int s = wave + kMergeWaves * kMergePre; s < splits; s += kMergeWaves) {
    const float c = weight[s];
#pragma unroll
    for (int e = 0; e < E; ++e) num[e] += partial[slot(s) * D + lane * E + e] * c;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) num_lds[wave][lane * E + e] = num[e];
  __syncthreads();
  if (wave == 0) {
    float o[E];
#pragma unroll
    for (int e = 0; e < E; ++e)
      o[e] = (((num_lds[0][lane * E + e] + num_lds[1][lane * E + e]) + num_lds[2][lane * E + e]) +
              num_lds[3][lane * E + e]) / den;
    if constexpr (E == 2) {
      *reinterpret_cast<uint32_t*>(out + (size_t)q * D + lane * 2) = pack_bf16(o[0], o[1]);
    } else {
      out[(size_t)q * D + lane] = (uint16_t)f32_to_bf16(o[0]);
    }
  }
}

// Registers of one lane, estimated from the compiler's counts (gfx950): two unit
// buffers of K and V plus the widened V rows (~18 per unit), query slice and
// softmax state (~17 per head), scores (one per head and unit), addressing.
constexpr bool attn_fits(int g, int u) { return 24 + 18 * u + 17 * g + g * u <= 230; }

template <int D, int G, int W, int U>
static hipError_t launch_partials(const AttnArgs& a, int grid, hipStream_t stream) {
  if constexpr (attn_fits(G, U)) {
    hipLaunchKernelGGL((attn_partials_kernel<D, G, W, U>), dim3((unsigned)grid), dim3(64 * W), 0, stream, a);
    return hipGetLastError();
  } else {
    return hipErrorInvalidValue;
  }
}

template <int D, int G>
static hipError_t launch_for_group(const AttnArgs& a, const AttnShape& s, hipStream_t stream) {
  const int grid = s.groups * s.splits;
  if (s.waves == 4 && s.unroll == 2) return launch_partials<D, G, 4, 2>(a, grid, stream);
  if (s.waves == 4 && s.unroll == 4) return launch_partials<D, G, 4, 4>(a, grid, stream);
  if (s.waves == 4 && s.unroll == 8) return launch_partials<D, G, 4, 8>(a, grid, stream);
  if (s.waves == 8 && s.unroll == 2) return launch_partials<D, G, 8, 2>(a, grid, stream);
  if (s.waves == 8 && s.unroll == 4) return launch_partials<D, G, 8, 4>(a, grid, stream);
  if (s.waves == 8 && s.unroll == 8) return launch_partials<D, G, 8, 8>(a, grid, stream);
  return hipErrorInvalidValue;
}

template <int D>
static hipError_t launch_for_dim(const AttnArgs& a, const AttnShape& s, hipStream_t stream) {
  switch (s.group_size) {
    case 1: return launch_for_group<D, 1>(a, s, stream);
    case 2: return launch_for_group<D, 2>(a, s, stream);
    case 3: return launch_for_group<D, 3>(a, s, stream);
    case 4: return launch_for_group<D, 4>(a, s, stream);
    case 5: return launch_for_group<D, 5>(a, s, stream);
    case 6: return launch_for_group<D, 6>(a, s, stream);
    case 7: return launch_for_group<D, 7>(a, s, stream);
    case 8: return launch_for_group<D, 8>(a, s, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int G, bool ROPE, bool FENCE>
static hipError_t launch_quad_for_group(const AttnArgs& a, const AttnShape& s, hipStream_t stream) {
  const dim3 grid((unsigned)(s.groups * s.splits));
  if (s.waves == 4 && s.unroll == 1)
    hipLaunchKernelGGL((attn_quad_kernel<G, 4, 1, ROPE, FENCE>), grid, dim3(256), 0, stream, a);
  else if (s.waves == 4 && s.unroll == 2)
    hipLaunchKernelGGL((attn_quad_kernel<G, 4, 2, ROPE, FENCE>), grid, dim3(256), 0, stream, a);
  else if (s.waves == 8 && s.unroll == 1)
    hipLaunchKernelGGL((attn_quad_kernel<G, 8, 1, ROPE, FENCE>), grid, dim3(512), 0, stream, a);
  else if (s.waves == 8 && s.unroll == 2)
    hipLaunchKernelGGL((attn_quad_kernel<G, 8, 2, ROPE, FENCE>), grid, dim3(512), 0, stream, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <bool ROPE, bool FENCE>
static hipError_t launch_quad(const AttnArgs& a, const AttnShape& s, hipStream_t stream) {
  switch (s.group_size) {
    case 1: return launch_quad_for_group<1, ROPE, FENCE>(a, s, stream);
    case 2: return launch_quad_for_group<2, ROPE, FENCE>(a, s, stream);
    case 3: return launch_quad_for_group<3, ROPE, FENCE>(a, s, stream);
    case 4: return launch_quad_for_group<4, ROPE, FENCE>(a, s, stream);
    default: return hipErrorInvalidValue;
  }
}

// Splits of up to this many slots take the RoPE prologue with the scheduling fence
// (measured on MI355X: B = 1 x 4K slots in 128-slot splits gains ~1 us with it;
// 1024- and 2048-slot splits lose 1-3.5 us).
constexpr int kAttnFenceMaxChunk = 256;

bool attn_supported(int kind, int dim, int group_size, int waves, int unroll) {
  if (waves != 4 && waves != 8) return false;
  if (group_size < 1 || group_size > kAttnMaxGroup) return false;
  if (kind == FTK_ATTN_QUAD) return dim == 128 && group_size <= 4 && (unroll == 1 || unroll == 2);
  if (kind != FTK_ATTN_ROWS) return false;
  if (dim != 64 && dim != 128) return false;
  if (unroll != 2 && unroll != 4 && unroll != 8) return false;
  return attn_fits(group_size, unroll);
}

hipError_t launch_attention(const AttnArgs& a, const AttnShape& s, hipStream_t stream) {
  // The head norm + RoPE prologue exists for the QUAD kind only (the caller checks).
  if (a.packed != nullptr && s.kind != FTK_ATTN_QUAD) return hipErrorInvalidValue;
  const bool rope = a.packed != nullptr, fence = s.chunk <= kAttnFenceMaxChunk;
  hipError_t e = s.kind == FTK_ATTN_QUAD ? (!rope   ? launch_quad<false, false>(a, s, stream)
                                            : fence ? launch_quad<true, true>(a, s, stream)
                                                    : launch_quad<true, false>(a, s, stream))
                 : s.dim == 128          ? launch_for_dim<128>(a, s, stream)
                                         : launch_for_dim<64>(a, s, stream);
  if (e != hipSuccess || s.splits == 1) return e;
  const unsigned heads = (unsigned)(s.groups * s.group_size);
  if (s.dim == 128)
    hipLaunchKernelGGL(attn_merge_kernel<128>, dim3(heads), dim3(64 * kMergeWaves), 0, stream, a.partial, a.stats, a.out, s.splits,
                       s.group_size);
  else
    hipLaunchKernelGGL(attn_merge_kernel<64>, dim3(heads), dim3(64 * kMergeWaves), 0, stream, a.partial, a.stats, a.out, s.splits,
                       s.group_size);
  return hipGetLastError();
}

}  // namespace ftk
