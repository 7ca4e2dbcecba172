// Device helpers shared by the gfx950 kernels: element conversions with the
// rounding Candle's CPU path uses (half::bf16::from_f32 is round-to-nearest-even
// with NaN kept quiet), 16-byte vector access and wave64 reductions built on
// DPP row operations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlse_kv.h"

namespace rlse {

// bf16 is carried as its raw 16-bit pattern.
struct bf16 {
  uint16_t bits;
};
typedef _Float16 f16;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// The same rounding with the NaN test as a select (v_cndmask) instead of an
// exec-masked branch: cheaper in straight-line element-wise code, at the cost
// of a few live registers.
__device__ __forceinline__ uint16_t f32_to_bf16_bits_sel(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x40u;
  return (uint16_t)(((u & 0x7fffffffu) > 0x7f800000u) ? qnan : rne);
}

template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static __device__ __forceinline__ float from_f32(float v) { return v; }
};

template <>
struct Elem<bf16> {
  static __device__ __forceinline__ float to_f32(bf16 v) { return bf16_bits_to_f32(v.bits); }
  static __device__ __forceinline__ bf16 from_f32(float v) {
    bf16 r;
    r.bits = f32_to_bf16_bits(v);
    return r;
  }
};

template <>
struct Elem<f16> {
  static __device__ __forceinline__ float to_f32(f16 v) { return (float)v; }
  static __device__ __forceinline__ f16 from_f32(float v) { return (f16)v; }
};

// Round a float to the precision of T (identity for float).
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  return Elem<T>::to_f32(Elem<T>::from_f32(v));
}

// ---------------------------------------------------------------------------
// 16-byte packets: unpack to floats and packed dot products.
// ---------------------------------------------------------------------------
template <typename T>
struct Packet;

template <>
struct Packet<float> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void unpack(const uint4& p, float* o) {
    o[0] = __uint_as_float(p.x);
    o[1] = __uint_as_float(p.y);
    o[2] = __uint_as_float(p.z);
    o[3] = __uint_as_float(p.w);
  }
  static __device__ __forceinline__ float dot(const uint4& a, const uint4& b, float c) {
    c = fmaf(__uint_as_float(a.x), __uint_as_float(b.x), c);
    c = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), c);
    c = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), c);
    c = fmaf(__uint_as_float(a.w), __uint_as_float(b.w), c);
    return c;
  }
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <>
struct Packet<bf16> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void unpack(const uint4& p, float* o) {
    const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
  }
  static __device__ __forceinline__ float dot(const uint4& a, const uint4& b, float c) {
    c = dot2(a.x, b.x, c);
    c = dot2(a.y, b.y, c);
    c = dot2(a.z, b.z, c);
    c = dot2(a.w, b.w, c);
    return c;
  }
  // Two floats rounded to nearest-even bf16, lo in the low half.
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
};

template <>
struct Packet<f16> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void unpack(const uint4& p, float* o) {
    const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f16x2_t h = __builtin_bit_cast(f16x2_t, w[i]);
      o[2 * i] = (float)h[0];
      o[2 * i + 1] = (float)h[1];
    }
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a),
                                  __builtin_bit_cast(f16x2_t, b), c, false);
  }
  // Two floats rounded to nearest-even f16, lo in the low half.
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    const f16x2_t v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float dot(const uint4& a, const uint4& b, float c) {
    c = dot2(a.x, b.x, c);
    c = dot2(a.y, b.y, c);
    c = dot2(a.z, b.z, c);
    c = dot2(a.w, b.w, c);
    return c;
  }
};

// ---------------------------------------------------------------------------
// Wave64 reductions. DPP controls (GCN/CDNA encoding): quad_perm [1,0,3,2]
// = 0xB1 (lane ^ 1), quad_perm [2,3,0,1] = 0x4E (lane ^ 2), row_half_mirror
// = 0x141 and row_mirror = 0x140. After the two quad steps every lane of a
// quad holds the same value, so the mirrors act as lane ^ 4 and lane ^ 8.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of LANES consecutive lanes; every lane of a group
// receives the group's sum. LANES is a power of two in [1, 64].
template <int LANES>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (LANES >= 2) x += dpp_f32<0xB1>(x);
  if constexpr (LANES >= 4) x += dpp_f32<0x4E>(x);
  if constexpr (LANES >= 8) x += dpp_f32<0x141>(x);
  if constexpr (LANES >= 16) x += dpp_f32<0x140>(x);
  if constexpr (LANES >= 32) x += __shfl_xor(x, 16, 64);
  if constexpr (LANES >= 64) x += __shfl_xor(x, 32, 64);
  return x;
}

// group_sum of N independent values, one butterfly step at a time across
// all of them: consecutive DPP adds are then independent, so none waits out
// the DPP read-after-write hazard of its predecessor.
template <int LANES, int N>
__device__ __forceinline__ void group_sum_n(float (&x)[N]) {
  if constexpr (LANES >= 2) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp_f32<0xB1>(x[i]);
  }
  if constexpr (LANES >= 4) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp_f32<0x4E>(x[i]);
  }
  if constexpr (LANES >= 8) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp_f32<0x141>(x[i]);
  }
  if constexpr (LANES >= 16) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp_f32<0x140>(x[i]);
  }
  if constexpr (LANES >= 32) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += __shfl_xor(x[i], 16, 64);
  }
  if constexpr (LANES >= 64) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += __shfl_xor(x[i], 32, 64);
  }
}

__device__ __forceinline__ float wave_sum(float x) { return group_sum<64>(x); }

__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_f32<0xB1>(x));
  x = fmaxf(x, dpp_f32<0x4E>(x));
  x = fmaxf(x, dpp_f32<0x141>(x));
  x = fmaxf(x, dpp_f32<0x140>(x));
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  x = fmaxf(x, __shfl_xor(x, 32, 64));
  return x;
}

__device__ __forceinline__ int wave_lane() { return __lane_id(); }

// ---------------------------------------------------------------------------
// Cross-workgroup hand-off of partial results within one launch.
// ---------------------------------------------------------------------------
// Partial records are written and read as single 32-bit words with
// device-scope (agent) atomic stores and loads: on gfx950 these carry the sc1
// bit, so each access is coherent across the XCDs' L2 caches by itself and a
// word is seen whole or not at all -- no whole-L2 writeback or invalidate is
// needed (a __threadfence() would emit both).
__device__ __forceinline__ void st_word(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_word(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Partial records handed between workgroups of one launch. Record words hold
// the complement of a float's bits, so a stored word is never 0 (the bits
// 0xFFFFFFFF, a NaN, are stored as another NaN) and 0 marks a word not yet
// written in this launch. Each word is stored once per launch with a single
// 32-bit agent-scope store, so a reader that sees it non-zero sees the whole
// value; the merging workgroup clears the words it read.
__device__ __forceinline__ uint32_t rec_encode(float v) {
  const uint32_t u = __float_as_uint(v);
  return ~(u == 0xFFFFFFFFu ? 0x7FFFFFFFu : u);
}
__device__ __forceinline__ float rec_decode(uint32_t x) { return __uint_as_float(~x); }
// A merge waits at most this long (wall clock ticks, 100 MHz: 100 ms) for a
// partial of an earlier workgroup before it gives up and writes NaN.
constexpr unsigned long long kMergeWaitTicks = 10000000ull;

// Four dwords as a native vector (element-wise copies, no memcpy).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
// Word 3 of a raw buffer descriptor on gfx9-family targets: 32-bit data
// format, no swizzle, no index stride. A raw buffer load whose byte offset
// is at or past the descriptor's record count returns zeros without
// accessing memory.
constexpr int kBufferWord3 = 0x00020000;

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima), fenced
// against compiler reordering on both sides.
__device__ __forceinline__ void wait_vm_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}


}  // namespace rlse
