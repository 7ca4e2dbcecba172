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

// A product or a sum rounded on its own: the operators sit under
// contract(off), so the compiler never fuses a product into the add that
// consumes it. (HIP's __fmul_rn / __fadd_rn are plain operators defined
// where contraction is allowed, so they do not prevent that fusion.)
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

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
  static __device__ __forceinline__ float dot0(const uint4& a, const uint4& b) {
    return dot(a, b, 0.f);
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

// Sum of squares of a row of n elements in the one order every RMSNorm that
// writes cached K follows (the fused decode step's q/k norm computes the same
// tree with one packet per lane): 16-byte packets of EPL = 16 / sizeof(T)
// elements, each packet's squares summed in element order from 0, then a
// balanced pairwise tree over the packets zero-padded to a power of two.
// One wave: lane c holds packets [c*M, c*M + M), added by the tree's bottom
// levels; the lane butterfly adds the upper ones. M = max(1, P2 / 64) for P2
// the packet count rounded up to a power of two. Every lane returns the sum.
template <typename T, int M>
__device__ __forceinline__ float sumsq_tree(const T* __restrict__ x, int n) {
  constexpr int EPL = 16 / (int)sizeof(T);
  const int lane = threadIdx.x & 63;
  float ps[M];
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const int base = (lane * M + j) * EPL;
    float a = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int i = base + e;
      const float v = i < n ? Elem<T>::to_f32(x[i]) : 0.f;
      a = add_rn(a, mul_rn(v, v));
    }
    ps[j] = a;
  }
#pragma unroll
  for (int span = 1; span < M; span <<= 1)
#pragma unroll
    for (int j = 0; j < M; j += 2 * span) ps[j] = add_rn(ps[j], ps[j + span]);
  return wave_sum(ps[0]);
}

// Packets per lane (the M of sumsq_tree) for a row of n elements of es
// bytes, or 0 when the row has more than 64 * 64 packets.
__host__ __device__ inline int sumsq_lane_packets(int n, int es) {
  const int epl = 16 / es;
  const int np = (n + epl - 1) / epl;
  int p2 = 1;
  while (p2 < np) p2 <<= 1;
  const int m = p2 > 64 ? p2 / 64 : 1;
  return m > 64 ? 0 : m;
}

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
// Partial records handed between workgroups of one launch are tagged 64-bit
// words: the launch's epoch in the high half, a float's bits in the low half,
// written and read with single 64-bit agent-scope atomics, so a reader sees
// a word whole or not at all. A word counts as written in this launch only
// if it carries this launch's epoch; words of earlier launches -- including
// a publication that landed after its merge had given up waiting -- are
// never taken, so records need no clearing between launches.
__device__ __forceinline__ void st_tagged(uint64_t* p, uint32_t tag, float v) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tagged(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_is(uint64_t w, uint32_t tag) {
  return (uint32_t)(w >> 32) == tag;
}
__device__ __forceinline__ float tag_value(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Launch epochs. Every wave of a launch that hands records between
// workgroups owns one counter word of the workspace: it reads the word at
// its start, tags what it publishes with next_epoch(word) and stores that
// value back before it ends. Each launch thus advances every counter word
// exactly once (waves of a launch with fewer waves than counters also
// advance the surplus words, which no wave of that launch reads), so all
// counters stay equal and a merging wave expects the tag its own counter
// gives. 0 is never an epoch: a zero-filled workspace holds no valid word.
__device__ __forceinline__ uint32_t next_epoch(uint32_t c) { return c + 1u == 0u ? 1u : c + 1u; }

// Workspace header shared by the kernels that hand records between
// workgroups: word 0 holds sticky error flags (RLSE_WS_ERR_*), raised by
// the device and read and cleared by rlse_workspace_check; the rest of the
// 256-byte header is reserved. Counter words follow, then the records.
__device__ __forceinline__ void ws_raise(uint32_t* err, uint32_t flag) {
  __hip_atomic_fetch_or(err, flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Default bound on a merge's wait for a partial of an earlier workgroup
// (wall clock ticks, 100 MHz: 100 ms); past it the merge gives up, writes
// NaN and raises RLSE_WS_ERR_MERGE_TIMEOUT.
constexpr unsigned long long kMergeWaitTicks = 10000000ull;

// Four dwords as a native vector (element-wise copies, no memcpy).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
// Word 3 of a raw buffer descriptor on gfx9-family targets: 32-bit data
// format, no swizzle, no index stride. A raw buffer load whose byte offset
// is at or past the descriptor's record count returns zeros without
// accessing memory.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of a buffer load that streams data read once: the
// non-temporal bit (bit 1), so the lines do not displace reused data in L2.
constexpr int kLoadNonTemporal = 2;

// Marks a loaded packet as used here (an empty asm reading its registers):
// the compiler waits for its load at this point, in straight-line code where
// it can count the loads issued since, instead of later inside a loop.
__device__ __forceinline__ void consume(const uint4& x) {
  asm volatile("" ::"v"(x.x), "v"(x.y), "v"(x.z), "v"(x.w));
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima), fenced
// against compiler reordering on both sides.
__device__ __forceinline__ void wait_vm_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}


}  // namespace rlse
