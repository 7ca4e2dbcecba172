// The rest of a batched decode step on the device: embedding gather, fused
// residual add + RMSNorm, the MLP activation, greedy argmax and the linear
// projections -- the ops of ModelForCausalLM::step_decode_batch
// (src/backends/qwen2.rs:628-764) around the attention of rlse_decode_step,
// so a step's activations and logits never leave HBM (the reference moves
// the logits to the host for sample_token, src/backends/candle.rs:737-751).
//
// Element-wise rounding follows Candle's per-op order on bf16/f16 tensors:
// every op computes in f32 and rounds its result to the tensor dtype, with
// no multiply-add contraction (a Candle op rounds its product before the
// next op adds to it).
#include <math.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.cuh"
#include "host_common.h"

#pragma clang fp contract(off)

namespace rlse {
namespace {

// One row per workgroup; 16-byte chunks (the row is a whole number of them).
template <typename T>
__global__ void embedding_kernel(const int32_t* __restrict__ ids, const T* __restrict__ table,
                                 T* __restrict__ out, int hidden, int vocab) {
  const int b = blockIdx.x;
  const int id = ids[b];
  const int chunks = hidden * (int)sizeof(T) / 16;
  uint4* dst = reinterpret_cast<uint4*>(out + (size_t)b * hidden);
  const bool ok = id >= 0 && id < vocab;
  const uint4* src = reinterpret_cast<const uint4*>(table + (size_t)(ok ? id : 0) * hidden);
  for (int c = threadIdx.x; c < chunks; c += blockDim.x)
    dst[c] = ok ? src[c] : make_uint4(0, 0, 0, 0);
}

// 16-byte packets of T as floats and back (round to nearest even).
template <typename T>
__device__ __forceinline__ uint4 pack_packet(const float* v) {
  if constexpr (sizeof(T) == 4) {
    return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                      __float_as_uint(v[3]));
  } else {
    return make_uint4(Packet<T>::pack2(v[0], v[1]), Packet<T>::pack2(v[2], v[3]),
                      Packet<T>::pack2(v[4], v[5]), Packet<T>::pack2(v[6], v[7]));
  }
}

// Sum over a workgroup of kThreads threads, the same order in every thread.
template <int kThreads>
__device__ __forceinline__ float block_sum(float v, float* s_part) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) t += s_part[w];
  return t;
}

// [residual <- residual + x (rounded)]; out <- RmsNorm(residual) * w, the
// reference's cast order (RmsNorm::forward). One workgroup per row, each
// thread holding up to kNormChunks 16-byte chunks of it in registers between
// the sum of squares and the scaling.
constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;
template <typename T, bool ADD>
__global__ __launch_bounds__(kNormThreads) void norm_rows_kernel(
    const T* __restrict__ x, T* __restrict__ residual, const T* __restrict__ w,
    T* __restrict__ out, int n, float inv_n, float eps, int packed_out) {
  constexpr int E = 16 / sizeof(T);
  __shared__ float s_part[kNormThreads / 64];
  const size_t base = (size_t)blockIdx.x * n;
  const int chunks = n / E;
  const uint4* rr = reinterpret_cast<const uint4*>(residual + base);
  // The weight is requested with the row, so its loads are not a second
  // round trip after the sum of squares.
  uint4 wp[kNormChunks];
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int ci = threadIdx.x + c * kNormThreads;
    wp[c] = ci < chunks ? reinterpret_cast<const uint4*>(w)[ci] : make_uint4(0, 0, 0, 0);
  }
  float h[kNormChunks][E];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int ci = threadIdx.x + c * kNormThreads;
    if (ci < chunks) {
      Packet<T>::unpack(rr[ci], h[c]);
      if constexpr (ADD) {
        float xv[E];
        Packet<T>::unpack(reinterpret_cast<const uint4*>(x + base)[ci], xv);
#pragma unroll
        for (int e = 0; e < E; ++e) h[c][e] = round_to<T>(h[c][e] + xv[e]);
        reinterpret_cast<uint4*>(residual + base)[ci] = pack_packet<T>(h[c]);
      }
#pragma unroll
      for (int e = 0; e < E; ++e) ss += h[c][e] * h[c][e];
    }
  }
  const float norm = sqrtf(block_sum<kNormThreads>(ss, s_part) * inv_n + eps);
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int ci = threadIdx.x + c * kNormThreads;
    if (ci < chunks) {
      float wv[E], o[E];
      Packet<T>::unpack(wp[c], wv);
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = round_to<T>(h[c][e] / norm) * wv[e];
      // Packed rows (16-bit): row r's packet ci (elements 8ci .. +8) goes to
      // ((r/16 * n/32 + ci/4) * 64 + r%16 + 16 (ci%4)) * 8, the order in
      // which dense_rows_kernel loads its B operands.
      const size_t at =
          packed_out ? (((size_t)(blockIdx.x >> 4) * (n >> 5) + (ci >> 2)) * 64 + (blockIdx.x & 15) +
                        16 * (ci & 3)) * 8
                     : base + (size_t)ci * E;
      *reinterpret_cast<uint4*>(out + at) = pack_packet<T>(o);
    }
  }
}

// The same for rows that are not whole 16-byte chunks or longer than the
// register-held form allows: one wave per row, element loads.
template <typename T, bool ADD>
__global__ __launch_bounds__(256) void norm_rows_any_kernel(const T* __restrict__ x,
                                                            T* __restrict__ residual,
                                                            const T* __restrict__ w,
                                                            T* __restrict__ out, int rows, int n,
                                                            float inv_n, float eps) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  T* rr = residual + row * n;
  T* orow = out + row * n;
  float ss = 0.f;
  for (int i = lane; i < n; i += 64) {
    float h = Elem<T>::to_f32(rr[i]);
    if constexpr (ADD) {
      h = round_to<T>(h + Elem<T>::to_f32(x[row * n + i]));
      rr[i] = Elem<T>::from_f32(h);
    }
    ss += h * h;
  }
  ss = wave_sum(ss);
  const float norm = sqrtf(ss * inv_n + eps);
  for (int i = lane; i < n; i += 64) {
    const float xn = round_to<T>(Elem<T>::to_f32(rr[i]) / norm);
    orow[i] = Elem<T>::from_f32(xn * Elem<T>::to_f32(w[i]));
  }
}

// out[r][i] = silu(gate[r][i]) * up[r][i] with gate_up = [rows][2*inter]
// (gate columns, then up columns): silu(v) = v / (1 + exp(-v)) rounded per
// op (exp, the sum, the quotient), then the product rounded.
template <typename T>
__device__ __forceinline__ float silu_mul_rounded(float g, float u) {
  const float e = round_to<T>(expf(-g));
  const float s = round_to<T>(g / round_to<T>(1.f + e));
  return s * u;
}

template <typename T>
__global__ void silu_mul_kernel(const T* __restrict__ gate_up, T* __restrict__ out, int inter) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= inter) return;
  const size_t r = blockIdx.y;
  const float g = Elem<T>::to_f32(gate_up[r * 2 * inter + c]);
  const float u = Elem<T>::to_f32(gate_up[r * 2 * inter + inter + c]);
  out[r * inter + c] = Elem<T>::from_f32(silu_mul_rounded<T>(g, u));
}

// y[r][c] = y[r][c] + bias[c], rounded (Candle's broadcast_add after matmul).
template <typename T>
__global__ void bias_add_kernel(T* __restrict__ y, const T* __restrict__ bias, int n) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= n) return;
  const size_t i = (size_t)blockIdx.y * n + c;
  y[i] = Elem<T>::from_f32(Elem<T>::to_f32(y[i]) + Elem<T>::to_f32(bias[c]));
}

// ---------------------------------------------------------------------------
// Greedy argmax with the sequential scan's answer (Tensor::argmax on the
// host copy): the first index whose value exceeds every earlier one. As a
// reduction: a NaN at index 0 wins outright; otherwise the first index of
// the largest non-NaN value. Each (value, index) becomes one 64-bit key --
// the value's bits mapped to an unsigned order (-0 taken as +0, which the
// scan treats as equal), then the complemented index -- so the largest key
// is the largest value at its first index, whatever order the partial
// maxima combine in. Pass 1: one workgroup per kArgChunk logits of a row
// writes its key; pass 2: one wave per row combines the row's keys.
// ---------------------------------------------------------------------------
constexpr int kArgThreads = 256;
constexpr int kArgChunk = 4096;

__device__ __forceinline__ unsigned long long arg_key(float v, int i) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) == 0) u = 0;
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)o << 32) | (0xffffffffu - (uint32_t)i);
}

__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t hi = (uint32_t)__shfl_xor((int)(k >> 32), off, 64);
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)k, off, 64);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    k = o > k ? o : k;
  }
  return k;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kArgThreads) void argmax_partial_kernel(
    const T* __restrict__ logits, unsigned long long* __restrict__ keys, int vocab, int parts) {
  const int part = blockIdx.x;
  const size_t row = blockIdx.y;
  const T* r = logits + row * vocab;
  const int begin = part * kArgChunk;
  const int end = min(vocab, begin + kArgChunk);
  unsigned long long best = 0;  // below every value's key
  auto take = [&](float v, int i) __attribute__((always_inline)) {
    if (v == v) {
      const unsigned long long k = arg_key(v, i);
      best = k > best ? k : best;
    }
  };
  if constexpr (VEC) {
    // Rows of whole 16-byte packets: each thread reads packets tid and
    // tid + kArgThreads of the chunk (kArgChunk = 2 * kArgThreads * E).
    constexpr int E = 16 / sizeof(T);
#pragma unroll
    for (int h = 0; h < kArgChunk / (kArgThreads * E); ++h) {
      const int i0 = begin + (threadIdx.x + h * kArgThreads) * E;
      if (i0 < end) {
        float v[E];
        Packet<T>::unpack(*reinterpret_cast<const uint4*>(r + i0), v);
#pragma unroll
        for (int e = 0; e < E; ++e) take(v[e], i0 + e);
      }
    }
  } else {
    for (int i = begin + threadIdx.x; i < end; i += kArgThreads) take(Elem<T>::to_f32(r[i]), i);
  }
  best = wave_max_key(best);
  __shared__ unsigned long long s_k[kArgThreads / 64];
  if ((threadIdx.x & 63) == 0) s_k[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kArgThreads / 64; ++w) best = s_k[w] > best ? s_k[w] : best;
    keys[row * parts + part] = best;
  }
}

template <typename T>
__global__ __launch_bounds__(64) void argmax_final_kernel(const T* __restrict__ logits,
                                                          const unsigned long long* __restrict__ keys,
                                                          int32_t* __restrict__ out, int vocab,
                                                          int parts) {
  const size_t row = blockIdx.x;
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < parts; i += 64) {
    const unsigned long long k = keys[row * parts + i];
    best = k > best ? k : best;
  }
  best = wave_max_key(best);
  if (threadIdx.x == 0) {
    const float v0 = Elem<T>::to_f32(logits[row * vocab]);
    out[row] = (v0 != v0 || best == 0) ? 0 : (int32_t)(0xffffffffu - (uint32_t)best);
  }
}

// ---------------------------------------------------------------------------
// Decode-shaped linear layers on MFMA: y[rows][N] = x[rows][K] . W[N][K]^T for
// rows <= 64 (one decode step's batch), bf16/f16 in, f32 accumulation.
//
// Work split: workgroup (g, ks) owns FT tiles of 16 output features, the
// whole batch and the ks-th of KS equal slices of K; its four waves split the
// slice again. Each streams its K range of the 16*FT weight rows from HBM once
// and the matching x columns from L2. Per 32-wide k step a wave issues
// v_mfma_f32_16x16x32_{bf16,f16} with A = 16 weight rows x 32 k and B = 32 k x
// 16 batch rows; lane l loads the 16 bytes at k = 8*(l/16) of weight row l%16
// (A) and of batch row l%16 (B), and holds D[4*(l/16) + v][l%16], v = 0..3 --
// four consecutive features of one batch row. U steps' loads are issued
// before their MFMAs. The waves' partial tiles are summed through LDS in wave
// order. With KS > 1 (few output tiles: the K split puts every compute unit
// to work) the slices' sums meet as in the decode kernel's merge: workgroups
// ks < KS-1 store theirs as self-validating records and leave; workgroup
// KS-1, dispatched after them, waits for the records, adds them in slice
// order (so the result does not depend on arrival order), clears them, and
// runs the epilogue:
//   kEpiStore     y = round(acc) [+ bias, rounded]               (Linear)
//   kEpiQkv       the same, columns [0,n1) to q, [n1,n2) to k, [n2,N) to v
//   kEpiResidual  x_res = round(x_res + round(acc))              (residual add)
//   kEpiSiluMul   act = round(silu(round(gate)) * round(up)): tile i holds
//                 gate rows 8i..8i+7 and up rows n1+8i..n1+8i+7
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T>
struct Mma16;
template <>
struct Mma16<bf16> {
  static __device__ __forceinline__ f32x4_t run(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <>
struct Mma16<f16> {
  static __device__ __forceinline__ f32x4_t run(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};
// f32 (the reference CPU path's dtype): a 16-byte operand load holds four
// floats, so a k step spans 16 elements, lane l holding elements
// 4*(l/16) .. +3 of its row. v_mfma_f32_16x16x4_f32 number m takes each
// lane's element m, for A and B alike: its four k indices are 4g + m over
// the lane groups g, and the four products cover the step. The accumulator
// layout is the 16-bit products' (lane l: D[4*(l/16) + v][l%16]).
template <>
struct Mma16<float> {
  static __device__ __forceinline__ f32x4_t run(u32x4_t a, u32x4_t b, f32x4_t c) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[m]), __uint_as_float(b[m]), c, 0,
                                               0, 0);
    return c;
  }
};
// Elements of one k step (four lanes groups' 16-byte loads) and of one
// lane's load.
template <typename T>
__host__ __device__ constexpr int dense_step_elems() { return 64 / (int)sizeof(T); }

enum : int { kEpiStore = 0, kEpiQkv = 1, kEpiResidual = 2, kEpiSiluMul = 3 };

struct DenseParams {
  const void* x;     // [rows][K]
  const void* w;     // [N][K]
  const void* bias;  // [N] or null (kEpiStore, kEpiQkv)
  void* out0;        // y [rows][N] | q [rows][n1] | x_res [rows][N] | act [rows][n1]
  void* out1;        // k [rows][n2 - n1] (kEpiQkv)
  void* out2;        // v [rows][N - n2] (kEpiQkv)
  // KS > 1: sticky error flags, one launch counter per wave slot
  // (kDenseCtrWords) and (tile groups) x (KS - 1) records of FT*RT*256
  // tagged 64-bit words.
  uint32_t* ws_err;
  uint32_t* ws_ctr;
  uint64_t* ws_rec;
  unsigned long long wait_ticks;
  int rows, K, N, n1, n2;
  int ksplit;        // KS
  int steps;         // 32-wide k steps per wave
  int packed;        // w in the tile order rlse_dense_pack writes
  int xpacked;       // x in the packed row order (RLSE_PACKED_ROWS)
  int opacked;       // kEpiSiluMul: act in the packed row order (RLSE_PACKED_OUT)
};

constexpr int kDenseWaves = 4;
constexpr int kDenseMaxRows = 64;
constexpr int kDenseMaxSplit = 8;
// Most K slices run inside one workgroup (kDenseWaves waves each; 1024
// threads at most).
constexpr int kDenseMaxInner = 4;
// Launch counters of a K-split workspace: one per wave of the largest split
// grid. A split grid has fewer than 512 workgroups: an output is split only
// when it has fewer than 256 tile groups, into ceil(256 / groups) slices.
constexpr int kDenseCtrWords = 512 * kDenseWaves;
constexpr int kDenseHeaderWords = 64;

template <typename T>
__device__ __forceinline__ void load4(const T* p, float* v) {
  if constexpr (sizeof(T) == 4) {
    const float4 u = *reinterpret_cast<const float4*>(p);
    v[0] = u.x;
    v[1] = u.y;
    v[2] = u.z;
    v[3] = u.w;
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    const uint4 q = make_uint4(u.x, u.y, 0, 0);
    float t[8];
    Packet<T>::unpack(q, t);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = t[e];
  }
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const float* v) {
  if constexpr (sizeof(T) == 4)
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  else
    *reinterpret_cast<uint2*>(p) = make_uint2(Packet<T>::pack2(v[0], v[1]),
                                              Packet<T>::pack2(v[2], v[3]));
}

// KV > 1: the K split runs inside the workgroup instead of across
// workgroups -- KV slices of kDenseWaves waves each, every wave on the k
// steps it would have in the split grid, their sums added in LDS in the
// order the split grid's merge adds its records (the waves of a slice in
// order, then the slices in order), so the results are the split grid's to
// the bit. No records, no launch counters, no second round trip to memory.
template <typename T, int RT, int FT, int EPI, int KV = 1>
__global__ __launch_bounds__(64 * kDenseWaves * KV) void dense_rows_kernel(DenseParams p) {
  constexpr int WV = kDenseWaves * KV;  // waves per workgroup
  if constexpr (KV > 1 && RT == 1 && (EPI == kEpiResidual || EPI == kEpiQkv)) {
    // Row tiles split over the grid's rows (the launcher does so only for
    // these instantiations): this workgroup takes row tile blockIdx.y.
    if (gridDim.y > 1) {
      const int r0 = 16 * (int)blockIdx.y;
      p.x = p.xpacked ? (const void*)((const T*)p.x + (size_t)(r0 >> 4) * (p.K >> 5) * 512)
                      : (const void*)((const T*)p.x + (size_t)r0 * p.K);
      if constexpr (EPI == kEpiQkv) {
        p.out0 = (void*)((T*)p.out0 + (size_t)r0 * p.n1);
        p.out1 = (void*)((T*)p.out1 + (size_t)r0 * (p.n2 - p.n1));
        p.out2 = (void*)((T*)p.out2 + (size_t)r0 * (p.N - p.n2));
      } else {
        p.out0 = (void*)((T*)p.out0 + (size_t)r0 * p.N);
      }
      p.rows = min(16, p.rows - r0);
    }
  }
  constexpr int U = FT == 1 ? 8 : 4;
  constexpr int SE = dense_step_elems<T>();  // elements of a k step (packed: 16-bit only)
  // An epilogue item is the four consecutive features one lane slot holds
  // (4*(slot/16).. of batch row slot%16); kEpiSiluMul pairs slot s (gate
  // features) with slot s+32 (the matching up features) in one item.
  constexpr int kPair = EPI == kEpiSiluMul ? 2 : 1;
  constexpr int kItems = FT * RT * 64 / kPair;
  constexpr int kItemsPerThread = (kItems + 64 * WV - 1) / (64 * WV);
  constexpr int kRecWords = FT * RT * 256;
  __shared__ float red[WV][FT][RT][256];
  const int lane = threadIdx.x & 63;
  // Wave-uniform (a scalar register): the k-step bounds below derive from
  // it, and a bound the compiler takes for a per-lane value puts the
  // unrolled steps' MFMAs under an exec mask instead of a branch -- steps
  // past the wave's last then fed their stale operands into the sums.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fi = lane & 15;
  const int g = lane >> 4;
  const int K = p.K;
  const int KS = p.ksplit;
  const int grp = blockIdx.x / KS;
  const int ks = blockIdx.x - grp * KS;
  // K split: this wave's launch counter (its epoch tags the records it
  // publishes and is expected on those it merges); the wave also advances
  // the counters of the wave slots this grid does not cover, so every
  // counter moves once per launch.
  const int gw = blockIdx.x * kDenseWaves + wave;
  uint32_t ep = 0;
  if (KS > 1)
    ep = next_epoch(__hip_atomic_load(p.ws_ctr + gw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  auto end_epoch = [&]() __attribute__((always_inline)) {
    if (KS > 1 && lane == 0)
      for (int c = gw; c < kDenseCtrWords; c += gridDim.x * kDenseWaves)
        __hip_atomic_store(p.ws_ctr + c, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  const T* wr[FT];
#pragma unroll
  for (int f = 0; f < FT; ++f) {
    const int tile = grp * FT + f;
    int row;
    if constexpr (EPI == kEpiSiluMul)
      row = fi < 8 ? tile * 8 + fi : p.n1 + tile * 8 + (fi - 8);
    else
      row = tile * 16 + fi;
    // Packed weights: tile t's operands of k step s are 64 lanes x 16
    // bytes at ((t * K/32 + s) * 64 + lane) * 8, one contiguous KiB per load.
    wr[f] = p.packed ? (const T*)p.w + ((size_t)tile * (K >> 5) * 64 + lane) * 8
                     : (const T*)p.w + (size_t)row * K + (SE / 4) * g;
  }
  const int wstep = p.packed ? 512 : SE;  // weight elements between k steps
  // x: row-major (rows past the batch read its last row), or packed rows:
  // row tile t's operands of k step s at ((t * K/32 + s) * 64 + lane) * 8
  // (the packed buffer holds whole 16-row tiles).
  const T* xr[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t)
    xr[t] = p.xpacked ? (const T*)p.x + ((size_t)t * (K >> 5) * 64 + lane) * 8
                      : (const T*)p.x + (size_t)min(16 * t + fi, p.rows - 1) * K + (SE / 4) * g;
  const int xstep = p.xpacked ? 512 : SE;  // x elements between k steps
  f32x4_t acc[FT][RT];
#pragma unroll
  for (int f = 0; f < FT; ++f)
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[f][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Epilogue operands read from memory (the residual, the bias) are
  // requested before the main loop: they arrive with its loads instead of
  // costing a round trip after it. Only the merging slice (or an unsplit
  // workgroup) needs them.
  float pre[kItemsPerThread][4];
#pragma unroll
  for (int k = 0; k < kItemsPerThread; ++k) {
    const int it = threadIdx.x + k * 64 * WV;
    const int l2 = it & (64 / kPair - 1);
    const int ft = it / (64 / kPair);
    const int t = ft % RT, f = ft / RT;
    const int b = 16 * t + (l2 & 15);
    const int n = (grp * FT + f) * 16 + 4 * (l2 >> 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) pre[k][e] = 0.f;
    if (it >= kItems || b >= p.rows || ks != KS - 1) continue;
    if constexpr (EPI == kEpiResidual) load4<T>((const T*)p.out0 + (size_t)b * p.N + n, pre[k]);
    if constexpr (EPI == kEpiStore || EPI == kEpiQkv)
      if (p.bias) load4<T>((const T*)p.bias + n, pre[k]);
  }

  const int S = K / SE;
  // The wave's k steps: slice sl of NS (a workgroup of the split grid, or a
  // slice of this workgroup's waves), its ws-th share.
  const int NS = KV > 1 ? KV : KS;
  const int sl = KV > 1 ? wave / kDenseWaves : ks;
  const int ws = KV > 1 ? wave % kDenseWaves : wave;
  const int slice_end = (sl + 1) * S / NS;
  const int s_begin = sl * S / NS + ws * p.steps;
  const int s_end = min(slice_end, s_begin + p.steps);
  for (int s = s_begin; s < s_end; s += U) {
    u32x4_t a[U][FT], b[U][RT];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      if (s + j < s_end) {
#pragma unroll
        for (int f = 0; f < FT; ++f)
          a[j][f] = *reinterpret_cast<const u32x4_t*>(wr[f] + (size_t)wstep * (s + j));
#pragma unroll
        for (int t = 0; t < RT; ++t)
          b[j][t] = *reinterpret_cast<const u32x4_t*>(xr[t] + (size_t)xstep * (s + j));
      }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      if (s + j < s_end) {
#pragma unroll
        for (int f = 0; f < FT; ++f)
#pragma unroll
          for (int t = 0; t < RT; ++t) acc[f][t] = Mma16<T>::run(a[j][f], b[j][t], acc[f][t]);
      }
    }
  }
#pragma unroll
  for (int f = 0; f < FT; ++f)
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][f][t][lane * 4 + v] = acc[f][t][v];
  __syncthreads();

  // This workgroup's sums of its items (waves in order), kPair slots each.
  float v[kItemsPerThread][kPair][4];
#pragma unroll
  for (int k = 0; k < kItemsPerThread; ++k) {
    const int it = threadIdx.x + k * 64 * WV;
    if (it < kItems) {
      const int l2 = it & (64 / kPair - 1);
      const int ft = it / (64 / kPair);
      const int t = ft % RT, f = ft / RT;
#pragma unroll
      for (int q = 0; q < kPair; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = 0.f;
#pragma unroll
          for (int c = 0; c < KV; ++c) {
            float y = red[c * kDenseWaves][f][t][(l2 + 32 * q) * 4 + e];
#pragma unroll
            for (int w = 1; w < kDenseWaves; ++w)
              y += red[c * kDenseWaves + w][f][t][(l2 + 32 * q) * 4 + e];
            x = c == 0 ? y : x + y;
          }
          v[k][q][e] = x;
        }
    }
  }

  bool ok = true;
  if (KS > 1) {
    // Record of slice sl: kItems items of kPair*4 tagged words.
    constexpr int kWords = kPair * 4;
    auto word_ptr = [&](int slice, int it, int j) {
      return p.ws_rec + ((size_t)grp * (KS - 1) + slice) * kRecWords + (size_t)it * kWords + j;
    };
    if (ks < KS - 1) {
#pragma unroll
      for (int k = 0; k < kItemsPerThread; ++k) {
        const int it = threadIdx.x + k * 64 * WV;
        if (it < kItems)
#pragma unroll
          for (int j = 0; j < kWords; ++j) st_tagged(word_ptr(ks, it, j), ep, v[k][j >> 2][j & 3]);
      }
      end_epoch();
      return;
    }
    // The merging workgroup: every slice's words are requested together,
    // then only those without this launch's epoch again; the sum runs in
    // slice order.
    const unsigned long long t0 = wall_clock64();
#pragma unroll
    for (int k = 0; k < kItemsPerThread; ++k) {
      const int it = threadIdx.x + k * 64 * WV;
      if (it >= kItems) continue;
      uint64_t r[kDenseMaxSplit - 1][kWords];
#pragma unroll
      for (int sl = 0; sl < kDenseMaxSplit - 1; ++sl)
#pragma unroll
        for (int j = 0; j < kWords; ++j) r[sl][j] = 0ull;
      for (;;) {
        bool all = true;
#pragma unroll
        for (int sl = 0; sl < kDenseMaxSplit - 1; ++sl) {
          if (sl >= KS - 1) break;
#pragma unroll
          for (int j = 0; j < kWords; ++j) {
            if (!tag_is(r[sl][j], ep)) r[sl][j] = ld_tagged(word_ptr(sl, it, j));
            all = all && tag_is(r[sl][j], ep);
          }
        }
        if (all) break;
        if (wall_clock64() - t0 > p.wait_ticks) {
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      float sum[kPair][4];
#pragma unroll
      for (int sl = 0; sl < kDenseMaxSplit - 1; ++sl) {
        if (sl >= KS - 1) break;
#pragma unroll
        for (int j = 0; j < kWords; ++j) {
          float& a = sum[j >> 2][j & 3];
          a = sl == 0 ? tag_value(r[sl][j]) : a + tag_value(r[sl][j]);
        }
      }
#pragma unroll
      for (int q = 0; q < kPair; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[k][q][e] = sum[q][e] + v[k][q][e];
    }
    if (!ok) ws_raise(p.ws_err, RLSE_WS_ERR_MERGE_TIMEOUT);
  }

#pragma unroll
  for (int k = 0; k < kItemsPerThread; ++k) {
    const int it = threadIdx.x + k * 64 * WV;
    if (it >= kItems) continue;
    const int l2 = it & (64 / kPair - 1);
    const int ft = it / (64 / kPair);
    const int t = ft % RT, f = ft / RT;
    const int b = 16 * t + (l2 & 15);
    const int fq = 4 * (l2 >> 4);
    if (b >= p.rows) continue;
    const int tile = grp * FT + f;
    float o[4];
    if constexpr (EPI == kEpiSiluMul) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = ok ? silu_mul_rounded<T>(round_to<T>(v[k][0][e]), round_to<T>(v[k][1][e]))
                  : __builtin_nanf("");
      const int c = tile * 8 + fq;  // act feature (4 of them)
      store4<T>((T*)p.out0 +
                    (p.opacked ? (((size_t)(b >> 4) * (p.n1 >> 5) + (c >> 5)) * 64 + (b & 15) +
                                  16 * ((c & 31) >> 3)) * 8 + (c & 7)
                               : (size_t)b * p.n1 + c),
                o);
    } else if constexpr (EPI == kEpiResidual) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = ok ? pre[k][e] + round_to<T>(v[k][0][e]) : __builtin_nanf("");
      store4<T>((T*)p.out0 + (size_t)b * p.N + tile * 16 + fq, o);
    } else {
      const int n = tile * 16 + fq;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = ok ? round_to<T>(v[k][0][e]) + (p.bias ? pre[k][e] : 0.f) : __builtin_nanf("");
      T* dst;
      if (EPI == kEpiQkv && n >= p.n2)
        dst = (T*)p.out2 + (size_t)b * (p.N - p.n2) + (n - p.n2);
      else if (EPI == kEpiQkv && n >= p.n1)
        dst = (T*)p.out1 + (size_t)b * (p.n2 - p.n1) + (n - p.n1);
      else if (EPI == kEpiQkv)
        dst = (T*)p.out0 + (size_t)b * p.n1 + n;
      else
        dst = (T*)p.out0 + (size_t)b * p.N + n;
      store4<T>(dst, o);
    }
  }
  end_epoch();
}

template <typename F>
int by_dtype(int dtype, F&& f) {
  switch (dtype) {
    case RLSE_DTYPE_F32: return f(float{});
    case RLSE_DTYPE_BF16: return f(bf16{});
    case RLSE_DTYPE_F16: return f(f16{});
  }
  return fail(RLSE_ERR_INVALID_VALUE, "bad dtype %d", dtype);
}

// One rocBLAS handle per device, created on first use.
std::mutex g_blas_mu;
rocblas_handle g_blas[64] = {nullptr};

bool aligned(const void* ptr, size_t a) { return ((uintptr_t)ptr % a) == 0; }

// 16-feature tiles per workgroup. Every workgroup reads the whole batch's x
// columns of its K range, so x costs (rows / (16 * tiles per group)) times
// the weight bytes in L2 reads: lm_head-sized outputs take four tiles
// (plain stores only); batches of more than 32 rows take two when the
// output still has 256 groups of two, so no K split is needed (the rows of
// the first 64-row chunk decide; every chunk uses the same grouping).
// Measured at 64 rows: gate/up of 9728 x 896, 18.4 -> 16.0 us; for outputs
// that then needed a K split (q/k/v 1152 x 896: 7.9 -> 11.6 us) two tiles
// cost more than they saved.
int dense_tiles_per_group(bool plain_store, int rows, int tiles) {
  if (plain_store && tiles % 4 == 0 && tiles >= 4096) return 4;
  const int rt = (std::min(rows, kDenseMaxRows) + 15) / 16;
  if (rt >= 3 && tiles % 2 == 0 && tiles / 2 >= 256) return 2;
  return 1;
}

// Header and launch-counter words at the start of a K-split workspace.
constexpr size_t dense_ws_fixed_words() { return kDenseHeaderWords + kDenseCtrWords; }

// K slices per output tile group: enough workgroups to cover every compute
// unit (256 on MI355X) when the output has few 16-feature tiles, each slice
// at least 4 k steps of 32. Outputs with 256 or more tiles are not split:
// measured, the merge's extra memory round trip costs them more than the
// added workgroups gain.
int dense_split(int groups, int K) {
  int ks = (256 + groups - 1) / groups;
  ks = std::min(ks, kDenseMaxSplit);
  ks = std::min(ks, std::max(1, (K / 32) / 4));
  return std::max(ks, 1);
}

// Launches dense_rows_kernel over the batch in chunks of kDenseMaxRows rows
// (each chunk streams the weights once). Shapes were checked by the caller:
// K % 32 == 0, 16-feature tiles that never straddle an output, 16-byte
// aligned x / W and 8-byte aligned outputs; ws holds ws_words words (zero
// before the first launch; every launch leaves it zero).
template <typename T, int EPI>
int launch_dense(DenseParams p, size_t x_stride, size_t o0_stride, size_t o1_stride,
                 size_t o2_stride, size_t ws_words, hipStream_t s) {
  const int total_rows = p.rows;
  const int tiles = EPI == kEpiSiluMul ? p.n1 / 8 : p.N / 16;
  const int ft = dense_tiles_per_group(EPI == kEpiStore, total_rows, tiles);
  const bool wide = ft == 4;
  const int groups = tiles / ft;
  const int ks = p.ws_rec ? dense_split(groups, p.K) : 1;
  // A split of one-tile groups runs inside the workgroup (KV slices of
  // kDenseWaves waves, at most kDenseMaxInner of them): the split grid's k
  // steps and sums, without its records. The residual and q/k/v
  // projections put each 16-row tile on its own workgroup row (grid rows;
  // one row tile per workgroup keeps the 16-wave workgroup within its
  // registers at any row count); plain stores do so up to 32 rows. The
  // SwiGLU epilogue's paired items would spill a 16-wave workgroup's 128
  // registers per lane, so it keeps the split grid.
  const int kv_inner =
      (ks > 1 && ft == 1 && EPI != kEpiSiluMul &&
       (total_rows <= 32 || EPI == kEpiResidual || EPI == kEpiQkv))
          ? std::min(ks, kDenseMaxInner)
          : 1;
  const int ns = kv_inner > 1 ? kv_inner : ks;
  const int steps_total = p.K / dense_step_elems<T>();
  const int slice = (steps_total + ns - 1) / ns;
  p.ksplit = kv_inner > 1 ? 1 : ks;
  p.steps = (slice + kDenseWaves - 1) / kDenseWaves;
  const char* base0 = (const char*)p.out0;
  const char* base1 = (const char*)p.out1;
  const char* base2 = (const char*)p.out2;
  const char* xb = (const char*)p.x;
  for (int r0 = 0; r0 < total_rows; r0 += kDenseMaxRows) {
    DenseParams q = p;
    q.rows = std::min(kDenseMaxRows, total_rows - r0);
    q.x = xb + (size_t)r0 * x_stride * sizeof(T);
    q.out0 = (void*)(base0 + (size_t)r0 * o0_stride * sizeof(T));
    q.out1 = base1 ? (void*)(base1 + (size_t)r0 * o1_stride * sizeof(T)) : nullptr;
    q.out2 = base2 ? (void*)(base2 + (size_t)r0 * o2_stride * sizeof(T)) : nullptr;
    const int rt = (q.rows + 15) / 16;
    if (q.ksplit > 1 && dense_ws_fixed_words() + (size_t)groups * (ks - 1) * ft * rt * 256 * 2 >
                            ws_words)
      return fail(RLSE_ERR_INVALID_VALUE, "dense: workspace too small");
    if (q.ksplit > 1 && groups * ks * kDenseWaves > kDenseCtrWords)
      return fail(RLSE_ERR_INVALID_VALUE, "dense: K-split grid larger than its counters");
    const dim3 block(64 * kDenseWaves);
    const dim3 grid(groups * q.ksplit);
    auto run = [&](auto rt_c) {
      constexpr int RT = decltype(rt_c)::value;
      if constexpr ((RT <= 2 || EPI == kEpiResidual || EPI == kEpiQkv) && EPI != kEpiSiluMul) {
        if (kv_inner > 1) {
          // A residual or q/k/v projection's row tiles go to separate
          // workgroups (grid rows): each streams the tile group's weights
          // (the others from L2/MALL) but only its 16 rows of the batch's
          // activations, which are most of a workgroup's bytes, and more
          // compute units take part. Same k steps and sums per row, so the
          // same bits. Measured in the whole decode step: o_proj and
          // down_proj 8.05 -> 6.14 us at 32 rows x hidden 1024; at 64 rows
          // x hidden 896, where it replaces the split grid's records, 11.86
          // -> 6.46 us, and q/k/v 8.96 -> 6.27 us.
          constexpr int RTL = (EPI == kEpiResidual || EPI == kEpiQkv) ? 1 : RT;
          const dim3 g(grid.x, RT / RTL);
          const dim3 big(64 * kDenseWaves * kv_inner);
          if (kv_inner == 2)
            hipLaunchKernelGGL((dense_rows_kernel<T, RTL, 1, EPI, 2>), g, big, 0, s, q);
          else if (kv_inner == 3)
            hipLaunchKernelGGL((dense_rows_kernel<T, RTL, 1, EPI, 3>), g, big, 0, s, q);
          else
            hipLaunchKernelGGL((dense_rows_kernel<T, RTL, 1, EPI, 4>), g, big, 0, s, q);
          return;
        }
      }
      if constexpr (EPI == kEpiStore) {
        if (wide) {
          hipLaunchKernelGGL((dense_rows_kernel<T, RT, 4, EPI>), grid, block, 0, s, q);
          return;
        }
      }
      if (ft == 2) {  // every chunk keeps the grouping (a short last chunk too)
        hipLaunchKernelGGL((dense_rows_kernel<T, RT, 2, EPI>), grid, block, 0, s, q);
        return;
      }
      hipLaunchKernelGGL((dense_rows_kernel<T, RT, 1, EPI>), grid, block, 0, s, q);
    };
    switch (rt) {
      case 1: run(std::integral_constant<int, 1>{}); break;
      case 2: run(std::integral_constant<int, 2>{}); break;
      case 3: run(std::integral_constant<int, 3>{}); break;
      default: run(std::integral_constant<int, 4>{}); break;
    }
    const int rc = launch_status("dense_rows_kernel");
    if (rc) return rc;
  }
  return RLSE_OK;
}

// Workspace words a fused projection needs for its K split (0: none): the
// header and the launch counters, then the tagged records (two 32-bit words
// each).
size_t dense_ws_words(int rows, int tiles, int K) {
  if (rows <= 0 || tiles <= 0 || K < 32) return 0;
  const int ft = dense_tiles_per_group(false, rows, tiles);
  const int ks = dense_split(tiles / ft, K);
  const int rt = (std::min(rows, kDenseMaxRows) + 15) / 16;
  return ks > 1 ? dense_ws_fixed_words() + (size_t)(tiles / ft) * (ks - 1) * ft * rt * 256 * 2
                : 0;
}

// Shape and alignment checks shared by the MFMA entry points.
int check_dense(const char* what, int dtype, int rows, int K, const void* x, const void* w,
                const void* const* outs, int nouts) {
  if (dtype != RLSE_DTYPE_BF16 && dtype != RLSE_DTYPE_F16)
    return fail(RLSE_ERR_INVALID_VALUE,
                "%s: bf16 or f16 only (f32 steps use rlse_linear with the element-wise ops)",
                what);
  if (rows < 0 || K <= 0 || K % 32)
    return fail(RLSE_ERR_INVALID_VALUE, "%s: rows %d, in_features %d (a multiple of 32)", what,
                rows, K);
  if (rows == 0) return RLSE_OK;
  if (!x || !w) return fail(RLSE_ERR_INVALID_VALUE, "%s: null pointer", what);
  if (!aligned(x, 16) || !aligned(w, 16))
    return fail(RLSE_ERR_INVALID_VALUE, "%s: x and weight must be 16-byte aligned", what);
  for (int i = 0; i < nouts; ++i) {
    if (!outs[i]) return fail(RLSE_ERR_INVALID_VALUE, "%s: null output", what);
    if (!aligned(outs[i], 8))
      return fail(RLSE_ERR_INVALID_VALUE, "%s: outputs must be 8-byte aligned", what);
  }
  return RLSE_OK;
}

template <int EPI>
int dense_by_dtype(int dtype, const DenseParams& p, size_t xs, size_t s0, size_t s1, size_t s2,
                   size_t ws_words, hipStream_t s) {
  return dtype == RLSE_DTYPE_BF16 ? launch_dense<bf16, EPI>(p, xs, s0, s1, s2, ws_words, s)
                                  : launch_dense<f16, EPI>(p, xs, s0, s1, s2, ws_words, s);
}

// The caller's workspace for a fused projection: NULL runs without a K
// split; otherwise it must hold dense_ws_words words, 4-byte aligned.
int dense_workspace(const char* what, DenseParams& p, void* workspace, size_t workspace_bytes,
                    size_t* words) {
  *words = 0;
  p.ws_err = p.ws_ctr = nullptr;
  p.ws_rec = nullptr;
  if (!workspace) return RLSE_OK;
  const size_t need = dense_ws_words(p.rows, p.N / 16, p.K);
  if (need == 0) return RLSE_OK;
  if (workspace_bytes < need * 4 || !aligned(workspace, 8))
    return fail(RLSE_ERR_INVALID_VALUE, "%s: workspace of %zu bytes (8-byte aligned) needed, %zu "
                                        "given", what, need * 4, workspace_bytes);
  uint32_t* base = (uint32_t*)workspace;
  p.ws_err = base;
  p.ws_ctr = base + kDenseHeaderWords;
  p.ws_rec = reinterpret_cast<uint64_t*>(base + dense_ws_fixed_words());
  p.wait_ticks = merge_wait_ticks();
  *words = need;
  return RLSE_OK;
}

// Weights in the tile order of dense_rows_kernel: one 16-byte packet per
// thread, packet i = ((tile * K/32 + s) * 64 + lane) holding row
// row(tile, lane % 16), elements 32s + 8(lane / 16) .. +8. Rows of a tile are
// 16 consecutive rows, or (n1 > 0, gate/up) gate rows 8t .. 8t+7 then up rows
// n1 + 8t .. n1 + 8t + 7.
template <typename T>
__global__ void dense_pack_kernel(const T* __restrict__ w, T* __restrict__ out, int K, int n1,
                                  long long packets) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= packets) return;
  const int S = K >> 5;
  const int lane = (int)(i & 63);
  const long long ts = i >> 6;
  const int st = (int)(ts % S);
  const long long tile = ts / S;
  const int fi = lane & 15, g = lane >> 4;
  const long long row = n1 > 0 ? (fi < 8 ? tile * 8 + fi : n1 + tile * 8 + (fi - 8))
                               : tile * 16 + fi;
  *reinterpret_cast<uint4*>(out + i * 8) =
      *reinterpret_cast<const uint4*>(w + row * K + 32 * st + 8 * g);
}

// Strips RLSE_DENSE_PACKED (weight), RLSE_PACKED_ROWS (x) and
// RLSE_PACKED_OUT (gate/up's act) from a dtype argument into p.
void take_packed(int& dtype, DenseParams& p) {
  p.packed = (dtype & RLSE_DENSE_PACKED) != 0;
  p.xpacked = (dtype & RLSE_PACKED_ROWS) != 0;
  p.opacked = (dtype & RLSE_PACKED_OUT) != 0;
  dtype &= ~(RLSE_DENSE_PACKED | RLSE_PACKED_ROWS | RLSE_PACKED_OUT);
}

}  // namespace
}  // namespace rlse

using namespace rlse;

extern "C" int rlse_embedding(const int32_t* ids, const void* table, void* out, int batch,
                              int hidden, int vocab, int dtype, rlse_stream_t stream) {
  const size_t es = dtype_size(dtype);
  if (!es || batch < 0 || hidden <= 0 || vocab <= 0 || (hidden * es) % 16)
    return fail(RLSE_ERR_INVALID_VALUE, "embedding: bad shape (hidden*dtype bytes must be a "
                                        "multiple of 16)");
  if (batch == 0) return RLSE_OK;
  if (!ids || !table || !out) return fail(RLSE_ERR_INVALID_VALUE, "embedding: null pointer");
  hipStream_t s = as_stream(stream);
  return by_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL(embedding_kernel<T>, dim3(batch), dim3(128), 0, s, ids,
                       (const T*)table, (T*)out, hidden, vocab);
    return launch_status("embedding");
  });
}

extern "C" int rlse_add_rmsnorm(const void* x, void* residual, const void* weight, void* out,
                                int rows, int n, float eps, int dtype, rlse_stream_t stream) {
  const bool packed_out = (dtype & RLSE_PACKED_ROWS) != 0;
  dtype &= ~RLSE_PACKED_ROWS;
  const size_t es = dtype_size(dtype);
  if (!es || rows < 0 || n <= 0 || !(eps >= 0.f))
    return fail(RLSE_ERR_INVALID_VALUE, "add_rmsnorm: bad arguments");
  if (rows == 0) return RLSE_OK;
  if (!residual || !weight || !out)
    return fail(RLSE_ERR_INVALID_VALUE, "add_rmsnorm: null pointer");
  const float inv_n = (float)(1.0 / (double)n);
  hipStream_t s = as_stream(stream);
  const bool chunked = (n * es) % 16 == 0 && n * es / 16 <= (size_t)kNormThreads * kNormChunks &&
                       aligned(residual, 16) && aligned(weight, 16) && aligned(out, 16) &&
                       (!x || aligned(x, 16));
  if (packed_out && (es != 2 || n % 32 || !chunked))
    return fail(RLSE_ERR_INVALID_VALUE,
                "add_rmsnorm: packed rows need bf16/f16, n a multiple of 32 (at most %d) and "
                "16-byte aligned buffers", kNormThreads * kNormChunks * 8);
  return by_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    const T* xp = (const T*)x;
    T* rp = (T*)residual;
    if (chunked) {
      if (x)
        hipLaunchKernelGGL((norm_rows_kernel<T, true>), dim3(rows), dim3(kNormThreads), 0, s,
                           xp, rp, (const T*)weight, (T*)out, n, inv_n, eps, (int)packed_out);
      else
        hipLaunchKernelGGL((norm_rows_kernel<T, false>), dim3(rows), dim3(kNormThreads), 0, s,
                           xp, rp, (const T*)weight, (T*)out, n, inv_n, eps, (int)packed_out);
    } else if (x) {
      hipLaunchKernelGGL((norm_rows_any_kernel<T, true>), dim3((rows + 3) / 4), dim3(256), 0, s,
                         xp, rp, (const T*)weight, (T*)out, rows, n, inv_n, eps);
    } else {
      hipLaunchKernelGGL((norm_rows_any_kernel<T, false>), dim3((rows + 3) / 4), dim3(256), 0,
                         s, xp, rp, (const T*)weight, (T*)out, rows, n, inv_n, eps);
    }
    return launch_status("add_rmsnorm");
  });
}

extern "C" int rlse_silu_mul(const void* gate_up, void* out, int rows, int inter, int dtype,
                             rlse_stream_t stream) {
  if (!dtype_size(dtype) || rows < 0 || inter <= 0 || rows > 65535)
    return fail(RLSE_ERR_INVALID_VALUE, "silu_mul: bad arguments");
  if (rows == 0) return RLSE_OK;
  if (!gate_up || !out) return fail(RLSE_ERR_INVALID_VALUE, "silu_mul: null pointer");
  hipStream_t s = as_stream(stream);
  return by_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL(silu_mul_kernel<T>, dim3((inter + 255) / 256, rows), dim3(256), 0, s,
                       (const T*)gate_up, (T*)out, inter);
    return launch_status("silu_mul");
  });
}

extern "C" int rlse_argmax_workspace_size(int rows, int vocab, size_t* bytes) {
  if (!bytes || rows < 0 || vocab <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "argmax_workspace_size: bad arguments");
  const size_t parts = ((size_t)vocab + kArgChunk - 1) / kArgChunk;
  *bytes = (size_t)rows * parts * sizeof(unsigned long long);
  return RLSE_OK;
}

extern "C" int rlse_argmax(const void* logits, int32_t* out, int rows, int vocab, int dtype,
                           void* workspace, size_t workspace_bytes, rlse_stream_t stream) {
  if (!dtype_size(dtype) || rows < 0 || vocab <= 0 || rows > 65535)
    return fail(RLSE_ERR_INVALID_VALUE, "argmax: bad arguments");
  if (rows == 0) return RLSE_OK;
  if (!logits || !out) return fail(RLSE_ERR_INVALID_VALUE, "argmax: null pointer");
  size_t need = 0;
  rlse_argmax_workspace_size(rows, vocab, &need);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 8))
    return fail(RLSE_ERR_INVALID_VALUE,
                "argmax: workspace of %zu bytes (8-byte aligned) needed, %zu given", need,
                workspace ? workspace_bytes : 0);
  const int parts = (vocab + kArgChunk - 1) / kArgChunk;
  auto* keys = (unsigned long long*)workspace;
  hipStream_t s = as_stream(stream);
  return by_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    // Whole 16-byte packets per row (and the chunk boundaries on packets):
    // vector loads.
    if (sizeof(T) == 2 && (vocab * sizeof(T)) % 16 == 0 && aligned(logits, 16))
      hipLaunchKernelGGL((argmax_partial_kernel<T, true>), dim3(parts, rows), dim3(kArgThreads),
                         0, s, (const T*)logits, keys, vocab, parts);
    else
      hipLaunchKernelGGL((argmax_partial_kernel<T, false>), dim3(parts, rows),
                         dim3(kArgThreads), 0, s, (const T*)logits, keys, vocab, parts);
    int rc = launch_status("argmax_partial");
    if (rc) return rc;
    hipLaunchKernelGGL(argmax_final_kernel<T>, dim3(rows), dim3(64), 0, s, (const T*)logits,
                       keys, out, vocab, parts);
    return launch_status("argmax_final");
  });
}

extern "C" int rlse_linear(const void* x, const void* weight, const void* bias, void* y,
                           int rows, int out_features, int in_features, int dtype,
                           rlse_stream_t stream) {
  DenseParams flags{};
  take_packed(dtype, flags);
  const bool packed = flags.packed || flags.xpacked;
  if (!dtype_size(dtype) || rows < 0 || out_features <= 0 || in_features <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "linear: bad arguments");
  if (rows == 0) return RLSE_OK;
  if (!x || !weight || !y) return fail(RLSE_ERR_INVALID_VALUE, "linear: null pointer");
  hipStream_t s = as_stream(stream);
  const bool mfma = (dtype == RLSE_DTYPE_BF16 || dtype == RLSE_DTYPE_F16) &&
                    in_features % 32 == 0 && out_features % 16 == 0 && aligned(x, 16) &&
                    aligned(weight, 16) && aligned(y, 8) && (!bias || aligned(bias, 8));
  // f32 at decode shapes: the same kernel on f32 MFMAs (16-element k steps,
  // 16-byte output and bias packets).
  const bool mfma32 = dtype == RLSE_DTYPE_F32 && !packed && rows <= kDenseMaxRows &&
                      in_features % 16 == 0 && out_features % 16 == 0 && aligned(x, 16) &&
                      aligned(weight, 16) && aligned(y, 16) && (!bias || aligned(bias, 16));
  if (mfma32) {
    DenseParams p{};
    p.x = x;
    p.w = weight;
    p.bias = bias;
    p.out0 = y;
    p.rows = rows;
    p.K = in_features;
    p.N = out_features;
    return launch_dense<float, kEpiStore>(p, in_features, out_features, 0, 0, 0, s);
  }
  if (packed && !mfma)
    return fail(RLSE_ERR_INVALID_VALUE,
                "linear: packed weights or rows need bf16/f16, in_features %% 32 == 0, "
                "out_features %% 16 == 0 and aligned buffers");
  // Decode-shaped products (a few rows) run on the MFMA kernel, as do
  // products over packed weights (64 rows at a time); larger unpacked
  // products (prefill-sized, one weight read serving many rows) are plain
  // library GEMMs.
  if (mfma && (rows <= kDenseMaxRows || packed)) {
    DenseParams p{};
    p.x = x;
    p.w = weight;
    p.bias = bias;
    p.out0 = y;
    p.rows = rows;
    p.K = in_features;
    p.N = out_features;
    p.packed = flags.packed;
    p.xpacked = flags.xpacked;
    return dense_by_dtype<kEpiStore>(dtype, p, in_features, out_features, 0, 0, 0, s);
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(RLSE_ERR_INVALID_VALUE, "linear: no current device");
  rocblas_handle h = nullptr;
  {
    std::lock_guard<std::mutex> g(g_blas_mu);
    if (!g_blas[dev] && rocblas_create_handle(&g_blas[dev]) != rocblas_status_success)
      return fail(RLSE_ERR_INVALID_VALUE, "linear: rocblas_create_handle failed");
    h = g_blas[dev];
  }
  if (rocblas_set_stream(h, s) != rocblas_status_success)
    return fail(RLSE_ERR_INVALID_VALUE, "linear: rocblas_set_stream failed");
  const rocblas_datatype t = dtype == RLSE_DTYPE_F32   ? rocblas_datatype_f32_r
                             : dtype == RLSE_DTYPE_BF16 ? rocblas_datatype_bf16_r
                                                        : rocblas_datatype_f16_r;
  const float alpha = 1.f, beta = 0.f;
  // Row-major y[rows][N] = x[rows][K] . W[N][K]^T is column-major
  // y^T[N][rows] = W^T . x^T: A = W (transposed, lda K), B = x (ldb K).
  const rocblas_status st = rocblas_gemm_ex(
      h, rocblas_operation_transpose, rocblas_operation_none, out_features, rows, in_features,
      &alpha, weight, t, in_features, x, t, in_features, &beta, y, t, out_features, y, t,
      out_features, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success)
    return fail(RLSE_ERR_INVALID_VALUE, "linear: rocblas_gemm_ex failed (%d)", (int)st);
  if (!bias) return RLSE_OK;
  if (rows > 65535) return fail(RLSE_ERR_INVALID_VALUE, "linear: bias add over %d rows", rows);
  return by_dtype(dtype, [&](auto tt) {
    using T = decltype(tt);
    hipLaunchKernelGGL(bias_add_kernel<T>, dim3((out_features + 255) / 256, rows), dim3(256), 0,
                       s, (T*)y, (const T*)bias, out_features);
    return launch_status("bias_add");
  });
}

extern "C" int rlse_dense_workspace_size(int rows, int out_features, int in_features,
                                         size_t* bytes) {
  if (!bytes || rows < 0 || out_features <= 0 || in_features <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "dense_workspace_size: bad arguments");
  *bytes = dense_ws_words(rows, out_features / 16, in_features) * 4;
  return RLSE_OK;
}

extern "C" int rlse_qkv_proj(const void* x, const void* w_qkv, const void* b_qkv, void* q,
                             void* k, void* v, int rows, int hidden, int q_features,
                             int kv_features, int dtype, void* workspace, size_t workspace_bytes,
                             rlse_stream_t stream) {
  DenseParams flags{};
  take_packed(dtype, flags);
  const void* outs[3] = {q, k, v};
  int rc = check_dense("qkv_proj", dtype, rows, hidden, x, w_qkv, outs, 3);
  if (rc || rows == 0) return rc;
  if (q_features <= 0 || kv_features <= 0 || q_features % 16 || kv_features % 16)
    return fail(RLSE_ERR_INVALID_VALUE,
                "qkv_proj: q_features %d and kv_features %d must be positive multiples of 16",
                q_features, kv_features);
  if (b_qkv && !aligned(b_qkv, 8))
    return fail(RLSE_ERR_INVALID_VALUE, "qkv_proj: bias must be 8-byte aligned");
  DenseParams p{};
  p.x = x;
  p.w = w_qkv;
  p.bias = b_qkv;
  p.out0 = q;
  p.out1 = k;
  p.out2 = v;
  p.rows = rows;
  p.K = hidden;
  p.n1 = q_features;
  p.n2 = q_features + kv_features;
  p.N = q_features + 2 * kv_features;
  p.packed = flags.packed;
  p.xpacked = flags.xpacked;
  size_t words = 0;
  rc = dense_workspace("qkv_proj", p, workspace, workspace_bytes, &words);
  if (rc) return rc;
  return dense_by_dtype<kEpiQkv>(dtype, p, hidden, q_features, kv_features, kv_features, words,
                                 as_stream(stream));
}

extern "C" int rlse_linear_residual(const void* x, const void* weight, void* residual, int rows,
                                    int out_features, int in_features, int dtype,
                                    void* workspace, size_t workspace_bytes,
                                    rlse_stream_t stream) {
  DenseParams flags{};
  take_packed(dtype, flags);
  const void* outs[1] = {residual};
  int rc = check_dense("linear_residual", dtype, rows, in_features, x, weight, outs, 1);
  if (rc || rows == 0) return rc;
  if (out_features <= 0 || out_features % 16)
    return fail(RLSE_ERR_INVALID_VALUE,
                "linear_residual: out_features %d must be a positive multiple of 16",
                out_features);
  DenseParams p{};
  p.x = x;
  p.w = weight;
  p.out0 = residual;
  p.rows = rows;
  p.K = in_features;
  p.N = out_features;
  p.packed = flags.packed;
  p.xpacked = flags.xpacked;
  size_t words = 0;
  rc = dense_workspace("linear_residual", p, workspace, workspace_bytes, &words);
  if (rc) return rc;
  return dense_by_dtype<kEpiResidual>(dtype, p, in_features, out_features, 0, 0, words,
                                      as_stream(stream));
}

extern "C" int rlse_gate_up_silu(const void* x, const void* w_gate_up, void* act, int rows,
                                 int hidden, int inter, int dtype, void* workspace,
                                 size_t workspace_bytes, rlse_stream_t stream) {
  DenseParams flags{};
  take_packed(dtype, flags);
  const void* outs[1] = {act};
  int rc = check_dense("gate_up_silu", dtype, rows, hidden, x, w_gate_up, outs, 1);
  if (rc || rows == 0) return rc;
  if (inter <= 0 || inter % 8)
    return fail(RLSE_ERR_INVALID_VALUE,
                "gate_up_silu: intermediate size %d must be a positive multiple of 8", inter);
  if (flags.opacked && (inter % 32 || !aligned(act, 16)))
    return fail(RLSE_ERR_INVALID_VALUE,
                "gate_up_silu: packed act needs inter a multiple of 32 (%d) and 16-byte alignment",
                inter);
  DenseParams p{};
  p.x = x;
  p.w = w_gate_up;
  p.out0 = act;
  p.rows = rows;
  p.K = hidden;
  p.N = 2 * inter;
  p.n1 = inter;
  p.packed = flags.packed;
  p.xpacked = flags.xpacked;
  p.opacked = flags.opacked;
  size_t words = 0;
  rc = dense_workspace("gate_up_silu", p, workspace, workspace_bytes, &words);
  if (rc) return rc;
  return dense_by_dtype<kEpiSiluMul>(dtype, p, hidden, inter, 0, 0, words, as_stream(stream));
}

extern "C" int rlse_dense_pack(const void* weight, void* packed, int out_features,
                               int in_features, int gate_up_inter, int dtype,
                               rlse_stream_t stream) {
  if (dtype != RLSE_DTYPE_BF16 && dtype != RLSE_DTYPE_F16)
    return fail(RLSE_ERR_INVALID_VALUE, "dense_pack: bf16 or f16 only");
  if (out_features <= 0 || in_features <= 0 || in_features % 32 || gate_up_inter < 0)
    return fail(RLSE_ERR_INVALID_VALUE,
                "dense_pack: out_features %d, in_features %d (a multiple of 32)", out_features,
                in_features);
  if (gate_up_inter > 0 ? (out_features != 2 * gate_up_inter || gate_up_inter % 8)
                        : out_features % 16)
    return fail(RLSE_ERR_INVALID_VALUE,
                "dense_pack: out_features %d must be a multiple of 16, or 2 * gate_up_inter "
                "with gate_up_inter %d a multiple of 8", out_features, gate_up_inter);
  if (!weight || !packed || weight == packed)
    return fail(RLSE_ERR_INVALID_VALUE, "dense_pack: null or in-place buffers");
  if (!aligned(weight, 16) || !aligned(packed, 16))
    return fail(RLSE_ERR_INVALID_VALUE, "dense_pack: buffers must be 16-byte aligned");
  const long long packets = (long long)out_features * in_features / 8;
  const dim3 grid((unsigned)((packets + 255) / 256));
  if (dtype == RLSE_DTYPE_BF16)
    hipLaunchKernelGGL(dense_pack_kernel<bf16>, grid, dim3(256), 0, as_stream(stream),
                       (const bf16*)weight, (bf16*)packed, in_features, gate_up_inter, packets);
  else
    hipLaunchKernelGGL(dense_pack_kernel<f16>, grid, dim3(256), 0, as_stream(stream),
                       (const f16*)weight, (f16*)packed, in_features, gate_up_inter, packets);
  return launch_status("dense_pack");
}
