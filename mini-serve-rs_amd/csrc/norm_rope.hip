// RMSNorm, NeoX rotary embedding and the fused q/k-norm + RoPE + KV append
// that forms the front half of Attention::forward
// (src/backends/qwen2.rs:291-313).
//
// Numerics follow Candle's op sequence on the reference's CPU path:
//   RmsNorm::forward (qwen2.rs:68-75): x -> f32; var = sum(x^2) * (1/n);
//     x / sqrt(var + eps) -> dtype; then * weight in dtype.
//   apply_rope (qwen2.rs:133-142): x*cos and rotate_half(x)*sin are each
//     rounded to dtype, then added and rounded, with no fused multiply-add.
// The sum of squares follows one fixed order (sumsq_tree: 16-byte packets,
// then a pairwise tree), the order of the fused decode step's q/k norm too,
// so cached K holds the same bytes whichever entry point wrote it.
//
// One wave handles one (token, head) row. For RoPE lane i holds the pair
// (x[i], x[i + d/2]) that rotate_half mixes, so no cross-lane traffic is
// needed beyond the norm's sum.
#include <math.h>
#include <string.h>

#include <type_traits>
#include <vector>

#include "common.cuh"
#include "host_common.h"

#pragma clang fp contract(off)

namespace rlse {

constexpr int kRowsPerBlock = 4;  // waves (rows) per 256-thread workgroup

template <typename T>
__device__ __forceinline__ float ld(const T* p, size_t i) {
  return Elem<T>::to_f32(p[i]);
}

template <typename T>
__device__ __forceinline__ void st(T* p, size_t i, float v) {
  p[i] = Elem<T>::from_f32(v);
}

// RMSNorm of one row held by one wave (M packets per lane in the sum of
// squares, see sumsq_tree).
template <typename T, int M>
__global__ __launch_bounds__(64 * kRowsPerBlock) void rmsnorm_kernel(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ out, int rows, int n,
    float inv_n, float eps) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * n;
  T* orow = out + row * n;
  const float ss = sumsq_tree<T, M>(xr, n);
  const float norm = sqrtf(ss * inv_n + eps);
  for (int i = lane; i < n; i += 64) {
    const float xn = round_to<T>(ld(xr, i) / norm);
    st(orow, i, xn * ld(w, i));
  }
}

// Applies (optional) RMSNorm with weight nw and then NeoX RoPE to a row of
// d elements read from src and written to dst. cs/sn are the table rows of
// the token's position (d/2 entries each).
template <typename T>
__device__ __forceinline__ void norm_rope_row(const T* __restrict__ src, T* __restrict__ dst,
                                              const T* __restrict__ nw, float inv_d, float eps,
                                              const T* __restrict__ cs,
                                              const T* __restrict__ sn, int d, bool do_rope) {
  const int lane = threadIdx.x & 63;
  const int half = d >> 1;
  constexpr int kMaxPairs = 4;  // d <= 512
  float x1[kMaxPairs], x2[kMaxPairs];
  int np = 0;
  for (int i = lane, k = 0; i < half && k < kMaxPairs; i += 64, ++k, ++np) {
    x1[k] = ld(src, i);
    x2[k] = ld(src, i + half);
  }
  if (nw) {
    // d <= 512: at most 128 packets (f32), two per lane
    const float ss = d * (int)sizeof(T) <= 1024 ? sumsq_tree<T, 1>(src, d)
                                                 : sumsq_tree<T, 2>(src, d);
    const float norm = sqrtf(ss * inv_d + eps);
    for (int k = 0; k < np; ++k) {
      const int i = lane + 64 * k;
      x1[k] = round_to<T>(round_to<T>(x1[k] / norm) * ld(nw, i));
      x2[k] = round_to<T>(round_to<T>(x2[k] / norm) * ld(nw, i + half));
    }
  }
  for (int k = 0; k < np; ++k) {
    const int i = lane + 64 * k;
    float y1 = x1[k], y2 = x2[k];
    if (do_rope) {
      const float c = ld(cs, i), s = ld(sn, i);
      y1 = round_to<T>(x1[k] * c) + round_to<T>(-x2[k] * s);
      y2 = round_to<T>(x2[k] * c) + round_to<T>(x1[k] * s);
    }
    st(dst, i, y1);
    st(dst, i + half, y2);
  }
}

// In-place RoPE of q rows then k rows.
template <typename T>
__global__ __launch_bounds__(64 * kRowsPerBlock) void rope_kernel(
    T* __restrict__ q, T* __restrict__ k, const T* __restrict__ cos_t,
    const T* __restrict__ sin_t, const int* __restrict__ positions, int num_tokens, int Hq,
    int Hkv, int d, int max_pos) {
  const long long row = (long long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const long long nq = q ? (long long)num_tokens * Hq : 0;
  const long long nk = k ? (long long)num_tokens * Hkv : 0;
  if (row >= nq + nk) return;
  int t;
  T* x;
  if (row < nq) {
    t = (int)(row / Hq);
    x = q + row * d;
  } else {
    t = (int)((row - nq) / Hkv);
    x = k + (row - nq) * d;
  }
  const int pos = positions[t];
  if (pos < 0 || pos >= max_pos) return;
  const size_t to = (size_t)pos * (d >> 1);
  norm_rope_row<T>(x, x, nullptr, 0.f, 0.f, cos_t + to, sin_t + to, d, true);
}

// Fused q/k RMSNorm + RoPE + append. Rows: num_tokens*Hq q rows, then
// num_tokens*Hkv k rows, then num_tokens*Hkv v rows (plain copies).
template <typename T>
__global__ __launch_bounds__(64 * kRowsPerBlock) void qk_norm_rope_append_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ qw, const T* __restrict__ kw, float inv_d, float eps,
    const T* __restrict__ cos_t, const T* __restrict__ sin_t, int max_pos,
    const int* __restrict__ positions, const int* __restrict__ tables, int num_seqs,
    const int* __restrict__ seq_index, int num_tokens, int Hq, int Hkv, int d, int mbps,
    int num_blocks, T* __restrict__ q_out, T* __restrict__ k_pool, T* __restrict__ v_pool) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const long long nq = (long long)num_tokens * Hq;
  const long long nkv = (long long)num_tokens * Hkv;
  if (row >= nq + 2 * nkv) return;
  int t;
  if (row < nq)
    t = (int)(row / Hq);
  else
    t = (int)(((row - nq) % nkv) / Hkv);
  const int pos = positions[t];
  const bool pos_ok = pos >= 0 && pos < max_pos;
  if (row < nq) {
    if (!pos_ok) return;
    const size_t to = (size_t)pos * (d >> 1);
    norm_rope_row<T>(q + row * d, q_out + row * d, qw, inv_d, eps, cos_t + to, sin_t + to, d,
                     true);
    return;
  }
  // K or V row: resolve the pool slot.
  const long long kr = (row - nq) % nkv;
  const bool is_v = (row - nq) >= nkv;
  const int h = (int)(kr % Hkv);
  const int seq = seq_index ? seq_index[t] : t;
  if (!pos_ok || seq < 0 || seq >= num_seqs || pos >= mbps * 16) return;
  const int blk = tables[(size_t)seq * mbps + (pos >> 4)];
  if ((unsigned)blk >= (unsigned)num_blocks) return;
  const size_t slot = (((size_t)blk * Hkv + h) * 16 + (pos & 15)) * d;
  if (is_v) {
    for (int i = lane; i < d; i += 64) v_pool[slot + i] = v[kr * d + i];
  } else {
    const size_t to = (size_t)pos * (d >> 1);
    norm_rope_row<T>(k + kr * d, k_pool + slot, kw, inv_d, eps, cos_t + to, sin_t + to, d,
                     true);
  }
}

static unsigned row_grid(long long rows) {
  return (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock);
}

}  // namespace rlse

using namespace rlse;

extern "C" int rlse_rmsnorm(const void* x, const void* weight, void* out, int rows, int n,
                            float eps, int dtype, rlse_stream_t stream) {
  if (rows <= 0 || n <= 0) return fail(RLSE_ERR_INVALID_VALUE, "rmsnorm: rows %d n %d", rows, n);
  if (!x || !weight || !out) return fail(RLSE_ERR_INVALID_VALUE, "rmsnorm: null pointer");
  if (!(eps >= 0.f)) return fail(RLSE_ERR_INVALID_VALUE, "rmsnorm: eps must be >= 0");
  const size_t es = dtype_size(dtype);
  if (es == 0) return fail(RLSE_ERR_INVALID_VALUE, "rmsnorm: bad dtype %d", dtype);
  const int m = sumsq_lane_packets(n, (int)es);
  if (m == 0)
    return fail(RLSE_ERR_INVALID_VALUE, "rmsnorm: n %d above %d elements", n,
                64 * 64 * (int)(16 / es));
  const float inv_n = (float)(1.0 / (double)n);
  const dim3 grid(row_grid(rows)), block(64 * kRowsPerBlock);
  hipStream_t s = as_stream(stream);
  auto run = [&](auto t) {
    using T = decltype(t);
    auto go = [&](auto mc) {
      constexpr int M = decltype(mc)::value;
      hipLaunchKernelGGL((rmsnorm_kernel<T, M>), grid, block, 0, s, (const T*)x,
                         (const T*)weight, (T*)out, rows, n, inv_n, eps);
    };
    switch (m) {
      case 1: go(std::integral_constant<int, 1>{}); break;
      case 2: go(std::integral_constant<int, 2>{}); break;
      case 4: go(std::integral_constant<int, 4>{}); break;
      case 8: go(std::integral_constant<int, 8>{}); break;
      case 16: go(std::integral_constant<int, 16>{}); break;
      case 32: go(std::integral_constant<int, 32>{}); break;
      default: go(std::integral_constant<int, 64>{}); break;
    }
  };
  if (dtype == RLSE_DTYPE_F32)
    run(float{});
  else if (dtype == RLSE_DTYPE_BF16)
    run(bf16{});
  else
    run(f16{});
  return launch_status("rmsnorm");
}

extern "C" int launch_rmsnorm_f32(const float* d_x, const float* d_w, float* d_out,
                                  int num_rows, int hidden_size, float eps) {
  return rlse_rmsnorm(d_x, d_w, d_out, num_rows, hidden_size, eps, RLSE_DTYPE_F32, nullptr);
}
extern "C" int launch_rmsnorm_f16(const void* d_x, const void* d_w, void* d_out, int num_rows,
                                  int hidden_size, float eps) {
  return rlse_rmsnorm(d_x, d_w, d_out, num_rows, hidden_size, eps, RLSE_DTYPE_F16, nullptr);
}
extern "C" int launch_rmsnorm_bf16(const void* d_x, const void* d_w, void* d_out, int num_rows,
                                   int hidden_size, float eps) {
  return rlse_rmsnorm(d_x, d_w, d_out, num_rows, hidden_size, eps, RLSE_DTYPE_BF16, nullptr);
}

// Host bf16/f16 rounding (round to nearest even, NaN kept quiet).
static uint16_t host_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

extern "C" int rlse_rope_tables(double theta, int head_dim, int max_pos, int dtype,
                                void* cos_out, void* sin_out) {
  if (!(theta > 0.0) || head_dim <= 0 || head_dim % 2 || max_pos <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "rope_tables: bad arguments");
  if (!cos_out || !sin_out) return fail(RLSE_ERR_INVALID_VALUE, "rope_tables: null output");
  if (dtype_size(dtype) == 0) return fail(RLSE_ERR_INVALID_VALUE, "rope_tables: bad dtype");
  const int half = head_dim / 2;
  std::vector<float> inv_freq(half);
  // inv_freq[i] = 1f32 / (theta.powf(2i / d) as f32)   (qwen2.rs:94-97)
  for (int i = 0; i < half; ++i)
    inv_freq[i] = 1.0f / (float)pow(theta, (double)(2 * i) / (double)head_dim);
  for (long long t = 0; t < max_pos; ++t) {
    for (int i = 0; i < half; ++i) {
      const float f = (float)t * inv_freq[i];  // t.matmul(inv_freq), one f32 product
      const float c = cosf(f), s = sinf(f);
      const size_t o = (size_t)t * half + i;
      switch (dtype) {
        case RLSE_DTYPE_F32:
          ((float*)cos_out)[o] = c;
          ((float*)sin_out)[o] = s;
          break;
        case RLSE_DTYPE_BF16:
          ((uint16_t*)cos_out)[o] = host_f32_to_bf16(c);
          ((uint16_t*)sin_out)[o] = host_f32_to_bf16(s);
          break;
        default: {
          const _Float16 hc = (_Float16)c, hs = (_Float16)s;
          memcpy((uint16_t*)cos_out + o, &hc, 2);
          memcpy((uint16_t*)sin_out + o, &hs, 2);
        }
      }
    }
  }
  return RLSE_OK;
}

extern "C" int rlse_rope(void* q, void* k, const void* cos_table, const void* sin_table,
                         const int32_t* positions, int num_tokens, int num_heads,
                         int num_kv_heads, int head_dim, int max_pos, int dtype,
                         rlse_stream_t stream) {
  if (num_tokens < 0 || head_dim <= 0 || head_dim % 2 || head_dim > 512 || max_pos <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "rope: bad sizes");
  if ((q && num_heads <= 0) || (k && num_kv_heads <= 0))
    return fail(RLSE_ERR_INVALID_VALUE, "rope: bad head counts");
  if (!cos_table || !sin_table || !positions)
    return fail(RLSE_ERR_INVALID_VALUE, "rope: null table/positions");
  const long long rows =
      (q ? (long long)num_tokens * num_heads : 0) + (k ? (long long)num_tokens * num_kv_heads : 0);
  if (rows == 0) return RLSE_OK;
  const dim3 grid(row_grid(rows)), block(64 * kRowsPerBlock);
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case RLSE_DTYPE_F32:
      hipLaunchKernelGGL(rope_kernel<float>, grid, block, 0, s, (float*)q, (float*)k,
                         (const float*)cos_table, (const float*)sin_table, positions,
                         num_tokens, num_heads, num_kv_heads, head_dim, max_pos);
      break;
    case RLSE_DTYPE_BF16:
      hipLaunchKernelGGL(rope_kernel<bf16>, grid, block, 0, s, (bf16*)q, (bf16*)k,
                         (const bf16*)cos_table, (const bf16*)sin_table, positions,
                         num_tokens, num_heads, num_kv_heads, head_dim, max_pos);
      break;
    case RLSE_DTYPE_F16:
      hipLaunchKernelGGL(rope_kernel<f16>, grid, block, 0, s, (f16*)q, (f16*)k,
                         (const f16*)cos_table, (const f16*)sin_table, positions, num_tokens,
                         num_heads, num_kv_heads, head_dim, max_pos);
      break;
    default:
      return fail(RLSE_ERR_INVALID_VALUE, "rope: bad dtype %d", dtype);
  }
  return launch_status("rope");
}

extern "C" int rlse_qk_norm_rope_append(
    const void* q, const void* k, const void* v, const void* q_norm_weight,
    const void* k_norm_weight, float eps, const void* cos_table, const void* sin_table,
    int max_pos, const int32_t* positions, const int32_t* block_tables, int num_seqs,
    const int32_t* seq_index, int num_tokens, int num_heads, int num_kv_heads, int head_dim,
    int max_blocks_per_seq, int num_blocks, void* q_out, void* k_pool, void* v_pool, int dtype,
    rlse_stream_t stream) {
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      head_dim % 2 || head_dim > 512 || max_pos <= 0 || max_blocks_per_seq <= 0 ||
      num_blocks <= 0 || num_seqs < 0)
    return fail(RLSE_ERR_INVALID_VALUE, "qk_norm_rope_append: bad sizes");
  if (!seq_index && num_seqs < num_tokens)
    return fail(RLSE_ERR_INVALID_VALUE, "qk_norm_rope_append: num_seqs < num_tokens");
  if (!(eps >= 0.f)) return fail(RLSE_ERR_INVALID_VALUE, "qk_norm_rope_append: eps < 0");
  if (num_tokens == 0) return RLSE_OK;
  if (!q || !k || !v || !cos_table || !sin_table || !positions || !block_tables || !q_out ||
      !k_pool || !v_pool)
    return fail(RLSE_ERR_INVALID_VALUE, "qk_norm_rope_append: null pointer argument");
  const long long rows = (long long)num_tokens * (num_heads + 2LL * num_kv_heads);
  const dim3 grid(row_grid(rows)), block(64 * kRowsPerBlock);
  const float inv_d = (float)(1.0 / (double)head_dim);
  hipStream_t s = as_stream(stream);
#define RLSE_QKNRA(T)                                                                         \
  hipLaunchKernelGGL(qk_norm_rope_append_kernel<T>, grid, block, 0, s, (const T*)q,          \
                     (const T*)k, (const T*)v, (const T*)q_norm_weight,                      \
                     (const T*)k_norm_weight, inv_d, eps, (const T*)cos_table,               \
                     (const T*)sin_table, max_pos, positions, block_tables, num_seqs,        \
                     seq_index, num_tokens, num_heads, num_kv_heads, head_dim,               \
                     max_blocks_per_seq, num_blocks, (T*)q_out, (T*)k_pool, (T*)v_pool)
  switch (dtype) {
    case RLSE_DTYPE_F32: RLSE_QKNRA(float); break;
    case RLSE_DTYPE_BF16: RLSE_QKNRA(bf16); break;
    case RLSE_DTYPE_F16: RLSE_QKNRA(f16); break;
    default: return fail(RLSE_ERR_INVALID_VALUE, "qk_norm_rope_append: bad dtype %d", dtype);
  }
#undef RLSE_QKNRA
  return launch_status("qk_norm_rope_append");
}
