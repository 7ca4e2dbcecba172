// The rest of a batched decode step on the device: embedding gather, fused
// residual add + RMSNorm, the MLP activation, greedy argmax and the linear
// projections -- the ops of ModelForCausalLM::step_decode_batch
// (src/backends/qwen2.rs:628-764) around the attention of rlse_decode_step,
// so a step's activations and logits never leave HBM (the reference moves
// the logits to the host for sample_token, src/backends/candle.rs:737-751).
//
// Element-wise rounding follows Candle's per-op order on bf16/f16 tensors:
// every op computes in f32 and rounds its result to the tensor dtype.
#include <math.h>
#include <rocblas/rocblas.h>

#include <mutex>

#include "common.cuh"
#include "host_common.h"

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

// residual <- residual + x (rounded); out <- RmsNorm(residual) * w. One wave
// per row, the sum of squares in the order of rmsnorm_kernel.
template <typename T>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const T* __restrict__ x,
                                                          T* __restrict__ residual,
                                                          const T* __restrict__ w,
                                                          T* __restrict__ out, int rows, int n,
                                                          float inv_n, float eps) {
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * n;
  T* rr = residual + row * n;
  T* orow = out + row * n;
  float ss = 0.f;
  for (int i = lane; i < n; i += 64) {
    const float h = round_to<T>(Elem<T>::to_f32(rr[i]) + Elem<T>::to_f32(xr[i]));
    rr[i] = Elem<T>::from_f32(h);
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
__global__ void silu_mul_kernel(const T* __restrict__ gate_up, T* __restrict__ out, int rows,
                                int inter) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)rows * inter) return;
  const long long r = i / inter, c = i - r * inter;
  const float g = Elem<T>::to_f32(gate_up[r * 2 * inter + c]);
  const float u = Elem<T>::to_f32(gate_up[r * 2 * inter + inter + c]);
  const float e = round_to<T>(expf(-g));
  const float s = round_to<T>(g / round_to<T>(1.f + e));
  out[i] = Elem<T>::from_f32(s * u);
}

// y[r][c] = y[r][c] + bias[c], rounded (Candle's broadcast_add after matmul).
template <typename T>
__global__ void bias_add_kernel(T* __restrict__ y, const T* __restrict__ bias, int rows, int n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)rows * n) return;
  y[i] = Elem<T>::from_f32(Elem<T>::to_f32(y[i]) + Elem<T>::to_f32(bias[i % n]));
}

// Greedy argmax of one row per workgroup with the sequential scan's answer
// (Tensor::argmax on the host copy): the first index whose value exceeds
// every earlier one -- the first maximum; a NaN never wins, except that a NaN
// at index 0 wins outright (nothing compares greater than it).
constexpr int kArgThreads = 256;
template <typename T>
__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const T* __restrict__ logits,
                                                             int32_t* __restrict__ out,
                                                             int vocab) {
  const T* row = logits + (size_t)blockIdx.x * vocab;
  float best = -INFINITY;
  int idx = 0x7fffffff;
  for (int i = threadIdx.x; i < vocab; i += kArgThreads) {
    const float v = Elem<T>::to_f32(row[i]);
    if (v > best || (v == best && i < idx)) {  // NaN compares false: skipped
      best = v;
      idx = i;
    }
  }
  // (value, index) pairs: larger value wins, ties go to the smaller index.
  for (int off = 32; off > 0; off >>= 1) {
    const float ob = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (ob > best || (ob == best && oi < idx)) {
      best = ob;
      idx = oi;
    }
  }
  __shared__ float s_b[kArgThreads / 64];
  __shared__ int s_i[kArgThreads / 64];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_b[wave] = best;
    s_i[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgThreads / 64; ++w)
      if (s_b[w] > best || (s_b[w] == best && s_i[w] < idx)) {
        best = s_b[w];
        idx = s_i[w];
      }
    const float v0 = Elem<T>::to_f32(row[0]);
    // Every value was -inf or NaN: the scan keeps index 0; a NaN first
    // element wins outright.
    out[blockIdx.x] = (v0 != v0 || idx == 0x7fffffff) ? 0 : idx;
  }
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
  if (!dtype_size(dtype) || rows < 0 || n <= 0 || !(eps >= 0.f))
    return fail(RLSE_ERR_INVALID_VALUE, "add_rmsnorm: bad arguments");
  if (rows == 0) return RLSE_OK;
  if (!x || !residual || !weight || !out)
    return fail(RLSE_ERR_INVALID_VALUE, "add_rmsnorm: null pointer");
  const float inv_n = (float)(1.0 / (double)n);
  hipStream_t s = as_stream(stream);
  return by_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL(add_rmsnorm_kernel<T>, dim3((rows + 3) / 4), dim3(256), 0, s,
                       (const T*)x, (T*)residual, (const T*)weight, (T*)out, rows, n, inv_n,
                       eps);
    return launch_status("add_rmsnorm");
  });
}

extern "C" int rlse_silu_mul(const void* gate_up, void* out, int rows, int inter, int dtype,
                             rlse_stream_t stream) {
  if (!dtype_size(dtype) || rows < 0 || inter <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "silu_mul: bad arguments");
  if (rows == 0) return RLSE_OK;
  if (!gate_up || !out) return fail(RLSE_ERR_INVALID_VALUE, "silu_mul: null pointer");
  const long long n = (long long)rows * inter;
  hipStream_t s = as_stream(stream);
  return by_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL(silu_mul_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       (const T*)gate_up, (T*)out, rows, inter);
    return launch_status("silu_mul");
  });
}

extern "C" int rlse_argmax(const void* logits, int32_t* out, int rows, int vocab, int dtype,
                           rlse_stream_t stream) {
  if (!dtype_size(dtype) || rows < 0 || vocab <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "argmax: bad arguments");
  if (rows == 0) return RLSE_OK;
  if (!logits || !out) return fail(RLSE_ERR_INVALID_VALUE, "argmax: null pointer");
  hipStream_t s = as_stream(stream);
  return by_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL(argmax_kernel<T>, dim3(rows), dim3(kArgThreads), 0, s, (const T*)logits,
                       out, vocab);
    return launch_status("argmax");
  });
}

extern "C" int rlse_linear(const void* x, const void* weight, const void* bias, void* y,
                           int rows, int out_features, int in_features, int dtype,
                           rlse_stream_t stream) {
  if (!dtype_size(dtype) || rows < 0 || out_features <= 0 || in_features <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "linear: bad arguments");
  if (rows == 0) return RLSE_OK;
  if (!x || !weight || !y) return fail(RLSE_ERR_INVALID_VALUE, "linear: null pointer");
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
  hipStream_t s = as_stream(stream);
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
  const long long n = (long long)rows * out_features;
  return by_dtype(dtype, [&](auto tt) {
    using T = decltype(tt);
    hipLaunchKernelGGL(bias_add_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       (T*)y, (const T*)bias, rows, out_features);
    return launch_status("bias_add");
  });
}
