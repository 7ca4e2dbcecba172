// Physical paged KV pool and its bit-exact data movement kernels: token
// append (scatter of new rows into pages), snapshot gather/scatter between
// pages and the reference's contiguous [Hkv, len, d] layout, and whole-block
// copy-on-write copies.
//
// Every kernel moves 16-byte packets (head_dim * elem_size is a multiple of
// 16), one packet per thread, consecutive threads on consecutive packets of a
// row so each wave touches contiguous 1 KB runs. The pool of one layer is
// [num_blocks][Hkv][16][head_dim] for K and the same for V; the layers of a
// pool handle are interleaved as K0 V0 K1 V1 ... in one allocation.
#include <new>

#include "common.cuh"
#include "host_common.h"

namespace rlse {

constexpr int kCopyThreads = 256;

__device__ __forceinline__ bool valid_block(int id, int num_blocks) {
  return (unsigned)id < (unsigned)num_blocks;
}

// Append: one thread per (token, head, packet).
__global__ __launch_bounds__(kCopyThreads) void kv_append_kernel(
    const uint4* __restrict__ k_new, const uint4* __restrict__ v_new, uint4* __restrict__ k_pool,
    uint4* __restrict__ v_pool, const int* __restrict__ tables, int num_seqs,
    const int* __restrict__ seq_index, const int* __restrict__ positions, int num_tokens,
    int Hkv, int ppr, int mbps, int num_blocks) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long n = (long long)num_tokens * Hkv * ppr;
  if (idx >= n) return;
  const int c = (int)(idx % ppr);
  const long long r = idx / ppr;
  const int h = (int)(r % Hkv);
  const int t = (int)(r / Hkv);
  const int seq = seq_index ? seq_index[t] : t;
  if (seq < 0 || seq >= num_seqs) return;
  const int pos = positions[t];
  if (pos < 0 || pos >= mbps * 16) return;
  const int blk = tables[(size_t)seq * mbps + (pos >> 4)];
  if (!valid_block(blk, num_blocks)) return;
  const size_t dst = (((size_t)blk * Hkv + h) * 16 + (pos & 15)) * ppr + c;
  k_pool[dst] = k_new[idx];
  v_pool[dst] = v_new[idx];
}

// Gather: one thread per (layer, head, token, packet) of the contiguous output.
__global__ __launch_bounds__(kCopyThreads) void kv_gather_kernel(
    const uint4* __restrict__ k_pool, const uint4* __restrict__ v_pool,
    long long layer_stride_pk, int num_layers, const int* __restrict__ table, int len,
    uint4* __restrict__ k_out, uint4* __restrict__ v_out, int Hkv, int ppr, int num_blocks) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long n = (long long)num_layers * Hkv * len * ppr;
  if (idx >= n) return;
  const int c = (int)(idx % ppr);
  long long r = idx / ppr;
  const int t = (int)(r % len);
  r /= len;
  const int h = (int)(r % Hkv);
  const int layer = (int)(r / Hkv);
  const int blk = table[t >> 4];
  if (!valid_block(blk, num_blocks)) {
    k_out[idx] = make_uint4(0, 0, 0, 0);
    v_out[idx] = make_uint4(0, 0, 0, 0);
    return;
  }
  const size_t src =
      (size_t)layer * layer_stride_pk + (((size_t)blk * Hkv + h) * 16 + (t & 15)) * ppr + c;
  k_out[idx] = k_pool[src];
  v_out[idx] = v_pool[src];
}

// Scatter: inverse of gather, writing positions start .. start+len-1.
__global__ __launch_bounds__(kCopyThreads) void kv_scatter_kernel(
    const uint4* __restrict__ k_in, const uint4* __restrict__ v_in, uint4* __restrict__ k_pool,
    uint4* __restrict__ v_pool, long long layer_stride_pk, int num_layers,
    const int* __restrict__ table, int start, int len, int Hkv, int ppr, int num_blocks) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long n = (long long)num_layers * Hkv * len * ppr;
  if (idx >= n) return;
  const int c = (int)(idx % ppr);
  long long r = idx / ppr;
  const int t = (int)(r % len);
  r /= len;
  const int h = (int)(r % Hkv);
  const int layer = (int)(r / Hkv);
  const int pos = start + t;
  const int blk = table[pos >> 4];
  if (!valid_block(blk, num_blocks)) return;
  const size_t dst =
      (size_t)layer * layer_stride_pk + (((size_t)blk * Hkv + h) * 16 + (pos & 15)) * ppr + c;
  k_pool[dst] = k_in[idx];
  v_pool[dst] = v_in[idx];
}

// Whole-block copies: one thread per (pair, layer, packet of a block).
__global__ __launch_bounds__(kCopyThreads) void kv_copy_blocks_kernel(
    uint4* __restrict__ k_pool, uint4* __restrict__ v_pool, long long layer_stride_pk,
    int num_layers, const int* __restrict__ src_blocks, const int* __restrict__ dst_blocks,
    int num_pairs, long long block_pk, int num_blocks) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long n = (long long)num_pairs * num_layers * block_pk;
  if (idx >= n) return;
  const long long c = idx % block_pk;
  const long long r = idx / block_pk;
  const int layer = (int)(r % num_layers);
  const int pr = (int)(r / num_layers);
  const int s = src_blocks[pr], d = dst_blocks[pr];
  if (!valid_block(s, num_blocks) || !valid_block(d, num_blocks)) return;
  const size_t lo = (size_t)layer * layer_stride_pk;
  k_pool[lo + (size_t)d * block_pk + c] = k_pool[lo + (size_t)s * block_pk + c];
  v_pool[lo + (size_t)d * block_pk + c] = v_pool[lo + (size_t)s * block_pk + c];
}

static unsigned grid_for(long long n) { return (unsigned)((n + kCopyThreads - 1) / kCopyThreads); }

// Packets per head_dim row, or 0 when the row is not a whole number of packets.
static int packets_per_row(int head_dim, int dtype) {
  const size_t es = dtype_size(dtype);
  if (es == 0 || head_dim <= 0) return 0;
  const size_t bytes = (size_t)head_dim * es;
  return bytes % 16 == 0 ? (int)(bytes / 16) : 0;
}

static int check_geom(const char* what, int num_kv_heads, int head_dim, int dtype,
                      int* ppr) {
  if (num_kv_heads <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "%s: num_kv_heads %d", what, num_kv_heads);
  *ppr = packets_per_row(head_dim, dtype);
  if (*ppr == 0)
    return fail(RLSE_ERR_INVALID_VALUE,
                "%s: head_dim %d x dtype %d is not a multiple of 16 bytes", what, head_dim,
                dtype);
  return RLSE_OK;
}

}  // namespace rlse

using namespace rlse;

struct rlse_kv_pool {
  void* base;
  int num_layers, num_blocks, num_kv_heads, head_dim, dtype;
  long long layer_elems;  // elements of one layer's K (or V) pool
};

extern "C" int rlse_pool_create(int num_layers, int num_blocks, int num_kv_heads, int head_dim,
                                int dtype, int block_size, rlse_kv_pool** out_pool) {
  if (!out_pool) return fail(RLSE_ERR_INVALID_VALUE, "pool_create: null output");
  *out_pool = nullptr;
  if (block_size != RLSE_BLOCK_SIZE)
    return fail(RLSE_ERR_INVALID_VALUE, "pool_create: block_size %d != 16", block_size);
  if (num_layers <= 0 || num_blocks <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "pool_create: layers %d / blocks %d", num_layers,
                num_blocks);
  int ppr = 0;
  int st = check_geom("pool_create", num_kv_heads, head_dim, dtype, &ppr);
  if (st) return st;
  const long long layer_elems = (long long)num_blocks * num_kv_heads * 16 * head_dim;
  const size_t bytes = (size_t)(2LL * num_layers * layer_elems) * dtype_size(dtype);
  void* base = nullptr;
  hipError_t e = hipMalloc(&base, bytes);
  if (e != hipSuccess)
    return fail((int)e, "pool_create: hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
  e = hipMemset(base, 0, bytes);
  if (e != hipSuccess) {
    (void)hipFree(base);
    return fail((int)e, "pool_create: hipMemset failed: %s", hipGetErrorString(e));
  }
  rlse_kv_pool* p = new (std::nothrow) rlse_kv_pool;
  if (!p) {
    (void)hipFree(base);
    return fail(RLSE_ERR_INVALID_VALUE, "pool_create: out of host memory");
  }
  p->base = base;
  p->num_layers = num_layers;
  p->num_blocks = num_blocks;
  p->num_kv_heads = num_kv_heads;
  p->head_dim = head_dim;
  p->dtype = dtype;
  p->layer_elems = layer_elems;
  *out_pool = p;
  return RLSE_OK;
}

extern "C" int rlse_pool_destroy(rlse_kv_pool* pool) {
  if (!pool) return fail(RLSE_ERR_INVALID_VALUE, "pool_destroy: null pool");
  hipError_t e = hipFree(pool->base);
  delete pool;
  if (e != hipSuccess) return fail((int)e, "pool_destroy: hipFree: %s", hipGetErrorString(e));
  return RLSE_OK;
}

extern "C" int rlse_pool_layer(const rlse_kv_pool* pool, int layer, void** k_pool,
                               void** v_pool) {
  if (!pool || !k_pool || !v_pool) return fail(RLSE_ERR_INVALID_VALUE, "pool_layer: null");
  if (layer < 0 || layer >= pool->num_layers)
    return fail(RLSE_ERR_INVALID_VALUE, "pool_layer: layer %d outside [0, %d)", layer,
                pool->num_layers);
  const size_t es = dtype_size(pool->dtype);
  char* b = reinterpret_cast<char*>(pool->base);
  *k_pool = b + (size_t)(2LL * layer) * pool->layer_elems * es;
  *v_pool = b + (size_t)(2LL * layer + 1) * pool->layer_elems * es;
  return RLSE_OK;
}

extern "C" int rlse_pool_info(const rlse_kv_pool* pool, int* num_layers, int* num_blocks,
                              int* num_kv_heads, int* head_dim, int* dtype,
                              long long* layer_stride_elems) {
  if (!pool) return fail(RLSE_ERR_INVALID_VALUE, "pool_info: null pool");
  if (num_layers) *num_layers = pool->num_layers;
  if (num_blocks) *num_blocks = pool->num_blocks;
  if (num_kv_heads) *num_kv_heads = pool->num_kv_heads;
  if (head_dim) *head_dim = pool->head_dim;
  if (dtype) *dtype = pool->dtype;
  if (layer_stride_elems) *layer_stride_elems = 2LL * pool->layer_elems;
  return RLSE_OK;
}

extern "C" int rlse_kv_append(const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                              const int32_t* block_tables, int num_seqs,
                              const int32_t* seq_index, const int32_t* positions,
                              int num_tokens, int num_kv_heads, int head_dim,
                              int max_blocks_per_seq, int num_blocks, int dtype,
                              rlse_stream_t stream) {
  int ppr = 0;
  int st = check_geom("kv_append", num_kv_heads, head_dim, dtype, &ppr);
  if (st) return st;
  if (num_tokens < 0 || num_seqs < 0 || max_blocks_per_seq <= 0 || num_blocks <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_append: bad sizes");
  if (!seq_index && num_seqs < num_tokens)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_append: num_seqs %d < num_tokens %d", num_seqs,
                num_tokens);
  if (num_tokens == 0) return RLSE_OK;
  if (!k_new || !v_new || !k_pool || !v_pool || !block_tables || !positions)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_append: null pointer argument");
  const long long n = (long long)num_tokens * num_kv_heads * ppr;
  hipLaunchKernelGGL(kv_append_kernel, dim3(grid_for(n)), dim3(kCopyThreads), 0,
                     as_stream(stream), (const uint4*)k_new, (const uint4*)v_new,
                     (uint4*)k_pool, (uint4*)v_pool, block_tables, num_seqs, seq_index,
                     positions, num_tokens, num_kv_heads, ppr, max_blocks_per_seq, num_blocks);
  return launch_status("kv_append");
}

static int check_layers(const char* what, long long layer_stride_elems, int num_layers,
                        int head_dim, int dtype, long long* stride_pk) {
  if (num_layers <= 0) return fail(RLSE_ERR_INVALID_VALUE, "%s: num_layers %d", what, num_layers);
  const long long bytes = layer_stride_elems * (long long)dtype_size(dtype);
  if (num_layers > 1 && (layer_stride_elems <= 0 || bytes % 16 != 0))
    return fail(RLSE_ERR_INVALID_VALUE, "%s: bad layer stride %lld", what, layer_stride_elems);
  *stride_pk = bytes / 16;
  (void)head_dim;
  return RLSE_OK;
}

extern "C" int rlse_kv_gather(const void* k_pool, const void* v_pool,
                              long long layer_stride_elems, int num_layers,
                              const int32_t* block_table, int len, void* k_out, void* v_out,
                              int num_kv_heads, int head_dim, int num_blocks, int dtype,
                              rlse_stream_t stream) {
  int ppr = 0;
  int st = check_geom("kv_gather", num_kv_heads, head_dim, dtype, &ppr);
  if (st) return st;
  long long stride_pk = 0;
  st = check_layers("kv_gather", layer_stride_elems, num_layers, head_dim, dtype, &stride_pk);
  if (st) return st;
  if (len < 0 || num_blocks <= 0) return fail(RLSE_ERR_INVALID_VALUE, "kv_gather: bad sizes");
  if (len == 0) return RLSE_OK;
  if (!k_pool || !v_pool || !block_table || !k_out || !v_out)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_gather: null pointer argument");
  const long long n = (long long)num_layers * num_kv_heads * len * ppr;
  hipLaunchKernelGGL(kv_gather_kernel, dim3(grid_for(n)), dim3(kCopyThreads), 0,
                     as_stream(stream), (const uint4*)k_pool, (const uint4*)v_pool, stride_pk,
                     num_layers, block_table, len, (uint4*)k_out, (uint4*)v_out, num_kv_heads,
                     ppr, num_blocks);
  return launch_status("kv_gather");
}

extern "C" int rlse_kv_scatter(const void* k_in, const void* v_in, void* k_pool, void* v_pool,
                               long long layer_stride_elems, int num_layers,
                               const int32_t* block_table, int start, int len,
                               int num_kv_heads, int head_dim, int num_blocks, int dtype,
                               rlse_stream_t stream) {
  int ppr = 0;
  int st = check_geom("kv_scatter", num_kv_heads, head_dim, dtype, &ppr);
  if (st) return st;
  long long stride_pk = 0;
  st = check_layers("kv_scatter", layer_stride_elems, num_layers, head_dim, dtype, &stride_pk);
  if (st) return st;
  if (len < 0 || start < 0 || num_blocks <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_scatter: bad sizes");
  if (len == 0) return RLSE_OK;
  if (!k_in || !v_in || !k_pool || !v_pool || !block_table)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_scatter: null pointer argument");
  const long long n = (long long)num_layers * num_kv_heads * len * ppr;
  hipLaunchKernelGGL(kv_scatter_kernel, dim3(grid_for(n)), dim3(kCopyThreads), 0,
                     as_stream(stream), (const uint4*)k_in, (const uint4*)v_in, (uint4*)k_pool,
                     (uint4*)v_pool, stride_pk, num_layers, block_table, start, len,
                     num_kv_heads, ppr, num_blocks);
  return launch_status("kv_scatter");
}

extern "C" int rlse_kv_copy_blocks(void* k_pool, void* v_pool, long long layer_stride_elems,
                                   int num_layers, const int32_t* src_blocks,
                                   const int32_t* dst_blocks, int num_pairs, int num_kv_heads,
                                   int head_dim, int num_blocks, int dtype,
                                   rlse_stream_t stream) {
  int ppr = 0;
  int st = check_geom("kv_copy_blocks", num_kv_heads, head_dim, dtype, &ppr);
  if (st) return st;
  long long stride_pk = 0;
  st = check_layers("kv_copy_blocks", layer_stride_elems, num_layers, head_dim, dtype,
                    &stride_pk);
  if (st) return st;
  if (num_pairs < 0 || num_blocks <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_copy_blocks: bad sizes");
  if (num_pairs == 0) return RLSE_OK;
  if (!k_pool || !v_pool || !src_blocks || !dst_blocks)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_copy_blocks: null pointer argument");
  const long long block_pk = (long long)num_kv_heads * 16 * ppr;
  const long long n = (long long)num_pairs * num_layers * block_pk;
  hipLaunchKernelGGL(kv_copy_blocks_kernel, dim3(grid_for(n)), dim3(kCopyThreads), 0,
                     as_stream(stream), (uint4*)k_pool, (uint4*)v_pool, stride_pk, num_layers,
                     src_blocks, dst_blocks, num_pairs, block_pk, num_blocks);
  return launch_status("kv_copy_blocks");
}
