// Split-K GQA decode attention over the paged KV pool (gfx950, wave64).
//
// Reference semantics: decode_attention_gqa_zero_copy
// (src/backends/qwen2.rs:177-203) -- for every KV head h, the G query heads
// h*G .. h*G+G-1 attend to that head's K/V with softmax(q K^T * scale) V --
// evaluated on the paged pool instead of a contiguous [Hkv, L, d] buffer.
//
// Work decomposition. The (sequence, KV head) rows are laid end to end as a
// single stream of 16-token blocks (row r = b*Hkv + h holds ceil(L_b/16)
// blocks). Worker w (one wave) takes the contiguous range
// [w*T/W, (w+1)*T/W) of that stream, so every worker streams the same number
// of bytes whatever the length mix. A worker walks its range one row segment
// at a time; all G query heads of the row are kept in registers so each K/V
// block is read from HBM exactly once (no repeat_kv). A row that lies wholly
// inside one worker is finished in place; a row cut by a range boundary
// leaves (m, l, acc) partials in the workspace and a second small kernel
// merges them with a log-sum-exp combine.
//
// Inside a wave a K/V block is read as 16-byte packets: LPR lanes cover one
// 16-token row's head_dim, RPL = 64/LPR rows are read per instruction and each
// lane owns NR = 16/RPL rows of the block. Scores are reduced over the LPR
// lanes of a row with DPP adds; each lane group keeps its own online-softmax
// state (running max m in log2 units, sum l, acc over its head_dim slice) and
// the groups are merged once per segment. Blocks are double-buffered in
// registers so the next block's loads are in flight during the math.
#include <math.h>

#include "common.cuh"
#include "host_common.h"

namespace rlse {

// Smallest number of blocks a worker is given (caps the number of partials
// when the batch is small).
constexpr int kMinBlocksPerWorker = 4;
// Largest batch handled per launch (prefix table lives in LDS).
constexpr int kMaxDecodeBatch = 16384;
// Workers launched per compute unit.
constexpr int kWorkersPerCU = 8;

template <typename T, int D>
struct DecodeShape {
  static constexpr int ES = sizeof(T);
  static constexpr int EPL = 16 / ES;   // elements per 16-byte packet
  static constexpr int LPR = D / EPL;   // lanes covering one K/V row
  static constexpr int RPL = 64 / LPR;  // rows per wave-wide packet load
  static constexpr int NR = 16 / RPL;   // packets per lane per 16-row block
  static_assert(D % EPL == 0, "head_dim must be a multiple of the packet size");
  static_assert(LPR >= 1 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "bad lanes per row");
  static_assert(RPL >= 1 && RPL <= 16, "bad rows per load");
};

__device__ __forceinline__ int clamp_len(int L, int mbps) {
  L = L < 0 ? 0 : L;
  const int cap = mbps * 16;
  return L > cap ? cap : L;
}

// Exclusive prefix of per-sequence block counts into s_pref[0..B]; returns
// the blocks of one KV head summed over the batch.
__device__ int block_prefix(const int* __restrict__ seq_lens, int B, int mbps,
                            int* s_pref) {
  const int lane = threadIdx.x;
  int carry = 0;
  for (int base = 0; base < B; base += 64) {
    const int b = base + lane;
    int nb = 0;
    if (b < B) nb = (clamp_len(seq_lens[b], mbps) + 15) >> 4;
    int x = nb;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (b < B) s_pref[b + 1] = carry + x;
    carry += __shfl(x, 63, 64);
  }
  if (lane == 0) s_pref[0] = 0;
  __syncthreads();
  return carry;
}

__device__ __forceinline__ long long effective_workers(long long total, int W) {
  long long we = total / kMinBlocksPerWorker;
  if (we < 1) we = 1;
  return we < W ? we : W;
}

__device__ __forceinline__ long long range_lo(long long w, long long total, long long we) {
  return (w * total) / we;
}

// Largest b in [0, B) with Hkv*s_pref[b] <= g (that sequence is non-empty).
__device__ __forceinline__ int locate_seq(const int* s_pref, int B, int Hkv, long long g) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((long long)Hkv * s_pref[mid] <= g)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// Floats of one partial record: acc[G][D], then m[G] and l[G], padded so
// records stay 16-byte aligned.
__host__ __device__ constexpr int rec_floats(int G, int D) { return G * D + ((2 * G + 3) & ~3); }

struct DecodeParams {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const int* tables;
  const int* seq_lens;
  void* out;
  float* ws;
  int B;
  int Hkv;
  int mbps;
  int num_blocks;
  int W;
  float c;  // scale * log2(e)
};

template <typename T, int D, int G>
struct Buf {
  uint4 k[DecodeShape<T, D>::NR];
  uint4 v[DecodeShape<T, D>::NR];
  int nvalid;  // valid rows (0 = block skipped)
};

template <typename T, int D, int G>
__global__ __launch_bounds__(64) void decode_split_kernel(DecodeParams p) {
  using S = DecodeShape<T, D>;
  constexpr int EPL = S::EPL, LPR = S::LPR, RPL = S::RPL, NR = S::NR;
  extern __shared__ int s_pref[];

  const int lane = threadIdx.x;
  const int col = lane % LPR;
  const int rsub = lane / LPR;
  const int B = p.B, Hkv = p.Hkv, mbps = p.mbps;
  const int Hq = Hkv * G;

  const int per_head = block_prefix(p.seq_lens, B, mbps, s_pref);
  const long long total = (long long)Hkv * per_head;
  if (total == 0) return;
  const long long we = effective_workers(total, p.W);
  const long long w = blockIdx.x;
  if (w >= we) return;
  long long lo = range_lo(w, total, we);
  const long long hi = range_lo(w + 1, total, we);

  const T* __restrict__ qb = reinterpret_cast<const T*>(p.q);
  const T* __restrict__ kp = reinterpret_cast<const T*>(p.k_pool);
  const T* __restrict__ vp = reinterpret_cast<const T*>(p.v_pool);
  const size_t tile = (size_t)16 * D;  // elements of one (block, head) tile
  const size_t lane_off = (size_t)rsub * D + (size_t)col * EPL;

  bool first_seg = true;
  while (lo < hi) {
    const int b = locate_seq(s_pref, B, Hkv, lo);
    const int nb = s_pref[b + 1] - s_pref[b];
    const long long o = lo - (long long)Hkv * s_pref[b];
    const int kvh = (int)(o / nb);
    const int blk0 = (int)(o % nb);
    const long long rem_row = nb - blk0;
    const int cnt = (int)((hi - lo) < rem_row ? (hi - lo) : rem_row);
    const int L = clamp_len(p.seq_lens[b], mbps);
    const int* __restrict__ trow = p.tables + (size_t)b * mbps + blk0;

    // Query packets of the G heads that share this KV head.
    uint4 qv[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
      qv[g] = *reinterpret_cast<const uint4*>(
          qb + ((size_t)b * Hq + (size_t)kvh * G + g) * D + (size_t)col * EPL);

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = -INFINITY;
      l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
    }

    // Physical ids of the segment's blocks, 64 at a time.
    int id_base = 0;
    int ids = lane < cnt ? trow[lane] : 0;
    auto issue = [&](Buf<T, D, G>& bf, int j) {
      if (j - id_base >= 64) {
        id_base += 64;
        ids = (id_base + lane) < cnt ? trow[id_base + lane] : 0;
      }
      const int id = __builtin_amdgcn_readlane(ids, j - id_base);
      int nv = L - (blk0 + j) * 16;
      nv = nv > 16 ? 16 : nv;
      if ((unsigned)id >= (unsigned)p.num_blocks) nv = 0;
      bf.nvalid = nv;
      if (nv > 0) {
        const size_t base = ((size_t)id * Hkv + kvh) * tile + lane_off;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          bf.k[i] = *reinterpret_cast<const uint4*>(kp + base + (size_t)i * RPL * D);
          bf.v[i] = *reinterpret_cast<const uint4*>(vp + base + (size_t)i * RPL * D);
        }
      }
    };
    auto compute = [&](const Buf<T, D, G>& bf) {
      const int nv = bf.nvalid;
      if (nv <= 0) return;
      float s[G][NR];
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < NR; ++i)
          s[g][i] = group_sum<LPR>(Packet<T>::dot(qv[g], bf.k[i], 0.f)) * p.c;
      float vf[NR][EPL];
#pragma unroll
      for (int i = 0; i < NR; ++i) Packet<T>::unpack(bf.v[i], vf[i]);
      if (nv < 16) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          if (i * RPL + rsub >= nv) {
#pragma unroll
            for (int g = 0; g < G; ++g) s[g][i] = -INFINITY;
#pragma unroll
            for (int e = 0; e < EPL; ++e) vf[i][e] = 0.f;
          }
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mx = m[g];
#pragma unroll
        for (int i = 0; i < NR; ++i) mx = fmaxf(mx, s[g][i]);
        const float ms = (mx == -INFINITY) ? 0.f : mx;
        const float alpha = __builtin_amdgcn_exp2f(m[g] - ms);
        float pr[NR];
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          pr[i] = __builtin_amdgcn_exp2f(s[g][i] - ms);
          psum += pr[i];
        }
        l[g] = fmaf(l[g], alpha, psum);
        m[g] = mx;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          float a = acc[g][e] * alpha;
#pragma unroll
          for (int i = 0; i < NR; ++i) a = fmaf(pr[i], vf[i][e], a);
          acc[g][e] = a;
        }
      }
    };

    Buf<T, D, G> bA, bB;
    issue(bA, 0);
    for (int j = 0;;) {
      issue(bB, j + 1 < cnt ? j + 1 : j);
      compute(bA);
      if (++j == cnt) break;
      issue(bA, j + 1 < cnt ? j + 1 : j);
      compute(bB);
      if (++j == cnt) break;
    }

    // Merge the RPL lane groups (each saw different rows of every block).
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float mo = __shfl_xor(m[g], off, 64);
        const float lo_ = __shfl_xor(l[g], off, 64);
        const float M = fmaxf(m[g], mo);
        const float Ms = (M == -INFINITY) ? 0.f : M;
        const float a = __builtin_amdgcn_exp2f(m[g] - Ms);
        const float bsc = __builtin_amdgcn_exp2f(mo - Ms);
        l[g] = l[g] * a + lo_ * bsc;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float ao = __shfl_xor(acc[g][e], off, 64);
          acc[g][e] = acc[g][e] * a + ao * bsc;
        }
        m[g] = M;
      }
    }

    const bool full_row = (blk0 == 0) && (cnt == nb);
    if (rsub == 0) {
      if (full_row) {
        T* ob = reinterpret_cast<T*>(p.out);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float inv = l[g] > 0.f ? 1.f / l[g] : 0.f;  // all pages skipped -> zeros
          T* dst = ob + ((size_t)b * Hq + (size_t)kvh * G + g) * D + (size_t)col * EPL;
#pragma unroll
          for (int e = 0; e < EPL; ++e) dst[e] = Elem<T>::from_f32(acc[g][e] * inv);
        }
      } else {
        const int slot = first_seg ? 0 : 1;
        float* rec = p.ws + ((size_t)w * 2 + slot) * (size_t)rec_floats(G, D);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float4* dst = reinterpret_cast<float4*>(rec + (size_t)g * D + (size_t)col * EPL);
#pragma unroll
          for (int e = 0; e < EPL; e += 4)
            dst[e / 4] = make_float4(acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]);
          if (col == 0) {
            rec[G * D + g] = m[g];
            rec[G * D + G + g] = l[g];
          }
        }
      }
    }
    first_seg = false;
    lo += cnt;
  }
}

// One wave per (sequence, KV head) row: combine the partials of rows that
// were cut by worker boundaries, and zero the rows of empty sequences.
template <typename T, int D, int G>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeParams p) {
  extern __shared__ int s_pref[];
  const int lane = threadIdx.x;
  const int B = p.B, Hkv = p.Hkv;
  const int Hq = Hkv * G;
  const int r = blockIdx.x;
  const int b = r / Hkv, kvh = r % Hkv;
  const int per_head = block_prefix(p.seq_lens, B, p.mbps, s_pref);
  const int nb = s_pref[b + 1] - s_pref[b];
  T* ob = reinterpret_cast<T*>(p.out) + ((size_t)b * Hq + (size_t)kvh * G) * D;
  if (nb == 0) {
    for (int i = lane; i < G * D; i += 64) ob[i] = Elem<T>::from_f32(0.f);
    return;
  }
  const long long total = (long long)Hkv * per_head;
  const long long we = effective_workers(total, p.W);
  const long long R = (long long)Hkv * s_pref[b] + (long long)kvh * nb;
  const long long wa = ((R + 1) * we - 1) / total;
  const long long wb = ((R + nb) * we - 1) / total;
  if (wa == wb) return;  // finished in place by the split kernel
  const long long lo_a = range_lo(wa, total, we);
  const size_t rec_stride = (size_t)rec_floats(G, D);
  for (int g = 0; g < G; ++g) {
    float M = -INFINITY;
    for (long long w = wa; w <= wb; ++w) {
      const int slot = (w == wa && lo_a != R) ? 1 : 0;
      const float* rec = p.ws + ((size_t)w * 2 + slot) * rec_stride;
      M = fmaxf(M, rec[G * D + g]);
    }
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float lsum = 0.f;
    float acc[(D + 63) / 64];
#pragma unroll
    for (int k = 0; k < (D + 63) / 64; ++k) acc[k] = 0.f;
    for (long long w = wa; w <= wb; ++w) {
      const int slot = (w == wa && lo_a != R) ? 1 : 0;
      const float* rec = p.ws + ((size_t)w * 2 + slot) * rec_stride;
      const float sc = __builtin_amdgcn_exp2f(rec[G * D + g] - Ms);
      lsum = fmaf(rec[G * D + G + g], sc, lsum);
#pragma unroll
      for (int k = 0; k < (D + 63) / 64; ++k) {
        const int d = lane + 64 * k;
        if (d < D) acc[k] = fmaf(rec[(size_t)g * D + d], sc, acc[k]);
      }
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
    for (int k = 0; k < (D + 63) / 64; ++k) {
      const int d = lane + 64 * k;
      if (d < D) ob[(size_t)g * D + d] = Elem<T>::from_f32(acc[k] * inv);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
static int decode_workers(int* W) {
  int cus = 0;
  int st = device_cu_count(&cus);
  if (st) return st;
  *W = cus * kWorkersPerCU;
  return RLSE_OK;
}

static size_t decode_ws_bytes(int W, int G, int D) {
  return (size_t)W * 2 * (size_t)rec_floats(G, D) * sizeof(float);
}

template <typename T, int D, int G>
static int launch_decode_t(const DecodeParams& p, hipStream_t stream) {
  const size_t lds = (size_t)(p.B + 1) * sizeof(int);
  hipLaunchKernelGGL((decode_split_kernel<T, D, G>), dim3(p.W), dim3(64), lds, stream, p);
  int st = launch_status("decode_split_kernel");
  if (st) return st;
  hipLaunchKernelGGL((decode_merge_kernel<T, D, G>), dim3(p.B * p.Hkv), dim3(64), lds, stream,
                     p);
  return launch_status("decode_merge_kernel");
}

template <typename T, int D>
static int launch_decode_g(int G, const DecodeParams& p, hipStream_t s) {
  switch (G) {
    case 1: return launch_decode_t<T, D, 1>(p, s);
    case 2: return launch_decode_t<T, D, 2>(p, s);
    case 3: return launch_decode_t<T, D, 3>(p, s);
    case 4: return launch_decode_t<T, D, 4>(p, s);
    case 5: return launch_decode_t<T, D, 5>(p, s);
    case 6: return launch_decode_t<T, D, 6>(p, s);
    case 7: return launch_decode_t<T, D, 7>(p, s);
    case 8: return launch_decode_t<T, D, 8>(p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode: unsupported group size %d", G);
}

template <typename T>
static int launch_decode_d(int D, int G, const DecodeParams& p, hipStream_t s) {
  switch (D) {
    case 64: return launch_decode_g<T, 64>(G, p, s);
    case 128: return launch_decode_g<T, 128>(G, p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode: unsupported head_dim %d", D);
}

// Library-owned workspace per device, for callers that pass none.
static void* g_ws_ptr[64] = {nullptr};
static size_t g_ws_size[64] = {0};

static int validate_decode(int batch, int num_heads, int num_kv_heads, int head_dim,
                           int max_blocks_per_seq, int num_blocks, int dtype) {
  if (batch <= 0 || batch > kMaxDecodeBatch)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: batch %d outside [1, %d]", batch,
                kMaxDecodeBatch);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: num_heads %d not a multiple of num_kv_heads %d",
                num_heads, num_kv_heads);
  const int G = num_heads / num_kv_heads;
  if (G > 8) return fail(RLSE_ERR_INVALID_VALUE, "decode: group size %d > 8", G);
  if (head_dim != 64 && head_dim != 128)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: head_dim %d not in {64, 128}", head_dim);
  if (max_blocks_per_seq <= 0 || num_blocks <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: max_blocks_per_seq %d / num_blocks %d",
                max_blocks_per_seq, num_blocks);
  if (dtype_size(dtype) == 0) return fail(RLSE_ERR_INVALID_VALUE, "decode: bad dtype %d", dtype);
  if ((long long)batch * num_heads * head_dim > (1LL << 40))
    return fail(RLSE_ERR_INVALID_VALUE, "decode: problem too large");
  return RLSE_OK;
}

}  // namespace rlse

using namespace rlse;

extern "C" int rlse_decode_workspace_size(int batch, int num_heads, int num_kv_heads,
                                          int head_dim, size_t* bytes) {
  if (!bytes) return fail(RLSE_ERR_INVALID_VALUE, "decode_workspace_size: null output");
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      head_dim <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_workspace_size: bad shape");
  int W = 0;
  int st = decode_workers(&W);
  if (st) return st;
  *bytes = decode_ws_bytes(W, num_heads / num_kv_heads, head_dim);
  return RLSE_OK;
}

extern "C" int rlse_paged_gqa_decode(const void* q, const void* k_pool, const void* v_pool,
                                     const int32_t* block_tables, const int32_t* seq_lens,
                                     void* out, int batch, int num_heads, int num_kv_heads,
                                     int head_dim, int max_blocks_per_seq, int num_blocks,
                                     float scale, int dtype, void* workspace,
                                     size_t workspace_bytes, rlse_stream_t stream) {
  int st = validate_decode(batch, num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                           num_blocks, dtype);
  if (st) return st;
  if (!q || !k_pool || !v_pool || !block_tables || !seq_lens || !out)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: null pointer argument");
  if (!(scale > 0.f) || !isfinite(scale))
    return fail(RLSE_ERR_INVALID_VALUE, "decode: scale must be finite and positive");
  int W = 0;
  st = decode_workers(&W);
  if (st) return st;
  const int G = num_heads / num_kv_heads;
  const size_t need = decode_ws_bytes(W, G, head_dim);
  if (workspace == nullptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64)
      return fail(RLSE_ERR_INVALID_VALUE, "decode: no current device");
    if (g_ws_size[dev] < need) {
      if (g_ws_ptr[dev]) (void)hipFree(g_ws_ptr[dev]);
      g_ws_ptr[dev] = nullptr;
      g_ws_size[dev] = 0;
      e = hipMalloc(&g_ws_ptr[dev], need);
      if (e != hipSuccess) return fail((int)e, "decode: workspace hipMalloc failed");
      g_ws_size[dev] = need;
    }
    workspace = g_ws_ptr[dev];
  } else if (workspace_bytes < need) {
    return fail(RLSE_ERR_BUFFER_TOO_SMALL, "decode: workspace %zu bytes < %zu needed",
                workspace_bytes, need);
  }
  DecodeParams p;
  p.q = q;
  p.k_pool = k_pool;
  p.v_pool = v_pool;
  p.tables = block_tables;
  p.seq_lens = seq_lens;
  p.out = out;
  p.ws = reinterpret_cast<float*>(workspace);
  p.B = batch;
  p.Hkv = num_kv_heads;
  p.mbps = max_blocks_per_seq;
  p.num_blocks = num_blocks;
  p.W = W;
  p.c = scale * 1.4426950408889634f;
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case RLSE_DTYPE_F32: return launch_decode_d<float>(head_dim, G, p, s);
    case RLSE_DTYPE_BF16: return launch_decode_d<bf16>(head_dim, G, p, s);
    case RLSE_DTYPE_F16: return launch_decode_d<f16>(head_dim, G, p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode: bad dtype %d", dtype);
}

static int compat_decode(const void* q, const void* k, const void* v, const int* tables,
                         const int* lens, void* out, int B, int Hq, int Hkv, int mbps,
                         float scale, int dtype) {
  return rlse_paged_gqa_decode(q, k, v, tables, lens, out, B, Hq, Hkv, 128, mbps, 0x7fffffff,
                               scale, dtype, nullptr, 0, nullptr);
}

extern "C" int launch_paged_gqa_decode_tiled_f32(const float* d_q, const float* d_k_pool,
                                                 const float* d_v_pool,
                                                 const int* d_block_tables,
                                                 const int* d_seq_lens, float* d_out,
                                                 int batch_size, int num_heads,
                                                 int num_kv_heads, int max_blocks_per_seq,
                                                 float scale) {
  return compat_decode(d_q, d_k_pool, d_v_pool, d_block_tables, d_seq_lens, d_out, batch_size,
                       num_heads, num_kv_heads, max_blocks_per_seq, scale, RLSE_DTYPE_F32);
}

extern "C" int launch_paged_gqa_decode_tiled_f16(const void* d_q, const void* d_k_pool,
                                                 const void* d_v_pool,
                                                 const int* d_block_tables,
                                                 const int* d_seq_lens, void* d_out,
                                                 int batch_size, int num_heads,
                                                 int num_kv_heads, int max_blocks_per_seq,
                                                 float scale) {
  return compat_decode(d_q, d_k_pool, d_v_pool, d_block_tables, d_seq_lens, d_out, batch_size,
                       num_heads, num_kv_heads, max_blocks_per_seq, scale, RLSE_DTYPE_F16);
}

extern "C" int launch_paged_gqa_decode_tiled_bf16(const void* d_q, const void* d_k_pool,
                                                  const void* d_v_pool,
                                                  const int* d_block_tables,
                                                  const int* d_seq_lens, void* d_out,
                                                  int batch_size, int num_heads,
                                                  int num_kv_heads, int max_blocks_per_seq,
                                                  float scale) {
  return compat_decode(d_q, d_k_pool, d_v_pool, d_block_tables, d_seq_lens, d_out, batch_size,
                       num_heads, num_kv_heads, max_blocks_per_seq, scale, RLSE_DTYPE_BF16);
}
