// Host side of the split-K GQA decode: argument checks, workspace, dispatch
// over (element type, head_dim, group size) and the C-ABI entry points. The
// kernel itself is in decode_kernel.cuh.
#include <math.h>

#include <mutex>

#include "decode_kernel.cuh"

namespace rlse {

RLSE_DECODE_INSTANCES(extern template, float, kModePlain)
RLSE_DECODE_INSTANCES(extern template, float, kModeFused)
RLSE_DECODE_INSTANCES(extern template, float, kModePlanned)
RLSE_DECODE_INSTANCES(extern template, float, kModePlannedStream)
RLSE_DECODE_INSTANCES(extern template, bf16, kModePlain)
RLSE_DECODE_INSTANCES(extern template, bf16, kModeFused)
RLSE_DECODE_INSTANCES(extern template, bf16, kModePlanned)
RLSE_DECODE_INSTANCES(extern template, bf16, kModePlannedStream)
RLSE_DECODE_INSTANCES(extern template, f16, kModePlain)
RLSE_DECODE_INSTANCES(extern template, f16, kModeFused)
RLSE_DECODE_INSTANCES(extern template, f16, kModePlanned)
RLSE_DECODE_INSTANCES(extern template, f16, kModePlannedStream)

// Per-step plan: for every wave of every workgroup of a decode launch, the
// descriptors of its first 64 blocks -- exactly what the wave would compute
// with the same lengths and tables (same prefix, ranges and block_desc) --
// followed, in a second array, by the new-token positions of the 64 rows
// from the wave's first row on (0 past the last row or for a wave without
// blocks), which rope its first query stage. One launch serves every layer
// of a step: the tables and lengths are the same in each.
__global__ __launch_bounds__(kThreads) void decode_plan_kernel(const int* __restrict__ tables,
                                                               const int* __restrict__ seq_lens,
                                                               int B, int Hkv, int mbps,
                                                               int num_blocks, int W, int w1,
                                                               int prefix,
                                                               const int* __restrict__ seq_pre,
                                                               int stamp,
                                                               int4* __restrict__ plan) {
  extern __shared__ int s_pref[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  if (wave == 0)
    block_prefix(seq_lens, B, mbps, s_pref, lane < B ? seq_lens[lane] : 0, prefix, seq_pre,
                 lane < B ? stream_skip(seq_pre, prefix, lane) : 0);
  __shared__ int s_bad;
  if (blockIdx.x == 0 && tid == 0) s_bad = 0;
  __syncthreads();
  if (blockIdx.x == 0) {
    // The one-prefix cascade contract, once for every layer of the step:
    // every sequence's first `prefix` table entries are sequence 0's, and
    // its length L has its new token past them and within its table
    // (16 prefix < L <= 16 mbps). The B x prefix entries are dealt over the
    // threads, four independent loads in flight per thread. (Prefix groups
    // are checked by the grouped plan.)
    bool bad = false;
    if (prefix > 0 && !seq_pre) {
      for (int b = tid; b < B; b += kThreads) {
        const int L = seq_lens[b];
        bad |= L <= 16 * prefix || L > 16 * mbps;
      }
      const int n = B * prefix;
      for (int e0 = tid; e0 < n; e0 += 4 * kThreads) {
        int a[4], z[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = e0 + u * kThreads < n ? e0 + u * kThreads : e0;
          const int b = e / prefix, i = e - b * prefix;
          a[u] = tables[(size_t)b * mbps + i];
          z[u] = tables[i];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) bad |= a[u] != z[u];
      }
    }
    if (__any(bad) && lane == 0) atomicOr(&s_bad, 1);
  }
  __syncthreads();
  if (blockIdx.x == 0 && tid == 0) {
    int* tail = const_cast<int*>(plan_tail(plan, W));
    tail[0] = stamp;
    tail[kPlanContractWord] = s_bad;
  }
  const long long w = blockIdx.x;
  const long long total = (long long)Hkv * s_pref[B];
  int4 d = make_int4(0, 0, -1, 0);
  if (total > 0) {
    const long long we = effective_groups(total, W);
    if (w < we) {
      const long long glo = range_lo(w, total, we, W, w1);
      const long long ghi = range_lo(w + 1, total, we, W, w1);
      const long long wlo = glo + (ghi - glo) * wave / kWaves;
      const long long whi = glo + (ghi - glo) * (wave + 1) / kWaves;
      d = block_desc(wlo + lane, whi, s_pref, tables, seq_lens, B, Hkv, mbps, num_blocks, prefix,
                     seq_pre);
    }
  }
  const size_t at = ((size_t)w * kWaves + wave) * 64 + lane;
  plan[at] = d;
  const int row0 = __shfl(d.z, 0, 64);
  int pos = 0;
  if (row0 >= 0 && row0 + lane < B * Hkv) {
    const int L = valid_len(seq_lens[(row0 + lane) / Hkv], mbps);
    pos = L > 0 ? L - 1 : 0;
  }
  reinterpret_cast<int*>(plan + (size_t)gridDim.x * kWaves * 64)[at] = pos;
}

// Grouped plan of a cascade step with prefix groups (one workgroup): from
// seq_group[b] (the prefix group of sequence b, -1 for none) and
// group_pages[g] (the pages group g's members share), into the plan's tail:
// each sequence's shared pages (0 for none), the grouped sequences group by
// group (in batch order within a group), the groups' member and column-tile
// offsets (G columns per member, 16 per tile) and pages. A group id outside
// [-1, NG) or a page count outside [1, min(mbps, kMaxPrefixPages)] sets the
// error word (the prefix launch raises RLSE_WS_ERR_PREFIX) and the sequence,
// or the group's members, are left unforked. So does a member that breaks
// its group's contract (error bit 4): its first P table entries must be the
// group's first member's and its length L within 16 P < L <= 16 mbps.
__global__ __launch_bounds__(1024) void group_plan_kernel(const int* __restrict__ seq_group,
                                                          const int* __restrict__ group_pages,
                                                          const int* __restrict__ tables,
                                                          const int* __restrict__ seq_lens,
                                                          int B, int NG, int G, int mbps,
                                                          int* __restrict__ tail) {
  __shared__ int s_cnt[kMaxPrefixGroups], s_pages[kMaxPrefixGroups], s_next[kMaxPrefixGroups];
  __shared__ int s_first[kMaxPrefixGroups], s_off[kMaxPrefixGroups + 1];
  __shared__ int s_tiles[kMaxPrefixGroups + 1], s_items[kMaxPrefixGroups + 1];
  __shared__ int s_err;
  int* seq_pre = tail + kPlanStampWords;
  int* members = seq_pre + kMaxDecodeBatch;
  int* grp = members + kMaxDecodeBatch;
  int4* items = reinterpret_cast<int4*>(grp + kGrpWords);
  int* item_rep = reinterpret_cast<int*>(items + kMaxGroupItems);
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid == 0) s_err = 0;
  if (tid < NG) {
    const int pg = group_pages[tid];
    const bool ok = pg >= 1 && pg <= mbps && pg <= kMaxPrefixPages;
    s_pages[tid] = ok ? pg : 0;
    s_cnt[tid] = 0;
    s_first[tid] = B;
  }
  __syncthreads();
  if (tid < NG && s_pages[tid] == 0) atomicOr(&s_err, 1);
  // A sequence's group, -1 when it has none or its group is invalid.
  auto group_of_seq = [&](int b) __attribute__((always_inline)) {
    const int g = seq_group[b];
    return (g >= 0 && g < NG && s_pages[g] > 0) ? g : -1;
  };
  for (int b = tid; b < B; b += 1024) {
    const int g = seq_group[b];
    if (g < -1 || g >= NG) atomicOr(&s_err, 2);
    const int gg = group_of_seq(b);
    if (gg >= 0) {
      atomicAdd(&s_cnt[gg], 1);
      atomicMin(&s_first[gg], b);
    }
    seq_pre[b] = gg >= 0 ? s_pages[gg] : 0;
  }
  __syncthreads();
  {
    // Each member against its group's first member: thread t takes
    // sequences t, t + 1024, ... (its length) and, for the table entries,
    // the members of four consecutive sequences at a time one entry column
    // per wave lane group -- independent loads, several in flight.
    bool bad = false;
    for (int b = tid; b < B; b += 1024) {
      const int gg = group_of_seq(b);
      if (gg < 0) continue;
      const int L = seq_lens[b], P = s_pages[gg];
      bad |= L <= 16 * P || L > 16 * mbps;
    }
    const int wave = tid >> 6;
    for (int b0 = 4 * wave; b0 < B; b0 += 4 * (1024 / 64)) {
      int P[4], f[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int gg = b0 + u < B ? group_of_seq(b0 + u) : -1;
        P[u] = gg >= 0 ? s_pages[gg] : 0;
        f[u] = gg >= 0 ? s_first[gg] : 0;
      }
      const int pmax = max(max(P[0], P[1]), max(P[2], P[3]));
      for (int i = lane; i < pmax; i += 64) {
        int a[4], z[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int ii = i < P[u] ? i : 0;
          const int bb = i < P[u] ? b0 + u : f[u];
          a[u] = tables[(size_t)bb * mbps + ii];
          z[u] = tables[(size_t)f[u] * mbps + ii];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) bad |= a[u] != z[u];
      }
    }
    if (__any(bad) && lane == 0) atomicOr(&s_err, 4);
  }
  __syncthreads();
  if (tid == 0) {
    int off = 0, tiles = 0, nitems = 0;
    for (int g = 0; g < NG; ++g) {
      grp[kGrpOff + g] = off;
      grp[kGrpTiles + g] = tiles;
      grp[kGrpPages + g] = s_pages[g];
      s_next[g] = s_off[g] = off;
      s_tiles[g] = tiles;
      s_items[g] = nitems;
      const int nt = (s_cnt[g] * G + 15) / 16;
      off += s_cnt[g];
      tiles += nt;
      nitems += nt * (s_cnt[g] > 0 ? prefix_splits(s_pages[g]) : 0);
    }
    grp[kGrpOff + NG] = s_off[NG] = off;
    grp[kGrpTiles + NG] = s_tiles[NG] = tiles;
    s_items[NG] = nitems;
    grp[kGrpErr] = s_err;
    grp[kGrpItems] = nitems;
  }
  __syncthreads();
  // The prefix launch's work items, slice-major within each group.
  for (int j = tid; j < s_items[NG]; j += 1024) {
    int g = 0;
    for (int k = 1; k < NG; ++k) g = s_items[k] <= j ? k : g;  // the last group starting at or before j
    const int nt = s_tiles[g + 1] - s_tiles[g], r = j - s_items[g];
    const int sp = r / nt, t = r - sp * nt;
    items[j] = make_int4(s_pages[g], t * 16, s_off[g], s_cnt[g]);
    item_rep[j] = s_first[g] | (sp << 16);
  }
  // Members in batch order within each group: wave 0 walks the batch 64
  // sequences at a time; the lanes of one group take consecutive slots.
  if (tid < 64) {
    for (int base = 0; base < B; base += 64) {
      const int b = base + lane;
      const int g = b < B ? group_of_seq(b) : -1;
      uint64_t pending = __ballot(g >= 0);
      while (pending) {
        const int g0 = __shfl(g, __builtin_ctzll(pending), 64);
        const uint64_t m = __ballot(g == g0);
        const int at = s_next[g0];
        if (g == g0) members[at + __builtin_popcountll(m & ((1ull << lane) - 1))] = b;
        if (lane == 0) s_next[g0] = at + __builtin_popcountll(m);
        pending &= ~m;
      }
    }
  }
}

static int decode_groups(int* W) {
  int cus = 0;
  int st = device_cu_count(&cus);
  if (st) return st;
  *W = cus * kGroupsPerCU;
  return RLSE_OK;
}

// Workspace: the header (sticky error flags), one launch counter per wave of
// the grid, then two tagged partial records per workgroup. Records carry
// their launch's epoch and need no clearing, so one zero-filled workspace
// stays valid across calls of any shape.
static size_t decode_ws_bytes(int W, int G, int D) {
  return (kWsHeaderWords + decode_ctr_words(W)) * sizeof(uint32_t) +
         (size_t)W * 2 * (size_t)rec_words(G, D) * sizeof(uint64_t);
}

// Points the kernel parameters at the parts of a workspace.
static void set_workspace(DecodeParams& p, void* workspace, int W) {
  uint32_t* base = reinterpret_cast<uint32_t*>(workspace);
  p.ws_err = base;
  p.ws_ctr = base + kWsHeaderWords;
  p.ws_rec = reinterpret_cast<uint64_t*>(base + kWsHeaderWords + decode_ctr_words(W));
  p.wait_ticks = merge_wait_ticks();
}

template <typename T, int D, int MODE>
static int launch_decode_g(int G, const DecodeParams& p, hipStream_t s) {
  switch (G) {
    case 1: return launch_decode_t<T, D, 1, MODE>(p, s);
    case 2: return launch_decode_t<T, D, 2, MODE>(p, s);
    case 3: return launch_decode_t<T, D, 3, MODE>(p, s);
    case 4: return launch_decode_t<T, D, 4, MODE>(p, s);
    case 5: return launch_decode_t<T, D, 5, MODE>(p, s);
    case 6: return launch_decode_t<T, D, 6, MODE>(p, s);
    case 7: return launch_decode_t<T, D, 7, MODE>(p, s);
    case 8: return launch_decode_t<T, D, 8, MODE>(p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode: unsupported group size %d", G);
}

template <typename T, int MODE>
static int launch_decode_d(int D, int G, const DecodeParams& p, hipStream_t s) {
  switch (D) {
    case 64: return launch_decode_g<T, 64, MODE>(G, p, s);
    case 128: return launch_decode_g<T, 128, MODE>(G, p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode: unsupported head_dim %d", D);
}

template <int MODE>
static int launch_decode_dtype(int dtype, int D, int G, const DecodeParams& p, hipStream_t s) {
  switch (dtype) {
    case RLSE_DTYPE_F32: return launch_decode_d<float, MODE>(D, G, p, s);
    case RLSE_DTYPE_BF16: return launch_decode_d<bf16, MODE>(D, G, p, s);
    case RLSE_DTYPE_F16: return launch_decode_d<f16, MODE>(D, G, p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode: bad dtype %d", dtype);
}

// Library-owned workspace per device, for callers that pass none. The mutex
// is held from the workspace lookup until the launch is queued, so a thread
// that grows (frees and reallocates) the buffer never frees one another
// thread is about to launch on; hipFree waits for launches already queued.
static void* g_ws_ptr[64] = {nullptr};
static size_t g_ws_size[64] = {0};
static std::mutex g_ws_mu;

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
  if ((long long)batch * num_kv_heads > kMaxDecodeRows)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: batch * num_kv_heads > %d", kMaxDecodeRows);
  if (head_dim != 64 && head_dim != 128)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: head_dim %d not in {64, 128}", head_dim);
  if (max_blocks_per_seq <= 0 || num_blocks <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: max_blocks_per_seq %d / num_blocks %d",
                max_blocks_per_seq, num_blocks);
  if (dtype_size(dtype) == 0) return fail(RLSE_ERR_INVALID_VALUE, "decode: bad dtype %d", dtype);
  if ((long long)max_blocks_per_seq * 16 > 0x7fffffffLL)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: max_blocks_per_seq too large");
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
  int st = decode_groups(&W);
  if (st) return st;
  *bytes = decode_ws_bytes(W, num_heads / num_kv_heads, head_dim);
  return RLSE_OK;
}

// Validates the shared decode arguments and fills p (workspace included).
// With a library-owned workspace, `lock` holds its mutex on return; the
// caller keeps it until the launch is queued.
#ifdef RLSE_DECODE_TIMELINE
// Measurement build: one timeline buffer per device, allocated and cleared
// on first use; every decode launch stamps it (see kTimelinePoints).
static unsigned long long* g_tl_ptr[64] = {nullptr};
static std::mutex g_tl_mu;
static unsigned long long* timeline_buffer() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(g_tl_mu);
  if (!g_tl_ptr[dev]) {
    const size_t bytes = (size_t)kTimelineMaxWaves * (kTimelinePoints + kPrefixTimelinePoints) *
                         sizeof(unsigned long long);
    void* ptr = nullptr;
    if (hipMalloc(&ptr, bytes) != hipSuccess) return nullptr;
    if (hipMemset(ptr, 0, bytes) != hipSuccess) return nullptr;
    g_tl_ptr[dev] = reinterpret_cast<unsigned long long*>(ptr);
  }
  return g_tl_ptr[dev];
}

// Copies the current device's timeline (kTimelineMaxWaves x kTimelinePoints
// stamps of the decode launches, then kTimelineMaxWaves x
// kPrefixTimelinePoints of the prefix launches; 100 MHz wall clock, 0 = not
// stamped since the last clear) into host (bytes at most) after the
// stream's work, then clears it when clear is nonzero. Exported by the
// measurement build only.
extern "C" int rlse_decode_timeline(void* host, size_t bytes, int clear, rlse_stream_t stream) {
  unsigned long long* tl = timeline_buffer();
  if (!tl) return fail(RLSE_ERR_INVALID_VALUE, "decode_timeline: no timeline buffer");
  const size_t all = (size_t)kTimelineMaxWaves * (kTimelinePoints + kPrefixTimelinePoints) *
                     sizeof(unsigned long long);
  hipStream_t s = as_stream(stream);
  hipError_t e = hipSuccess;
  if (host) e = hipMemcpyAsync(host, tl, bytes < all ? bytes : all, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess && clear) e = hipMemsetAsync(tl, 0, all, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return e == hipSuccess ? RLSE_OK : fail((int)e, "decode_timeline: copy or clear failed");
}
#endif

static int prepare_decode(DecodeParams& p, std::unique_lock<std::mutex>& lock, const void* q,
                          const void* k_pool, const void* v_pool, const int32_t* block_tables,
                          const int32_t* seq_lens, void* out, int batch, int num_heads,
                          int num_kv_heads, int head_dim, int max_blocks_per_seq, int num_blocks,
                          float scale, int dtype, void* workspace, size_t workspace_bytes) {
  int st = validate_decode(batch, num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                           num_blocks, dtype);
  if (st) return st;
  if (!q || !k_pool || !v_pool || !block_tables || !seq_lens || !out)
    return fail(RLSE_ERR_INVALID_VALUE, "decode: null pointer argument");
  if (!(scale > 0.f) || !isfinite(scale))
    return fail(RLSE_ERR_INVALID_VALUE, "decode: scale must be finite and positive");
  int W = 0;
  st = decode_groups(&W);
  if (st) return st;
  const int G = num_heads / num_kv_heads;
  const size_t need = decode_ws_bytes(W, G, head_dim);
  if (workspace == nullptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64)
      return fail(RLSE_ERR_INVALID_VALUE, "decode: no current device");
    lock = std::unique_lock<std::mutex>(g_ws_mu);
    if (g_ws_size[dev] < need) {
      if (g_ws_ptr[dev]) (void)hipFree(g_ws_ptr[dev]);
      g_ws_ptr[dev] = nullptr;
      g_ws_size[dev] = 0;
      e = hipMalloc(&g_ws_ptr[dev], need);
      if (e != hipSuccess) return fail((int)e, "decode: workspace hipMalloc failed");
      e = hipMemset(g_ws_ptr[dev], 0, need);
      if (e != hipSuccess) return fail((int)e, "decode: workspace hipMemset failed");
      g_ws_size[dev] = need;
    }
    workspace = g_ws_ptr[dev];
  } else if (workspace_bytes < need) {
    return fail(RLSE_ERR_BUFFER_TOO_SMALL, "decode: workspace %zu bytes < %zu needed",
                workspace_bytes, need);
  } else if ((uintptr_t)workspace % 8) {
    return fail(RLSE_ERR_INVALID_VALUE, "decode: workspace must be 8-byte aligned");
  }
  p = DecodeParams{};
  p.q = q;
  p.k_pool = k_pool;
  p.v_pool = v_pool;
  p.tables = block_tables;
  p.seq_lens = seq_lens;
  p.out = out;
  set_workspace(p, workspace, W);
  p.B = batch;
  p.Hkv = num_kv_heads;
  p.mbps = max_blocks_per_seq;
  p.num_blocks = num_blocks;
  p.W = W;
  p.w1 = kSlot1Weight;
  p.c = scale * 1.4426950408889634f;
#ifdef RLSE_DECODE_TIMELINE
  p.timeline = timeline_buffer();
#endif
  return RLSE_OK;
}

extern "C" int rlse_paged_gqa_decode(const void* q, const void* k_pool, const void* v_pool,
                                     const int32_t* block_tables, const int32_t* seq_lens,
                                     void* out, int batch, int num_heads, int num_kv_heads,
                                     int head_dim, int max_blocks_per_seq, int num_blocks,
                                     float scale, int dtype, void* workspace,
                                     size_t workspace_bytes, rlse_stream_t stream) {
  DecodeParams p;
  std::unique_lock<std::mutex> lock;
  const int st = prepare_decode(p, lock, q, k_pool, v_pool, block_tables, seq_lens, out, batch,
                                num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                                num_blocks, scale, dtype, workspace, workspace_bytes);
  if (st) return st;
  return launch_decode_dtype<kModePlain>(dtype, head_dim, num_heads / num_kv_heads, p,
                                         as_stream(stream));
}

extern "C" int rlse_decode_plan_size(size_t* bytes) {
  if (!bytes) return fail(RLSE_ERR_INVALID_VALUE, "decode_plan_size: null output");
  int W = 0;
  const int st = decode_groups(&W);
  if (st) return st;
  *bytes = plan_bytes(W);
  return RLSE_OK;
}

static int decode_plan_impl(const int32_t* block_tables, const int32_t* seq_lens, int batch,
                            int num_kv_heads, int max_blocks_per_seq, int num_blocks, int prefix,
                            void* plan, size_t plan_bytes, rlse_stream_t stream,
                            const int32_t* seq_group = nullptr,
                            const int32_t* group_pages = nullptr, int num_groups = 0,
                            int group_size = 1) {
  if (prefix < 0 || prefix > max_blocks_per_seq || prefix > kMaxPrefixPages)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_plan: prefix_pages %d outside [0, min(%d, %d)]",
                prefix, max_blocks_per_seq, kMaxPrefixPages);
  if (batch <= 0 || batch > kMaxDecodeBatch || num_kv_heads <= 0 ||
      (long long)batch * num_kv_heads > kMaxDecodeRows || max_blocks_per_seq <= 0 ||
      num_blocks <= 0 || (long long)max_blocks_per_seq * 16 > 0x7fffffffLL)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_plan: bad shape");
  if (!block_tables || !seq_lens || !plan)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_plan: null pointer argument");
  size_t need = 0;
  int st = rlse_decode_plan_size(&need);
  if (st) return st;
  if (plan_bytes < need || (uintptr_t)plan % 16)
    return fail(RLSE_ERR_BUFFER_TOO_SMALL, "decode_plan: %zu bytes (16-byte aligned) needed, %zu "
                                           "given", need, plan_bytes);
  int W = 0;
  st = decode_groups(&W);
  if (st) return st;
  int4* pl = reinterpret_cast<int4*>(plan);
  const int* seq_pre = nullptr;
  int stamp = plan_stamp(1, prefix);
  if (num_groups > 0) {
    int* tail = const_cast<int*>(plan_tail(pl, W));
    hipLaunchKernelGGL(group_plan_kernel, dim3(1), dim3(1024), 0, as_stream(stream), seq_group,
                       group_pages, block_tables, seq_lens, batch, num_groups, group_size,
                       max_blocks_per_seq, tail);
    st = launch_status("group_plan_kernel");
    if (st) return st;
    seq_pre = tail + kPlanStampWords;
    stamp = group_stamp(num_groups, group_size);
  }
  const size_t lds = (size_t)(batch + 1) * sizeof(int);
  hipLaunchKernelGGL(decode_plan_kernel, dim3(W), dim3(kThreads), lds, as_stream(stream),
                     block_tables, seq_lens, batch, num_kv_heads, max_blocks_per_seq, num_blocks,
                     W, kSlot1Weight, prefix, seq_pre, stamp, pl);
  return launch_status("decode_plan_kernel");
}

extern "C" int rlse_decode_plan(const int32_t* block_tables, const int32_t* seq_lens, int batch,
                                int num_kv_heads, int max_blocks_per_seq, int num_blocks,
                                void* plan, size_t plan_bytes, rlse_stream_t stream) {
  return decode_plan_impl(block_tables, seq_lens, batch, num_kv_heads, max_blocks_per_seq,
                          num_blocks, 0, plan, plan_bytes, stream);
}

extern "C" int rlse_decode_plan_cascade(const int32_t* block_tables, const int32_t* seq_lens,
                                        int batch, int num_kv_heads, int max_blocks_per_seq,
                                        int num_blocks, int prefix_pages, void* plan,
                                        size_t plan_bytes, rlse_stream_t stream) {
  return decode_plan_impl(block_tables, seq_lens, batch, num_kv_heads, max_blocks_per_seq,
                          num_blocks, prefix_pages, plan, plan_bytes, stream);
}

extern "C" int rlse_decode_plan_groups(const int32_t* block_tables, const int32_t* seq_lens,
                                       const int32_t* seq_group, const int32_t* group_pages,
                                       int num_groups, int batch, int num_heads,
                                       int num_kv_heads, int max_blocks_per_seq, int num_blocks,
                                       void* plan, size_t plan_bytes, rlse_stream_t stream) {
  if (num_groups < 1 || num_groups > kMaxPrefixGroups)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_plan_groups: num_groups %d outside [1, %d]",
                num_groups, kMaxPrefixGroups);
  if (!seq_group || !group_pages)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_plan_groups: null pointer argument");
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      num_heads / num_kv_heads > 8)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_plan_groups: bad head counts (group size <= 8)");
  return decode_plan_impl(block_tables, seq_lens, batch, num_kv_heads, max_blocks_per_seq,
                          num_blocks, 0, plan, plan_bytes, stream, seq_group, group_pages,
                          num_groups, num_heads / num_kv_heads);
}

extern "C" int rlse_decode_prefix_size(int batch, int num_heads, int head_dim,
                                       int prefix_pages, size_t* bytes) {
  if (!bytes) return fail(RLSE_ERR_INVALID_VALUE, "decode_prefix_size: null output");
  if (batch <= 0 || num_heads <= 0 || head_dim <= 0 || prefix_pages < 0 ||
      prefix_pages > kMaxPrefixPages)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_prefix_size: bad shape");
  // The slices' states, then the decode's parked row states.
  *bytes = (size_t)prefix_regions(prefix_pages) * batch * num_heads *
           prefix_row_floats(head_dim) * sizeof(float);
  return RLSE_OK;
}

static int decode_step_impl(const void* q, const void* k_new, const void* v_new,
                                const void* q_norm_weight, const void* k_norm_weight, float eps,
                                const void* cos_table, const void* sin_table, int max_pos,
                                void* k_pool, void* v_pool, const int32_t* block_tables,
                                const int32_t* seq_lens, void* out, int batch, int num_heads,
                                int num_kv_heads, int head_dim, int max_blocks_per_seq,
                                int num_blocks, float scale, int dtype, void* workspace,
                                size_t workspace_bytes, const void* plan, int flags,
                                int prefix, void* prefix_buf, size_t prefix_bytes,
                                rlse_stream_t stream, int num_groups = 0,
                                int max_group_pages = 0) {
  if (flags & ~RLSE_DECODE_STREAM)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_step: unknown flags 0x%x", flags);
  DecodeParams p;
  std::unique_lock<std::mutex> lock;
  const int st = prepare_decode(p, lock, q, k_pool, v_pool, block_tables, seq_lens, out, batch,
                                num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                                num_blocks, scale, dtype, workspace, workspace_bytes);
  if (st) return st;
  if (!k_new || !v_new || !cos_table || !sin_table)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_step: null pointer argument");
  if (!(eps >= 0.f)) return fail(RLSE_ERR_INVALID_VALUE, "decode_step: eps must be >= 0");
  if ((long long)max_pos < (long long)max_blocks_per_seq * 16)
    return fail(RLSE_ERR_INVALID_VALUE,
                "decode_step: max_pos %d < max_blocks_per_seq * 16 (%lld): every position the "
                "block table can hold needs a RoPE table row",
                max_pos, (long long)max_blocks_per_seq * 16);
  p.k_new = k_new;
  p.v_new = v_new;
  p.qw = q_norm_weight;
  p.kw = k_norm_weight;
  p.cos_t = cos_table;
  p.sin_t = sin_table;
  p.eps = eps;
  p.inv_d = (float)(1.0 / (double)head_dim);
  if (plan && (uintptr_t)plan % 16)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_step: plan must be 16-byte aligned");
  p.plan = reinterpret_cast<const int4*>(plan);
  const int G = num_heads / num_kv_heads;
  const hipStream_t s = as_stream(stream);
  p.plan_stamp = num_groups > 0 ? group_stamp(num_groups, G) : plan_stamp(1, prefix);
  const int* tail = plan ? plan_tail(p.plan, p.W) : nullptr;
  if (num_groups > 0) {
    // Prefix groups: every sequence's shared pages come from the plan, and
    // the bound max_group_pages sizes the prefix launch and buffer.
    if (!plan)
      return fail(RLSE_ERR_INVALID_VALUE, "decode_step_groups: a plan from "
                                          "rlse_decode_plan_groups is required");
    if (num_groups > kMaxPrefixGroups)
      return fail(RLSE_ERR_INVALID_VALUE, "decode_step_groups: num_groups %d > %d", num_groups,
                  kMaxPrefixGroups);
    if (max_group_pages < 1 || max_group_pages > max_blocks_per_seq ||
        max_group_pages > kMaxPrefixPages)
      return fail(RLSE_ERR_INVALID_VALUE,
                  "decode_step_groups: max_group_pages %d outside [1, min(%d, %d)]",
                  max_group_pages, max_blocks_per_seq, kMaxPrefixPages);
    prefix = max_group_pages;
  }
  if (prefix > 0) {
    // Cascade step: the shared prefix's partials first, on the same stream.
    if (dtype != RLSE_DTYPE_BF16 && dtype != RLSE_DTYPE_F16)
      return fail(RLSE_ERR_INVALID_VALUE, "decode_step_cascade: dtype %d (bf16/f16 only)", dtype);
    if (prefix > max_blocks_per_seq || prefix > kMaxPrefixPages)
      return fail(RLSE_ERR_INVALID_VALUE,
                  "decode_step_cascade: prefix_pages %d above min(max_blocks_per_seq %d, %d)",
                  prefix, max_blocks_per_seq, kMaxPrefixPages);
    size_t need = 0;
    int st2 = rlse_decode_prefix_size(batch, num_heads, head_dim, prefix, &need);
    if (st2) return st2;
    if (!prefix_buf || prefix_bytes < need || (uintptr_t)prefix_buf % 16)
      return fail(RLSE_ERR_BUFFER_TOO_SMALL,
                  "decode_step_cascade: prefix buffer of %zu bytes (16-byte aligned) needed, %zu "
                  "given", need, prefix_bytes);
    PrefixParams pp;
    pp.q = q;
    pp.k_pool = k_pool;
    pp.v_pool = v_pool;
    pp.tables = block_tables;
    pp.seq_lens = seq_lens;
    pp.qw = q_norm_weight;
    pp.cos_t = cos_table;
    pp.sin_t = sin_table;
    pp.eps = eps;
    pp.inv_d = p.inv_d;
    pp.c = p.c;
    pp.B = batch;
    pp.Hkv = num_kv_heads;
    pp.mbps = max_blocks_per_seq;
    pp.num_blocks = num_blocks;
    pp.prefix = prefix;
    pp.pre = reinterpret_cast<float*>(prefix_buf);
    pp.ws_err = p.ws_err;
    pp.members = nullptr;
    pp.grp = nullptr;
    pp.num_groups = 0;
    pp.tiles = 0;
    // A planned one-prefix step reads the plan's verdict on its contract.
    pp.contract = (plan && num_groups == 0)
                      ? plan_tail(reinterpret_cast<const int4*>(plan), p.W) + kPlanContractWord
                      : nullptr;
#ifdef RLSE_DECODE_TIMELINE
    pp.timeline = p.timeline ? p.timeline + (size_t)kTimelineMaxWaves * kTimelinePoints : nullptr;
#endif
    if (num_groups > 0) {
      const int* seq_pre = tail + kPlanStampWords;
      pp.members = seq_pre + kMaxDecodeBatch;
      pp.grp = pp.members + kMaxDecodeBatch;
      pp.num_groups = num_groups;
      pp.tiles = (batch * G + 15) / 16 + num_groups;  // each group adds at most one part tile
      p.seq_pre = seq_pre;
    }
    st2 = launch_decode_prefix(dtype, head_dim, G, pp, s);
    if (st2) return st2;
    p.prefix = num_groups > 0 ? 0 : prefix;
    p.pre = pp.pre;
    p.pre_slices = prefix_splits(prefix);
    p.pre_stride = (long long)batch * num_heads * prefix_row_floats(head_dim);
    p.pre_own = pp.pre + (size_t)p.pre_slices * p.pre_stride;
  }
  if (!plan) return launch_decode_dtype<kModeFused>(dtype, head_dim, G, p, s);
  return (flags & RLSE_DECODE_STREAM)
             ? launch_decode_dtype<kModePlannedStream>(dtype, head_dim, G, p, s)
             : launch_decode_dtype<kModePlanned>(dtype, head_dim, G, p, s);
}

extern "C" int rlse_decode_step(const void* q, const void* k_new, const void* v_new,
                                const void* q_norm_weight, const void* k_norm_weight, float eps,
                                const void* cos_table, const void* sin_table, int max_pos,
                                void* k_pool, void* v_pool, const int32_t* block_tables,
                                const int32_t* seq_lens, void* out, int batch, int num_heads,
                                int num_kv_heads, int head_dim, int max_blocks_per_seq,
                                int num_blocks, float scale, int dtype, void* workspace,
                                size_t workspace_bytes, rlse_stream_t stream) {
  return decode_step_impl(q, k_new, v_new, q_norm_weight, k_norm_weight, eps, cos_table,
                          sin_table, max_pos, k_pool, v_pool, block_tables, seq_lens, out, batch,
                          num_heads, num_kv_heads, head_dim, max_blocks_per_seq, num_blocks,
                          scale, dtype, workspace, workspace_bytes, nullptr, 0, 0, nullptr, 0,
                          stream);
}

extern "C" int rlse_decode_step_planned(
    const void* q, const void* k_new, const void* v_new, const void* q_norm_weight,
    const void* k_norm_weight, float eps, const void* cos_table, const void* sin_table,
    int max_pos, void* k_pool, void* v_pool, const int32_t* block_tables,
    const int32_t* seq_lens, void* out, int batch, int num_heads, int num_kv_heads, int head_dim,
    int max_blocks_per_seq, int num_blocks, float scale, int dtype, void* workspace,
    size_t workspace_bytes, const void* plan, int flags, rlse_stream_t stream) {
  if (!plan) return fail(RLSE_ERR_INVALID_VALUE, "decode_step_planned: null plan");
  return decode_step_impl(q, k_new, v_new, q_norm_weight, k_norm_weight, eps, cos_table,
                          sin_table, max_pos, k_pool, v_pool, block_tables, seq_lens, out, batch,
                          num_heads, num_kv_heads, head_dim, max_blocks_per_seq, num_blocks,
                          scale, dtype, workspace, workspace_bytes, plan, flags, 0, nullptr, 0,
                          stream);
}

extern "C" int rlse_decode_step_cascade(
    const void* q, const void* k_new, const void* v_new, const void* q_norm_weight,
    const void* k_norm_weight, float eps, const void* cos_table, const void* sin_table,
    int max_pos, void* k_pool, void* v_pool, const int32_t* block_tables,
    const int32_t* seq_lens, void* out, int batch, int num_heads, int num_kv_heads, int head_dim,
    int max_blocks_per_seq, int num_blocks, float scale, int dtype, void* workspace,
    size_t workspace_bytes, const void* plan, int flags, int prefix_pages, void* prefix_buf,
    size_t prefix_bytes, rlse_stream_t stream) {
  if (prefix_pages < 0)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_step_cascade: prefix_pages %d < 0", prefix_pages);
  return decode_step_impl(q, k_new, v_new, q_norm_weight, k_norm_weight, eps, cos_table,
                          sin_table, max_pos, k_pool, v_pool, block_tables, seq_lens, out, batch,
                          num_heads, num_kv_heads, head_dim, max_blocks_per_seq, num_blocks,
                          scale, dtype, workspace, workspace_bytes, plan, flags, prefix_pages,
                          prefix_buf, prefix_bytes, stream);
}

extern "C" int rlse_decode_step_groups(
    const void* q, const void* k_new, const void* v_new, const void* q_norm_weight,
    const void* k_norm_weight, float eps, const void* cos_table, const void* sin_table,
    int max_pos, void* k_pool, void* v_pool, const int32_t* block_tables,
    const int32_t* seq_lens, void* out, int batch, int num_heads, int num_kv_heads, int head_dim,
    int max_blocks_per_seq, int num_blocks, float scale, int dtype, void* workspace,
    size_t workspace_bytes, const void* plan, int flags, int num_groups, int max_group_pages,
    void* prefix_buf, size_t prefix_bytes, rlse_stream_t stream) {
  if (num_groups < 1)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_step_groups: num_groups %d < 1", num_groups);
  return decode_step_impl(q, k_new, v_new, q_norm_weight, k_norm_weight, eps, cos_table,
                          sin_table, max_pos, k_pool, v_pool, block_tables, seq_lens, out, batch,
                          num_heads, num_kv_heads, head_dim, max_blocks_per_seq, num_blocks,
                          scale, dtype, workspace, workspace_bytes, plan, flags, 0, prefix_buf,
                          prefix_bytes, stream, num_groups, max_group_pages);
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

// ---------------------------------------------------------------------------
// Allocation-free fused decode step (rlse_decode_step_noalloc). Its
// workspace is `scratch`, a file-scope device array sized for the largest
// decode workspace it serves: kStaticMaxGroups workgroups (2 per compute
// unit on a device of up to 256 CUs) and records of group size <= 8 at
// head_dim <= 128 -- 8.5 MB, held by every device the library runs on until
// the process ends. Like every static-storage object it starts zero-filled
// (error flags clear, launch counters equal, no record carrying an epoch);
// the kernels keep it consistent from then on. Host code never passes
// `scratch` itself to a kernel: each device holds its own copy at its own
// address, taken once per device with hipGetSymbolAddress and kept in
// g_scratch_ptr. Calls on one device share it, so calls that overlap on one
// device (different streams, different host threads) race.
// ---------------------------------------------------------------------------
constexpr int kStaticMaxGroups = 512;
constexpr size_t kScratchWords = kWsHeaderWords + decode_ctr_words(kStaticMaxGroups) +
                                 (size_t)kStaticMaxGroups * 2 * rec_words(8, 128) * 2;
static __device__ __align__(256) uint32_t scratch[kScratchWords];

static void* g_scratch_ptr[64] = {nullptr};
static std::mutex g_scratch_mu;

// The current device's copy of `scratch` (set up on the first call per
// device, with that device current).
static int scratch_address(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64)
    return fail(RLSE_ERR_INVALID_VALUE, "decode_step_noalloc: no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(e != hipSuccess ? (int)e : RLSE_ERR_INVALID_VALUE,
                  "decode_step_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return RLSE_OK;
}

extern "C" int rlse_decode_step_noalloc(
    const void* q, const void* k_new, const void* v_new, const void* q_norm_weight,
    const void* k_norm_weight, float eps, const void* cos_table, const void* sin_table,
    int max_pos, void* k_pool, void* v_pool, const int32_t* block_tables,
    const int32_t* seq_lens, void* out, int batch, int num_heads, int num_kv_heads, int head_dim,
    int max_blocks_per_seq, int num_blocks, float scale, int dtype, rlse_stream_t stream) {
  int st = validate_decode(batch, num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                           num_blocks, dtype);
  if (st) return st;
  int W = 0;
  st = decode_groups(&W);
  if (st) return st;
  if (W > kStaticMaxGroups)
    return fail(RLSE_ERR_INVALID_VALUE,
                "decode_step_noalloc: %d workgroups exceed the static scratch's %d", W,
                kStaticMaxGroups);
  const size_t need = decode_ws_bytes(W, num_heads / num_kv_heads, head_dim);
  if (need > sizeof(scratch))
    return fail(RLSE_ERR_INVALID_VALUE,
                "decode_step_noalloc: workspace of %zu bytes exceeds the static scratch (%zu)",
                need, sizeof(scratch));
  void* ws = nullptr;
  st = scratch_address(&ws);
  if (st) return st;
  return decode_step_impl(q, k_new, v_new, q_norm_weight, k_norm_weight, eps, cos_table,
                          sin_table, max_pos, k_pool, v_pool, block_tables, seq_lens, out, batch,
                          num_heads, num_kv_heads, head_dim, max_blocks_per_seq, num_blocks,
                          scale, dtype, ws, need, nullptr, 0, 0, nullptr, 0, stream);
}

extern "C" int rlse_workspace_check(void* workspace, rlse_stream_t stream, unsigned* flags) {
  if (flags) *flags = 0;
  hipStream_t s = as_stream(stream);
  if (workspace) return read_and_clear_ws_flags(workspace, s, flags);
  // The library's own decode workspaces of the current device: the
  // allocated one and the static scratch, each if a call has used it. Each
  // one's mutex is held until its flags are read and cleared, so a call
  // that grows the allocated workspace (hipFree, then hipMalloc) cannot free
  // it between the lookup and the clear.
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(RLSE_ERR_INVALID_VALUE, "workspace_check: no current device");
  int rc = RLSE_OK;
  auto check_one = [&](std::mutex& mu, void* const* slot) {
    std::lock_guard<std::mutex> lock(mu);
    if (!*slot) return;
    unsigned f = 0;
    const int r = read_and_clear_ws_flags(*slot, s, &f);
    if (flags) *flags |= f;
    if (rc == RLSE_OK || r == RLSE_ERR_DEVICE_TIMEOUT) rc = r ? r : rc;
  };
  check_one(g_ws_mu, &g_ws_ptr[dev]);
  check_one(g_scratch_mu, &g_scratch_ptr[dev]);
  return rc;
}
