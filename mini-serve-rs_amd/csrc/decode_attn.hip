// Split-K GQA decode attention over the paged KV pool (gfx950, wave64).
//
// Reference semantics: decode_attention_gqa_zero_copy
// (src/backends/qwen2.rs:177-203) -- for every KV head h, the G query heads
// h*G .. h*G+G-1 attend to that head's K/V with softmax(q K^T * scale) V --
// evaluated on the paged pool instead of a contiguous [Hkv, L, d] buffer.
//
// Work decomposition. The (sequence, KV head) rows are laid end to end as one
// stream of 16-token blocks (row r = b*Hkv + h holds ceil(L_b/16) blocks).
// Workgroup w -- a group of kWaves wavefronts -- takes the contiguous range
// [w*T/W, (w+1)*T/W) of that stream, so every workgroup streams the same number
// of bytes whatever the length mix. The group walks its range one row segment
// at a time; inside a segment its waves take interleaved blocks, each wave
// keeping all G query heads of the KV head in registers, so every K/V block
// is read from HBM exactly once (no repeat_kv) and shared by the G heads. The
// waves' online-softmax states (running max m in log2 units, sum l, acc) are
// combined through LDS. A row that lies wholly inside one group's range is
// finished there; a row cut by a range boundary leaves one (m, l, acc)
// partial per group in the workspace, and the group that finishes the row
// last (a per-row arrival counter) merges the partials with a log-sum-exp
// combine in the same launch. The counters return to zero after every
// launch, so a workspace only needs zero-filling once, before first use.
//
// Inside a wave a K/V block is read as 16-byte packets: LPR lanes cover one
// 16-token row's head_dim, RPL = 64/LPR rows are read per instruction and each
// lane owns NR = 16/RPL rows of the block. Scores are reduced over the LPR
// lanes of a row with DPP adds (bf16/f16 dot products with v_dot2); each lane
// group keeps its own online-softmax state and the groups are merged once per
// segment. Blocks are double-buffered in registers so the next block's loads
// are in flight during the math.
#include <math.h>

#include "common.cuh"
#include "host_common.h"

namespace rlse {

constexpr int kWaves = 4;               // wavefronts per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kGroupsPerCU = 2;         // workgroups launched per compute unit
constexpr int kMinBlocksPerGroup = 8;   // smallest share of blocks per workgroup
constexpr int kMaxDecodeBatch = 8192;   // prefix table lives in LDS
constexpr int kMaxDecodeRows = 65536;   // batch * num_kv_heads (arrival counters)
constexpr int kMergeChunk = 8;          // partials loaded per batch in a merge

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

// Exclusive prefix of per-sequence block counts into s_pref[0..B] (one wave).
__device__ void block_prefix(const int* __restrict__ seq_lens, int B, int mbps, int* s_pref) {
  const int lane = threadIdx.x & 63;
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
}

__device__ __forceinline__ long long effective_groups(long long total, int W) {
  long long we = total / kMinBlocksPerGroup;
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

// Partial records and arrival counters are accessed with device-scope
// (agent) atomic loads and stores: on gfx950 these carry the sc1 bit, so each
// access is coherent across the XCDs' L2 caches by itself. A group's record
// stores are therefore visible device-wide once they complete, and waiting for
// them (vmcnt(0)) before the counter increment orders them ahead of it -- no
// whole-L2 writeback or invalidate is needed (a __threadfence() would emit
// both, once per partial).
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima), fenced
// against compiler reordering on both sides.
__device__ __forceinline__ void wait_vm_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

struct DecodeParams {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const int* tables;
  const int* seq_lens;
  void* out;
  float* ws;      // partial records, two slots per workgroup
  int* counters;  // per-row arrival counters, zero between launches
  int B;
  int Hkv;
  int mbps;
  int num_blocks;
  int W;    // workgroups launched
  float c;  // scale * log2(e)
};

// Combines (m, l, a) with (mo, lo, ao), all in log2 units; -inf maxima mean
// "empty" and never produce NaN.
__device__ __forceinline__ void lse_combine(float& m, float& l, float& a, float mo, float lo,
                                            float ao) {
  const float M = fmaxf(m, mo);
  const float Ms = (M == -INFINITY) ? 0.f : M;
  const float sa = __builtin_amdgcn_exp2f(m - Ms);
  const float sb = __builtin_amdgcn_exp2f(mo - Ms);
  l = l * sa + lo * sb;
  a = a * sa + ao * sb;
  m = M;
}

template <typename T, int D>
struct Buf {
  uint4 k[DecodeShape<T, D>::NR];
  uint4 v[DecodeShape<T, D>::NR];
  int nvalid;  // valid rows of the block (0 = block skipped)
};

template <typename T, int D, int G>
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeParams p) {
  using S = DecodeShape<T, D>;
  constexpr int EPL = S::EPL, LPR = S::LPR, RPL = S::RPL, NR = S::NR;
  constexpr int REC = rec_floats(G, D);
  extern __shared__ int s_pref[];           // [B + 1]
  __shared__ float s_st[kWaves][G][D + 2];  // per wave: acc[D], m, l for each head
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int col = lane % LPR, rsub = lane / LPR;
  const int B = p.B, Hkv = p.Hkv, mbps = p.mbps;
  const int Hq = Hkv * G;
  T* __restrict__ ob = reinterpret_cast<T*>(p.out);

  if (wave == 0) block_prefix(p.seq_lens, B, mbps, s_pref);
  __syncthreads();
  const long long w = blockIdx.x;
  if (w == 0) {  // rows of sequences without keys produce zeros
    for (int b = 0; b < B; ++b) {
      if (s_pref[b + 1] != s_pref[b]) continue;
      for (int i = tid; i < Hq * D; i += kThreads)
        ob[(size_t)b * Hq * D + i] = Elem<T>::from_f32(0.f);
    }
  }
  const long long total = (long long)Hkv * s_pref[B];
  if (total == 0) return;
  const long long we = effective_groups(total, p.W);
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

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = -INFINITY;
      l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
    }

    // This wave's blocks of the segment: j = wave, wave + kWaves, ...
    const int mine = cnt > wave ? (cnt - wave + kWaves - 1) / kWaves : 0;
    if (mine > 0) {
      uint4 qv[G];  // query packets of the G heads sharing this KV head
#pragma unroll
      for (int g = 0; g < G; ++g)
        qv[g] = *reinterpret_cast<const uint4*>(
            qb + ((size_t)b * Hq + (size_t)kvh * G + g) * D + (size_t)col * EPL);
      int id_base = 0;
      int ids = lane < mine ? trow[wave + lane * kWaves] : 0;
      auto issue = [&](Buf<T, D>& bf, int i) {
        if (i - id_base >= 64) {
          id_base += 64;
          ids = (id_base + lane) < mine ? trow[wave + (id_base + lane) * kWaves] : 0;
        }
        const int id = __builtin_amdgcn_readlane(ids, i - id_base);
        int nv = L - (blk0 + wave + i * kWaves) * 16;
        nv = nv > 16 ? 16 : nv;
        if ((unsigned)id >= (unsigned)p.num_blocks) nv = 0;
        bf.nvalid = nv;
        if (nv > 0) {
          const size_t base = ((size_t)id * Hkv + kvh) * tile + lane_off;
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            bf.k[r] = *reinterpret_cast<const uint4*>(kp + base + (size_t)r * RPL * D);
            bf.v[r] = *reinterpret_cast<const uint4*>(vp + base + (size_t)r * RPL * D);
          }
        }
      };
      auto compute = [&](const Buf<T, D>& bf) {
        const int nv = bf.nvalid;
        if (nv <= 0) return;
        float s[G][NR];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int r = 0; r < NR; ++r)
            s[g][r] = group_sum<LPR>(Packet<T>::dot(qv[g], bf.k[r], 0.f)) * p.c;
        float vf[NR][EPL];
#pragma unroll
        for (int r = 0; r < NR; ++r) Packet<T>::unpack(bf.v[r], vf[r]);
        if (nv < 16) {  // tail block: mask rows past the sequence end
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            if (r * RPL + rsub >= nv) {
#pragma unroll
              for (int g = 0; g < G; ++g) s[g][r] = -INFINITY;
#pragma unroll
              for (int e = 0; e < EPL; ++e) vf[r][e] = 0.f;
            }
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float mx = m[g];
#pragma unroll
          for (int r = 0; r < NR; ++r) mx = fmaxf(mx, s[g][r]);
          const float ms = (mx == -INFINITY) ? 0.f : mx;
          const float alpha = __builtin_amdgcn_exp2f(m[g] - ms);
          float pr[NR];
          float psum = 0.f;
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            pr[r] = __builtin_amdgcn_exp2f(s[g][r] - ms);
            psum += pr[r];
          }
          l[g] = fmaf(l[g], alpha, psum);
          m[g] = mx;
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            float a = acc[g][e] * alpha;
#pragma unroll
            for (int r = 0; r < NR; ++r) a = fmaf(pr[r], vf[r][e], a);
            acc[g][e] = a;
          }
        }
      };

      Buf<T, D> bA, bB;
      issue(bA, 0);
      for (int i = 0;;) {
        issue(bB, i + 1 < mine ? i + 1 : i);
        compute(bA);
        if (++i == mine) break;
        issue(bA, i + 1 < mine ? i + 1 : i);
        compute(bB);
        if (++i == mine) break;
      }

      // Merge the RPL lane groups of the wave (each saw different rows).
#pragma unroll
      for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float mo = __shfl_xor(m[g], off, 64);
          const float lo_ = __shfl_xor(l[g], off, 64);
          const float M = fmaxf(m[g], mo);
          const float Ms = (M == -INFINITY) ? 0.f : M;
          const float sa = __builtin_amdgcn_exp2f(m[g] - Ms);
          const float sb = __builtin_amdgcn_exp2f(mo - Ms);
          l[g] = l[g] * sa + lo_ * sb;
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            const float ao = __shfl_xor(acc[g][e], off, 64);
            acc[g][e] = acc[g][e] * sa + ao * sb;
          }
          m[g] = M;
        }
      }
    }
    if (rsub == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) s_st[wave][g][col * EPL + e] = acc[g][e];
        if (col == 0) {
          s_st[wave][g][D] = m[g];
          s_st[wave][g][D + 1] = l[g];
        }
      }
    }
    __syncthreads();

    // Combine the waves: one thread per (head, dim) output element.
    const bool full_row = (blk0 == 0) && (cnt == nb);
    float* rec = p.ws + ((size_t)w * 2 + (first_seg ? 0 : 1)) * (size_t)REC;
    for (int idx = tid; idx < G * D; idx += kThreads) {
      const int g = idx / D, d = idx - g * D;
      float M = -INFINITY, ls = 0.f, a = 0.f;
#pragma unroll
      for (int wv = 0; wv < kWaves; ++wv)
        lse_combine(M, ls, a, s_st[wv][g][D], s_st[wv][g][D + 1], s_st[wv][g][d]);
      if (full_row) {
        const float inv = ls > 0.f ? 1.f / ls : 0.f;  // all pages skipped -> zeros
        ob[((size_t)b * Hq + (size_t)kvh * G + g) * D + d] = Elem<T>::from_f32(a * inv);
      } else {
        st_dev(rec + (size_t)g * D + d, a);
        if (d == 0) {
          st_dev(rec + G * D + g, M);
          st_dev(rec + G * D + G + g, ls);
        }
      }
    }

    if (!full_row) {
      // Publish the partial and count the arrival; the last of the row's np
      // groups merges. Records of group w: slot 0 = its first segment, slot 1
      // = a later one; group wa (holding the row's first block) used slot 0
      // only if its range starts exactly at the row start.
      const int row = b * Hkv + kvh;
      const long long R = (long long)Hkv * s_pref[b] + (long long)kvh * nb;
      const long long wa = ((R + 1) * we - 1) / total;
      const long long wb = ((R + nb) * we - 1) / total;
      const int np = (int)(wb - wa + 1);
      const bool wa_slot1 = range_lo(wa, total, we) != R;
      wait_vm_stores();
      __syncthreads();
      if (tid == 0)
        s_last = __hip_atomic_fetch_add(p.counters + row, 1, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == np - 1;
      __syncthreads();
      if (s_last) {
        for (int idx = tid; idx < G * D; idx += kThreads) {
          const int g = idx / D, d = idx - g * D;
          float M = -INFINITY, ls = 0.f, a = 0.f;
          for (int c = 0; c < np; c += kMergeChunk) {
            float mv[kMergeChunk], lv[kMergeChunk], av[kMergeChunk];
#pragma unroll
            for (int i = 0; i < kMergeChunk; ++i) {  // issue the chunk's loads together
              const int j = c + i < np ? c + i : np - 1;
              const int slot = (j == 0 && wa_slot1) ? 1 : 0;
              const float* r = p.ws + ((size_t)(wa + j) * 2 + slot) * (size_t)REC;
              mv[i] = ld_dev(r + G * D + g);
              lv[i] = ld_dev(r + G * D + G + g);
              av[i] = ld_dev(r + (size_t)g * D + d);
            }
#pragma unroll
            for (int i = 0; i < kMergeChunk; ++i)
              if (c + i < np) lse_combine(M, ls, a, mv[i], lv[i], av[i]);
          }
          const float inv = ls > 0.f ? 1.f / ls : 0.f;
          ob[((size_t)b * Hq + (size_t)kvh * G + g) * D + d] = Elem<T>::from_f32(a * inv);
        }
        if (tid == 0)
          __hip_atomic_store(p.counters + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();  // s_st and s_last are reused by the next segment
    first_seg = false;
    lo += cnt;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
static int decode_groups(int* W) {
  int cus = 0;
  int st = device_cu_count(&cus);
  if (st) return st;
  *W = cus * kGroupsPerCU;
  return RLSE_OK;
}

// Workspace: a fixed region of kMaxDecodeRows arrival counters, then two
// partial records per workgroup. The counter region does not depend on the
// call's shape, so one zero-filled workspace stays valid across calls of any
// batch.
static size_t decode_counter_bytes() { return (size_t)kMaxDecodeRows * sizeof(int); }
static size_t decode_ws_bytes(int W, int G, int D) {
  return decode_counter_bytes() + (size_t)W * 2 * (size_t)rec_floats(G, D) * sizeof(float);
}

template <typename T, int D, int G>
static int launch_decode_t(const DecodeParams& p, hipStream_t stream) {
  const size_t lds = (size_t)(p.B + 1) * sizeof(int);
  hipLaunchKernelGGL((decode_kernel<T, D, G>), dim3(p.W), dim3(kThreads), lds, stream, p);
  return launch_status("decode_kernel");
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
  st = decode_groups(&W);
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
      e = hipMemset(g_ws_ptr[dev], 0, need);
      if (e != hipSuccess) return fail((int)e, "decode: workspace hipMemset failed");
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
  p.counters = reinterpret_cast<int*>(workspace);
  p.ws = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + decode_counter_bytes());
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
