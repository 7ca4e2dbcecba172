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
// [w*T/W, (w+1)*T/W) of that stream and each of its waves a contiguous quarter
// of it, so every wave streams the same number of bytes whatever the length
// mix. A wave keeps all G query heads of the current KV head in registers, so
// every K/V block is read from HBM exactly once (no repeat_kv) and shared by
// the G heads. A row that lies wholly inside a wave's share is finished by the
// wave; pieces of rows cut between waves are parked in LDS and combined after
// one barrier at the end; rows cut by the group's range boundary leave one
// (m, l, acc) partial per group in the workspace, and the group that finishes
// such a row last (a per-row arrival counter) merges the partials with a
// log-sum-exp combine in the same launch. The counters return to zero after
// every launch, so a workspace only needs zero-filling once, before first use.
//
// Inside a wave a K/V block is read as 16-byte packets: LPR lanes cover one
// 16-token row's head_dim, RPL = 64/LPR rows are read per instruction and each
// lane owns NR = 16/RPL rows of the block. Scores are reduced over the LPR
// lanes of a row with DPP adds (bf16/f16 dot products with v_dot2); each lane
// group keeps its own online-softmax state (running max m in log2 units, sum
// l, acc) and the groups are merged when the wave's part of a row ends. The
// page ids of 64 blocks are fetched at once (one per lane), blocks are
// double-buffered in registers so the next block's loads -- and the query of
// a new row -- are in flight during the math, and no barrier is taken while
// streaming.
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
// The running max of a softmax moves only when a score exceeds it by more
// than this many powers of two.
constexpr float kLazyLog2 = 8.f;

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
  // Fused decode step only (rlse_decode_step): raw new-token k/v
  // [B][Hkv][D], q/k RMSNorm weights [D] (null: no norm), RoPE tables
  // [max_pos][D/2]. The new token of sequence b sits at seq_lens[b] - 1.
  const void* k_new;
  const void* v_new;
  const void* qw;
  const void* kw;
  const void* cos_t;
  const void* sin_t;
  float eps;
  float inv_d;
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

template <typename T, int D, int G>
struct Buf {
  uint4 k[DecodeShape<T, D>::NR];
  uint4 v[DecodeShape<T, D>::NR];
  uint4 q[G];   // query packets, loaded with the first block of a row
  uint4 cs, sn; // fused step: RoPE cos/sin packets of the row's new token
  uint4 kn, vn; // fused step: raw new-token k/v packets (last block of a row)
  int nvalid;   // valid rows of the block (0 = block skipped)
  int row;      // b * Hkv + kvh
  int id;       // physical block
  bool newrow;  // first block of its row in this wave's range
  bool last;    // last block of its row (holds the new token)
};

// Packs EPL floats of a row slice into a 16-byte packet of T.
template <typename T>
__device__ __forceinline__ uint4 pack_packet(const float* y) {
  if constexpr (sizeof(T) == 4) {
    return make_uint4(__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]),
                      __float_as_uint(y[3]));
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const T a = Elem<T>::from_f32(y[2 * i]), b = Elem<T>::from_f32(y[2 * i + 1]);
      uint16_t ua, ub;
      __builtin_memcpy(&ua, &a, 2);
      __builtin_memcpy(&ub, &b, 2);
      w[i] = (uint32_t)ua | ((uint32_t)ub << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// RMSNorm (optional) then NeoX RoPE of one row held as packets: lane col of
// an LPR-lane group holds elements [col*EPL, col*EPL + EPL); rotate_half
// pairs element i with i + D/2, held by lane col ^ LPR/2. Rounding follows
// Candle's op sequence (RmsNorm::forward, apply_rope; src/backends/qwen2.rs:
// 68-75, 133-142): x/norm and *w rounded to T, x*cos and rot*sin rounded,
// then the sum rounded; no fused multiply-adds.
template <typename T, int D>
__device__ __forceinline__ uint4 norm_rope_packet(uint4 x, bool norm, uint4 w, float inv_d,
                                                  float eps, uint4 cs, uint4 sn, int col) {
  using S = DecodeShape<T, D>;
  constexpr int EPL = S::EPL, LPR = S::LPR;
  float xf[EPL], wf[EPL], cf[EPL], sf[EPL];
  Packet<T>::unpack(x, xf);
  if (norm) {
    Packet<T>::unpack(w, wf);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) ss = __fadd_rn(ss, __fmul_rn(xf[e], xf[e]));
    ss = group_sum<LPR>(ss);
    const float nrm = sqrtf(__fadd_rn(__fmul_rn(ss, inv_d), eps));
#pragma unroll
    for (int e = 0; e < EPL; ++e) xf[e] = round_to<T>(__fmul_rn(round_to<T>(xf[e] / nrm), wf[e]));
  }
  Packet<T>::unpack(cs, cf);
  Packet<T>::unpack(sn, sf);
  const bool upper = col >= LPR / 2;
  float y[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float pf = __shfl_xor(xf[e], LPR / 2, 64);
    const float a = round_to<T>(__fmul_rn(xf[e], cf[e]));
    const float bb = round_to<T>(__fmul_rn(upper ? pf : -pf, sf[e]));
    y[e] = __fadd_rn(a, bb);
  }
  return pack_packet<T>(y);
}

template <typename T, int D, int G, bool FUSED>
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeParams p) {
  using S = DecodeShape<T, D>;
  constexpr int EPL = S::EPL, LPR = S::LPR, RPL = S::RPL, NR = S::NR;
  constexpr int REC = rec_floats(G, D);
  constexpr int NPART = 2 * kWaves;
  constexpr int DPL = (D + 63) / 64;  // output dims per lane in the row epilogue
  // Register buffers per wave: three when the block and query packets fit
  // beside two waves per SIMD, else two.
  constexpr int kNumBufs = (sizeof(T) == 2 && G <= 2 && !FUSED) ? 3 : 2;
  extern __shared__ int s_pref[];             // [B + 1]
  __shared__ float s_part[NPART][G][D + 2];   // wave partials: acc[D], m, l per head
  __shared__ int s_part_row[NPART];           // their rows (-1 = unused)

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int col = lane % LPR, rsub = lane / LPR;
  const int B = p.B, Hkv = p.Hkv, mbps = p.mbps;
  const int Hq = Hkv * G;
  T* __restrict__ ob = reinterpret_cast<T*>(p.out);

  if (wave == 0) block_prefix(p.seq_lens, B, mbps, s_pref);
  if (tid < NPART) s_part_row[tid] = -1;
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
  const long long glo = range_lo(w, total, we);
  const long long ghi = range_lo(w + 1, total, we);
  // This wave's contiguous share of the group's range.
  const long long wlo = glo + (ghi - glo) * wave / kWaves;
  const long long whi = glo + (ghi - glo) * (wave + 1) / kWaves;
  const int nblk = (int)(whi - wlo);

  // Row start in the block stream and its block count.
  auto row_extent = [&](int row, long long& R, int& nb) __attribute__((always_inline)) {
    const int b = row / Hkv, kvh = row - b * Hkv;
    nb = s_pref[b + 1] - s_pref[b];
    R = (long long)Hkv * s_pref[b] + (long long)kvh * nb;
  };

  if (nblk > 0) {
    const T* __restrict__ qb = reinterpret_cast<const T*>(p.q);
    const T* __restrict__ kp = reinterpret_cast<const T*>(p.k_pool);
    const T* __restrict__ vp = reinterpret_cast<const T*>(p.v_pool);
    const size_t tile = (size_t)16 * D;  // elements of one (block, head) tile
    const size_t lane_off = (size_t)rsub * D + (size_t)col * EPL;

    // Descriptors of 64 consecutive blocks, one per lane: page id, valid
    // rows and row, read back with readlane when the block is issued.
    // d_nv holds the valid rows in bits 0-7 and "last block of its row" in
    // bit 8; d_pos is the row's new-token position (fused step).
    int d_id = 0, d_nv = 0, d_row = -1, d_pos = 0, cbase = 0;
    auto load_chunk = [&](int base) __attribute__((always_inline)) {
      cbase = base;
      const long long f = wlo + base + lane;
      d_id = 0;
      d_nv = 0;
      d_row = -1;
      d_pos = 0;
      if (f < whi) {
        const int b = locate_seq(s_pref, B, Hkv, f);
        const int nb = s_pref[b + 1] - s_pref[b];
        const long long o = f - (long long)Hkv * s_pref[b];
        const int kvh = (int)(o / nb), blk = (int)(o % nb);
        d_row = b * Hkv + kvh;
        d_id = p.tables[(size_t)b * mbps + blk];
        const int L = clamp_len(p.seq_lens[b], mbps);
        const int nv = L - blk * 16;
        d_nv = nv > 16 ? 16 : nv;
        d_pos = L - 1;
        if ((unsigned)d_id >= (unsigned)p.num_blocks)
          d_nv = 0;
        else if (blk == nb - 1)
          d_nv |= 256;
      }
    };
    load_chunk(0);

    int issued_row = -1;
    auto issue = [&](Buf<T, D, G>& bf, int j) __attribute__((always_inline)) {
      if (j - cbase >= 64) load_chunk(cbase + 64);
      const int k = j - cbase;
      const int id = __builtin_amdgcn_readlane(d_id, k);
      const int nvf = __builtin_amdgcn_readlane(d_nv, k);
      const int row = __builtin_amdgcn_readlane(d_row, k);
      const int b = row / Hkv, kvh = row - b * Hkv;
      const int nv = nvf & 255;
      bf.nvalid = nv;
      bf.row = row;
      bf.id = id;
      bf.newrow = row != issued_row;
      bf.last = (nvf >> 8) != 0;
      if (bf.newrow) {
        issued_row = row;
#pragma unroll
        for (int g = 0; g < G; ++g)
          bf.q[g] = *reinterpret_cast<const uint4*>(
              qb + ((size_t)b * Hq + (size_t)kvh * G + g) * D + (size_t)col * EPL);
        if constexpr (FUSED) {
          const int pos = __builtin_amdgcn_readlane(d_pos, k);
          const size_t to = (size_t)pos * (D / 2) + (size_t)(col % (LPR / 2)) * EPL;
          bf.cs = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.cos_t) + to);
          bf.sn = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.sin_t) + to);
        }
      }
      if constexpr (FUSED) {
        if (bf.last) {
          const size_t no = ((size_t)b * Hkv + kvh) * D + (size_t)col * EPL;
          bf.kn = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.k_new) + no);
          bf.vn = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.v_new) + no);
        }
      }
      if (nv > 0) {
        const size_t base = ((size_t)id * Hkv + kvh) * tile + lane_off;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          bf.k[r] = *reinterpret_cast<const uint4*>(kp + base + (size_t)r * RPL * D);
          bf.v[r] = *reinterpret_cast<const uint4*>(vp + base + (size_t)r * RPL * D);
        }
      }
    };

    float m[G], l[G], acc[G][EPL];
    uint4 qv[G];
    uint4 cs_cur = make_uint4(0, 0, 0, 0), sn_cur = make_uint4(0, 0, 0, 0);
    uint4 qw_pk = make_uint4(0, 0, 0, 0), kw_pk = make_uint4(0, 0, 0, 0);
    if constexpr (FUSED) {
      if (p.qw) qw_pk = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.qw) + col * EPL);
      if (p.kw) kw_pk = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.kw) + col * EPL);
    }
    int cur_row = -1;
    auto reset = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
      }
    };
    // Ends the wave's part of cur_row: merge the lane groups, then write the
    // output (row wholly inside this wave) or park the state in LDS.
    auto finalize = [&]() __attribute__((always_inline)) {
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
      long long R;
      int nb;
      row_extent(cur_row, R, nb);
      const int b = cur_row / Hkv, kvh = cur_row - b * Hkv;
      if (R >= wlo && R + nb <= whi) {
        if (rsub == 0) {
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float inv = l[g] > 0.f ? 1.f / l[g] : 0.f;  // all pages skipped -> zeros
            T* dst = ob + ((size_t)b * Hq + (size_t)kvh * G + g) * D + (size_t)col * EPL;
#pragma unroll
            for (int e = 0; e < EPL; ++e) dst[e] = Elem<T>::from_f32(acc[g][e] * inv);
          }
        }
      } else {
        const int slot = 2 * wave + (R < wlo ? 0 : 1);
        if (rsub == 0) {
#pragma unroll
          for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) s_part[slot][g][col * EPL + e] = acc[g][e];
            if (col == 0) {
              s_part[slot][g][D] = m[g];
              s_part[slot][g][D + 1] = l[g];
            }
          }
        }
        if (lane == 0) s_part_row[slot] = cur_row;
      }
    };
    auto compute = [&](const Buf<T, D, G>& bf) __attribute__((always_inline)) {
      if (bf.newrow) {
        if (cur_row >= 0) finalize();
        reset();
        cur_row = bf.row;
        if constexpr (FUSED) {  // q_norm + RoPE of the row's query heads
          cs_cur = bf.cs;
          sn_cur = bf.sn;
#pragma unroll
          for (int g = 0; g < G; ++g)
            qv[g] = norm_rope_packet<T, D>(bf.q[g], p.qw != nullptr, qw_pk, p.inv_d, p.eps,
                                           cs_cur, sn_cur, col);
        } else {
#pragma unroll
          for (int g = 0; g < G; ++g) qv[g] = bf.q[g];
        }
      }
      const int nv = bf.nvalid;
      if (nv <= 0) return;
      uint4 kr[NR], vr[NR];
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        kr[r] = bf.k[r];
        vr[r] = bf.v[r];
      }
      if constexpr (FUSED) {
        if (bf.last) {
          // The new token is the row's last key (slot nv-1 of this block):
          // k_norm + RoPE it, append k and raw v to the pool, and use them in
          // place of whatever the slot held.
          const uint4 kn = norm_rope_packet<T, D>(bf.kn, p.kw != nullptr, kw_pk, p.inv_d,
                                                  p.eps, cs_cur, sn_cur, col);
          const int slot = nv - 1;
          const int kvh = bf.row % Hkv;
          if (rsub == slot % RPL) {
#pragma unroll
            for (int r = 0; r < NR; ++r)
              if (r == slot / RPL) {
                kr[r] = kn;
                vr[r] = bf.vn;
              }
            const size_t dst = (((size_t)bf.id * Hkv + kvh) * 16 + slot) * D + (size_t)col * EPL;
            *reinterpret_cast<uint4*>(const_cast<T*>(kp) + dst) = kn;
            *reinterpret_cast<uint4*>(const_cast<T*>(vp) + dst) = bf.vn;
          }
        }
      }
      // Raw scores q.k, summed over the LPR lanes of each row.
      float s[G][NR];
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int r = 0; r < NR; ++r)
          s[g][r] = group_sum<LPR>(Packet<T>::dot(qv[g], kr[r], 0.f));
      if (nv < 16) {  // tail block: rows past the sequence end get p = 0 and V = 0
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          if (r * RPL + rsub >= nv) {
#pragma unroll
            for (int g = 0; g < G; ++g) s[g][r] = -INFINITY;
            vr[r] = make_uint4(0, 0, 0, 0);
          }
        }
      }
      // 16-bit V: pair rows (r, r+1) element-wise so one v_dot2 applies two
      // probabilities; the pairing is shared by all G heads.
      constexpr bool kPacked = sizeof(T) == 2;
      uint32_t vpair[kPacked ? NR / 2 : 1][4][2];
      float vf[kPacked ? 1 : NR][EPL];
      if constexpr (kPacked) {
#pragma unroll
        for (int r = 0; r < NR; r += 2) {
          const uint32_t w0[4] = {vr[r].x, vr[r].y, vr[r].z, vr[r].w};
          const uint32_t w1[4] = {vr[r + 1].x, vr[r + 1].y, vr[r + 1].z, vr[r + 1].w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            vpair[r / 2][k][0] = __builtin_amdgcn_perm(w1[k], w0[k], 0x05040100u);  // low halves
            vpair[r / 2][k][1] = __builtin_amdgcn_perm(w1[k], w0[k], 0x07060302u);  // high halves
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < NR; ++r) Packet<T>::unpack(vr[r], vf[r]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mx = s[g][0];
#pragma unroll
        for (int r = 1; r < NR; ++r) mx = fmaxf(mx, s[g][r]);
        const float cand = mx * p.c;
        // Lazy rescaling: the running max moves only when a score exceeds it
        // by more than kLazyLog2 (probabilities then stay below 2^kLazyLog2).
        if (__any(cand > m[g] + kLazyLog2)) {
          const float mn = fmaxf(m[g], cand);
          const float alpha = (mn == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m[g] - mn);
          l[g] *= alpha;
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
          m[g] = mn;
        }
        const float nms = (m[g] == -INFINITY) ? 0.f : -m[g];
        float pr[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          pr[r] = __builtin_amdgcn_exp2f(fmaf(s[g][r], p.c, nms));
          l[g] += pr[r];
        }
        if constexpr (kPacked) {
#pragma unroll
          for (int r = 0; r < NR; r += 2) {
            const uint32_t pp = Packet<T>::pack2(pr[r], pr[r + 1]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              acc[g][2 * k] = Packet<T>::dot2(vpair[r / 2][k][0], pp, acc[g][2 * k]);
              acc[g][2 * k + 1] = Packet<T>::dot2(vpair[r / 2][k][1], pp, acc[g][2 * k + 1]);
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            float a = acc[g][e];
#pragma unroll
            for (int r = 0; r < NR; ++r) a = fmaf(pr[r], vf[r][e], a);
            acc[g][e] = a;
          }
        }
      }
    };

    // kNumBufs blocks in flight: kNumBufs-1 are loading while one is
    // computed (indices past the end re-load the last block, never computed).
    const int last = nblk - 1;
    if constexpr (kNumBufs == 3) {
      Buf<T, D, G> b0, b1, b2;
      issue(b0, 0);
      issue(b1, last < 1 ? last : 1);
      for (int i = 0;;) {
        issue(b2, i + 2 < last ? i + 2 : last);
        compute(b0);
        if (++i == nblk) break;
        issue(b0, i + 2 < last ? i + 2 : last);
        compute(b1);
        if (++i == nblk) break;
        issue(b1, i + 2 < last ? i + 2 : last);
        compute(b2);
        if (++i == nblk) break;
      }
    } else {
      Buf<T, D, G> b0, b1;
      issue(b0, 0);
      for (int i = 0;;) {
        issue(b1, i + 1 < last ? i + 1 : last);
        compute(b0);
        if (++i == nblk) break;
        issue(b0, i + 1 < last ? i + 1 : last);
        compute(b1);
        if (++i == nblk) break;
      }
    }
    finalize();
  }
  __syncthreads();

  // Rows this group holds in pieces. The wave holding the group's last piece
  // of a row finishes it: it combines the pieces parked by earlier waves
  // (waves own consecutive ranges, so a row's pieces sit in consecutive
  // waves), then writes the output (row inside the group's range) or
  // publishes one group partial and merges the row if it arrives last. Waves
  // handle their rows independently, so the publication chains overlap.
  for (int s = 0; s < 2; ++s) {
    const int row = s_part_row[2 * wave + s];
    if (row < 0) continue;
    long long R;
    int nb;
    row_extent(row, R, nb);
    if (R + nb > whi && whi < ghi) continue;  // a later wave holds more of the row
    const int b = row / Hkv, kvh = row - b * Hkv;
    const bool inside = R >= glo && R + nb <= ghi;
    float M[G][DPL], Ls[G][DPL], A[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
        M[g][k] = -INFINITY;
        Ls[g][k] = 0.f;
        A[g][k] = 0.f;
      }
    for (int wv = wave; wv >= 0; --wv) {
      bool any = false;
      for (int s2 = 1; s2 >= 0; --s2) {
        const int slot = 2 * wv + s2;
        if ((wv == wave && s2 != s) || s_part_row[slot] != row) continue;
        any = true;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int k = 0; k < DPL; ++k) {
            const int d = lane + 64 * k;
            if (d < D)
              lse_combine(M[g][k], Ls[g][k], A[g][k], s_part[slot][g][D], s_part[slot][g][D + 1],
                          s_part[slot][g][d]);
          }
      }
      if (!any) break;
    }
    if (inside) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < DPL; ++k) {
          const int d = lane + 64 * k;
          if (d < D) {
            const float inv = Ls[g][k] > 0.f ? 1.f / Ls[g][k] : 0.f;
            ob[((size_t)b * Hq + (size_t)kvh * G + g) * D + d] = Elem<T>::from_f32(A[g][k] * inv);
          }
        }
      continue;
    }
    // Group partial: slot 0 = the group's first segment, 1 = a later one.
    float* rec = p.ws + ((size_t)w * 2 + (R <= glo ? 0 : 1)) * (size_t)REC;
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
        const int d = lane + 64 * k;
        if (d < D) st_dev(rec + (size_t)g * D + d, A[g][k]);
      }
      if (lane == 0) {
        st_dev(rec + G * D + g, M[g][0]);
        st_dev(rec + G * D + G + g, Ls[g][0]);
      }
    }
    // Count the arrival; the last of the row's np groups merges. Group wa
    // (holding the row's first block) used slot 0 only if its range starts
    // exactly at the row start.
    const long long wa = ((R + 1) * we - 1) / total;
    const long long wb = ((R + nb) * we - 1) / total;
    const int np = (int)(wb - wa + 1);
    const bool wa_slot1 = range_lo(wa, total, we) != R;
    wait_vm_stores();
    int prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(p.counters + row, 1, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0, 64);
    if (prev != np - 1) continue;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
        M[g][k] = -INFINITY;
        Ls[g][k] = 0.f;
        A[g][k] = 0.f;
      }
    for (int c = 0; c < np; c += kMergeChunk) {
      float mv[kMergeChunk][G], lv[kMergeChunk][G], av[kMergeChunk][G][DPL];
#pragma unroll
      for (int i = 0; i < kMergeChunk; ++i) {  // issue the chunk's loads together
        const int j = c + i < np ? c + i : np - 1;
        const int slot = (j == 0 && wa_slot1) ? 1 : 0;
        const float* r = p.ws + ((size_t)(wa + j) * 2 + slot) * (size_t)REC;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          mv[i][g] = ld_dev(r + G * D + g);
          lv[i][g] = ld_dev(r + G * D + G + g);
#pragma unroll
          for (int k = 0; k < DPL; ++k) {
            const int d = lane + 64 * k;
            av[i][g][k] = d < D ? ld_dev(r + (size_t)g * D + d) : 0.f;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < kMergeChunk; ++i)
        if (c + i < np)
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int k = 0; k < DPL; ++k)
              lse_combine(M[g][k], Ls[g][k], A[g][k], mv[i][g], lv[i][g], av[i][g][k]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
        const int d = lane + 64 * k;
        if (d < D) {
          const float inv = Ls[g][k] > 0.f ? 1.f / Ls[g][k] : 0.f;
          ob[((size_t)b * Hq + (size_t)kvh * G + g) * D + d] = Elem<T>::from_f32(A[g][k] * inv);
        }
      }
    if (lane == 0)
      __hip_atomic_store(p.counters + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

template <typename T, int D, int G, bool FUSED>
static int launch_decode_t(const DecodeParams& p, hipStream_t stream) {
  const size_t lds = (size_t)(p.B + 1) * sizeof(int);
  hipLaunchKernelGGL((decode_kernel<T, D, G, FUSED>), dim3(p.W), dim3(kThreads), lds, stream,
                     p);
  return launch_status("decode_kernel");
}

template <typename T, int D, bool FUSED>
static int launch_decode_g(int G, const DecodeParams& p, hipStream_t s) {
  switch (G) {
    case 1: return launch_decode_t<T, D, 1, FUSED>(p, s);
    case 2: return launch_decode_t<T, D, 2, FUSED>(p, s);
    case 3: return launch_decode_t<T, D, 3, FUSED>(p, s);
    case 4: return launch_decode_t<T, D, 4, FUSED>(p, s);
    case 5: return launch_decode_t<T, D, 5, FUSED>(p, s);
    case 6: return launch_decode_t<T, D, 6, FUSED>(p, s);
    case 7: return launch_decode_t<T, D, 7, FUSED>(p, s);
    case 8: return launch_decode_t<T, D, 8, FUSED>(p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode: unsupported group size %d", G);
}

template <typename T, bool FUSED>
static int launch_decode_d(int D, int G, const DecodeParams& p, hipStream_t s) {
  switch (D) {
    case 64: return launch_decode_g<T, 64, FUSED>(G, p, s);
    case 128: return launch_decode_g<T, 128, FUSED>(G, p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode: unsupported head_dim %d", D);
}

template <bool FUSED>
static int launch_decode_dtype(int dtype, int D, int G, const DecodeParams& p, hipStream_t s) {
  switch (dtype) {
    case RLSE_DTYPE_F32: return launch_decode_d<float, FUSED>(D, G, p, s);
    case RLSE_DTYPE_BF16: return launch_decode_d<bf16, FUSED>(D, G, p, s);
    case RLSE_DTYPE_F16: return launch_decode_d<f16, FUSED>(D, G, p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode: bad dtype %d", dtype);
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

// Validates the shared decode arguments and fills p (workspace included).
static int prepare_decode(DecodeParams& p, const void* q, const void* k_pool,
                          const void* v_pool, const int32_t* block_tables,
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
  p = DecodeParams{};
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
  return RLSE_OK;
}

extern "C" int rlse_paged_gqa_decode(const void* q, const void* k_pool, const void* v_pool,
                                     const int32_t* block_tables, const int32_t* seq_lens,
                                     void* out, int batch, int num_heads, int num_kv_heads,
                                     int head_dim, int max_blocks_per_seq, int num_blocks,
                                     float scale, int dtype, void* workspace,
                                     size_t workspace_bytes, rlse_stream_t stream) {
  DecodeParams p;
  const int st = prepare_decode(p, q, k_pool, v_pool, block_tables, seq_lens, out, batch,
                                num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                                num_blocks, scale, dtype, workspace, workspace_bytes);
  if (st) return st;
  return launch_decode_dtype<false>(dtype, head_dim, num_heads / num_kv_heads, p,
                                    as_stream(stream));
}

extern "C" int rlse_decode_step(const void* q, const void* k_new, const void* v_new,
                                const void* q_norm_weight, const void* k_norm_weight, float eps,
                                const void* cos_table, const void* sin_table, int max_pos,
                                void* k_pool, void* v_pool, const int32_t* block_tables,
                                const int32_t* seq_lens, void* out, int batch, int num_heads,
                                int num_kv_heads, int head_dim, int max_blocks_per_seq,
                                int num_blocks, float scale, int dtype, void* workspace,
                                size_t workspace_bytes, rlse_stream_t stream) {
  DecodeParams p;
  const int st = prepare_decode(p, q, k_pool, v_pool, block_tables, seq_lens, out, batch,
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
  return launch_decode_dtype<true>(dtype, head_dim, num_heads / num_kv_heads, p,
                                   as_stream(stream));
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
