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
// (m, l, acc) partial per earlier group in the workspace, and the group
// holding the row's last block merges them with a log-sum-exp combine in the
// same launch, taking each partial as soon as all of its words have arrived
// (record words carry the launch's epoch, so a word of an earlier launch is
// never taken for one of this launch). Groups are dispatched in index order
// and the grid never exceeds two groups per compute unit, so a merging group
// only ever waits for groups that are running or done; the wait is bounded,
// and a merge that gives up writes NaN and raises a sticky error flag in the
// workspace. A workspace only needs zero-filling once, before first use.
//
// Inside a wave a K/V block is read as 16-byte packets (16 rows of head_dim
// elements); the page ids of 64 blocks are fetched at once (one per lane),
// NBUF blocks are buffered in registers so the next blocks' loads -- and the
// query of a new row -- are in flight during the math, and no barrier is
// taken while streaming. The math per block:
//  - 16-bit K/V (decode_mma): MFMAs give S^T = K . Q^T (16 keys x the G heads
//    padded to 16) and accumulate O^T += V^T . P^T, V transposed through LDS;
//    a lane holds one head's scores of four keys and 16 of its output
//    dimensions, and only the online softmax runs on the VALU;
//  - 32-bit K/V: LPR lanes cover one row's head_dim, RPL = 64/LPR rows are
//    read per instruction and each lane owns NR = 16/RPL rows of the block;
//    scores are reduced over the LPR lanes of a row with DPP adds, each lane
//    group keeps its own online-softmax state (running max m in log2 units,
//    sum l, acc) and the groups are merged when the wave's part of a row ends.
#pragma once

#include <math.h>

#include "common.cuh"
#include "host_common.h"

namespace rlse {

constexpr int kWaves = 4;               // wavefronts per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kGroupsPerCU = 2;         // workgroups launched per compute unit
constexpr int kMinBlocksPerGroup = 8;   // smallest share of blocks per workgroup
constexpr int kMaxDecodeBatch = 8192;   // prefix table lives in LDS
constexpr int kMaxDecodeRows = 65536;   // batch * num_kv_heads
// Share of the block stream taken by the second workgroup of each compute
// unit, in sixteenths of the first's (16: equal shares; see share_cum).
constexpr int kSlot1Weight = 16;
// Kernel modes: the paged decode (rlse_paged_gqa_decode), the fused step
// (rlse_decode_step), the fused step with a plan (rlse_decode_step_planned),
// and the same streaming its pages with non-temporal loads (flag
// RLSE_DECODE_STREAM: no page is read by more than one row of the batch).
enum : int { kModePlain = 0, kModeFused = 1, kModePlanned = 2, kModePlannedStream = 3 };
// The running max of a softmax moves only when a score exceeds it by more
// than this many powers of two.
constexpr float kLazyLog2 = 8.f;

// Per-phase timeline of a launch, in the measurement build only (`make
// timeline` defines RLSE_DECODE_TIMELINE; the library then exports
// rlse_decode_timeline): every wave reads the wall clock (100 MHz ticks) at
// kTimelinePoints points of its launch into registers, and lane 0 stores them
// once, when the wave has finished, at p.timeline[(block * kWaves + wave) *
// kTimelinePoints + point] -- a store per point would wait behind the loads
// in flight and move the points after it. The points:
//   0 entry, 1 plan arrived (planned), 2 first pages requested (planned),
//   3 prologue barrier passed, 4 prologue done (queries staged, appends
//   stored), 5 first page computed, 6 streaming loop ended, 7 group
//   barrier passed (the epilogue's), 8 the group's own pieces of a row
//   combined (waves that finish or publish a row held in pieces; the last
//   such row), 9 earlier groups' records arrived and combined (the merging
//   wave), 10 finished (outputs, publications and the launch counter
//   stored).
// A point a wave does not reach reads 0. Other builds compile no stamp.
constexpr int kTimelinePoints = 11;
constexpr int kTimelineMaxWaves = 8192;
// The cascade step's prefix launch stamps its own region, after the
// decode's: kPrefixTimelinePoints per wave, at
// [kTimelineMaxWaves * kTimelinePoints + (block * 8 + wave) * points]:
//   0 entry, 1 page ids and query loads issued, 2 first blocks requested,
//   3 queries staged (normed, roped, in LDS behind the barrier), 4 first
//   block computed, 5 loop ended, 6 waves' states combined (behind the
//   second barrier), 7 slice state stored, 8 finished (the contract check
//   included). Waves with no work leave their row at 0.
constexpr int kPrefixTimelinePoints = 9;
struct TimelineStamps {
  unsigned long long t[kTimelinePoints];
};
#ifdef RLSE_DECODE_TIMELINE
#define RLSE_TL(k) (tl.t[k] = wall_clock64())
#else
#define RLSE_TL(k) ((void)0)
#endif

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

// Keys of a row: its length, or 0 for a row with no keys (L <= 0) and for
// an invalid row whose length exceeds its block table (L > mbps*16).
__device__ __forceinline__ int valid_len(int L, int mbps) {
  return (L <= 0 || L > mbps * 16) ? 0 : L;
}

// Leading table entries of sequence b left out of the page stream: a
// shared prefix attended separately (cascade step), the same `prefix` for
// every sequence or, with seq_pre (prefix groups), each sequence's own.
__device__ __forceinline__ int stream_skip(const int* __restrict__ seq_pre, int prefix, int b) {
  return seq_pre ? seq_pre[b] : prefix;
}

// Exclusive prefix of per-sequence block counts into s_pref[0..B] (one wave).
// first / first_pre: seq_lens[lane] and the lane's skipped entries for
// lane < B, requested by the caller beforehand. (The first chunk issues no
// load, so a caller with loads in flight does not wait for them here.)
__device__ void block_prefix(const int* __restrict__ seq_lens, int B, int mbps, int* s_pref,
                             int first, int prefix, const int* __restrict__ seq_pre,
                             int first_pre) {
  const int lane = threadIdx.x & 63;
  int carry = 0;
  auto chunk = [&](int base, int len, int pre) __attribute__((always_inline)) {
    const int b = base + lane;
    int x = b < B ? (valid_len(len, mbps) + 15) >> 4 : 0;
    x = x > pre ? x - pre : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (b < B) s_pref[b + 1] = carry + x;
    carry += __shfl(x, 63, 64);
  };
  chunk(0, first, first_pre);
  for (int base = 64; base < B; base += 64) {
    const int b = base + lane < B ? base + lane : B - 1;
    chunk(base, base + lane < B ? seq_lens[b] : 0, stream_skip(seq_pre, prefix, b));
  }
  if (lane == 0) s_pref[0] = 0;
}

__device__ __forceinline__ long long effective_groups(long long total, int W) {
  long long we = total / kMinBlocksPerGroup;
  if (we < 1) we = 1;
  return we < W ? we : W;
}

// Shares of the block stream. With the full grid, workgroups [0, W/2) --
// dispatched first, one per compute unit -- weigh 16 and the second
// workgroup of each compute unit weighs w1 (a per-launch constant): the
// second workgroup's waves start later and lose issue arbitration to the
// first's, so an equal share would leave its compute units streaming alone
// at the end. Fewer groups (small batches) share evenly.
__device__ __forceinline__ long long share_cum(long long w, long long we, int W, int w1) {
  if (we < W || w1 == 16) return w * 16;
  const long long h = W / 2;
  return w <= h ? w * 16 : h * 16 + (w - h) * w1;
}
__device__ __forceinline__ long long range_lo(long long w, long long total, long long we, int W,
                                              int w1) {
  return total * share_cum(w, we, W, w1) / share_cum(we, we, W, w1);
}
// The workgroup whose range holds block f: the largest w with
// range_lo(w) <= f, i.e. with total * share_cum(w) < (f + 1) * S (S the
// whole stream's share): the largest w whose share_cum is at most
// c = ((f + 1) * S - 1) / total. One division, on the merge's critical path.
__device__ __forceinline__ long long group_of(long long f, long long total, long long we, int W,
                                              int w1) {
  const long long S = share_cum(we, we, W, w1);
  const long long c = ((f + 1) * S - 1) / total;
  if (we < W || w1 == 16) return c / 16;
  const long long h16 = (long long)(W / 2) * 16;
  return c <= h16 ? c / 16 : W / 2 + (c - h16) / w1;
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

// Descriptor of block f of the page stream (f < the wave's end): the page id,
// the valid rows in bits 0-7 (0 for a page id outside the pool) with bit 8
// set on the last block of its row, the (sequence, KV head) row and the
// row's new-token position. Blocks past the wave's end get {0, 0, -1, 0}.
// A row's stream starts at table entry stream_skip(b) (block_prefix).
__device__ __forceinline__ int4 block_desc(long long f, long long whi, const int* s_pref,
                                           const int* __restrict__ tables,
                                           const int* __restrict__ seq_lens, int B, int Hkv,
                                           int mbps, int num_blocks, int prefix,
                                           const int* __restrict__ seq_pre) {
  int4 d = make_int4(0, 0, -1, 0);
  if (f < whi) {
    const int b = locate_seq(s_pref, B, Hkv, f);
    const int nb = s_pref[b + 1] - s_pref[b];
    const long long o = f - (long long)Hkv * s_pref[b];
    const int kvh = (int)(o / nb), blk = (int)(o % nb);
    const int pre = stream_skip(seq_pre, prefix, b);
    d.z = b * Hkv + kvh;
    d.x = tables[(size_t)b * mbps + pre + blk];
    const int L = valid_len(seq_lens[b], mbps);
    const int nv = L - (pre + blk) * 16;
    d.y = nv > 16 ? 16 : nv;
    d.w = L - 1;
    if ((unsigned)d.x >= (unsigned)num_blocks)
      d.y = 0;
    else if (blk == nb - 1)
      d.y |= 256;
  }
  return d;
}

// Tagged 64-bit words of one partial record: acc[G][D], then m[G] and l[G].
__host__ __device__ constexpr int rec_words(int G, int D) { return G * D + 2 * G; }

// Workspace layout (32-bit words): the 256-byte header (word 0: sticky
// error flags), one launch counter per wave of the grid (rounded up to 256
// bytes), then two records per workgroup.
constexpr int kWsHeaderWords = 64;
__host__ __device__ constexpr size_t decode_ctr_words(int W) {
  return ((size_t)W * kWaves + 63) & ~(size_t)63;
}


struct DecodeParams {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const int* tables;
  const int* seq_lens;
  void* out;
  uint32_t* ws_err;  // workspace word 0: sticky RLSE_WS_ERR_* flags
  uint32_t* ws_ctr;  // one launch counter per wave of the grid
  uint64_t* ws_rec;  // tagged partial records, two slots per workgroup
  unsigned long long wait_ticks;  // bound on a merge's wait (100 MHz ticks)
  int B;
  int Hkv;
  int mbps;
  int num_blocks;
  int W;    // workgroups launched
  int w1;   // weight of the second workgroup per compute unit (16 = even shares)
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
  // Optional per-step plan (rlse_decode_plan): the first 64 block
  // descriptors of every wave, as block_desc computes them. Null: each wave
  // derives them from the lengths and the block tables.
  const int4* plan;
  // Shared-prefix (cascade) step, 16-bit K/V only: the first `prefix` table
  // entries of every sequence are left out of the stream, and every row's
  // result is combined with `pre`, the softmax state of its query heads over
  // those pages ([B][Hq][D + 4] floats: acc[D], m, l in log2 units), when the
  // row is finished. prefix 0 and pre null: none.
  int prefix;
  const float* pre;      // cascade step: pre_slices states over the shared prefix
  int pre_slices;        // (regions pre_stride floats apart), combined in order
  long long pre_stride;
  // Prefix groups (several shared prefixes and unforked sequences in one
  // cascade step): the shared pages of each sequence ([B], 0 = none; its
  // prefix states take prefix_splits of them slices), or null (`prefix` for
  // every sequence).
  const int* seq_pre;
  // The stamp a planned launch expects in its plan (plan_stamp).
  int plan_stamp;
  // Cascade step: rows finished inside one wave's range park their state
  // here ([B][Hq][prefix_row_floats(D)] floats) and are combined with the
  // prefix states after the wave's stream, all slices' loads at once.
  float* pre_own;
#ifdef RLSE_DECODE_TIMELINE
  unsigned long long* timeline;  // [waves][kTimelinePoints] wall-clock stamps
#endif
};

// Floats per (sequence, query head) of a prefix partial: acc[D], m, l, and
// two of padding so that rows stay 16-byte aligned.
__host__ __device__ constexpr int prefix_row_floats(int D) { return D + 4; }

// Shared-prefix partial attention of a cascade decode step
// (decode_prefix.hip): the softmax state of every query head over the first
// `prefix` table entries, which every sequence of the batch shares.
struct PrefixParams {
  const void* q;  // [B][Hq][D] raw queries (q_norm + RoPE applied here, as the decode does)
  const void* k_pool;
  const void* v_pool;
  const int* tables;  // [B][mbps]; sequence 0's first `prefix` entries are the shared pages
  const int* seq_lens;
  const void* qw;  // q RMSNorm weight [D] (null: no norm)
  const void* cos_t;
  const void* sin_t;
  float eps;
  float inv_d;
  float c;  // scale * log2(e)
  int B;
  int Hkv;
  int mbps;
  int num_blocks;
  int prefix;
  float* pre;        // prefix_splits(prefix) x [B][Hq][prefix_row_floats(D)] floats
  uint32_t* ws_err;  // sticky flags: RLSE_WS_ERR_PREFIX
  // Prefix groups (null members: one group, every sequence, `prefix`
  // pages): the grouped sequences, group by group, then the grouped plan's
  // offsets, pages and column tiles (group_plan_kernel); num_groups groups,
  // `prefix` then bounds every group's pages and tiles the launch's column
  // tiles.
  const int* members;
  const int* grp;
  int num_groups;
  int tiles;
  // Planned one-prefix step: the plan's verdict on the cascade contract
  // (kPlanContractWord, nonzero: violated), checked once per step by the
  // plan; null: the launch checks the tables and lengths itself.
  const int* contract;
#ifdef RLSE_DECODE_TIMELINE
  unsigned long long* timeline;  // the prefix launch's region of the timeline buffer
#endif
};
// Most prefix groups one grouped cascade step takes.
constexpr int kMaxPrefixGroups = 64;
// The grouped plan, after the per-wave descriptors of a plan buffer:
// seq_pre[kMaxDecodeBatch] (shared pages per sequence), members
// [kMaxDecodeBatch] (grouped sequences, group by group, in batch order within
// a group), then grp: member offsets [kMaxPrefixGroups + 1], column-tile
// offsets [kMaxPrefixGroups + 1], pages [kMaxPrefixGroups], one word of error
// bits (a group id or a page count out of range) and the number of work
// items, padded to 16 bytes; then the work items of the prefix launch. An
// item is one (column tile, prefix slice) of a group -- G columns per member,
// 16 per tile, prefix_splits(pages) slices -- in group order, slice-major
// within a group: {pages, the tile's first column within its group, the
// group's member offset, its member count} and, after all of those, the
// group's first member (whose table rows hold the pages) | slice << 16. A
// prefix workgroup reads its item's two entries, the count and the stamp in
// one round of loads, and no other word of the plan before it requests page
// ids.
constexpr int kGrpOff = 0, kGrpTiles = kMaxPrefixGroups + 1, kGrpPages = 2 * kGrpTiles,
              kGrpErr = kGrpPages + kMaxPrefixGroups, kGrpItems = kGrpErr + 1,
              kGrpWords = (kGrpItems + 1 + 3) & ~3;
// Column tiles a grouped prefix launch may have (every member's G <= 8
// columns, one part tile per group), and its work items (at most 8 slices a
// tile).
constexpr int kMaxGroupTiles = kMaxDecodeBatch * 8 / 16 + kMaxPrefixGroups;
constexpr int kMaxGroupItems = 8 * kMaxGroupTiles;
__host__ __device__ constexpr size_t group_plan_words() {
  return 2 * (size_t)kMaxDecodeBatch + kGrpWords + 5 * (size_t)kMaxGroupItems;
}
// A plan buffer: the descriptors of the first 64 blocks of every wave
// (int4), the new-token positions of the 64 rows from each wave's first row
// (int), then the tail: 64 words whose first is the plan's stamp, and the
// grouped plan.
constexpr int kPlanStampWords = 64;
// Tail word 1: the one-prefix cascade contract's verdict (0: every
// sequence's first `prefix` table entries are sequence 0's and its new token
// lies past them; 1: some sequence breaks it), written by the plan.
constexpr int kPlanContractWord = 1;
__host__ __device__ inline const int* plan_tail(const int4* plan, int W) {
  return reinterpret_cast<const int*>(plan + (size_t)W * kWaves * 64) + (size_t)W * kWaves * 64;
}
__host__ __device__ constexpr size_t plan_bytes(int W) {
  return (size_t)W * kWaves * 64 * (sizeof(int4) + sizeof(int)) +
         (kPlanStampWords + group_plan_words()) * sizeof(int);
}
// The stamp of a plan: mode 1 with the shared prefix's pages (0 for a
// plain plan), mode 2 with the number of prefix groups and the query heads
// per KV head (the grouped plan's column tiles depend on both).
__host__ __device__ constexpr int plan_stamp(int mode, int value) { return (mode << 24) | value; }
__host__ __device__ constexpr int group_stamp(int num_groups, int G) {
  return plan_stamp(2, num_groups | (G << 8));
}
// Longest shared prefix a cascade step takes, in pages (8192 tokens).
constexpr int kMaxPrefixPages = 512;
// Slices of the prefix attended by separate workgroups (each leaves its own
// softmax state; the decode combines them into each row): about 16 pages per
// slice, at most 8 slices.
__host__ __device__ constexpr int prefix_splits(int prefix) {
  return prefix <= 16 ? 1 : ((prefix + 15) / 16 > 8 ? 8 : (prefix + 15) / 16);
}
// Regions of a cascade step's prefix buffer: one state per slice, then the
// decode's parked row states.
__host__ __device__ constexpr int prefix_regions(int prefix) { return prefix_splits(prefix) + 1; }

int launch_decode_prefix(int dtype, int D, int G, const PrefixParams& p, hipStream_t s);

template <typename T, int D>
struct Buf {
  uint4 k[DecodeShape<T, D>::NR];
  uint4 v[DecodeShape<T, D>::NR];
  int nvalid;   // valid rows of the block (0 = block skipped)
  int row;      // b * Hkv + kvh
  int sub;      // fused step: s_new entry holding the block's new row (-1: none)
  bool newrow;  // first block of its row in this wave's range
};

// LDS bytes per wave for staged query packets: the queries of QR consecutive
// rows are staged at once (QR = kQStageBytes / (G * D * sizeof(T)), at least 1).
constexpr int kQStageBytes = 4096;
template <typename T, int D, int G>
__host__ __device__ constexpr int q_stage_rows() {
  return kQStageBytes / (G * D * (int)sizeof(T)) > 0 ? kQStageBytes / (G * D * (int)sizeof(T))
                                                      : 1;
}

// Matrix-core decode for 16-bit K/V: per 16-key block, S^T = K . Q^T on
// 16x16x32 MFMAs (keys x heads, the heads padded to 16 with zero queries) and
// O^T += V^T . P^T on 16x16x16 MFMAs, so the q.k and p.V dot products leave
// the VALU. Every mode takes it, so the cache-policy flag never changes a
// result.
template <typename T, int D, int G>
__host__ __device__ constexpr bool decode_mma() {
  return sizeof(T) == 2;
}

typedef float mma_f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 mma_bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 mma_f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 mma_f16x4_t __attribute__((ext_vector_type(4)));
typedef short mma_i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) mma_i16x4_t mma_lds_i16x4_t;

// 16x16 MFMAs on 16-bit operands (lane l: A[l%16][k], B[k][l%16] for its
// k-slots, accumulator rows 4*(l/16) .. +3 of column l%16). k32: eight
// elements per lane and operand; k16: four.
template <typename T>
struct Mma16;
template <>
struct Mma16<bf16> {
  static __device__ __forceinline__ mma_f32x4_t k32(uint4 a, uint4 b, mma_f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mma_bf16x8_t, a),
                                                   __builtin_bit_cast(mma_bf16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ mma_f32x4_t k16(mma_i16x4_t a, uint2 b, mma_f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, __builtin_bit_cast(mma_i16x4_t, b), c, 0,
                                                     0, 0);
  }
};
template <>
struct Mma16<f16> {
  static __device__ __forceinline__ mma_f32x4_t k32(uint4 a, uint4 b, mma_f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mma_f16x8_t, a),
                                                  __builtin_bit_cast(mma_f16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ mma_f32x4_t k16(mma_i16x4_t a, uint2 b, mma_f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(mma_f16x4_t, a),
                                                 __builtin_bit_cast(mma_f16x4_t, b), c, 0, 0, 0);
  }
};

// Rounding to T for the prologue's element-wise math: bf16 uses the
// select-form conversion (same result as round_to).
template <typename T>
__device__ __forceinline__ uint16_t bits_sel(float v) {
  if constexpr (sizeof(T) == 2 && !__is_same(T, f16)) {
    return f32_to_bf16_bits_sel(v);
  } else {
    const T h = Elem<T>::from_f32(v);
    uint16_t u;
    __builtin_memcpy(&u, &h, 2);
    return u;
  }
}
template <typename T>
__device__ __forceinline__ float round_sel(float v) {
  if constexpr (sizeof(T) == 4) {
    return v;
  } else if constexpr (!__is_same(T, f16)) {
    return bf16_bits_to_f32(f32_to_bf16_bits_sel(v));
  } else {
    return round_to<T>(v);
  }
}

// Packs EPL floats of a row slice into a 16-byte packet of T.
template <typename T>
__device__ __forceinline__ uint4 pack_packet(const float* y) {
  if constexpr (sizeof(T) == 4) {
    return make_uint4(__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]),
                      __float_as_uint(y[3]));
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)bits_sel<T>(y[2 * i]) | ((uint32_t)bits_sel<T>(y[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// RMSNorm (optional) then NeoX RoPE of one row held as packets: lane col of
// an LPR-lane group holds elements [col*EPL, col*EPL + EPL); rotate_half
// pairs element i with i + D/2, held by lane col ^ LPR/2. Rounding follows
// Candle's op sequence (RmsNorm::forward, apply_rope; src/backends/qwen2.rs:
// 68-75, 133-142): x/norm and *w rounded to T, x*cos and rot*sin rounded,
// then the sum rounded; no fused multiply-adds (mul_rn / add_rn). The sum
// of squares is sumsq_tree's order with one packet per lane, so every entry
// point that writes K stores the same bytes.
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
    for (int e = 0; e < EPL; ++e) ss = add_rn(ss, mul_rn(xf[e], xf[e]));
    ss = group_sum<LPR>(ss);
    const float nrm = sqrtf(add_rn(mul_rn(ss, inv_d), eps));
#pragma unroll
    for (int e = 0; e < EPL; ++e) xf[e] = round_sel<T>(mul_rn(round_sel<T>(xf[e] / nrm), wf[e]));
  }
  Packet<T>::unpack(cs, cf);
  Packet<T>::unpack(sn, sf);
  const bool upper = col >= LPR / 2;
  float y[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float pf = __shfl_xor(xf[e], LPR / 2, 64);
    const float a = round_sel<T>(mul_rn(xf[e], cf[e]));
    const float bb = round_sel<T>(mul_rn(upper ? pf : -pf, sf[e]));
    y[e] = add_rn(a, bb);
  }
  return pack_packet<T>(y);
}

// Appended rows per wave kept in LDS: the blocks of a wave's first kNewCap
// appends take the new row from there, so their loads never wait for the
// append stores.
template <typename T>
__host__ __device__ constexpr int new_row_cap() { return sizeof(T) == 2 ? 4 : 2; }

// Static LDS of one decode workgroup (the block prefix is dynamic LDS).
template <typename T, int D, int G, bool FUSED>
struct DecodeLds {
  static constexpr int LPR = DecodeShape<T, D>::LPR;
  static constexpr int QR = q_stage_rows<T, D, G>();
  static constexpr int kNew = new_row_cap<T>();
  float part[2 * kWaves][G][D + 2];  // wave partials: acc[D], m, l per head
  int part_row[2 * kWaves];          // their rows (-1 = unused)
  uint4 q[kWaves][QR][G][LPR];       // staged query packets per wave
  uint4 nw[FUSED ? kWaves : 1][FUSED ? kNew : 1][2][LPR];  // appended k, v rows
  // Matrix-core decode: the V block of each wave, row-major with 16 elements
  // of padding per row (transposing reads free of bank conflicts).
  static constexpr bool kMma = decode_mma<T, D, G>();
  uint4 vt[kMma ? kWaves : 1][kMma ? 16 : 1][(D + 16) / 8];
};

// The decode of one workgroup. POL is the cache-policy operand of the page
// loads: kLoadNonTemporal when every page is read by one row only (streamed
// once: the lines do not displace the small per-launch data -- plan, tables,
// queries, records -- from L2); 0 otherwise, so that a page shared by many
// rows (a forked prefix) is served from the caches after its first read.
// plan_d, ctr0, len_t0, pre_t0 and stamp were requested by decode_kernel:
// the wave's plan descriptors (planned modes), its launch counter,
// seq_lens[tid], the leading table entries sequence tid leaves out of the
// stream and the plan's stamp.
template <typename T, int D, int G, int MODE, int POL>
__device__ __forceinline__ void decode_body(const DecodeParams& p,
                                            DecodeLds<T, D, G, MODE != kModePlain>& lds,
                                            int* s_pref, int4 plan_d, int plan_pos,
                                            uint32_t ctr0, int len_t0, int pre_t0, int stamp,
                                            TimelineStamps& tl) {
  constexpr bool FUSED = MODE != kModePlain;
  constexpr bool PLANNED = MODE >= kModePlanned;
  constexpr bool kMma = decode_mma<T, D, G>();
  using S = DecodeShape<T, D>;
  constexpr int EPL = S::EPL, LPR = S::LPR, RPL = S::RPL, NR = S::NR;
  constexpr int REC = rec_words(G, D);
  constexpr int NPART = 2 * kWaves;
  constexpr int DPL = (D + 63) / 64;  // output dims per lane in the row epilogue
  constexpr int QR = q_stage_rows<T, D, G>();
  // Partial records loaded per batch in a merge: G*DPL + 2 words per lane
  // each, about 48 words (96 VGPRs) a batch -- at 64 words the batch's
  // registers cost the d = 128, G = 7 kernel its second wave per SIMD.
  constexpr int MC = 48 / (G * DPL + 2) > 8 ? 8 : (48 / (G * DPL + 2) < 2 ? 2 : 48 / (G * DPL + 2));
  // Register buffers per wave: while one block is computed, NBUF - 1 are in
  // flight. The matrix-core decode (16-bit K/V) takes three: the bytes in
  // flight then also cover the stretches in which the compute unit's other
  // workgroup is not streaming (its late start, the end of the launch), and
  // its state per head is small enough to keep two waves per SIMD. 32-bit
  // K/V lacks the registers for a third.
  constexpr int NBUF = kMma ? 3 : 2;
  // Blocks a planned launch requests before the prologue's appends: three
  // at d = 128 (measured 0.6 us faster at Qwen3-0.6B's shape) except in a
  // cascade step (1 us slower there), two otherwise.
  constexpr int kPreIssued = kMma && D == 128 && NBUF == 3 ? 3 : 2;
  constexpr int kNewCap = new_row_cap<T>();
  static_assert(kNewCap >= kPreIssued, "pre-issued blocks must find their new rows in LDS");
  auto& s_part = lds.part;
  auto& s_part_row = lds.part_row;
  auto& s_q = lds.q;
  auto& s_new = lds.nw;
  auto& s_vt = lds.vt;

  const int tid = threadIdx.x;
  // The wave index and everything derived from LDS-held prefixes below are
  // wave-uniform; readfirstlane tells the compiler so, which keeps the
  // streaming loop a scalar loop (a divergent trip count would make it an
  // exec-masked loop, with conservative waits on the loads in flight).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane % LPR, rsub = lane / LPR;
  const int B = p.B, Hkv = p.Hkv, mbps = p.mbps;
  const int Hq = Hkv * G;
  T* __restrict__ ob = reinterpret_cast<T*>(p.out);

  int* s_len = s_pref + B + 1;  // fused step: valid sequence lengths
  const T* __restrict__ kp = reinterpret_cast<const T*>(p.k_pool);
  const T* __restrict__ vp = reinterpret_cast<const T*>(p.v_pool);
  const size_t tile = (size_t)16 * D;  // elements of one (block, head) tile
  const int voff = (int)(((size_t)rsub * D + (size_t)col * EPL) * sizeof(T));
  // Matrix-core decode: K is read straight into the MFMA operand layout --
  // lane l takes key row l%16, elements 32r + 8*(l/16) .. +8 in its r-th
  // load; the four lanes of a key read 64 contiguous bytes per load, so the
  // requests are those of the coalesced load. V keeps the coalesced layout
  // (it is transposed through LDS).
  const int koff =
      kMma ? (int)(((size_t)(lane & 15) * D + (size_t)(lane >> 4) * EPL) * sizeof(T)) : voff;
  // K and V packets of one block, as raw buffer loads through a descriptor
  // of the block's tile: a block not fetched (past the wave's end, or an
  // invalid page) gets a descriptor of zero records, which returns zeros
  // without a memory access. With loads under a branch instead the compiler
  // cannot count the loads in flight and waits for every earlier block
  // before reusing a buffer's registers, which would serialize the pipeline.
  // (POL: see above.)
  auto load_pages = [&](Buf<T, D>& bf, int id, int kvh, bool fetch) __attribute__((always_inline)) {
    const size_t tb = ((size_t)(fetch ? id : 0) * Hkv + kvh) * tile;
    const int nrec = fetch ? (int)(tile * sizeof(T)) : 0;
    const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(kp + tb), 0, nrec,
                                                      kBufferWord3);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(vp + tb), 0, nrec,
                                                      kBufferWord3);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int o = voff + r * RPL * D * (int)sizeof(T);
      const int ok = kMma ? koff + r * 32 * (int)sizeof(T) : o;
      const u32x4_t kx = __builtin_amdgcn_raw_buffer_load_b128(rk, ok, 0, POL);
      const u32x4_t vx = __builtin_amdgcn_raw_buffer_load_b128(rv, o, 0, POL);
      bf.k[r] = make_uint4(kx.x, kx.y, kx.z, kx.w);
      bf.v[r] = make_uint4(vx.x, vx.y, vx.z, vx.w);
    }
  };
  Buf<T, D> b0, b1, b2;
  // With a plan the wave's first kPreIssued blocks are requested as soon as
  // its descriptors arrive: HBM starts streaming one round trip into the
  // launch, while the prefix, the query staging and the appends run.
  uint32_t* const ctr = p.ws_ctr + (size_t)blockIdx.x * kWaves + wave;
  auto end_epoch = [&](uint32_t ep) __attribute__((always_inline)) {
    if (lane == 0) __hip_atomic_store(ctr, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  const T* __restrict__ qb = reinterpret_cast<const T*>(p.q);
  // Descriptors of 64 consecutive blocks, one per lane: page id, valid
  // rows and row, read back with readlane when the block is issued.
  // d_nv holds the valid rows in bits 0-7 and "last block of its row" in
  // bit 8; d_pos is the row's new-token position (fused step).
  int d_id = 0, d_nv = 0, d_row = -1, d_pos = 0, cbase = 0;
  // RoPE cos/sin packets of position pos for lane column col: rotate_half
  // pairs element i with i + D/2, so both halves use table columns
  // (col % (LPR/2)) * EPL onwards.
  auto rope_packets = [&](int pos, uint4& cs, uint4& sn) __attribute__((always_inline)) {
    const size_t to = (size_t)pos * (D / 2) + (size_t)(col % (LPR / 2)) * EPL;
    cs = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.cos_t) + to);
    sn = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.sin_t) + to);
  };
  // RMSNorm weight packet of lane column col (zeros when w is null), read
  // where it is used (an L1 hit) rather than held across the streaming loop.
  // RMSNorm weight packet of lane column col, read where it is used (an L1
  // hit) rather than held across the streaming loop. A null weight (no
  // norm) reads q instead, which norm_rope_packet then ignores.
  auto load_weight = [&](const void* w) __attribute__((always_inline)) {
    const T* wp = reinterpret_cast<const T*>(w ? w : p.q);
    return *reinterpret_cast<const uint4*>(wp + col * EPL);
  };
  // Query packets of QR consecutive rows from q_base on, staged in this
  // wave's LDS slice (fused step: q_norm + RoPE at the row's new position).
  // Staging is split into loads and then math + LDS stores, so the first
  // stage's loads are in flight together with the first blocks' loads.
  constexpr int QITEMS = QR * G;
  constexpr int QPASSES = (QITEMS + RPL - 1) / RPL;
  int q_base = 0, q_top = 0;  // staged rows [q_base, q_top)
  uint4 sq_q[QPASSES], sq_c[QPASSES], sq_s[QPASSES], sq_w;
  // Every staging load is unconditional, with its indices clamped into
  // range (items past the end re-read a valid row and are never used): a
  // load under a branch with a zero default would make the compiler copy
  // its result at the join and wait for it right after issue.
  // Issues the query staging loads of QR rows from row0 on (items past the
  // last row re-read a clamped row and are never stored). The fused step
  // ropes each query at its row's new position: from the plan (lane t holds
  // row row0 + t's) when it is loaded before the barrier, else from s_len.
  auto stage_q_load = [&](int row0) __attribute__((always_inline)) {
    const int nrows = B * Hkv;
    q_base = row0;
    if constexpr (FUSED) sq_w = load_weight(p.qw);
#pragma unroll
    for (int ps = 0; ps < QPASSES; ++ps) {
      const int item = ps * RPL + rsub;
      const int t = item / G, g = item - t * G;
      const int r = row0 + t < nrows ? row0 + t : nrows - 1;
      const int b = r / Hkv, kvh = r - b * Hkv;
      sq_q[ps] = *reinterpret_cast<const uint4*>(
          qb + ((size_t)b * Hq + (size_t)kvh * G + g) * D + (size_t)col * EPL);
      if constexpr (FUSED) {
        const int pos = PLANNED ? __shfl(plan_pos, t, 64) : s_len[b] - 1;
        rope_packets(pos > 0 ? pos : 0, sq_c[ps], sq_s[ps]);
      }
    }
  };
  uint64_t amask = 0;
  int a_src = -1, a_slot = -1;
  int a_ord = 0;  // appends started so far (wave-uniform)
  uint4 a_k, a_v, a_c, a_s, a_w;  // one pass's loads (append_load)
  auto append_load = [&]() __attribute__((always_inline)) {
    int src = -1, ord = -1;
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      if (amask) {
        const int k = __builtin_ctzll(amask);
        amask &= amask - 1;
        if (rsub == i) {
          src = k;
          ord = a_ord;
        }
        ++a_ord;
      }
    }
    a_src = src;
    a_slot = ord;
    // Lane groups without a row load lane 0's (a valid block of the chunk)
    // and store nothing.
    const int sl = src >= 0 ? src : 0;
    const int rw = __shfl(d_row, sl, 64), pos = __shfl(d_pos, sl, 64);
    const int row = rw > 0 ? rw : 0;  // a wave without blocks loads row 0
    a_w = load_weight(p.kw);
    const size_t no = (size_t)row * D + (size_t)col * EPL;
    a_k = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.k_new) + no);
    a_v = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.v_new) + no);
    rope_packets(pos, a_c, a_s);
  };
  if constexpr (PLANNED) {
    // A plan built for another step shape (another prefix, prefix groups
    // where none are expected, or the reverse) does not describe this
    // launch's page stream: nothing of it is used, the launch does no work
    // (every wave still advances its launch counter) and the error is
    // flagged, as the caller's.
    if (__builtin_amdgcn_readfirstlane(stamp) != p.plan_stamp) {
      if (blockIdx.x == 0 && tid == 0) ws_raise(p.ws_err, RLSE_WS_ERR_PREFIX);
      end_epoch(next_epoch(ctr0));
      return;
    }
    RLSE_TL(1);
    // The plan gives the first row and the appends of the first 64 blocks:
    // their query and append loads go out ahead of the first blocks', so the
    // prologue's math waits for them alone and not behind the launch's first
    // wave of block loads (loads complete in order).
    d_id = plan_d.x;
    d_nv = plan_d.y;
    d_row = plan_d.z;
    d_pos = plan_d.w;
    const int row0 = __builtin_amdgcn_readfirstlane(plan_d.z);
    stage_q_load(row0 > 0 ? row0 : 0);
    amask = __ballot((d_nv & 256) != 0);
    append_load();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < kPreIssued; ++k) {
      if (k == 2 && p.pre) break;
      const int nv = __builtin_amdgcn_readlane(plan_d.y, k) & 255;
      const int row = __builtin_amdgcn_readlane(plan_d.z, k);
      const int kvh = nv > 0 ? row % Hkv : 0;
      load_pages(k == 0 ? b0 : (k == 1 ? b1 : b2), __builtin_amdgcn_readlane(plan_d.x, k), kvh,
                 nv > 0);
    }
    RLSE_TL(2);
  }
  if (wave == 0) block_prefix(p.seq_lens, B, mbps, s_pref, len_t0, p.prefix, p.seq_pre, pre_t0);
  if constexpr (FUSED) {
    if (tid < B) s_len[tid] = valid_len(len_t0, mbps);
    for (int b = tid + kThreads; b < B; b += kThreads) s_len[b] = valid_len(p.seq_lens[b], mbps);
  }
  if (tid < NPART) s_part_row[tid] = -1;
  __syncthreads();
  RLSE_TL(3);
  const long long w = blockIdx.x;
  if (w == 0) {  // rows without keys and invalid rows produce zeros
    for (int b = 0; b < B; ++b) {
      if (s_pref[b + 1] != s_pref[b]) continue;
      if (tid == 0 && p.seq_lens[b] > mbps * 16) ws_raise(p.ws_err, RLSE_WS_ERR_LENGTH);
      for (int i = tid; i < Hq * D; i += kThreads)
        ob[(size_t)b * Hq * D + i] = Elem<T>::from_f32(0.f);
    }
  }
  const uint32_t ep = next_epoch(ctr0);
  const long long total = (long long)Hkv * __builtin_amdgcn_readfirstlane(s_pref[B]);
  if (total == 0) {
    end_epoch(ep);
    return;
  }
  const long long we = effective_groups(total, p.W);
  if (w >= we) {
    end_epoch(ep);
    return;
  }
  const long long glo = range_lo(w, total, we, p.W, p.w1);
  const long long ghi = range_lo(w + 1, total, we, p.W, p.w1);
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

  // This wave's parked pieces (slot 0: the row that started before the
  // wave's range, 1: the row that continues after it), kept in registers
  // beside the LDS copy the group reads: row (-1 = none), start and blocks.
  int part_row0 = -1, part_row1 = -1, part_nb0 = 0, part_nb1 = 0;
  long long part_R0 = 0, part_R1 = 0;
  // Cascade step: the first and last row finished inside this wave's range
  // (consecutive rows, their states parked in pre_own).
  int def_lo = -1, def_hi = -1;

  if (nblk > 0) {
    // Descriptors of 64 consecutive blocks, one per lane: page id, valid
    // rows and row, read back with readlane when the block is issued.
    // d_nv holds the valid rows in bits 0-7 and "last block of its row" in
    // bit 8; d_pos is the row's new-token position (fused step).
    auto load_chunk = [&](int base) __attribute__((always_inline)) {
      cbase = base;
      int4 d;
      if (PLANNED && base == 0)  // the plan's copy, loaded before the barrier
        d = plan_d;
      else
        d = block_desc(wlo + base + lane, whi, s_pref, p.tables, p.seq_lens, B, Hkv, mbps,
                       p.num_blocks, p.prefix, p.seq_pre);
      d_id = d.x;
      d_nv = d.y;
      d_row = d.z;
      d_pos = d.w;
    };
    load_chunk(0);

    // The wave's last row; staging never goes past it.
    int last_row;
    {
      const long long f = whi - 1;
      const int b = locate_seq(s_pref, B, Hkv, f);
      const int nb = s_pref[b + 1] - s_pref[b];
      last_row = __builtin_amdgcn_readfirstlane(b * Hkv + (int)((f - (long long)Hkv * s_pref[b]) / nb));
    }
    int q_items = 0;  // staged (row, head) items: (q_top - q_base) * G
    auto stage_bounds = [&](int row0) __attribute__((always_inline)) {
      q_base = row0;
      q_top = row0 + QR < last_row + 1 ? row0 + QR : last_row + 1;
      q_items = (q_top - q_base) * G;
    };
    // In-loop restaging (a wave whose range holds more than QR rows): one
    // pass at a time in a rolled loop, which keeps the streaming loop's code
    // (unrolled over the block buffers) small.
    auto stage_q_refill = [&](int row0) __attribute__((always_inline)) {
      const int nrows = B * Hkv;
      stage_bounds(row0);
      const uint4 w = FUSED ? load_weight(p.qw) : make_uint4(0, 0, 0, 0);
#pragma unroll 1
      for (int ps = 0; ps * RPL < q_items; ++ps) {
        const int item = ps * RPL + rsub;
        const int t = item / G, g = item - t * G;
        const int r = row0 + t < nrows ? row0 + t : nrows - 1;
        const int b = r / Hkv, kvh = r - b * Hkv;
        uint4 x = *reinterpret_cast<const uint4*>(
            qb + ((size_t)b * Hq + (size_t)kvh * G + g) * D + (size_t)col * EPL);
        consume(x);  // every load used on every path (see after_pre_issue)
        if constexpr (FUSED) {
          const int pos = s_len[b] - 1;
          uint4 cs, sn;
          rope_packets(pos > 0 ? pos : 0, cs, sn);
          consume(cs);
          consume(sn);
          x = norm_rope_packet<T, D>(x, p.qw != nullptr, w, p.inv_d, p.eps, cs, sn, col);
        }
        if (item < q_items) s_q[wave][t][g][col] = x;
      }
    };
    // Passes past the staged items skip their math (the loads above were
    // issued for every pass, clamped, so no wait depends on the item count).
    auto stage_q_store = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int ps = 0; ps < QPASSES; ++ps) {
        if (ps > 0 && ps * RPL >= q_items) break;
        const int item = ps * RPL + rsub;
        const int t = item / G, g = item - t * G;
        uint4 y = sq_q[ps];
        if constexpr (FUSED)
          y = norm_rope_packet<T, D>(sq_q[ps], p.qw != nullptr, sq_w, p.inv_d, p.eps, sq_c[ps],
                                     sq_s[ps], col);
        if (item < q_items) s_q[wave][t][g][col] = y;
      }
    };

    // Fused step: the new token of every row whose last block lies in this
    // wave's range is appended by this wave (k_norm + RoPE of k, raw v), as
    // that block is read by this wave only. The first kPreIssued blocks are
    // issued before the appends are stored. The wave's first kNewCap appends
    // (in stream order) also go to LDS (s_new) and their blocks take the new
    // row from there whenever they are loaded, so no load waits for an append
    // store. A wave with more appends waits for its stores (vmcnt(0)) before
    // issuing any later block -- the compute unit's write-through L1 then shows
    // them to its loads -- and only blocks issued after that wait can hold an
    // append past the first kNewCap. A pass appends up to RPL rows, one per
    // lane group.
    auto append_store = [&]() __attribute__((always_inline)) {
      const int sl = a_src >= 0 ? a_src : 0;
      const int row = __shfl(d_row, sl, 64), pos = __shfl(d_pos, sl, 64);
      const int id = __shfl(d_id, sl, 64);
      const uint4 kr = norm_rope_packet<T, D>(a_k, p.kw != nullptr, a_w, p.inv_d, p.eps, a_c, a_s,
                                              col);
      if (a_src >= 0) {
        const int kvh = row % Hkv;
        const size_t dst = (((size_t)id * Hkv + kvh) * 16 + (pos & 15)) * D + (size_t)col * EPL;
        *reinterpret_cast<uint4*>(const_cast<T*>(kp) + dst) = kr;
        *reinterpret_cast<uint4*>(const_cast<T*>(vp) + dst) = a_v;
        if (a_slot < kNewCap) {
          s_new[wave][a_slot][0][col] = kr;
          s_new[wave][a_slot][1][col] = a_v;
        }
      }
    };

    // Before the first blocks are issued (planned launches: at the start):
    // the first row's query loads and the first append pass's loads.
    if constexpr (!PLANNED) {
      stage_q_load(__builtin_amdgcn_readfirstlane(d_row));
      if constexpr (FUSED) {
        amask = __ballot((d_nv & 256) != 0);
        append_load();
      }
    }
    stage_bounds(q_base);
    // Keep these loads ahead of the block loads: the math after the first
    // issues waits for them, and a wait for a load issued after the blocks
    // would wait for the blocks too (loads complete in order).
    __builtin_amdgcn_sched_barrier(0);
    // After the first kPreIssued blocks are issued: finish the query stage
    // and every append.
    auto after_pre_issue = [&]() __attribute__((always_inline)) {
      stage_q_store();
      if constexpr (FUSED) append_store();
      // Every prologue load is consumed here, in straight-line code: a
      // staging pass past the staged items, or an append pass with nothing to
      // store, would otherwise leave its load pending into the streaming loop,
      // where the compiler cannot count the loads issued since and drains
      // every block in flight (vmcnt(0)) before it first reuses the register.
#pragma unroll
      for (int ps = 0; ps < QPASSES; ++ps) {
        consume(sq_q[ps]);
        if constexpr (FUSED) {
          consume(sq_c[ps]);
          consume(sq_s[ps]);
        }
      }
      if constexpr (FUSED) {
        consume(sq_w);
        consume(a_k);
        consume(a_v);
        consume(a_c);
        consume(a_s);
        consume(a_w);
        for (int base = 0; base < nblk; base += 64) {
          if (base) {
            load_chunk(base);
            amask = __ballot((d_nv & 256) != 0);
          }
          while (amask) {
            append_load();
            append_store();
          }
        }
        if (nblk > 64) load_chunk(0);
        if (a_ord > kNewCap) wait_vm_stores();
      }
    };

    int issued_row = -1;
    int n_last = 0;  // last blocks of rows issued so far = their append ordinal
    // Block j of the wave's range (j >= nblk: past the end, never computed):
    // its bookkeeping, then (unless the plan's early requests already made
    // them) its loads, issued for every j (load_pages).
    auto issue = [&](Buf<T, D>& bf, int j, bool loads) __attribute__((always_inline)) {
      const bool real = j < nblk;
      j = real ? j : nblk - 1;
      if (j - cbase >= 64) load_chunk(cbase + 64);
      const int k = j - cbase;
      const int id = __builtin_amdgcn_readlane(d_id, k);
      const int nvf = __builtin_amdgcn_readlane(d_nv, k);
      const int row = __builtin_amdgcn_readlane(d_row, k);
      const int kvh = row % Hkv;
      const int nv = nvf & 255;
      bf.nvalid = nv;
      bf.row = row;
      bf.newrow = row != issued_row;
      const bool row_end = FUSED && (nvf & 256);
      bf.sub = (row_end && n_last < kNewCap) ? n_last : -1;
      if (real) {
        if (row_end) ++n_last;
        issued_row = row;
      }
      if (loads) load_pages(bf, id, kvh, real && nv > 0);
    };

    // nms[g] is the exponent offset -m[g] (0 while m[g] is -inf) and thr[g]
    // the raw score above which the running max must move, (m[g] +
    // kLazyLog2) / c (-inf while m[g] is -inf); both are kept beside m[g],
    // as they change only when the running max moves.
    float m[G], l[G], acc[G][EPL], nms[G], thr[G];
    int cur_row = -1;
    const float inv_c = 1.f / p.c;
    uint4 qv[G];
    // Matrix-core decode state: lane l works for head l%16 (heads past G have
    // zero queries and are never stored) and holds keys 4*(l/16) .. +3 of
    // each block's S^T column and rows 16t + 4*(l/16) .. +3 of O^T tile t;
    // m1, nms1 and thr1 are the head's running max, exponent offset and
    // rescale threshold (equal in the head's four lanes), l1 the lane's part
    // of the head's sum. mqv holds the head's query in the K operand layout.
    const int mh = lane & 15, mq = lane >> 4;
    uint4 mqv[kMma ? NR : 1];
    mma_f32x4_t macc[kMma ? D / 16 : 1];
    float m1 = -INFINITY, l1 = 0.f, nms1 = 0.f, thr1 = -INFINITY;
    auto reset = [&]() __attribute__((always_inline)) {
      if constexpr (kMma) {
        m1 = -INFINITY;
        l1 = 0.f;
        nms1 = 0.f;
        thr1 = -INFINITY;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) macc[t] = mma_f32x4_t{0.f, 0.f, 0.f, 0.f};
        return;
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        nms[g] = 0.f;
        thr[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
      }
    };
    // Ends the wave's part of cur_row: merge the lane groups, then write the
    // output (row wholly inside this wave) or park the state in LDS.
    auto finalize = [&]() __attribute__((always_inline)) {
      if constexpr (kMma) {
        // The head's sum over its four lanes; m1 is already common to them.
        float lt = l1 + __shfl_xor(l1, 16, 64);
        lt = lt + __shfl_xor(lt, 32, 64);
        long long R;
        int nb;
        row_extent(cur_row, R, nb);
        const int b = cur_row / Hkv, kvh = cur_row - b * Hkv;
        if (R >= wlo && R + nb <= whi) {
          if (p.pre) {
            // Cascade step: park the row's state; the prefix states are
            // combined into it after the stream.
            if (mh < G) {
              float* dst = p.pre_own + ((size_t)b * Hq + (size_t)kvh * G + mh) *
                                           prefix_row_floats(D);
#pragma unroll
              for (int t = 0; t < D / 16; ++t)
                *reinterpret_cast<float4*>(dst + 16 * t + 4 * mq) =
                    make_float4(macc[t][0], macc[t][1], macc[t][2], macc[t][3]);
              if (mq == 0) *reinterpret_cast<float2*>(dst + D) = make_float2(m1, lt);
            }
            def_lo = def_lo < 0 ? cur_row : def_lo;
            def_hi = cur_row;
          } else if (mh < G) {
            const float inv = lt > 0.f ? 1.f / lt : 0.f;  // all pages skipped -> zeros
            T* dst = ob + ((size_t)b * Hq + (size_t)kvh * G + mh) * D + 4 * mq;
#pragma unroll
            for (int t = 0; t < D / 16; ++t) {
              const uint32_t w0 = (uint32_t)bits_sel<T>(macc[t][0] * inv) |
                                  ((uint32_t)bits_sel<T>(macc[t][1] * inv) << 16);
              const uint32_t w1 = (uint32_t)bits_sel<T>(macc[t][2] * inv) |
                                  ((uint32_t)bits_sel<T>(macc[t][3] * inv) << 16);
              *reinterpret_cast<uint2*>(dst + 16 * t) = make_uint2(w0, w1);
            }
          }
        } else {
          const int slot = 2 * wave + (R < wlo ? 0 : 1);
          if (R < wlo) {
            part_row0 = cur_row;
            part_R0 = R;
            part_nb0 = nb;
          } else {
            part_row1 = cur_row;
            part_R1 = R;
            part_nb1 = nb;
          }
          if (mh < G) {
#pragma unroll
            for (int t = 0; t < D / 16; ++t)
#pragma unroll
              for (int i = 0; i < 4; ++i) s_part[slot][mh][16 * t + 4 * mq + i] = macc[t][i];
            if (mq == 0) {
              s_part[slot][mh][D] = m1;
              s_part[slot][mh][D + 1] = lt;
            }
          }
          if (lane == 0) s_part_row[slot] = cur_row;
        }
        return;
      }
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
          l[g] = fmaf(l[g], sa, mul_rn(lo_, sb));
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            const float ao = __shfl_xor(acc[g][e], off, 64);
            acc[g][e] = fmaf(acc[g][e], sa, mul_rn(ao, sb));
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
            float y[EPL];
#pragma unroll
            for (int e = 0; e < EPL; ++e) y[e] = acc[g][e] * inv;
            *reinterpret_cast<uint4*>(dst) = pack_packet<T>(y);
          }
        }
      } else {
        const int slot = 2 * wave + (R < wlo ? 0 : 1);
        if (R < wlo) {
          part_row0 = cur_row;
          part_R0 = R;
          part_nb0 = nb;
        } else {
          part_row1 = cur_row;
          part_R1 = R;
          part_nb1 = nb;
        }
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
    auto compute = [&](const Buf<T, D>& bf) __attribute__((always_inline)) {
      if constexpr (kMma) {
        if (bf.newrow) {
          if (cur_row >= 0) finalize();
          reset();
          cur_row = bf.row;
          if (cur_row < q_base || cur_row >= q_top) stage_q_refill(cur_row);
          const int hq = mh < G ? mh : G - 1;
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const uint4 x = s_q[wave][cur_row - q_base][hq][4 * r + mq];
            mqv[r] = mh < G ? x : make_uint4(0, 0, 0, 0);
          }
        }
        const int nv = bf.nvalid;
        uint4 kr[NR], vr[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          kr[r] = bf.k[r];
          vr[r] = bf.v[r];
        }
        if constexpr (FUSED) {
          if (bf.sub >= 0) {  // the new token (slot nv-1) may not be stored yet: take it from LDS
            const int slot = nv - 1;
            if (mh == slot) {
#pragma unroll
              for (int r = 0; r < NR; ++r) kr[r] = s_new[wave][bf.sub][0][4 * r + mq];
            }
            if (rsub == slot % RPL) {
              const uint4 vn = s_new[wave][bf.sub][1][col];
#pragma unroll
              for (int r = 0; r < NR; ++r)
                if (r == slot / RPL) vr[r] = vn;
            }
          }
        }
        // Rows past the sequence end: V = 0 (their p is 0, and 0 * garbage
        // could be NaN), scores -inf below.
        if (nv < 16) {
#pragma unroll
          for (int r = 0; r < NR; ++r)
            if (r * RPL + rsub >= nv) vr[r] = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) s_vt[wave][r * RPL + rsub][col] = vr[r];
        // S^T (keys x heads) = K . Q^T
        mma_f32x4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < NR; ++r) sacc = Mma16<T>::k32(kr[r], mqv[r], sacc);
        float sv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = 4 * mq + i < nv ? sacc[i] : -INFINITY;
        // Lazy rescaling (as below): the head's new max is taken over its
        // four lanes.
        const float cand = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        if (__any(cand > thr1)) {
          float cm = fmaxf(cand, __shfl_xor(cand, 16, 64));
          cm = fmaxf(cm, __shfl_xor(cm, 32, 64));
          const float mn = fmaxf(m1, cm * p.c);
          const float alpha = (mn == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m1 - mn);
          l1 *= alpha;
#pragma unroll
          for (int t = 0; t < D / 16; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) macc[t][i] *= alpha;
          m1 = mn;
          nms1 = (mn == -INFINITY) ? 0.f : -mn;
          thr1 = (mn == -INFINITY) ? -INFINITY : (mn + kLazyLog2) * inv_c;
        }
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], p.c, nms1));
          l1 += pr[i];
        }
        // P^T in the accumulator layout is the B operand of O^T += V^T . P^T;
        // V^T tile t comes from LDS by transposing reads: within each 16-lane
        // group, lane 4j+a points at key row 4*(l/16)+j, columns 16t+4a .. +3,
        // and lane 4a+e receives column 16t+4a+e of those four keys.
        const uint2 pp = make_uint2(Packet<T>::pack2(pr[0], pr[1]), Packet<T>::pack2(pr[2], pr[3]));
        const uint16_t* vrow =
            reinterpret_cast<const uint16_t*>(&s_vt[wave][4 * mq + ((lane & 15) >> 2)][0]) +
            4 * (lane & 3);
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
          const mma_i16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((mma_lds_i16x4_t*)(vrow + 16 * t));
          macc[t] = Mma16<T>::k16(a, pp, macc[t]);
        }
      } else {
        // 32-bit K/V: the lane-group math on the VALU.
        if (bf.newrow) {
          if (cur_row >= 0) finalize();
          reset();
          cur_row = bf.row;
          if (cur_row < q_base || cur_row >= q_top) stage_q_refill(cur_row);
#pragma unroll
          for (int g = 0; g < G; ++g) qv[g] = s_q[wave][cur_row - q_base][g][col];
        }
        // A skipped block (nv = 0) runs the same math with every row masked,
        // which leaves m, l and acc unchanged; consuming its registers on every
        // path keeps the compiler's count of loads in flight exact.
        const int nv = bf.nvalid;
        uint4 kr[NR], vr[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          kr[r] = bf.k[r];
          vr[r] = bf.v[r];
        }
        if constexpr (FUSED) {
          if (bf.sub >= 0) {  // the new token (slot nv-1) may not be stored yet: take it from LDS
            const int slot = nv - 1;
            if (rsub == slot % RPL) {
              const uint4 kn = s_new[wave][bf.sub][0][col], vn = s_new[wave][bf.sub][1][col];
#pragma unroll
              for (int r = 0; r < NR; ++r)
                if (r == slot / RPL) {
                  kr[r] = kn;
                  vr[r] = vn;
                }
            }
          }
        }
        // Raw scores q.k, summed over the LPR lanes of each row (all G*NR
        // partial dots first, then the reduction steps across all of them).
        float s[G][NR];
        {
          float part[G * NR];
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int r = 0; r < NR; ++r) part[g * NR + r] = Packet<T>::dot0(qv[g], kr[r]);
          group_sum_n<LPR>(part);
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int r = 0; r < NR; ++r) s[g][r] = part[g * NR + r];
        }
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
        float vf[NR][EPL];
#pragma unroll
        for (int r = 0; r < NR; ++r) Packet<T>::unpack(vr[r], vf[r]);
        // Lazy rescaling: a running max moves only when a scaled score exceeds
        // it by more than kLazyLog2 (probabilities then stay below
        // 2^kLazyLog2). The test compares raw scores with thr (c > 0), every
        // head at once; when any lane of the wave needs it, every head's max
        // moves to its largest score so far.
        float cand[G];
        bool move = false;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          cand[g] = s[g][0];
#pragma unroll
          for (int r = 1; r < NR; ++r) cand[g] = fmaxf(cand[g], s[g][r]);
          move = move || cand[g] > thr[g];
        }
        if (__any(move)) {
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float mn = fmaxf(m[g], cand[g] * p.c);
            const float alpha = (mn == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m[g] - mn);
            l[g] *= alpha;
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
            m[g] = mn;
            nms[g] = (mn == -INFINITY) ? 0.f : -mn;
            thr[g] = (mn == -INFINITY) ? -INFINITY : (mn + kLazyLog2) * inv_c;
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float pr[NR];
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            pr[r] = __builtin_amdgcn_exp2f(fmaf(s[g][r], p.c, nms[g]));
            l[g] += pr[r];
          }
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

    // While block i is computed, blocks i + 1 .. i + NBUF - 1 are in flight
    // (an index past the end loads nothing and is never computed). With a
    // plan, blocks 0 and 1 were requested at the start of the launch.
    issue(b0, 0, !PLANNED);
    if constexpr (PLANNED) issue(b1, 1, false);
    after_pre_issue();
    RLSE_TL(4);
    if constexpr (!PLANNED) issue(b1, 1, true);
    if constexpr (NBUF == 3) issue(b2, 2, !PLANNED || kPreIssued < 3 || p.pre);
    for (int i = 0;;) {
      compute(b0);
#ifdef RLSE_DECODE_TIMELINE
      if (i == 0) RLSE_TL(5);
#endif
      if (++i == nblk) break;
      issue(b0, i + NBUF - 1, true);
      compute(b1);
      if (++i == nblk) break;
      issue(b1, i + NBUF - 1, true);
      if constexpr (NBUF == 3) {
        compute(b2);
        if (++i == nblk) break;
        issue(b2, i + 2, true);
      }
    }
    finalize();
    RLSE_TL(6);
  }
  // A row that began in earlier groups and ends in this one is finished by
  // wave 0 (its slot 0 row), which merges the records of groups wa .. w-1;
  // group wa used record slot 0 only if its range starts exactly at the row
  // start. Found before the barrier (two 64-bit divisions), so the wave's
  // wait there covers them.
  long long wa = 0;
  int np = 0;
  bool wa_slot1 = false;
  if (wave == 0 && part_row0 >= 0 && part_R0 < glo && part_R0 + part_nb0 <= ghi) {
    wa = group_of(part_R0, total, we, p.W, p.w1);
    np = (int)(w - wa);
    wa_slot1 = range_lo(wa, total, we, p.W, p.w1) != part_R0;
  }
  __syncthreads();
  RLSE_TL(7);

  // Rows this group holds in pieces. A row that started in an earlier group
  // and ends in this one is finished by wave 0, which merges the partials of
  // the earlier groups as they arrive; every other row is finished by the
  // wave holding its last piece in the group, which writes the output (row
  // inside the group's range) or publishes one group partial (the row
  // continues in a later group: always the group's last wave). The finishing
  // wave first combines the pieces parked by the group's waves (a row's
  // pieces sit in consecutive waves), from the last piece down. No wave both
  // publishes and merges: a wave's waits count its own stores too, so a
  // merge in the publishing wave would stand behind the publication's write
  // round trip, and a publication behind a merge would chain merges from
  // group to group. Every slot's row is read once (lane j < NPART holds slot
  // j's), so the pieces of a row are found with one ballot and their LDS
  // reads issued together.
  // Epilogue softmax states: head g's running max and sum sit in lane g
  // (hm, hl; lanes past G hold values that are never read), its
  // accumulators in A[g][k] (dimension lane + 64k) of every lane.
  // combine_heads folds a piece (pm, pl in the heads' lanes, pa) into them,
  // all in log2 units: M = max(m, mo), scales sa = 2^(m - M) and
  // sb = 2^(mo - M) (M = 0 when both are -inf, so empty states never give
  // NaN), l = l*sa + lo*sb and a = a*sa + ao*sb. The scales are computed
  // once, in the heads' own lanes, and read back per head for the
  // accumulators: one exponential pair per piece instead of one per head
  // and output dimension in every lane, on the wave's critical path at the
  // end of the launch. The sums are one fma over a product rounded on its
  // own, so every instantiation rounds them alike (left to contraction,
  // x*sa + y*sb may fuse either product).
  const int hj = lane < G ? lane : 0;  // the head a lane's hm, hl belong to
  auto combine_heads = [&](float& hm, float& hl, float(&A)[G][DPL], float pm, float pl,
                           const float(&pa)[G][DPL]) __attribute__((always_inline)) {
    const float mx = fmaxf(hm, pm);
    const float ms = (mx == -INFINITY) ? 0.f : mx;
    const float sa = __builtin_amdgcn_exp2f(hm - ms);
    const float sb = __builtin_amdgcn_exp2f(pm - ms);
    hl = fmaf(hl, sa, mul_rn(pl, sb));
    hm = mx;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float ag = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sa), g));
      const float bg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sb), g));
#pragma unroll
      for (int k = 0; k < DPL; ++k) A[g][k] = fmaf(A[g][k], ag, mul_rn(pa[g][k], bg));
    }
  };
  // Cascade step: combines the prefix slices' states of row (b, kvh) into
  // (hm, hl, A) in slice order, the loads of SB slices in flight at once
  // (a slice index past the last reloads the first of the batch, unused).
  constexpr int SB = 32 / (G * DPL) < 1 ? 1 : (32 / (G * DPL) > 8 ? 8 : 32 / (G * DPL));
  auto combine_prefix = [&](int b, int kvh, float& hm, float& hl, float(&A)[G][DPL])
      __attribute__((always_inline)) {
    constexpr int PF = prefix_row_floats(D);
    const float* pr = p.pre + ((size_t)b * Hq + (size_t)kvh * G) * PF;
    int ns = p.pre_slices;
    if (p.seq_pre) {  // prefix groups: the slices of this sequence's group, none if unforked
      const int pg = p.seq_pre[b];
      ns = pg > 0 ? (prefix_splits(pg) < ns ? prefix_splits(pg) : ns) : 0;  // at most the buffer's
    }
#pragma unroll 1
    for (int s0 = 0; s0 < ns; s0 += SB) {
      float sm[SB], sl[SB], sa[SB][G][DPL];
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const float* r = pr + (size_t)(s0 + i < ns ? s0 + i : s0) * (size_t)p.pre_stride;
        sm[i] = r[hj * PF + D];
        sl[i] = r[hj * PF + D + 1];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int k = 0; k < DPL; ++k)
            sa[i][g][k] = lane + 64 * k < D ? r[g * PF + lane + 64 * k] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < SB; ++i)
        if (s0 + i < ns) combine_heads(hm, hl, A, sm[i], sl[i], sa[i]);
    }
  };
  // Output of a finished row (NaN if a partial did not arrive within the
  // wait bound).
  auto write_row = [&](int b, int kvh, bool ok, float hl, const float(&A)[G][DPL])
      __attribute__((always_inline)) {
    const float inv = hl > 0.f ? 1.f / hl : 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float ig = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), g));
#pragma unroll
      for (int k = 0; k < DPL; ++k) {
        const int d = lane + 64 * k;
        if (d < D)
          ob[((size_t)b * Hq + (size_t)kvh * G + g) * D + d] =
              Elem<T>::from_f32(ok ? A[g][k] * ig : __builtin_nanf(""));
      }
    }
  };
  const int prow = lane < NPART ? s_part_row[lane] : -1;
#pragma unroll 1
  for (int s = 1; s >= 0; --s) {
    const int row = s ? part_row1 : part_row0;
    if (row < 0) continue;
    const long long R = s ? part_R1 : part_R0;
    const int nb = s ? part_nb1 : part_nb0;
    const bool merge = R < glo && R + nb <= ghi;  // only ever wave 0's slot 0 in wave 0
    if (merge ? wave != 0 : (R + nb > whi && whi < ghi)) continue;
    const int b = row / Hkv, kvh = row - b * Hkv;
    float hm = -INFINITY, hl = 0.f, A[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int k = 0; k < DPL; ++k) A[g][k] = 0.f;
    // Cascade step: a row finished here starts from its prefix slices'
    // states (written by the prefix launch, so ready from the launch's
    // start): their round trip then runs under the LDS reads of the pieces
    // and, for a merged row, under the wait for the earlier groups'
    // records. A published piece leaves them to the row's finisher.
    if (p.pre && R + nb <= ghi) combine_prefix(b, kvh, hm, hl, A);
    // Slots holding pieces of the row: this wave's slot s and, in the waves
    // below it (every wave when merging), the slot naming the same row. A
    // row's pieces sit in consecutive waves, at most one slot per wave.
    const int top = merge ? kWaves - 1 : wave;
    const uint64_t hit = __ballot(lane < 2 * top + 2 && prow == row &&
                                  ((lane >> 1) != wave || (lane & 1) == s));
    float pm[kWaves], pl[kWaves], pa[kWaves][G][DPL];
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) {
      const int slot = 2 * wv + (int)((hit >> (2 * wv + 1)) & 1);
      pm[wv] = s_part[slot][hj][D];
      pl[wv] = s_part[slot][hj][D + 1];
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < DPL; ++k) {
          const int d = lane + 64 * k;
          pa[wv][g][k] = d < D ? s_part[slot][g][d] : 0.f;
        }
    }
#pragma unroll
    for (int wv = kWaves - 1; wv >= 0; --wv) {
      if (((hit >> (2 * wv)) & 3) == 0) continue;
      combine_heads(hm, hl, A, pm[wv], pl[wv], pa[wv]);
    }
    RLSE_TL(8);
    if (R + nb > ghi) {
      // The row continues in a later group: publish this group's piece
      // (slot 0 = the group's first segment, 1 = a later one) and leave.
      uint64_t* rec = p.ws_rec + ((size_t)w * 2 + (R <= glo ? 0 : 1)) * (size_t)REC;
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < DPL; ++k) {
          const int d = lane + 64 * k;
          if (d < D) st_tagged(rec + (size_t)g * D + d, ep, A[g][k]);
        }
      // m then l of every head: lane g < G stores words G*D + g and G*D + G + g.
      if (lane < G) {
        st_tagged(rec + G * D + lane, ep, hm);
        st_tagged(rec + G * D + G + lane, ep, hl);
      }
      continue;
    }
    bool ok = true;
    if (R < glo) {
      // The row's last block is in this group (wave 0's slot 0 row, whose
      // wa, np and wa_slot1 were found before the barrier): combine the
      // pieces of the earlier groups with this one's, each record once all
      // of its words carry this launch's epoch.
      auto record = [&](int j) __attribute__((always_inline)) {
        const int slot = (j == 0 && wa_slot1) ? 1 : 0;
        return p.ws_rec + ((size_t)(wa + j) * 2 + slot) * (size_t)REC;
      };
      const unsigned long long t0 = wall_clock64();
      auto timed_out = [&]() __attribute__((always_inline)) {
        return wall_clock64() - t0 > p.wait_ticks;
      };
      // Records are loaded MC at a time, each as G*DPL words of acc per lane
      // plus the m and l words of head j in lane j < G, and loaded again
      // (after a short sleep) until every word carries this launch's epoch.
      for (int c = 0; c < np && ok; c += MC) {
        uint64_t mm[MC], ml[MC], av[MC][G][DPL];
        for (int attempt = 0;; ++attempt) {
          if (attempt > 0) {
            if (timed_out()) {
              ok = false;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
          const uint64_t fill = (uint64_t)ep << 32;  // words not loaded count as arrived
#pragma unroll
          for (int i = 0; i < MC; ++i) {  // issue the batch's loads together
            if (c + i >= np) {
              mm[i] = fill;
              ml[i] = fill;
#pragma unroll
              for (int g = 0; g < G; ++g)
#pragma unroll
                for (int k = 0; k < DPL; ++k) av[i][g][k] = fill;
              continue;
            }
            const uint64_t* r = record(c + i);
            mm[i] = lane < G ? ld_tagged(r + G * D + lane) : fill;
            ml[i] = lane < G ? ld_tagged(r + G * D + G + lane) : fill;
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
              for (int k = 0; k < DPL; ++k) {
                const int d = lane + 64 * k;
                av[i][g][k] = d < D ? ld_tagged(r + (size_t)g * D + d) : fill;
              }
          }
          bool ready = true;
#pragma unroll
          for (int i = 0; i < MC; ++i) {
            ready = ready && tag_is(mm[i], ep) && tag_is(ml[i], ep);
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
              for (int k = 0; k < DPL; ++k) ready = ready && tag_is(av[i][g][k], ep);
          }
          if (__all(ready)) break;
        }
        if (!ok) break;
#pragma unroll
        for (int i = 0; i < MC; ++i)
          if (c + i < np) {
            float ra[G][DPL];
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
              for (int k = 0; k < DPL; ++k) ra[g][k] = tag_value(av[i][g][k]);
            combine_heads(hm, hl, A, tag_value(mm[i]), tag_value(ml[i]), ra);
          }
      }
      if (!ok && lane == 0) ws_raise(p.ws_err, RLSE_WS_ERR_MERGE_TIMEOUT);
      RLSE_TL(9);
    }
    write_row(b, kvh, ok, hl, A);
  }
  if constexpr (kMma) {
    // Cascade step: the rows this wave finished inside its range, their
    // states parked in pre_own, combined with the prefix states.
    if (p.pre && def_lo >= 0) {
      constexpr int PF = prefix_row_floats(D);
#pragma unroll 1
      for (int row = def_lo; row <= def_hi; ++row) {
        long long R;
        int nb;
        row_extent(row, R, nb);
        if (nb == 0) continue;  // no keys of its own: written by group 0
        const int b = row / Hkv, kvh = row - b * Hkv;
        const float* own = p.pre_own + ((size_t)b * Hq + (size_t)kvh * G) * PF;
        float hm = own[hj * PF + D], hl = own[hj * PF + D + 1], A[G][DPL];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int k = 0; k < DPL; ++k) {
            const int d = lane + 64 * k;
            A[g][k] = d < D ? own[g * PF + d] : 0.f;
          }
        combine_prefix(b, kvh, hm, hl, A);
        write_row(b, kvh, true, hl, A);
      }
    }
  }
  end_epoch(ep);
}

template <typename T, int D, int G, int MODE>
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeParams p) {
  constexpr bool PLANNED = MODE >= kModePlanned;
  extern __shared__ int s_pref[];  // [B + 1]; fused step: then s_len[B]
  __shared__ DecodeLds<T, D, G, MODE != kModePlain> lds;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  // Requested first of all: with a plan, the wave's first descriptors; its
  // launch counter (the epoch tags its records and is expected on those it
  // merges); seq_lens[tid] (0 past the batch) for the block prefix's first
  // chunk and the fused step's first pass over the lengths -- a raw buffer
  // load over the B lengths, so no exec-masked branch and no copy at a join
  // that would wait for it early. The lengths arrive with the descriptors,
  // so the prefix never waits behind the first blocks.
  TimelineStamps tl = {};
  RLSE_TL(0);
  int4 plan_d = make_int4(0, 0, -1, 0);
  int plan_pos = 0, stamp = 0;
  if constexpr (PLANNED) {
    const size_t at = ((size_t)blockIdx.x * kWaves + wave) * 64 + lane;
    plan_d = p.plan[at];
    plan_pos = reinterpret_cast<const int*>(p.plan + (size_t)p.W * kWaves * 64)[at];
    stamp = plan_tail(p.plan, p.W)[0];
  }
  const uint32_t ctr0 = __hip_atomic_load(p.ws_ctr + (size_t)blockIdx.x * kWaves + wave,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int len_t0 = (int)__builtin_amdgcn_raw_buffer_load_b32(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int*>(p.seq_lens), 0, p.B * 4, kBufferWord3),
      tid * 4, 0, 0);
  // The lane's skipped table entries for the block prefix's first chunk (a
  // null seq_pre gets a descriptor of zero records: zeros, no access).
  const int pre_t0 = p.seq_pre ? (int)__builtin_amdgcn_raw_buffer_load_b32(
                                     __builtin_amdgcn_make_buffer_rsrc(
                                         const_cast<int*>(p.seq_pre), 0, p.B * 4, kBufferWord3),
                                     tid * 4, 0, 0)
                               : p.prefix;
  (void)lane;
  decode_body<T, D, G, MODE, MODE == kModePlannedStream ? kLoadNonTemporal : 0>(
      p, lds, s_pref, plan_d, plan_pos, ctr0, len_t0, pre_t0, stamp, tl);
#ifdef RLSE_DECODE_TIMELINE
  RLSE_TL(10);
  if (p.timeline && lane == 0) {
    unsigned long long* dst =
        p.timeline + ((size_t)blockIdx.x * kWaves + wave) * kTimelinePoints;
#pragma unroll
    for (int k = 0; k < kTimelinePoints; ++k) dst[k] = tl.t[k];
  }
#endif
}


// Launches one instantiation of the kernel on stream (defined here, instantiated
// explicitly per element type and mode in the decode_inst_*.hip units so they
// compile in parallel).
template <typename T, int D, int G, int MODE>
int launch_decode_t(const DecodeParams& p, hipStream_t stream) {
  // Dynamic LDS: block prefix [B + 1], then (fused step) lengths [B].
  const size_t lds = (size_t)(p.B + 1 + (MODE != kModePlain ? p.B : 0)) * sizeof(int);
  hipLaunchKernelGGL((decode_kernel<T, D, G, MODE>), dim3(p.W), dim3(kThreads), lds, stream, p);
  return launch_status("decode_kernel");
}

#define RLSE_DECODE_INST_G(PREFIX, T, D, MODE)                              \
  PREFIX int launch_decode_t<T, D, 1, MODE>(const DecodeParams&, hipStream_t); \
  PREFIX int launch_decode_t<T, D, 2, MODE>(const DecodeParams&, hipStream_t); \
  PREFIX int launch_decode_t<T, D, 3, MODE>(const DecodeParams&, hipStream_t); \
  PREFIX int launch_decode_t<T, D, 4, MODE>(const DecodeParams&, hipStream_t); \
  PREFIX int launch_decode_t<T, D, 5, MODE>(const DecodeParams&, hipStream_t); \
  PREFIX int launch_decode_t<T, D, 6, MODE>(const DecodeParams&, hipStream_t); \
  PREFIX int launch_decode_t<T, D, 7, MODE>(const DecodeParams&, hipStream_t); \
  PREFIX int launch_decode_t<T, D, 8, MODE>(const DecodeParams&, hipStream_t);
// Every supported (head_dim, group size) of one element type and mode.
#define RLSE_DECODE_INSTANCES(PREFIX, T, MODE) \
  RLSE_DECODE_INST_G(PREFIX, T, 64, MODE)      \
  RLSE_DECODE_INST_G(PREFIX, T, 128, MODE)

}  // namespace rlse
