// Chunked-prefill attention over the paged KV pool, on MFMA tiles (gfx950).
//
// Reference semantics: the prefill branch of Attention::forward
// (src/backends/qwen2.rs:329-345) with prepare_causal_attention_mask
// (src/backends/qwen2.rs:476-503). A chunk of Tq query tokens sits at
// positions offset .. offset+Tq-1 of its sequence (offset = ctx_len - Tq, the
// chunk's own K/V already appended); query token t attends to keys
// 0 .. offset+t with softmax(q K^T * scale) V, query head hq reading KV head
// hq / G -- evaluated here on the paged pool, without repeat_kv and without
// materialising the score matrix.
//
// Work decomposition. For KV head h the (token, head-in-group) pairs form
// Tq*G rows (row = t*G + g). A workgroup of 8 waves takes 256 rows of one KV
// head, each wave 32 of them, and streams that head's keys in tiles of 64:
// the tile's K and V rows are staged in LDS once and shared by the 8
// waves. When there are too few row tiles to fill the chip, the keys
// are also split across workgroups: each stores its (m, l, acc) partial and
// a second launch merges them with a log-sum-exp combine. Workgroups are mapped to
// work so that consecutive work items -- the row tiles reading the same K/V
// range -- run on one XCD and share its L2.
//
// Per wave and tile (v_mfma_f32_32x32x16_{bf16,f16}; lane l holds
// A[l%32][8*(l/32)+j], B[8*(l/32)+j][l%32] and accumulator element i at
// [8*(i/4) + 4*(l/32) + i%4][l%32]):
//   S^T (keys x queries) = K (keys x d) . Q^T (d x queries)
// so each lane owns one query column: the softmax max and sum are 16 values
// in the lane plus one exchange with lane l^32. The probabilities stay in the
// accumulator layout and feed
//   O^T (d x queries) += V^T (d x keys) . P^T (keys x queries)
// directly as the B operand; the keys of each 16-key MFMA block are taken in
// the order the accumulator holds them (lane half h: keys 4h..4h+3 and
// 8+4h..11+4h). V is staged in LDS row-major, as K is, and its V^T A operand
// is read with two ds_read_b64_tr_b16: within each 16-lane group, lane 4j+a
// points at key row j, columns 4a..4a+3, and lane 4a+e receives column 4a+e
// of the four key rows -- four consecutive keys of one dimension.
#include <math.h>

#include <mutex>

#include "common.cuh"
#include "host_common.h"

namespace rlse {
namespace {

// Eight waves share each staged K/V tile: twice the rows per tile of four
// waves, so half the staging and L2 reads per row (measured 6% faster on the
// Qwen3-8B chunk); one workgroup per compute unit.
constexpr int kPWaves = 8;
constexpr int kPThreads = 64 * kPWaves;
constexpr int kBM = 32 * kPWaves;  // rows per workgroup
constexpr int kBN = 64;            // keys per tile
// LDS row padding (elements), for the 64 four-byte banks of the gfx950
// LDS. K rows are read as 16-byte packets, 16 lanes (16 rows, one column)
// per cycle: a row stride of 68 words puts the rows 4 banks apart. V rows
// are read by transposing 8-byte reads, 32 lanes per cycle: 4 rows (keys)
// times two 16-column blocks of 8 words each; a row stride of 80 words
// (D = 128) or 48 (D = 64) puts the 4 rows 16 banks apart, so both column
// blocks of every row have banks of their own. (A stride of 72 words, a
// padding of 16, put row j's first block on row j-1's second: 2 conflict
// cycles per read.)
constexpr int kPadK = 8;
constexpr int kPadV = 32;
constexpr int kMinKeysPerSplit = 512;
constexpr int kMaxSplits = 16;
constexpr int kMaxSplitPages = 1024;  // page ids of a split staged in LDS (16384 keys)
// The running max of a query's softmax moves only when a score exceeds it by
// more than this many powers of two (probabilities stay below 2^kLazyLog2).
constexpr float kLazyLog2 = 8.f;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
// 16-byte packets are staged as u32x4_t, a native vector, so copies are
// vector loads and stores (HIP's uint4 struct is copied with memcpy, which
// keeps an array of them in scratch memory when it is later written to LDS).

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16> {
  static __device__ __forceinline__ f32x16_t mma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<f16> {
  static __device__ __forceinline__ f32x16_t mma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};

struct PrefillParams {
  const void* q;       // [Tq][Hq][D]
  const void* k_pool;  // [num_blocks][Hkv][16][D]
  const void* v_pool;
  const int* table;    // [mbps] page ids of the sequence
  void* out;           // [Tq][Hq][D]
  float* part;         // per-workgroup partial blocks (S > 1), see the kernel's tail
  int Tq, L, offset, Hq, Hkv, G, num_blocks, mbps;
  int row_tiles, splits, split_keys;
  float c;  // scale * log2(e)
};

// The partial block of split sp for (KV head h, row tile rt): (4*D/32 + 1)
// float4 slots per thread of the workgroup.
template <int D>
__device__ __forceinline__ float4* part_block(const PrefillParams& p, int sp, int h, int rt) {
  const size_t wgi = ((size_t)sp * p.Hkv + h) * p.row_tiles + rt;
  return reinterpret_cast<float4*>(p.part) + wgi * (4 * (D / 32) + 1) * kPThreads;
}

template <typename T, int D>
__global__ __launch_bounds__(kPThreads, 1) void prefill_kernel(PrefillParams p) {
  constexpr int KB = D / 16;                  // 16-wide k-blocks of q.k
  constexpr int DB = D / 32;                  // 32-row blocks of O^T
  constexpr int CPR = D / 8;                  // 16-byte chunks per key row
  constexpr int KPK = kBN * CPR;              // K packets per tile
  constexpr int KPT = KPK / kPThreads;        // per thread
  static_assert(KPK % kPThreads == 0, "K tile must split evenly");
  __shared__ __align__(16) uint16_t s_k[2][kBN][D + kPadK];  // K rows
  __shared__ __align__(16) uint16_t s_v[2][kBN][D + kPadV];  // V rows
  __shared__ int s_valid[2];                                 // page-valid bits of the tile
  __shared__ __align__(16) int s_pages[kMaxSplitPages];      // the split's page ids (-1: invalid)

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int half = lane >> 5, col = lane & 31;

  // XCD-aware work index: workgroup b runs on XCD b % 8; give each XCD a
  // contiguous run of work items.
  const int nwg = gridDim.x;
  const int b = blockIdx.x;
  const int wid = (nwg % 8 == 0) ? (b % 8) * (nwg / 8) + b / 8 : b;
  const int rt = wid % p.row_tiles;
  const int h = (wid / p.row_tiles) % p.Hkv;
  const int split = wid / (p.row_tiles * p.Hkv);

  const int G = p.G, Hq = p.Hq, Hkv = p.Hkv;
  const int rows = p.Tq * G;
  const int myrow = rt * kBM + wave * 32 + col;
  const int row_c = myrow < rows ? myrow : rows - 1;
  const int t = row_c / G, g = row_c - t * G, qh = h * G + g;
  const int kmax = p.offset + t;  // last key this query sees
  // Last key every query of this wave sees (its first row has the smallest t).
  const int kmin_wave = p.offset + min(rt * kBM + wave * 32, rows - 1) / G;

  // Keys of this workgroup: up to the last query's diagonal, this split's share.
  const int last_row = min(rows - 1, rt * kBM + kBM - 1);
  const int wg_keys = min(p.L, p.offset + last_row / G + 1);
  const int k_begin = split * p.split_keys;
  const int k_end = min(wg_keys, k_begin + p.split_keys);

  const T* __restrict__ qb = reinterpret_cast<const T*>(p.q);
  const T* __restrict__ kp = reinterpret_cast<const T*>(p.k_pool);
  const T* __restrict__ vp = reinterpret_cast<const T*>(p.v_pool);

  // Page ids of this split's keys, staged once (whole 4-page tiles, indices
  // past the context clamped to its last page).
  {
    const int npg = k_begin < k_end ? (((k_end - k_begin + 15) >> 4) + 3) & ~3 : 0;
    const int plast = (p.L - 1) >> 4;
    for (int i = tid; i < npg; i += kPThreads) {
      const int pi = min((k_begin >> 4) + i, plast);
      const int id = p.table[pi];
      s_pages[i] = ((unsigned)id < (unsigned)p.num_blocks) ? id : -1;
    }
    __syncthreads();
  }

  f32x16_t o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m = -INFINITY, lsum = 0.f;

  if (k_begin < k_end) {
    uint4 qreg[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      qreg[kb] = *reinterpret_cast<const uint4*>(qb + ((size_t)t * Hq + qh) * D + kb * 16 +
                                                 half * 8);

   const int last_tile = k_begin + ((k_end - 1 - k_begin) / kBN) * kBN;
    static_assert(kBN == 64, "a tile spans 4 pages");
    // Packet u of this thread: key kk of the tile, 16-byte chunk dc of its
    // row. Its page, kk >> 4, is the same for the whole wave; its offset in
    // the page tile is a per-lane constant.
    int voff[KPT], pg_of[KPT];
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int pk = tid + u * kPThreads;
      const int kk = pk / CPR, dc = pk - kk * CPR;
      voff[u] = (((kk & 15) * D) + dc * 8) * (int)sizeof(T);
      pg_of[u] = __builtin_amdgcn_readfirstlane(kk >> 4);
    }
    u32x4_t kst[KPT], vst[KPT];
    int4 pid;  // page ids of the tile's 4 pages (-1: invalid), for the valid bits
    // Global loads of the tile at kt: raw buffer loads through a descriptor
    // of the packet's (page, head) tile, built in scalar registers. An
    // invalid page id gets a descriptor of zero records (zeros, no memory
    // access); page indices past the context read the last page; both are
    // masked in the math.
    const size_t tile_elems = (size_t)16 * D;
    auto load_tile = [&](int kt) __attribute__((always_inline)) {
      pid = *reinterpret_cast<const int4*>(&s_pages[(kt - k_begin) >> 4]);
#pragma unroll
      for (int u = 0; u < KPT; ++u) {
        const int r = __builtin_amdgcn_readfirstlane(s_pages[((kt - k_begin) >> 4) + pg_of[u]]);
        const size_t tb = ((size_t)(r < 0 ? 0 : r) * Hkv + h) * tile_elems;
        const int nrec = r < 0 ? 0 : (int)(tile_elems * sizeof(T));
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(kp + tb), 0, nrec,
                                                          kBufferWord3);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(vp + tb), 0, nrec,
                                                          kBufferWord3);
        kst[u] = __builtin_amdgcn_raw_buffer_load_b128(rk, voff[u], 0, 0);
        vst[u] = __builtin_amdgcn_raw_buffer_load_b128(rv, voff[u], 0, 0);
      }
    };
    // Staged registers -> LDS buffer bf: K and V rows as they are.
    auto store_tile = [&](int bf) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < KPT; ++u) {
        const int pk = tid + u * kPThreads;
        const int kk = pk / CPR, dc = pk - kk * CPR;
        *reinterpret_cast<u32x4_t*>(&s_k[bf][kk][dc * 8]) = kst[u];
        *reinterpret_cast<u32x4_t*>(&s_v[bf][kk][dc * 8]) = vst[u];
      }
      if (tid == 0) {
        s_valid[bf] = (pid.x >= 0 ? 1 : 0) | (pid.y >= 0 ? 2 : 0) | (pid.z >= 0 ? 4 : 0) |
                      (pid.w >= 0 ? 8 : 0);
      }
    };
    // V^T operand reads: lane = (group g of 16, j = key row in the group's
    // 4, a = 4-column block); half h = g / 2 takes keys 4h.. (first read) and
    // 8+4h.. (second), dimension block g % 2 the columns 16 (g % 2) + 4a.
    const int tr_g = lane >> 4, tr_j = (lane & 15) >> 2, tr_a = lane & 3;
    const int tr_row = (tr_g >> 1) * 4 + tr_j, tr_col = (tr_g & 1) * 16 + tr_a * 4;

    load_tile(k_begin);
    store_tile(0);
    __syncthreads();
    int bf = 0;
    for (int kt = k_begin;; kt += kBN) {
      const bool more = kt < last_tile;
      load_tile(more ? kt + kBN : kt);  // in flight during this tile's math
      const int vbits = s_valid[bf];

      // S^T for the two 32-key halves of the tile.
      // (The two halves' MFMA chains are interleaved: consecutive MFMAs then
      // never wait on each other's accumulator.)
      f32x16_t s[2];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) s[sb][i] = 0.f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          const uint4 a =
              *reinterpret_cast<const uint4*>(&s_k[bf][sb * 32 + col][kb * 16 + half * 8]);
          s[sb] = Mfma<T>::mma(a, qreg[kb], s[sb]);
        }
      // Mask (causal, past the split's end, invalid pages) only on tiles that
      // need it: the test is wave-uniform and most tiles are fully visible.
      if (!(kt + kBN - 1 <= kmin_wave && kt + kBN <= k_end && vbits == 15)) {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int kk = sb * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
            const int ka = kt + kk;
            if (!(ka <= kmax && ka < k_end && ((vbits >> (kk >> 4)) & 1))) s[sb][i] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[sb][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // Online softmax in log2 units (the scale folded into the exponent's
      // FMA). The running max moves only when a score exceeds it by more
      // than kLazyLog2, so the accumulator rescale is rare.
      const float cand = mx * p.c;
      if (__any(cand > m + kLazyLog2)) {
        const float mn = fmaxf(m, cand);
        const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
        lsum *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        m = mn;
      }
      const float nms = m == -INFINITY ? 0.f : -m;
      float rs = 0.f;
      uint4 pk[4];  // P^T operands of the four 16-key blocks
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        float pr[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          pr[i] = __builtin_amdgcn_exp2f(fmaf(s[sb][i], p.c, nms));
          rs += pr[i];
        }
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2) {
          const float* v8 = pr + kb2 * 8;
          pk[sb * 2 + kb2] = make_uint4(Packet<T>::pack2(v8[0], v8[1]), Packet<T>::pack2(v8[2], v8[3]),
                                        Packet<T>::pack2(v8[4], v8[5]), Packet<T>::pack2(v8[6], v8[7]));
        }
      }
      rs += __shfl_xor(rs, 32, 64);
      lsum += rs;
      // O^T += V^T . P^T
#pragma unroll
      for (int kq = 0; kq < 4; ++kq)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const uint16_t* v0 = &s_v[bf][kq * 16 + tr_row][db * 32 + tr_col];
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)v0);
          const i16x4_t hi =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(v0 + 8 * (D + kPadV)));
          const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
          o[db] = Mfma<T>::mma(make_uint4(l2.x, l2.y, h2.x, h2.y), pk[kq], o[db]);
        }

      if (!more) break;
      store_tile(bf ^ 1);
      __syncthreads();
      bf ^= 1;
    }
  }

  // Lane holds O^T rows d = 32*db + 8*(i/4) + 4*half + i%4 of its query.
  T* dst = reinterpret_cast<T*>(p.out) + ((size_t)t * Hq + qh) * D;
  auto write_out = [&](const f32x16_t* acc, float inv) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d0 = db * 32 + i4 * 8 + half * 4;
        const f32x16_t& y = acc[db];
        *reinterpret_cast<uint2*>(dst + d0) =
            make_uint2(Packet<T>::pack2(y[i4 * 4] * inv, y[i4 * 4 + 1] * inv),
                       Packet<T>::pack2(y[i4 * 4 + 2] * inv, y[i4 * 4 + 3] * inv));
      }
  };
  if (p.splits == 1) {
    if (myrow < rows) write_out(o, lsum > 0.f ? 1.f / lsum : 0.f);
    return;
  }
  // Key splits: store this split's (acc, m, l) for the workgroup's rows in
  // its register layout -- float4 slot k of thread tid at
  // blk + (k*kPThreads + tid)*4 floats, slots 0..4*DB-1 holding acc and slot 4*DB
  // (m, l) -- so every store covers 1 KB of consecutive bytes. The merge
  // launch reads them back with the same thread-to-row map.
  float4* blk = part_block<D>(p, split, h, rt) + tid;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4)
      blk[(db * 4 + i4) * kPThreads] =
          make_float4(o[db][i4 * 4], o[db][i4 * 4 + 1], o[db][i4 * 4 + 2], o[db][i4 * 4 + 3]);
  blk[4 * DB * kPThreads] = make_float4(m, lsum, 0.f, 0.f);
}

// The same chunked prefill with f32 K/V and queries (the dtype of the
// reference's CPU path), on v_mfma_f32_32x32x2_f32: lane l holds
// A[l%32][l/32], B[l/32][l%32] and accumulator element i at
// [8*(i/4) + 4*(l/32) + i%4][l%32], the layout of the 16-bit kernel's 32x32
// tiles, so the softmax, the masks, the partial records and the merge are
// the same. Per 2-wide k step:
//   S^T += K . Q^T: lane half h contracts dimension h*D/2 + j at step j, so
//   a lane's query operand is D/2 consecutive elements of its query (held in
//   registers) and its K operand comes from LDS four steps at a time;
//   O^T += V^T . P^T: step j pairs the keys the two lane halves hold in
//   accumulator element j (8*(j/4) + 4h + j%4), so the B operand is the
//   lane's own probability and the A operand one float of V's key row.
// K and V rows are staged in LDS as they are (f32). K rows are read as
// 16-byte packets, 16 rows per cycle: a stride of D + 4 words puts them 4
// banks apart. A V read takes 32 consecutive columns of one row in each lane
// half, the halves four rows apart: a stride of D + 8 words puts those rows
// 32 banks apart.
constexpr int kPadF = 4;
constexpr int kPadFV = 8;
template <int D>
__global__ __launch_bounds__(kPThreads, 1) void prefill_kernel_f32(PrefillParams p) {
  constexpr int DB = D / 32;                  // 32-row blocks of O^T
  constexpr int KH = D / 2;                   // k steps of q.k
  constexpr int CPR = D / 4;                  // 16-byte chunks per key row
  constexpr int KPK = kBN * CPR;              // K packets per tile
  constexpr int KPT = KPK / kPThreads;        // per thread
  static_assert(KPK % kPThreads == 0, "K tile must split evenly");
  __shared__ __align__(16) float s_k[2][kBN][D + kPadF];  // K rows
  __shared__ __align__(16) float s_v[2][kBN][D + kPadFV];  // V rows
  __shared__ int s_valid[2];                               // page-valid bits of the tile
  __shared__ __align__(16) int s_pages[kMaxSplitPages];    // the split's page ids (-1: invalid)

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int half = lane >> 5, col = lane & 31;

  // XCD-aware work index, as in the 16-bit kernel.
  const int nwg = gridDim.x;
  const int b = blockIdx.x;
  const int wid = (nwg % 8 == 0) ? (b % 8) * (nwg / 8) + b / 8 : b;
  const int rt = wid % p.row_tiles;
  const int h = (wid / p.row_tiles) % p.Hkv;
  const int split = wid / (p.row_tiles * p.Hkv);

  const int G = p.G, Hq = p.Hq, Hkv = p.Hkv;
  const int rows = p.Tq * G;
  const int myrow = rt * kBM + wave * 32 + col;
  const int row_c = myrow < rows ? myrow : rows - 1;
  const int t = row_c / G, g = row_c - t * G, qh = h * G + g;
  const int kmax = p.offset + t;
  const int kmin_wave = p.offset + min(rt * kBM + wave * 32, rows - 1) / G;
  const int last_row = min(rows - 1, rt * kBM + kBM - 1);
  const int wg_keys = min(p.L, p.offset + last_row / G + 1);
  const int k_begin = split * p.split_keys;
  const int k_end = min(wg_keys, k_begin + p.split_keys);

  const float* __restrict__ qb = reinterpret_cast<const float*>(p.q);
  const float* __restrict__ kp = reinterpret_cast<const float*>(p.k_pool);
  const float* __restrict__ vp = reinterpret_cast<const float*>(p.v_pool);

  {
    const int npg = k_begin < k_end ? (((k_end - k_begin + 15) >> 4) + 3) & ~3 : 0;
    const int plast = (p.L - 1) >> 4;
    for (int i = tid; i < npg; i += kPThreads) {
      const int pi = min((k_begin >> 4) + i, plast);
      const int id = p.table[pi];
      s_pages[i] = ((unsigned)id < (unsigned)p.num_blocks) ? id : -1;
    }
    __syncthreads();
  }

  f32x16_t o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m = -INFINITY, lsum = 0.f;

  if (k_begin < k_end) {
    // Dimensions half*D/2 .. +D/2 of the lane's query.
    float qreg[KH];
#pragma unroll
    for (int j = 0; j < KH; j += 4) {
      const float4 x = *reinterpret_cast<const float4*>(qb + ((size_t)t * Hq + qh) * D +
                                                        half * KH + j);
      qreg[j] = x.x;
      qreg[j + 1] = x.y;
      qreg[j + 2] = x.z;
      qreg[j + 3] = x.w;
    }
    const int last_tile = k_begin + ((k_end - 1 - k_begin) / kBN) * kBN;
    static_assert(kBN == 64, "a tile spans 4 pages");
    int voff[KPT], pg_of[KPT];
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int pk = tid + u * kPThreads;
      const int kk = pk / CPR, dc = pk - kk * CPR;
      voff[u] = (((kk & 15) * D) + dc * 4) * (int)sizeof(float);
      pg_of[u] = __builtin_amdgcn_readfirstlane(kk >> 4);
    }
    u32x4_t kst[KPT], vst[KPT];
    int4 pid;
    const size_t tile_elems = (size_t)16 * D;
    auto load_tile = [&](int kt) __attribute__((always_inline)) {
      pid = *reinterpret_cast<const int4*>(&s_pages[(kt - k_begin) >> 4]);
#pragma unroll
      for (int u = 0; u < KPT; ++u) {
        const int r = __builtin_amdgcn_readfirstlane(s_pages[((kt - k_begin) >> 4) + pg_of[u]]);
        const size_t tb = ((size_t)(r < 0 ? 0 : r) * Hkv + h) * tile_elems;
        const int nrec = r < 0 ? 0 : (int)(tile_elems * sizeof(float));
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(kp + tb), 0, nrec,
                                                          kBufferWord3);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(vp + tb), 0, nrec,
                                                          kBufferWord3);
        kst[u] = __builtin_amdgcn_raw_buffer_load_b128(rk, voff[u], 0, 0);
        vst[u] = __builtin_amdgcn_raw_buffer_load_b128(rv, voff[u], 0, 0);
      }
    };
    auto store_tile = [&](int bf) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < KPT; ++u) {
        const int pk = tid + u * kPThreads;
        const int kk = pk / CPR, dc = pk - kk * CPR;
        *reinterpret_cast<u32x4_t*>(&s_k[bf][kk][dc * 4]) = kst[u];
        *reinterpret_cast<u32x4_t*>(&s_v[bf][kk][dc * 4]) = vst[u];
      }
      if (tid == 0) {
        s_valid[bf] = (pid.x >= 0 ? 1 : 0) | (pid.y >= 0 ? 2 : 0) | (pid.z >= 0 ? 4 : 0) |
                      (pid.w >= 0 ? 8 : 0);
      }
    };

    load_tile(k_begin);
    store_tile(0);
    __syncthreads();
    int bf = 0;
    for (int kt = k_begin;; kt += kBN) {
      const bool more = kt < last_tile;
      load_tile(more ? kt + kBN : kt);  // in flight during this tile's math
      const int vbits = s_valid[bf];

      f32x16_t s[2];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) s[sb][i] = 0.f;
#pragma unroll
      for (int j = 0; j < KH; j += 4)
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          const float4 a = *reinterpret_cast<const float4*>(&s_k[bf][sb * 32 + col][half * KH + j]);
          s[sb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qreg[j], s[sb], 0, 0, 0);
          s[sb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qreg[j + 1], s[sb], 0, 0, 0);
          s[sb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qreg[j + 2], s[sb], 0, 0, 0);
          s[sb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qreg[j + 3], s[sb], 0, 0, 0);
        }
      if (!(kt + kBN - 1 <= kmin_wave && kt + kBN <= k_end && vbits == 15)) {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int kk = sb * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
            const int ka = kt + kk;
            if (!(ka <= kmax && ka < k_end && ((vbits >> (kk >> 4)) & 1))) s[sb][i] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[sb][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float cand = mx * p.c;
      if (__any(cand > m + kLazyLog2)) {
        const float mn = fmaxf(m, cand);
        const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
        lsum *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        m = mn;
      }
      const float nms = m == -INFINITY ? 0.f : -m;
      float rs = 0.f;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          s[sb][i] = __builtin_amdgcn_exp2f(fmaf(s[sb][i], p.c, nms));
          rs += s[sb][i];
        }
      rs += __shfl_xor(rs, 32, 64);
      lsum += rs;
      // O^T += V^T . P^T, step j of key half sb: the lane's half takes key
      // sb*32 + 8*(j/4) + 4*half + j%4 (its accumulator element j).
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float* vrow = &s_v[bf][sb * 32 + (j >> 2) * 8 + half * 4 + (j & 3)][col];
#pragma unroll
          for (int db = 0; db < DB; ++db)
            o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[db * 32], s[sb][j], o[db], 0, 0, 0);
        }

      if (!more) break;
      store_tile(bf ^ 1);
      __syncthreads();
      bf ^= 1;
    }
  }

  // Lane holds O^T rows d = 32*db + 8*(i/4) + 4*half + i%4 of its query.
  if (p.splits == 1) {
    if (myrow < rows) {
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
      float* dst = reinterpret_cast<float*>(p.out) + ((size_t)t * Hq + qh) * D;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
          *reinterpret_cast<float4*>(dst + db * 32 + i4 * 8 + half * 4) =
              make_float4(o[db][i4 * 4] * inv, o[db][i4 * 4 + 1] * inv, o[db][i4 * 4 + 2] * inv,
                          o[db][i4 * 4 + 3] * inv);
    }
    return;
  }
  // Key splits: the partial block in the 16-bit kernel's layout.
  float4* blk = part_block<D>(p, split, h, rt) + tid;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4)
      blk[(db * 4 + i4) * kPThreads] =
          make_float4(o[db][i4 * 4], o[db][i4 * 4 + 1], o[db][i4 * 4 + 2], o[db][i4 * 4 + 3]);
  blk[4 * DB * kPThreads] = make_float4(m, lsum, 0.f, 0.f);
}

// Log-sum-exp merge of the key splits. Workgroup (row tile, KV head, q)
// combines slots 4q..4q+3 of every row: thread tid reads what thread tid of
// each split stored, so all the loads of kMergeBatch splits are in flight
// together and D/32 workgroups share a tile. The splits combine online in
// split order (a deterministic result): with (M, L, A) so far and a split's
// (m, l, a), M' = max(M, m) and L, A scale by 2^(M - M') and 2^(m - M').
constexpr int kMergeBatch = 4;
template <typename T, int D>
__global__ __launch_bounds__(kPThreads) void prefill_merge_kernel(PrefillParams p) {
  constexpr int DB = D / 32;
  constexpr int KQ = 4;  // float4 slots per thread: 4*DB slots over DB workgroups
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, half = lane >> 5, col = lane & 31;
  const int q = blockIdx.x % DB;
  const int tile = blockIdx.x / DB;
  const int rt = tile % p.row_tiles, h = tile / p.row_tiles;
  const int G = p.G, Hq = p.Hq;
  const int rows = p.Tq * G;
  const int myrow = rt * kBM + wave * 32 + col;
  if (myrow >= rows) return;
  const int t = myrow / G, qh = h * G + (myrow - (myrow / G) * G);
  float M = -INFINITY, L = 0.f;
  float acc[KQ * 4];
#pragma unroll
  for (int i = 0; i < KQ * 4; ++i) acc[i] = 0.f;
  for (int s0 = 0; s0 < p.splits; s0 += kMergeBatch) {
    float4 ml[kMergeBatch], a[kMergeBatch][KQ];
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) {
      // Past the last split: re-read the last one (never combined).
      const int sp = s0 + j < p.splits ? s0 + j : p.splits - 1;
      const float4* blk = part_block<D>(p, sp, h, rt) + tid;
      ml[j] = blk[4 * DB * kPThreads];
#pragma unroll
      for (int kk = 0; kk < KQ; ++kk) a[j][kk] = blk[(q * KQ + kk) * kPThreads];
    }
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) {
      if (s0 + j >= p.splits) break;
      const float m = ml[j].x;
      const float Mn = fmaxf(M, m);
      if (Mn == -INFINITY) continue;  // no visible key so far
      const float sa = __builtin_amdgcn_exp2f(M - Mn);
      const float sb = __builtin_amdgcn_exp2f(m - Mn);
      L = L * sa + ml[j].y * sb;
#pragma unroll
      for (int kk = 0; kk < KQ; ++kk) {
        acc[kk * 4] = acc[kk * 4] * sa + a[j][kk].x * sb;
        acc[kk * 4 + 1] = acc[kk * 4 + 1] * sa + a[j][kk].y * sb;
        acc[kk * 4 + 2] = acc[kk * 4 + 2] * sa + a[j][kk].z * sb;
        acc[kk * 4 + 3] = acc[kk * 4 + 3] * sa + a[j][kk].w * sb;
      }
      M = Mn;
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  T* dst = reinterpret_cast<T*>(p.out) + ((size_t)t * Hq + qh) * D;
#pragma unroll
  for (int kk = 0; kk < KQ; ++kk) {
    // slot k = (db, i4): dims 32*db + 8*i4 + 4*half .. +3
    const int k = q * KQ + kk;
    const int d0 = (k >> 2) * 32 + (k & 3) * 8 + half * 4;
    if constexpr (sizeof(T) == 4) {
      *reinterpret_cast<float4*>(dst + d0) = make_float4(acc[kk * 4] * inv,
                                                         acc[kk * 4 + 1] * inv,
                                                         acc[kk * 4 + 2] * inv,
                                                         acc[kk * 4 + 3] * inv);
    } else {
      *reinterpret_cast<uint2*>(dst + d0) =
          make_uint2(Packet<T>::pack2(acc[kk * 4] * inv, acc[kk * 4 + 1] * inv),
                     Packet<T>::pack2(acc[kk * 4 + 2] * inv, acc[kk * 4 + 3] * inv));
    }
  }
}

// Workspace (key splits only): the partial blocks of every workgroup.
struct PrefillPlan {
  int row_tiles, splits, split_keys;
  size_t ws_bytes;
};

int plan_prefill(int Tq, int ctx_len, int Hq, int Hkv, int D, PrefillPlan* plan) {
  int cus = 0;
  const int st = device_cu_count(&cus);
  if (st) return st;
  const int G = Hq / Hkv;
  plan->row_tiles = (Tq * G + kBM - 1) / kBM;
  const long long base = (long long)plan->row_tiles * Hkv;
  int s = (int)(((long long)cus + base - 1) / base);  // one group per compute unit
  const int by_len = (ctx_len + kMinKeysPerSplit - 1) / kMinKeysPerSplit;
  s = s < by_len ? s : by_len;
  s = s < kMaxSplits ? s : kMaxSplits;
  const int by_pages = (ctx_len + kMaxSplitPages * 16 - 1) / (kMaxSplitPages * 16);
  s = s > by_pages ? s : by_pages;  // a split's page ids must fit the LDS stage
  s = s < 1 ? 1 : s;
  int per = (ctx_len + s - 1) / s;
  per = (per + kBN - 1) / kBN * kBN;
  s = (ctx_len + per - 1) / per;  // drop splits left empty by the rounding
  plan->splits = s;
  plan->split_keys = per;
  plan->ws_bytes = s > 1 ? (size_t)s * Hkv * plan->row_tiles * (4 * (D / 32) + 1) * kPThreads *
                               4 * sizeof(float)
                         : 0;
  return RLSE_OK;
}

template <typename T, int D>
int launch_prefill(PrefillParams& pp, hipStream_t stream) {
  const int nwg = pp.row_tiles * pp.Hkv * pp.splits;
  if constexpr (sizeof(T) == 4)
    hipLaunchKernelGGL((prefill_kernel_f32<D>), dim3(nwg), dim3(kPThreads), 0, stream, pp);
  else
    hipLaunchKernelGGL((prefill_kernel<T, D>), dim3(nwg), dim3(kPThreads), 0, stream, pp);
  const int st = launch_status("prefill_kernel");
  if (st || pp.splits == 1) return st;
  hipLaunchKernelGGL((prefill_merge_kernel<T, D>), dim3(pp.row_tiles * pp.Hkv * (D / 32)),
                     dim3(kPThreads), 0, stream, pp);
  return launch_status("prefill_merge_kernel");
}

// Library-owned workspace per device, for callers that pass none. The mutex
// is held from the lookup until the launches are queued, so a thread that
// grows (frees and reallocates) the buffer never frees one another thread
// is about to launch on; hipFree waits for launches already queued.
void* g_pws_ptr[64] = {nullptr};
size_t g_pws_size[64] = {0};
std::mutex g_pws_mu;

int validate_prefill(int num_tokens, int ctx_len, int Hq, int Hkv, int D, int mbps,
                     int num_blocks, int dtype) {
  if (num_tokens <= 0 || ctx_len < num_tokens)
    return fail(RLSE_ERR_INVALID_VALUE, "prefill: need 1 <= num_tokens (%d) <= ctx_len (%d)",
                num_tokens, ctx_len);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
    return fail(RLSE_ERR_INVALID_VALUE, "prefill: num_heads %d not a multiple of num_kv_heads %d",
                Hq, Hkv);
  if (D != 64 && D != 128)
    return fail(RLSE_ERR_INVALID_VALUE, "prefill: head_dim %d not in {64, 128}", D);
  if (dtype != RLSE_DTYPE_BF16 && dtype != RLSE_DTYPE_F16 && dtype != RLSE_DTYPE_F32)
    return fail(RLSE_ERR_INVALID_VALUE, "prefill: bad dtype %d", dtype);
  if (mbps <= 0 || num_blocks <= 0 || (long long)mbps * 16 < ctx_len)
    return fail(RLSE_ERR_INVALID_VALUE,
                "prefill: ctx_len %d exceeds the table's %d blocks of 16 (num_blocks %d)",
                ctx_len, mbps, num_blocks);
  if ((long long)num_tokens * Hq > 0x7fffffffLL / 256)
    return fail(RLSE_ERR_INVALID_VALUE, "prefill: num_tokens * num_heads too large");
  return RLSE_OK;
}

}  // namespace
}  // namespace rlse

using namespace rlse;

extern "C" int rlse_prefill_workspace_size(int num_tokens, int ctx_len, int num_heads,
                                           int num_kv_heads, int head_dim, size_t* bytes) {
  if (!bytes) return fail(RLSE_ERR_INVALID_VALUE, "prefill_workspace_size: null output");
  if (num_tokens <= 0 || ctx_len < num_tokens || num_heads <= 0 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0 || (head_dim != 64 && head_dim != 128))
    return fail(RLSE_ERR_INVALID_VALUE, "prefill_workspace_size: bad shape");
  PrefillPlan plan;
  const int st = plan_prefill(num_tokens, ctx_len, num_heads, num_kv_heads, head_dim, &plan);
  if (st) return st;
  *bytes = plan.ws_bytes;
  return RLSE_OK;
}

extern "C" int rlse_prefill_attn(const void* q, const void* k_pool, const void* v_pool,
                                 const int32_t* block_table, int ctx_len, int num_tokens,
                                 void* out, int num_heads, int num_kv_heads, int head_dim,
                                 int max_blocks, int num_blocks, float scale, int dtype,
                                 void* workspace, size_t workspace_bytes, rlse_stream_t stream) {
  int st = validate_prefill(num_tokens, ctx_len, num_heads, num_kv_heads, head_dim, max_blocks,
                            num_blocks, dtype);
  if (st) return st;
  if (!q || !k_pool || !v_pool || !block_table || !out)
    return fail(RLSE_ERR_INVALID_VALUE, "prefill: null pointer argument");
  if (!(scale > 0.f) || !isfinite(scale))
    return fail(RLSE_ERR_INVALID_VALUE, "prefill: scale must be finite and positive");
  PrefillPlan plan;
  st = plan_prefill(num_tokens, ctx_len, num_heads, num_kv_heads, head_dim, &plan);
  if (st) return st;
  std::unique_lock<std::mutex> lock;
  if (plan.ws_bytes > 0) {
    if (workspace == nullptr) {
      int dev = 0;
      hipError_t e = hipGetDevice(&dev);
      if (e != hipSuccess || dev < 0 || dev >= 64)
        return fail(RLSE_ERR_INVALID_VALUE, "prefill: no current device");
      lock = std::unique_lock<std::mutex>(g_pws_mu);
      if (g_pws_size[dev] < plan.ws_bytes) {
        if (g_pws_ptr[dev]) (void)hipFree(g_pws_ptr[dev]);
        g_pws_ptr[dev] = nullptr;
        g_pws_size[dev] = 0;
        e = hipMalloc(&g_pws_ptr[dev], plan.ws_bytes);
        if (e != hipSuccess) return fail((int)e, "prefill: workspace hipMalloc failed");
        g_pws_size[dev] = plan.ws_bytes;
      }
      workspace = g_pws_ptr[dev];
    } else if (workspace_bytes < plan.ws_bytes) {
      return fail(RLSE_ERR_BUFFER_TOO_SMALL, "prefill: workspace %zu bytes < %zu needed",
                  workspace_bytes, plan.ws_bytes);
    }
  }
  PrefillParams pp{};
  pp.q = q;
  pp.k_pool = k_pool;
  pp.v_pool = v_pool;
  pp.table = block_table;
  pp.out = out;
  pp.part = reinterpret_cast<float*>(workspace);
  pp.Tq = num_tokens;
  pp.L = ctx_len;
  pp.offset = ctx_len - num_tokens;
  pp.Hq = num_heads;
  pp.Hkv = num_kv_heads;
  pp.G = num_heads / num_kv_heads;
  pp.num_blocks = num_blocks;
  pp.mbps = max_blocks;
  pp.row_tiles = plan.row_tiles;
  pp.splits = plan.splits;
  pp.split_keys = plan.split_keys;
  pp.c = scale * 1.4426950408889634f;
  const hipStream_t s = as_stream(stream);
  if (dtype == RLSE_DTYPE_BF16)
    return head_dim == 128 ? launch_prefill<bf16, 128>(pp, s) : launch_prefill<bf16, 64>(pp, s);
  if (dtype == RLSE_DTYPE_F32)
    return head_dim == 128 ? launch_prefill<float, 128>(pp, s)
                           : launch_prefill<float, 64>(pp, s);
  return head_dim == 128 ? launch_prefill<f16, 128>(pp, s) : launch_prefill<f16, 64>(pp, s);
}
