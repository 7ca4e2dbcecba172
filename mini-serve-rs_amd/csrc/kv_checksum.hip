// Checksums of the paged pool's K and V rows: for every (sequence, KV head)
// row, the order-independent sum (mod 2^32) over its attended positions
// t < L and the 32-bit words j of each position's head_dim elements of
//     mix(w, t, j) = (w ^ (t * 0x9E3779B1 + j * 0x85EBCA77)) * 0xC2B2AE3D,
// separately for K and V. Pages whose id lies outside the pool contribute
// nothing (as the decode skips them).
//
// No counterpart in the reference, whose tests compare snapshot buffers
// byte for byte on the host (src/backends/candle.rs:1281-1292); at the
// benched sizes the pool holds hundreds of MB per layer, and these sums let a
// test compare it with the expected contents without copying it back.
//
// The kernel splits the pages as the decode does -- the same stream of
// (sequence, KV head) rows cut into contiguous ranges of 2 x CUs workgroups
// of four waves, raw non-temporal buffer loads of whole K and V tiles -- and
// does no other work, so its duration is the time a launch of this shape
// takes to read the decode's K/V bytes: the ceiling the decode's bandwidth
// is measured against. Each wave keeps one page (its 16-row K and V tiles)
// in flight: of one, two and three pages per wave, one reads fastest at the
// Qwen3-0.6B batch's 140 MB (about 16 MB in flight over the chip; more
// only lengthens HBM's queues), so this is the fastest read of those bytes
// with this split.
#include "decode_kernel.cuh"

namespace rlse {
namespace {

__device__ __forceinline__ uint32_t mix_word(uint32_t w, uint32_t t, uint32_t j) {
  return (w ^ (t * 0x9E3779B1u + j * 0x85EBCA77u)) * 0xC2B2AE3Du;
}

struct ChecksumParams {
  const void* k_pool;
  const void* v_pool;
  const int* tables;
  const int* seq_lens;
  uint32_t* out;  // [B][Hkv][2]: K, V
  int B, Hkv, mbps, num_blocks, W;
  // Optional decode plan (rlse_decode_plan of the same tables and lengths):
  // its descriptors give each wave's first page before the block prefix is
  // built, as in a planned decode launch. Null, or a plan of another step
  // shape (its stamp is not a plain plan's): the walk builds them itself.
  const int4* plan;
};

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void checksum_kernel(ChecksumParams p) {
  using S = DecodeShape<T, D>;
  constexpr int EPL = S::EPL, LPR = S::LPR, RPL = S::RPL, NR = S::NR;
  constexpr int WPP = 4;  // 32-bit words per 16-byte packet
  extern __shared__ int s_pref[];  // [B + 1]
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane % LPR, rsub = lane / LPR;
  const int B = p.B, Hkv = p.Hkv, mbps = p.mbps;
  const T* __restrict__ kp = reinterpret_cast<const T*>(p.k_pool);
  const T* __restrict__ vp = reinterpret_cast<const T*>(p.v_pool);
  const size_t tile = (size_t)16 * D;
  const int voff = (int)(((size_t)rsub * D + (size_t)col * EPL) * sizeof(T));
  struct Page {
    uint4 k[NR], v[NR];
    int nv, row, blk;
  };
  // K and V tiles of page id for KV head kvh (a descriptor of zero records,
  // no memory access, unless fetch).
  auto load_pages = [&](Page& pg, int id, int kvh, bool fetch) __attribute__((always_inline)) {
    const size_t tb = ((size_t)(fetch ? id : 0) * Hkv + kvh) * tile;
    const int nrec = fetch ? (int)(tile * sizeof(T)) : 0;
    const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(kp + tb), 0, nrec,
                                                      kBufferWord3);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(vp + tb), 0, nrec,
                                                      kBufferWord3);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int o = voff + r * RPL * D * (int)sizeof(T);
      const u32x4_t kx = __builtin_amdgcn_raw_buffer_load_b128(rk, o, 0, kLoadNonTemporal);
      const u32x4_t vx = __builtin_amdgcn_raw_buffer_load_b128(rv, o, 0, kLoadNonTemporal);
      pg.k[r] = make_uint4(kx.x, kx.y, kx.z, kx.w);
      pg.v[r] = make_uint4(vx.x, vx.y, vx.z, vx.w);
    }
  };
  // With a plain plan, the wave's first page is requested before anything
  // else (its block index is filled in once the prefix is built).
  int4 plan_d = make_int4(0, 0, -1, 0);
  bool planned = false;
  Page page;
  if (p.plan) {
    plan_d = p.plan[((size_t)blockIdx.x * kWaves + wave) * 64 + lane];
    planned = __builtin_amdgcn_readfirstlane(plan_tail(p.plan, p.W)[0]) == plan_stamp(1, 0);
    if (planned) {
      const int nv = __builtin_amdgcn_readlane(plan_d.y, 0) & 255;
      page.nv = nv;
      page.row = __builtin_amdgcn_readlane(plan_d.z, 0);
      load_pages(page, __builtin_amdgcn_readlane(plan_d.x, 0), nv > 0 ? page.row % Hkv : 0,
                 nv > 0);
    }
  }
  if (wave == 0)
    block_prefix(p.seq_lens, B, mbps, s_pref, lane < B ? p.seq_lens[lane] : 0, 0, nullptr, 0);
  __syncthreads();
  const long long total = (long long)Hkv * __builtin_amdgcn_readfirstlane(s_pref[B]);
  const long long we = total > 0 ? effective_groups(total, p.W) : 0;
  const long long w = blockIdx.x;
  long long wlo = 0, whi = 0;
  if (w < we) {
    const long long glo = range_lo(w, total, we, p.W, 16);
    const long long ghi = range_lo(w + 1, total, we, p.W, 16);
    wlo = glo + (ghi - glo) * wave / kWaves;
    whi = glo + (ghi - glo) * (wave + 1) / kWaves;
  }
  const int nblk = (int)(whi - wlo);
  if (nblk <= 0) {
    if (planned) {  // the early request (none past the wave's end) is consumed before leaving
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        consume(page.k[r]);
        consume(page.v[r]);
      }
    }
    return;
  }

  // Descriptors of 64 consecutive blocks, one per lane: page id, valid rows
  // (0 for an id outside the pool), row, and the block's index in its row.
  // The plan's copy of the first 64 has no block index: it follows from the
  // block's place in the stream and its row's start.
  int d_id = 0, d_nv = 0, d_row = -1, d_blk = 0, cbase = 0;
  auto load_chunk = [&](int base) __attribute__((always_inline)) {
    cbase = base;
    const long long f = wlo + base + lane;
    d_id = 0;
    d_nv = 0;
    d_row = -1;
    d_blk = 0;
    if (planned && base == 0) {
      if (f < whi && plan_d.z >= 0) {
        const int b = plan_d.z / Hkv, kvh = plan_d.z - b * Hkv;
        const int nb = s_pref[b + 1] - s_pref[b];
        d_id = plan_d.x;
        d_nv = plan_d.y & 255;
        d_row = plan_d.z;
        d_blk = (int)(f - (long long)Hkv * s_pref[b] - (long long)kvh * nb);
      }
    } else if (f < whi) {
      const int b = locate_seq(s_pref, B, Hkv, f);
      const int nb = s_pref[b + 1] - s_pref[b];
      const long long o = f - (long long)Hkv * s_pref[b];
      const int kvh = (int)(o / nb), blk = (int)(o % nb);
      d_row = b * Hkv + kvh;
      d_blk = blk;
      d_id = p.tables[(size_t)b * mbps + blk];
      const int nv = valid_len(p.seq_lens[b], mbps) - blk * 16;
      d_nv = (unsigned)d_id < (unsigned)p.num_blocks ? (nv > 16 ? 16 : nv) : 0;
    }
  };
  auto issue = [&](Page& pg, int j) __attribute__((always_inline)) {
    const bool real = j < nblk;
    j = real ? j : nblk - 1;
    if (j - cbase >= 64) load_chunk(cbase + 64);
    const int k = j - cbase;
    const int id = __builtin_amdgcn_readlane(d_id, k);
    const int nv = real ? __builtin_amdgcn_readlane(d_nv, k) : 0;
    pg.nv = nv;
    pg.row = __builtin_amdgcn_readlane(d_row, k);
    pg.blk = __builtin_amdgcn_readlane(d_blk, k);
    load_pages(pg, id, pg.row % Hkv, nv > 0);
  };
  int cur_row = -1;
  uint32_t hk = 0, hv = 0;
  auto flush = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      hk += (uint32_t)__shfl_xor((int)hk, o, 64);
      hv += (uint32_t)__shfl_xor((int)hv, o, 64);
    }
    if (lane == 0) {
      atomicAdd(p.out + (size_t)cur_row * 2, hk);
      atomicAdd(p.out + (size_t)cur_row * 2 + 1, hv);
    }
    hk = hv = 0;
  };
  auto sum_page = [&](const Page& pg) __attribute__((always_inline)) {
    if (pg.row != cur_row) {
      if (cur_row >= 0) flush();
      cur_row = pg.row;
    }
    const uint32_t j0 = (uint32_t)(col * WPP);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int slot = r * RPL + rsub;
      const uint32_t t = (uint32_t)(pg.blk * 16 + slot);
      const uint32_t kw[4] = {pg.k[r].x, pg.k[r].y, pg.k[r].z, pg.k[r].w};
      const uint32_t vw[4] = {pg.v[r].x, pg.v[r].y, pg.v[r].z, pg.v[r].w};
      uint32_t sk = 0, sv = 0;
#pragma unroll
      for (int i = 0; i < WPP; ++i) {
        sk += mix_word(kw[i], t, j0 + i);
        sv += mix_word(vw[i], t, j0 + i);
      }
      hk += slot < pg.nv ? sk : 0u;
      hv += slot < pg.nv ? sv : 0u;
    }
  };
  load_chunk(0);
  if (planned)
    page.blk = __builtin_amdgcn_readlane(d_blk, 0);  // requested above
  else
    issue(page, 0);
  for (int i = 0;;) {
    sum_page(page);
    if (++i == nblk) break;
    issue(page, i);
  }
  flush();
}

template <typename T, int D>
int launch_checksum(const ChecksumParams& p, hipStream_t s) {
  hipLaunchKernelGGL((checksum_kernel<T, D>), dim3(p.W), dim3(kThreads),
                     (size_t)(p.B + 1) * sizeof(int), s, p);
  return launch_status("checksum_kernel");
}

}  // namespace
}  // namespace rlse

using namespace rlse;

static int kv_checksum_impl(const void* k_pool, const void* v_pool, const int32_t* block_tables,
                            const int32_t* seq_lens, int batch, int num_kv_heads, int head_dim,
                            int max_blocks_per_seq, int num_blocks, int dtype, const void* plan,
                            uint32_t* out, rlse_stream_t stream) {
  if (batch <= 0 || batch > kMaxDecodeBatch || num_kv_heads <= 0 ||
      (long long)batch * num_kv_heads > kMaxDecodeRows || max_blocks_per_seq <= 0 ||
      num_blocks <= 0 || (long long)max_blocks_per_seq * 16 > 0x7fffffffLL)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_checksum: bad shape");
  if (head_dim != 64 && head_dim != 128)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_checksum: head_dim %d not in {64, 128}", head_dim);
  if (!k_pool || !v_pool || !block_tables || !seq_lens || !out)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_checksum: null pointer argument");
  int cus = 0;
  const int st = device_cu_count(&cus);
  if (st) return st;
  if ((uintptr_t)plan % 16)
    return fail(RLSE_ERR_INVALID_VALUE, "kv_checksum: plan must be 16-byte aligned");
  ChecksumParams p{k_pool, v_pool, block_tables, seq_lens, out, batch, num_kv_heads,
                   max_blocks_per_seq, num_blocks, cus * kGroupsPerCU,
                   reinterpret_cast<const int4*>(plan)};
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case RLSE_DTYPE_F32:
      return head_dim == 128 ? launch_checksum<float, 128>(p, s) : launch_checksum<float, 64>(p, s);
    case RLSE_DTYPE_BF16:
      return head_dim == 128 ? launch_checksum<bf16, 128>(p, s) : launch_checksum<bf16, 64>(p, s);
    case RLSE_DTYPE_F16:
      return head_dim == 128 ? launch_checksum<f16, 128>(p, s) : launch_checksum<f16, 64>(p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "kv_checksum: bad dtype %d", dtype);
}

extern "C" int rlse_kv_checksum(const void* k_pool, const void* v_pool,
                                const int32_t* block_tables, const int32_t* seq_lens, int batch,
                                int num_kv_heads, int head_dim, int max_blocks_per_seq,
                                int num_blocks, int dtype, uint32_t* out, rlse_stream_t stream) {
  return kv_checksum_impl(k_pool, v_pool, block_tables, seq_lens, batch, num_kv_heads, head_dim,
                          max_blocks_per_seq, num_blocks, dtype, nullptr, out, stream);
}

extern "C" int rlse_kv_checksum_planned(const void* k_pool, const void* v_pool,
                                        const int32_t* block_tables, const int32_t* seq_lens,
                                        int batch, int num_kv_heads, int head_dim,
                                        int max_blocks_per_seq, int num_blocks, int dtype,
                                        const void* plan, uint32_t* out, rlse_stream_t stream) {
  if (!plan) return fail(RLSE_ERR_INVALID_VALUE, "kv_checksum_planned: null plan");
  return kv_checksum_impl(k_pool, v_pool, block_tables, seq_lens, batch, num_kv_heads, head_dim,
                          max_blocks_per_seq, num_blocks, dtype, plan, out, stream);
}
