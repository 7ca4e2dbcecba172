// Shared-prefix (cascade) attention of a decode step, 16-bit K/V.
//
// When every sequence of a batch was forked from one cached prefix, the first
// P entries of all block tables are the same pages (refcounted, see
// rlse_bm_fork / rlse_pc_fork). Attending them once per sequence reads each
// prefix page B times; here they are attended once for the whole batch: per
// KV head h, the B*G query vectors of h are taken 16 at a time as the columns
// of the decode's matrix-core block math (S^T = K . Q^T on 16x16x32 MFMAs,
// O^T += V^T . P^T on 16x16x16 MFMAs with V transposed through LDS). The
// prefix is cut into NS = prefix_splits(P) slices of about 16 pages, one
// workgroup per (column tile, KV head, slice), and each wave of a workgroup
// takes its own pages of the slice. The waves' partial softmax states meet
// in LDS, where wave t combines accumulator tile t of all waves (in wave
// order) into the slice's state --
// acc[D], m, l of each query in the decode's log2 units -- and the decode
// launch combines the slices' states, in slice order, into each row it
// finishes; it leaves the prefix out of its page stream. Workgroups are
// numbered so that the column tiles reading one slice's pages run on one XCD
// and share its L2.
// The queries get q_norm + RoPE at their sequence's new position exactly as
// the decode stages them, so both launches see the same query bytes.
//
// Reference semantics are those of decode_attention_gqa_zero_copy
// (src/backends/qwen2.rs:177-203) over the sequence's full key range; the
// split of the keys into prefix and suffix changes only the order of the
// softmax sums.
#include "decode_kernel.cuh"

namespace rlse {
namespace {

constexpr int kPrefixWaves = 8;
static_assert(kMaxPrefixPages <= 64 * kPrefixWaves, "a wave holds the page ids of 64 blocks");

// Measurement build: the wall clock at the points of kPrefixTimelinePoints,
// kept in registers and stored by lane 0 when the wave has finished.
#ifdef RLSE_DECODE_TIMELINE
#define RLSE_PTL(k) (ptl[k] = wall_clock64())
#else
#define RLSE_PTL(k) ((void)0)
#endif

// SELF_CHECK: the launch checks the one-prefix contract itself (a step
// without a plan); planned steps take the plan's verdict.
template <typename T, int D, int G, bool SELF_CHECK>
__global__ __launch_bounds__(64 * kPrefixWaves) void decode_prefix_kernel(PrefixParams p) {
  using S = DecodeShape<T, D>;
  constexpr int EPL = S::EPL, LPR = S::LPR, RPL = S::RPL, NR = S::NR;
  constexpr int NT = D / 16;                   // O^T tiles
  constexpr int PF = prefix_row_floats(D);     // floats per stored (sequence, head)
  constexpr int PL = 2 + 4 * NT;               // a lane's partial: m, l, acc
  struct Lds {
    uint4 q[16][LPR];  // the tile's 16 queries, normed and roped
    union {
      uint4 vt[kPrefixWaves][16][(D + 16) / 8];  // each wave's V block (padded rows)
      float part[kPrefixWaves][PL][64];          // every wave's partial
    } u;
  };
  __shared__ Lds lds;

#ifdef RLSE_DECODE_TIMELINE
  unsigned long long ptl[kPrefixTimelinePoints] = {};
#endif
  RLSE_PTL(0);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane % LPR, rsub = lane / LPR;
  const int mh = lane & 15, mq = lane >> 4;
  const int B = p.B, Hkv = p.Hkv, Hq = Hkv * G;
  const bool grouped = p.members != nullptr;
  // Workgroup id -> (KV head h, prefix slice sp, column tile c). One prefix:
  // slice set ps = sp * Hkv + h and tile c, where the tiles of one slice set
  // share id % 8, i.e. one XCD (workgroups are dealt to the XCDs
  // round-robin), and heads run fastest in ps, so that with Hkv a multiple
  // of 8 an XCD takes every slice of its heads; ids past the last slice set
  // have no work. Prefix groups: id = j * Hkv + h, where item j of the plan
  // names the group's tile and slice. The items are dense, so the ids with
  // work come first and are dispatched first, one workgroup a CU while they
  // last; the launch is sized by bounds (p.prefix bounds every group's
  // pages, p.tiles its column tiles) and the ids past the plan's items have
  // no work.
  const int NS = prefix_splits(p.prefix), NC = grouped ? p.tiles : (B * G + 15) / 16;
  const int id = blockIdx.x;
  int h, sp, ps = 0, c = 0;
  int P = p.prefix, ncols = B * G, c0 = 0, first = 0;
  const int* __restrict__ mem = nullptr;  // grouped: the group's members
  if (grouped) {
    // One round of loads: the item's entries, the plan's item count, stamp
    // and error word (and, in workgroup 0, every group's pages). A plan built
    // for another step shape (no items, another group count or group size)
    // is not used: the error is flagged and the decode launch that follows
    // does nothing either. Every entry is clamped into the batch, so no plan
    // makes an access leave its buffers.
    const int j = id / Hkv;
    h = id - j * Hkv;
    if (j >= kMaxGroupItems) return;
    const int* tail = p.members - kMaxDecodeBatch - kPlanStampWords;
    const int4* items = reinterpret_cast<const int4*>(p.grp + kGrpWords);
    const int4 te = items[j];
    const int rep = reinterpret_cast<const int*>(items + kMaxGroupItems)[j];
    const int stamp = tail[0], err = p.grp[kGrpErr], nitems = p.grp[kGrpItems];
    const int gpages = id == 0 && lane < p.num_groups ? p.grp[kGrpPages + lane] : 0;
    if (__builtin_amdgcn_readfirstlane(stamp) != group_stamp(p.num_groups, G)) {
      if (id == 0 && tid == 0) ws_raise(p.ws_err, RLSE_WS_ERR_PREFIX);
      return;
    }
    if (id == 0 && wave == 0) {
      // a group above the bound that sized the launch and the buffer, or
      // the plan's own error bits
      if (__any(gpages > p.prefix) && lane == 0) ws_raise(p.ws_err, RLSE_WS_ERR_PREFIX);
      if (err != 0 && lane == 0) ws_raise(p.ws_err, RLSE_WS_ERR_PREFIX);
    }
    if (j >= __builtin_amdgcn_readfirstlane(nitems)) return;
    P = __builtin_amdgcn_readfirstlane(te.x);
    const int r = __builtin_amdgcn_readfirstlane(rep);
    sp = r >> 16;
    if (P <= 0 || P > p.prefix || sp >= prefix_splits(P)) return;
    const int moff = min(max(__builtin_amdgcn_readfirstlane(te.z), 0), B);
    const int n_g = min(__builtin_amdgcn_readfirstlane(te.w), B - moff);
    c0 = __builtin_amdgcn_readfirstlane(te.y);
    if (n_g <= 0 || c0 < 0 || c0 >= n_g * G) return;
    ncols = n_g * G;
    first = min(max(r & 0xffff, 0), B - 1);
    mem = p.members + moff;
  } else {
    const int xq = id >> 3;
    ps = (xq / NC) * 8 + (id & 7);
    c = xq % NC;
    if (ps >= Hkv * NS) return;
    sp = ps / Hkv;
    h = ps - sp * Hkv;
    c0 = c * 16;
  }
  const int NSg = prefix_splits(P);
  // Sequence of column j (one per query head of the sequence); member
  // indices are clamped into the batch.
  auto seq_of = [&](int j) __attribute__((always_inline)) {
    const int b = mem ? mem[j / G] : j / G;
    return b < 0 ? 0 : (b < B ? b : B - 1);
  };
  const int* __restrict__ ptab = p.tables + (size_t)first * p.mbps;  // the group's pages
  const T* __restrict__ qb = reinterpret_cast<const T*>(p.q);
  const T* __restrict__ kp = reinterpret_cast<const T*>(p.k_pool);
  const T* __restrict__ vp = reinterpret_cast<const T*>(p.v_pool);


  // This wave's pages: slice sp of the prefix, then the wave's share of it.
  const int PS = (P + NSg - 1) / NSg;
  const int slo = sp * PS < P ? sp * PS : P, shi = slo + PS < P ? slo + PS : P;
  const int per = (shi - slo + kPrefixWaves - 1) / kPrefixWaves;
  const int lo = slo + wave * per < shi ? slo + wave * per : shi;
  const int hi = lo + per < shi ? lo + per : shi;
  // Lane i holds the page id of block lo + i (a wave takes at most 64).
  const int ids = lo + lane < hi ? ptab[lo + lane] : 0;
  // The contract: every sequence's first P table entries are the group's
  // first sequence's (sequence 0's without groups), and its new token
  // (position L - 1) lies past them. A plan checks it once per step (the
  // grouped plan's error word, read above; a one-prefix plan's verdict word,
  // read here by workgroup 0 and acted on at its end). Without a plan, wave 1
  // of each workgroup checks a share of the batch: every nwork-th of
  // sequences [k0, B), dealt over the workgroups. The first sequence's
  // entries are requested here, ahead of the page loads, and compared once
  // those are issued; further ones, when there are more sequences than
  // workgroups, are read at the end.
  constexpr int kChk = kMaxPrefixPages / 64;
  constexpr bool self_check = SELF_CHECK;
  const int k0 = ps * NC + c, kend = B, nwork = Hkv * NS * NC;
  const int verdict = !grouped && p.contract && id == 0 && wave == 1 ? *p.contract : 0;
  int chk_len = 0, chk_t[kChk], chk_0[kChk];
  bool bad = false;
  if (self_check && wave == 1 && k0 < kend) {
    const int b = seq_of(k0 * G);
    chk_len = p.seq_lens[b];
#pragma unroll
    for (int k = 0; k < kChk; ++k) {
      const int i = lane + 64 * k;
      chk_t[k] = i < P ? p.tables[(size_t)b * p.mbps + i] : 0;
      chk_0[k] = i < P ? ptab[i] : 0;
    }
  }

  // The tile's queries: column j = c0 + i is (sequence j / G, head h*G + j % G).
  // Their loads go out with the page ids, ahead of the first blocks' loads
  // (loads complete in order); their math follows those.
  constexpr int QPASS = 16 / RPL;  // staging passes, one per wave
  const bool stager = wave < QPASS;
  const int it = wave * RPL + rsub;
  const int qj = c0 + it;
  uint4 sq_x = make_uint4(0, 0, 0, 0), sq_c = sq_x, sq_s = sq_x, sq_w = sq_x;
  if (stager) {
    const int jj = qj < ncols ? qj : ncols - 1;
    const int b = seq_of(jj), g = jj % G;
    sq_x = *reinterpret_cast<const uint4*>(qb + ((size_t)b * Hq + (size_t)h * G + g) * D +
                                           (size_t)col * EPL);
    const int L = valid_len(p.seq_lens[b], p.mbps);
    const int pos = L > 0 ? L - 1 : 0;
    const size_t to = (size_t)pos * (D / 2) + (size_t)(col % (LPR / 2)) * EPL;
    sq_c = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.cos_t) + to);
    sq_s = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(p.sin_t) + to);
    const T* wp = reinterpret_cast<const T*>(p.qw ? p.qw : p.q);
    sq_w = *reinterpret_cast<const uint4*>(wp + col * EPL);
  }
  RLSE_PTL(1);

  uint4 qv[NR];
  float m1 = -INFINITY, l1 = 0.f, nms1 = 0.f, thr1 = -INFINITY;
  const float inv_c = 1.f / p.c;
  mma_f32x4_t macc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) macc[t] = mma_f32x4_t{0.f, 0.f, 0.f, 0.f};

  {
    // K in the MFMA operand layout, V coalesced (as the decode loads them);
    // a block past the range or on an id outside the pool gets a descriptor
    // of zero records (zeros, no memory access) and is masked.
    const size_t tile = (size_t)16 * D;
    const int koff = (int)(((size_t)(lane & 15) * D + (size_t)(lane >> 4) * EPL) * sizeof(T));
    const int voff = (int)(((size_t)rsub * D + (size_t)col * EPL) * sizeof(T));
    struct PBuf {
      uint4 k[NR];
      uint4 v[NR];
      int nv;
    };
    auto load = [&](PBuf& bf, int i) __attribute__((always_inline)) {
      const bool real = i < hi;
      const int id = __builtin_amdgcn_readlane(ids, real ? i - lo : 0);
      const bool fetch = real && (unsigned)id < (unsigned)p.num_blocks;
      bf.nv = fetch ? 16 : 0;
      const size_t tb = ((size_t)(fetch ? id : 0) * Hkv + h) * tile;
      const int nrec = fetch ? (int)(tile * sizeof(T)) : 0;
      const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(kp + tb), 0, nrec,
                                                        kBufferWord3);
      const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(vp + tb), 0, nrec,
                                                        kBufferWord3);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const u32x4_t kx =
            __builtin_amdgcn_raw_buffer_load_b128(rk, koff + r * 32 * (int)sizeof(T), 0, 0);
        const u32x4_t vx =
            __builtin_amdgcn_raw_buffer_load_b128(rv, voff + r * RPL * D * (int)sizeof(T), 0, 0);
        bf.k[r] = make_uint4(kx.x, kx.y, kx.z, kx.w);
        bf.v[r] = make_uint4(vx.x, vx.y, vx.z, vx.w);
      }
    };
    // The queries' math, then the barrier that publishes them, between the
    // first blocks' requests and their math.
    auto stage = [&]() __attribute__((always_inline)) {
      if (self_check && wave == 1 && k0 < kend) {
        bad = chk_len <= 16 * P || chk_len > p.mbps * 16;
#pragma unroll
        for (int k = 0; k < kChk; ++k) bad = bad || chk_t[k] != chk_0[k];
      }
      if (stager) {
        const uint4 y = norm_rope_packet<T, D>(sq_x, p.qw != nullptr, sq_w, p.inv_d, p.eps, sq_c,
                                               sq_s, col);
        lds.q[it][col] = qj < ncols ? y : make_uint4(0, 0, 0, 0);
      }
      consume(sq_x);
      consume(sq_c);
      consume(sq_s);
      consume(sq_w);
      __syncthreads();
      RLSE_PTL(3);
#pragma unroll
      for (int r = 0; r < NR; ++r) qv[r] = lds.q[mh][4 * r + mq];
    };
    // The decode's block math (decode_body, matrix-core path) on one block.
    auto compute = [&](const PBuf& bf) __attribute__((always_inline)) {
      const int nv = bf.nv;
#pragma unroll
      for (int r = 0; r < NR; ++r)
        lds.u.vt[wave][r * RPL + rsub][col] = nv > 0 ? bf.v[r] : make_uint4(0, 0, 0, 0);
      mma_f32x4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < NR; ++r) sacc = Mma16<T>::k32(bf.k[r], qv[r], sacc);
      float sv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = 4 * mq + i < nv ? sacc[i] : -INFINITY;
      const float cand = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      if (__any(cand > thr1)) {
        float cm = fmaxf(cand, __shfl_xor(cand, 16, 64));
        cm = fmaxf(cm, __shfl_xor(cm, 32, 64));
        const float mn = fmaxf(m1, cm * p.c);
        const float alpha = (mn == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m1 - mn);
        l1 *= alpha;
#pragma unroll
        for (int t = 0; t < NT; ++t)
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
      const uint2 pp = make_uint2(Packet<T>::pack2(pr[0], pr[1]), Packet<T>::pack2(pr[2], pr[3]));
      const uint16_t* vrow =
          reinterpret_cast<const uint16_t*>(&lds.u.vt[wave][4 * mq + ((lane & 15) >> 2)][0]) +
          4 * (lane & 3);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const mma_i16x4_t a =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((mma_lds_i16x4_t*)(vrow + 16 * t));
        macc[t] = Mma16<T>::k16(a, pp, macc[t]);
      }
    };
    PBuf b0, b1;
    if (per <= 2) {
      // At most two blocks a wave (per is the workgroup's share, so every
      // wave takes this branch or none does): both requested up front and
      // no third buffer, whose zero-size loads would still pass through the
      // compute unit's address unit ahead of the real ones.
      load(b0, lo);
      load(b1, lo + 1);
      RLSE_PTL(2);
      stage();
      if (lo < hi) {
        compute(b0);
        RLSE_PTL(4);
        if (lo + 1 < hi) compute(b1);
      }
    } else {
      PBuf b2;
      load(b0, lo);
      load(b1, lo + 1);
      load(b2, lo + 2);
      RLSE_PTL(2);
      stage();
      // Blocks i + 1 and i + 2 in flight while block i is computed.
      for (int i = lo; i < hi;) {
        compute(b0);
        if (i == lo) RLSE_PTL(4);
        if (++i == hi) break;
        load(b0, i + 2);
        compute(b1);
        if (++i == hi) break;
        load(b1, i + 2);
        compute(b2);
        if (++i == hi) break;
        load(b2, i + 2);
      }
    }
  }
  RLSE_PTL(5);

  // Every wave parks its partial in LDS (the V blocks are dead here); after
  // one barrier wave t combines accumulator tile t of all waves, in wave
  // order, and stores it in region sp; wave 0 also stores m and l.
  __syncthreads();
  {
    float(&dst)[PL][64] = lds.u.part[wave];
    dst[0][lane] = m1;
    dst[1][lane] = l1;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[2 + 4 * t + i][lane] = macc[t][i];
  }
  __syncthreads();
  RLSE_PTL(6);
  const int j = c0 + mh;
  if (wave < NT && j < ncols) {
    float pm[kPrefixWaves], M = -INFINITY;
#pragma unroll
    for (int v = 0; v < kPrefixWaves; ++v) {
      pm[v] = lds.u.part[v][0][lane];
      M = fmaxf(M, pm[v]);
    }
    const float Ms = (M == -INFINITY) ? 0.f : M;
    float l = 0.f, a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < kPrefixWaves; ++v) {
      const float sc = __builtin_amdgcn_exp2f(pm[v] - Ms);
      l = fmaf(lds.u.part[v][1][lane], sc, l);
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = fmaf(lds.u.part[v][2 + 4 * wave + i][lane], sc, a[i]);
    }
    // The head's sum over its four lanes; M is common to them.
    l = l + __shfl_xor(l, 16, 64);
    l = l + __shfl_xor(l, 32, 64);
    const int b = seq_of(j), g = j % G;
    const size_t slice = (size_t)B * Hq * PF;  // floats of one region
    float* dst = p.pre + (size_t)sp * slice + ((size_t)b * Hq + (size_t)h * G + g) * PF;
    *reinterpret_cast<float4*>(dst + 16 * wave + 4 * mq) = make_float4(a[0], a[1], a[2], a[3]);
    if (wave == 0 && mq == 0) *reinterpret_cast<float2*>(dst + D) = make_float2(M, l);
  }
  RLSE_PTL(7);
  if (verdict != 0 && lane == 0) ws_raise(p.ws_err, RLSE_WS_ERR_PREFIX);
  if (self_check && wave == 1 && k0 < kend) {
    for (int k = k0 + nwork; k < kend; k += nwork) {
      const int b = seq_of(k * G);
      const int L = p.seq_lens[b];
      bad = bad || L <= 16 * P || L > p.mbps * 16;
      for (int i = lane; i < P; i += 64) bad = bad || p.tables[(size_t)b * p.mbps + i] != ptab[i];
    }
    if (__any(bad) && lane == 0) ws_raise(p.ws_err, RLSE_WS_ERR_PREFIX);
  }
#ifdef RLSE_DECODE_TIMELINE
  RLSE_PTL(8);
  const size_t tw = (size_t)blockIdx.x * kPrefixWaves + wave;
  if (p.timeline && lane == 0 && tw < (size_t)kTimelineMaxWaves) {
    unsigned long long* dstt = p.timeline + tw * kPrefixTimelinePoints;
#pragma unroll
    for (int k = 0; k < kPrefixTimelinePoints; ++k) dstt[k] = ptl[k];
  }
#endif
}

template <typename T, int D, int G>
int launch_prefix_t(const PrefixParams& p, hipStream_t s) {
  // Grouped steps are checked by the grouped plan, planned one-prefix steps
  // by the plan (its verdict word): only a step without a plan checks here.
  const bool self_check = !p.members && !p.contract;
  // One prefix: 8 ids per group of 8 slice sets and column tile; prefix
  // groups: Hkv ids per work item the bounds allow (see the kernel).
  const int nps = p.Hkv * prefix_splits(p.prefix);
  const unsigned grid = p.members ? (unsigned)(nps * p.tiles)
                                  : (unsigned)(8 * ((p.B * G + 15) / 16) * ((nps + 7) / 8));
  if (self_check)
    hipLaunchKernelGGL((decode_prefix_kernel<T, D, G, true>), dim3(grid), dim3(64 * kPrefixWaves),
                       0, s, p);
  else
    hipLaunchKernelGGL((decode_prefix_kernel<T, D, G, false>), dim3(grid),
                       dim3(64 * kPrefixWaves), 0, s, p);
  return launch_status("decode_prefix_kernel");
}

template <typename T, int D>
int launch_prefix_g(int G, const PrefixParams& p, hipStream_t s) {
  switch (G) {
    case 1: return launch_prefix_t<T, D, 1>(p, s);
    case 2: return launch_prefix_t<T, D, 2>(p, s);
    case 3: return launch_prefix_t<T, D, 3>(p, s);
    case 4: return launch_prefix_t<T, D, 4>(p, s);
    case 5: return launch_prefix_t<T, D, 5>(p, s);
    case 6: return launch_prefix_t<T, D, 6>(p, s);
    case 7: return launch_prefix_t<T, D, 7>(p, s);
    case 8: return launch_prefix_t<T, D, 8>(p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode_prefix: unsupported group size %d", G);
}

template <typename T>
int launch_prefix_d(int D, int G, const PrefixParams& p, hipStream_t s) {
  switch (D) {
    case 64: return launch_prefix_g<T, 64>(G, p, s);
    case 128: return launch_prefix_g<T, 128>(G, p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode_prefix: unsupported head_dim %d", D);
}

}  // namespace

int launch_decode_prefix(int dtype, int D, int G, const PrefixParams& p, hipStream_t s) {
  switch (dtype) {
    case RLSE_DTYPE_BF16: return launch_prefix_d<bf16>(D, G, p, s);
    case RLSE_DTYPE_F16: return launch_prefix_d<f16>(D, G, p, s);
  }
  return fail(RLSE_ERR_INVALID_VALUE, "decode_prefix: dtype %d (16-bit K/V only)", dtype);
}

}  // namespace rlse
