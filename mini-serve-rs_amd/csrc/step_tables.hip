// Per-step block-table hand-off from the host block manager to the device:
// the successor of the scheduler's per-step block reservation
// (src/scheduler/scheduler.rs:422-449), which grows each active sequence by
// a block when blocks_needed(next_len) exceeds the blocks it holds and
// drops -- cancel + release -- a sequence that cannot grow.
//
// rlse_st_prepare runs that loop over the step's batch and lays out the
// packed block-table rows and lengths the decode kernels read (row i =
// request i of the batch). It remembers, per row, which request and which
// version of its block list the device copy holds, so a row whose request
// only grew costs one (row, column, page) triple per new page, and only a
// row that changed request (or whose list was replaced) is sent whole.
// rlse_st_upload stages the lengths and the triples in pinned host memory
// (two buffers, so the host can fill one while the other is in flight),
// copies them in one transfer and applies them with one scatter kernel: at
// long contexts this replaces a full-table upload per step (1 MB at 128
// sequences of 32 K tokens) with a few hundred bytes.
#include <string.h>

#include <string>
#include <vector>

#include "block_manager.h"
#include "common.cuh"
#include "host_common.h"

namespace rlse {
namespace {

// Lengths into seq_lens, then (row, col, page) triples into the table.
__global__ void apply_step_kernel(const int32_t* __restrict__ stage, int batch, int ndelta,
                                  int mbps, int32_t* __restrict__ tables,
                                  int32_t* __restrict__ seq_lens) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < batch) seq_lens[i] = stage[i];
  if (i < ndelta) {
    const int32_t* d = stage + batch + 3 * (size_t)i;
    tables[(size_t)d[0] * mbps + d[1]] = d[2];
  }
}

}  // namespace
}  // namespace rlse

using namespace rlse;

struct rlse_step_tables {
  int max_batch = 0, mbps = 0;
  // What the device copy of each row holds.
  std::vector<std::string> row_req;
  std::vector<unsigned long long> row_version;
  std::vector<int> row_count;
  // This step: the host image of the tables, the lengths and the pending
  // triples (rows < batch).
  int batch = 0;
  std::vector<int32_t> tables, lens, deltas;
  // Upload staging, grown on demand: two pinned host buffers and two device
  // buffers, each pair reused once the event recorded after its scatter
  // kernel has completed.
  int device = -1;
  size_t cap_ints = 0;
  int32_t* h_stage[2] = {nullptr, nullptr};
  int32_t* d_stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int cur = 0;

  void free_staging() {
    for (int k = 0; k < 2; ++k) {
      if (done[k]) (void)hipEventSynchronize(done[k]);
      if (h_stage[k]) (void)hipHostFree(h_stage[k]);
      if (d_stage[k]) (void)hipFree(d_stage[k]);
      h_stage[k] = d_stage[k] = nullptr;
    }
    cap_ints = 0;
  }
};

extern "C" int rlse_st_create(int max_batch, int max_blocks_per_seq, rlse_step_tables** out) {
  if (!out) return fail(RLSE_ERR_INVALID_VALUE, "st_create: null output");
  *out = nullptr;
  if (max_batch <= 0 || max_blocks_per_seq <= 0 ||
      (long long)max_batch * max_blocks_per_seq > 0x7fffffffLL)
    return fail(RLSE_ERR_INVALID_VALUE, "st_create: max_batch %d max_blocks_per_seq %d",
                max_batch, max_blocks_per_seq);
  rlse_step_tables* st = new (std::nothrow) rlse_step_tables;
  if (!st) return fail(RLSE_ERR_INVALID_VALUE, "st_create: out of memory");
  st->max_batch = max_batch;
  st->mbps = max_blocks_per_seq;
  st->row_req.assign(max_batch, std::string());
  st->row_version.assign(max_batch, 0);
  st->row_count.assign(max_batch, 0);
  st->tables.assign((size_t)max_batch * max_blocks_per_seq, -1);
  st->lens.assign(max_batch, 0);
  *out = st;
  return RLSE_OK;
}

extern "C" int rlse_st_destroy(rlse_step_tables* st) {
  if (!st) return fail(RLSE_ERR_INVALID_VALUE, "st_destroy: null");
  st->free_staging();
  for (int k = 0; k < 2; ++k)
    if (st->done[k]) (void)hipEventDestroy(st->done[k]);
  delete st;
  return RLSE_OK;
}

extern "C" int rlse_st_reset(rlse_step_tables* st) {
  if (!st) return fail(RLSE_ERR_INVALID_VALUE, "st_reset: null");
  for (int r = 0; r < st->max_batch; ++r) {
    st->row_req[r].clear();
    st->row_version[r] = 0;
    st->row_count[r] = 0;
  }
  st->deltas.clear();
  return RLSE_OK;
}

extern "C" int rlse_st_prepare(rlse_step_tables* st, rlse_block_manager* bm,
                               const char* const* request_ids, const long long* next_lens,
                               int batch, int* status) {
  if (!st || !bm || batch < 0 || (batch > 0 && (!request_ids || !next_lens || !status)))
    return fail(RLSE_ERR_INVALID_VALUE, "st_prepare: bad arguments");
  if (batch > st->max_batch)
    return fail(RLSE_ERR_INVALID_VALUE, "st_prepare: batch %d > max_batch %d", batch,
                st->max_batch);
  const int mbps = st->mbps;
  // Triples still pending from an earlier prepare (no upload since): a row
  // prepared again supersedes its pending triples from the column it now
  // starts at, so one upload never carries two pages for one table cell.
  const size_t prev = st->deltas.size() / 3;
  std::vector<std::vector<size_t>> pending_of_row;
  if (prev > 0) {
    pending_of_row.resize(st->max_batch);
    for (size_t t = 0; t < prev; ++t) pending_of_row[st->deltas[3 * t]].push_back(t);
  }
  bool dropped = false;
  auto drop_pending = [&](int row, int from_col) {
    if (prev == 0) return;
    for (size_t t : pending_of_row[row])
      if (st->deltas[3 * t + 1] >= from_col) {
        st->deltas[3 * t] = -1;  // removed below
        dropped = true;
      }
  };
  for (int i = 0; i < batch; ++i) {
    st->lens[i] = 0;
    status[i] = RLSE_OK;
    const char* id = request_ids[i];
    const long long len = next_lens[i];
    if (!id || len < 0 || len > 0x7fffffffLL) {
      status[i] = RLSE_ERR_INVALID_VALUE;
      continue;
    }
    auto it = bm->allocations.find(id);
    if (it == bm->allocations.end()) {
      status[i] = RLSE_ERR_UNKNOWN_REQUEST;
      continue;
    }
    const long long need = bm->blocks_needed(len);
    if (need > mbps) {
      status[i] = RLSE_ERR_INVALID_VALUE;
      continue;
    }
    // scheduler.rs:427-445: grow to blocks_needed(next_len); a sequence that
    // cannot grow is released and leaves the batch (length 0 here: the
    // decode kernels write zeros for it).
    while ((long long)it->second.size() < need) {
      int32_t b = 0;
      const int rc = rlse_bm_allocate_block(bm, id, &b);
      if (rc != RLSE_OK) {
        status[i] = rc;
        break;
      }
    }
    if (status[i] != RLSE_OK) {
      rlse_bm_release(bm, id, nullptr);
      continue;
    }
    st->lens[i] = (int32_t)len;
    const std::vector<int>& pages = it->second;
    const int count = (int)std::min<size_t>(pages.size(), (size_t)mbps);
    const unsigned long long ver = bm->list_version[id];
    int from = st->row_count[i];
    if (st->row_req[i] != id || st->row_version[i] != ver || from > count) {
      st->row_req[i] = id;
      st->row_version[i] = ver;
      from = 0;
    }
    drop_pending(i, from);
    int32_t* row = st->tables.data() + (size_t)i * mbps;
    for (int j = from; j < count; ++j) {
      row[j] = pages[(size_t)j];
      st->deltas.insert(st->deltas.end(), {(int32_t)i, (int32_t)j, (int32_t)pages[(size_t)j]});
    }
    st->row_count[i] = count;
  }
  if (dropped) {
    size_t w = 0;
    for (size_t t = 0; t < st->deltas.size() / 3; ++t) {
      if (st->deltas[3 * t] < 0) continue;
      for (int c = 0; c < 3; ++c) st->deltas[3 * w + c] = st->deltas[3 * t + c];
      ++w;
    }
    st->deltas.resize(3 * w);
  }
  st->batch = batch;
  return RLSE_OK;
}

extern "C" int rlse_st_host(const rlse_step_tables* st, const int32_t** tables,
                            const int32_t** seq_lens, int* batch, const int32_t** pending,
                            int* num_pending) {
  if (!st) return fail(RLSE_ERR_INVALID_VALUE, "st_host: null");
  if (tables) *tables = st->tables.data();
  if (seq_lens) *seq_lens = st->lens.data();
  if (batch) *batch = st->batch;
  if (pending) *pending = st->deltas.data();
  if (num_pending) *num_pending = (int)(st->deltas.size() / 3);
  return RLSE_OK;
}

extern "C" int rlse_st_mark_uploaded(rlse_step_tables* st) {
  if (!st) return fail(RLSE_ERR_INVALID_VALUE, "st_mark_uploaded: null");
  st->deltas.clear();
  return RLSE_OK;
}

extern "C" int rlse_st_upload(rlse_step_tables* st, int32_t* tables, int32_t* seq_lens,
                              rlse_stream_t stream) {
  if (!st || !tables || !seq_lens) return fail(RLSE_ERR_INVALID_VALUE, "st_upload: bad args");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "st_upload: no current device");
  if (st->device >= 0 && st->device != dev)
    return fail(RLSE_ERR_INVALID_VALUE, "st_upload: created its staging on device %d, now %d",
                st->device, dev);
  const int ndelta = (int)(st->deltas.size() / 3);
  const size_t ints = (size_t)st->batch + 3 * (size_t)ndelta;
  if (ints == 0) return RLSE_OK;
  if (ints > st->cap_ints) {
    st->free_staging();
    const size_t cap = std::max(ints + ints / 2, (size_t)4096);
    for (int k = 0; k < 2; ++k) {
      e = hipHostMalloc((void**)&st->h_stage[k], cap * sizeof(int32_t), hipHostMallocDefault);
      if (e == hipSuccess) e = hipMalloc((void**)&st->d_stage[k], cap * sizeof(int32_t));
      if (e == hipSuccess && !st->done[k])
        e = hipEventCreateWithFlags(&st->done[k], hipEventDisableTiming);
      if (e != hipSuccess) {
        st->free_staging();
        return fail((int)e, "st_upload: staging allocation failed");
      }
    }
    st->cap_ints = cap;
    st->device = dev;
  }
  const int k = st->cur;
  // The pinned buffer and its device twin are free once the scatter kernel
  // of the upload that last used them has run.
  e = hipEventSynchronize(st->done[k]);
  if (e != hipSuccess) return fail((int)e, "st_upload: waiting for the previous upload failed");
  memcpy(st->h_stage[k], st->lens.data(), (size_t)st->batch * sizeof(int32_t));
  memcpy(st->h_stage[k] + st->batch, st->deltas.data(), st->deltas.size() * sizeof(int32_t));
  e = hipMemcpyAsync(st->d_stage[k], st->h_stage[k], ints * sizeof(int32_t),
                     hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return fail((int)e, "st_upload: copy failed");
  const int items = std::max(st->batch, ndelta);
  hipLaunchKernelGGL(apply_step_kernel, dim3((items + 255) / 256), dim3(256), 0, s,
                     st->d_stage[k], st->batch, ndelta, st->mbps, tables, seq_lens);
  const int rc = launch_status("apply_step_kernel");
  if (rc) return rc;
  e = hipEventRecord(st->done[k], s);
  if (e != hipSuccess) return fail((int)e, "st_upload: event record failed");
  st->deltas.clear();
  st->cur ^= 1;
  return RLSE_OK;
}
