// Host block manager: the physical-page successor of the reference's logical
// block allocator KVCache (src/cache/kv_cache.rs:15-145).
//
// Kept from the reference, so a scheduler sees the same ids and errors:
//   - a free stack filled so that pops yield 0, 1, 2, ... (kv_cache.rs:23-35);
//   - blocks_needed(t) = 1 for t == 0, else ceil(t / block_size) (:53-59);
//   - allocate replaces the request's list (HashMap insert, :61-84) and fails
//     with the reference's CachePressure text when too few blocks are free;
//   - allocate_block appends one block (:86-99); release pushes the request's
//     blocks back in list order and reports how many it held (:101-111);
//   - stats: utilization and fragmentation rounded to 3 decimals (:113-145).
// Added for physical pages: a refcount per block, so a prefix can be shared by
// several sequences (fork), with copy-on-write of a trailing partial block.
// A block is pushed back on the free stack only when its last holder releases it.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <new>

#include "block_manager.h"

namespace rlse {
int fail(int code, const char* fmt, ...);
}
using rlse::fail;

static float round3(float x) { return roundf(x * 1000.0f) / 1000.0f; }

// An allocation of n pages that the attached budget cannot hold: counted as a
// rejection (TensorMemoryBudget::record_rejection) and refused before any change.
static int budget_pressure(rlse_block_manager* bm, long long n) {
  long long avail = 0;
  {
    std::lock_guard<std::mutex> g(bm->budget->mu);
    ++bm->budget->rejections;
    avail = bm->budget->available;
  }
  return fail(RLSE_ERR_CACHE_PRESSURE,
              "Tensor memory budget exhausted: %lld pages of %lld bytes requested, %lld bytes "
              "available",
              n, bm->page_bytes, avail);
}

extern "C" int rlse_bm_create(int total_blocks, int block_size, rlse_block_manager** out) {
  if (!out) return fail(RLSE_ERR_INVALID_VALUE, "bm_create: null output");
  *out = nullptr;
  if (total_blocks < 0 || block_size <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "bm_create: total_blocks %d block_size %d",
                total_blocks, block_size);
  rlse_block_manager* bm = new (std::nothrow) rlse_block_manager;
  if (!bm) return fail(RLSE_ERR_INVALID_VALUE, "bm_create: out of memory");
  bm->total_blocks = total_blocks;
  bm->block_size = block_size;
  bm->free_stack.reserve(total_blocks);
  for (int i = total_blocks - 1; i >= 0; --i) bm->free_stack.push_back(i);
  bm->refcount.assign(total_blocks, 0);
  bm->cache_refs.assign(total_blocks, 0);
  *out = bm;
  return RLSE_OK;
}

extern "C" int rlse_bm_destroy(rlse_block_manager* bm) {
  if (!bm) return fail(RLSE_ERR_INVALID_VALUE, "bm_destroy: null");
  if (bm->budget) rlse_bm_attach_budget(bm, nullptr, 0);  // uncharge every held page
  delete bm;
  return RLSE_OK;
}

extern "C" int rlse_bm_blocks_needed(const rlse_block_manager* bm, long long tokens) {
  if (!bm || tokens < 0) return -1;
  const long long n = bm->blocks_needed(tokens);
  return n > 0x7fffffffLL ? -1 : (int)n;
}

extern "C" int rlse_bm_free_count(const rlse_block_manager* bm) {
  return bm ? (int)bm->free_stack.size() : -1;
}

extern "C" int rlse_bm_allocate(rlse_block_manager* bm, const char* request_id,
                                long long num_tokens, int32_t* out_blocks, int capacity,
                                int* num_out) {
  if (!bm || !request_id || num_tokens < 0)
    return fail(RLSE_ERR_INVALID_VALUE, "bm_allocate: bad arguments");
  const long long needed = bm->blocks_needed(num_tokens);
  if (needed > (long long)bm->free_stack.size())
    return fail(RLSE_ERR_CACHE_PRESSURE,
                "Requested %lld blocks (%lld tokens), but only %zu free blocks remain", needed,
                num_tokens, bm->free_stack.size());
  if (out_blocks && capacity < needed)
    return fail(RLSE_ERR_BUFFER_TOO_SMALL, "bm_allocate: capacity %d < %lld blocks", capacity,
                needed);
  if (!bm->reserve_pages(needed)) return budget_pressure(bm, needed);
  std::vector<int> blocks;
  blocks.reserve((size_t)needed);
  for (long long i = 0; i < needed; ++i) blocks.push_back(bm->pop());
  if (out_blocks)
    for (size_t i = 0; i < blocks.size(); ++i) out_blocks[i] = blocks[i];
  if (num_out) *num_out = (int)needed;
  bm->set_list(request_id, std::move(blocks));
  return RLSE_OK;
}

extern "C" int rlse_bm_allocate_block(rlse_block_manager* bm, const char* request_id,
                                      int32_t* out_block) {
  if (!bm || !request_id) return fail(RLSE_ERR_INVALID_VALUE, "bm_allocate_block: bad args");
  if (bm->free_stack.empty())
    return fail(RLSE_ERR_CACHE_PRESSURE,
                "KV cache pressure: no free blocks remaining for incremental allocation");
  if (!bm->reserve_pages(1)) return budget_pressure(bm, 1);
  const int b = bm->pop();
  auto& list = bm->allocations[request_id];
  if (list.empty()) bm->list_version[request_id] = ++bm->next_version;  // a new request
  list.push_back(b);
  if (out_block) *out_block = b;
  return RLSE_OK;
}

extern "C" int rlse_bm_release(rlse_block_manager* bm, const char* request_id,
                               int* num_released) {
  if (!bm || !request_id) return fail(RLSE_ERR_INVALID_VALUE, "bm_release: bad args");
  auto it = bm->allocations.find(request_id);
  int count = 0;
  if (it != bm->allocations.end()) {
    count = (int)it->second.size();
    for (int b : it->second) bm->unref_request(b);
    bm->allocations.erase(it);
    bm->list_version.erase(request_id);
  }
  if (num_released) *num_released = count;
  return RLSE_OK;
}

extern "C" int rlse_bm_release_all(rlse_block_manager* bm, int* num_requests) {
  if (!bm) return fail(RLSE_ERR_INVALID_VALUE, "bm_release_all: null");
  // In request-id order, so the free stack (and the ids handed out next) does
  // not depend on the hash map's iteration order.
  std::vector<std::string> ids;
  ids.reserve(bm->allocations.size());
  for (const auto& kv : bm->allocations) ids.push_back(kv.first);
  std::sort(ids.begin(), ids.end());
  for (const std::string& id : ids) {
    for (int b : bm->allocations[id]) bm->unref_request(b);
    bm->allocations.erase(id);
    bm->list_version.erase(id);
  }
  if (num_requests) *num_requests = (int)ids.size();
  return RLSE_OK;
}

extern "C" int rlse_bm_fork(rlse_block_manager* bm, const char* parent_id, const char* child_id,
                            long long num_tokens, int32_t* cow_src, int32_t* cow_dst,
                            int cow_capacity, int* num_cow) {
  if (!bm || !parent_id || !child_id || num_tokens < 0)
    return fail(RLSE_ERR_INVALID_VALUE, "bm_fork: bad arguments");
  if (strcmp(parent_id, child_id) == 0)
    return fail(RLSE_ERR_INVALID_VALUE, "bm_fork: parent and child are the same request");
  auto pit = bm->allocations.find(parent_id);
  if (pit == bm->allocations.end())
    return fail(RLSE_ERR_UNKNOWN_REQUEST, "bm_fork: unknown parent '%s'", parent_id);
  auto cit = bm->allocations.find(child_id);
  if (cit != bm->allocations.end() && !cit->second.empty())
    return fail(RLSE_ERR_INVALID_VALUE, "bm_fork: child '%s' already holds blocks", child_id);
  const long long full = num_tokens / bm->block_size;
  const bool partial = (num_tokens % bm->block_size) != 0;
  const std::vector<int>& parent = pit->second;
  if ((long long)parent.size() < full + (partial ? 1 : 0))
    return fail(RLSE_ERR_INVALID_VALUE, "bm_fork: parent holds %zu blocks, %lld tokens need %lld",
                parent.size(), num_tokens, full + (partial ? 1 : 0));
  if (partial && bm->free_stack.empty())
    return fail(RLSE_ERR_CACHE_PRESSURE,
                "KV cache pressure: no free block for the copy-on-write of a partial block");
  if (partial && (!cow_src || !cow_dst || cow_capacity < 1))
    return fail(RLSE_ERR_BUFFER_TOO_SMALL, "bm_fork: no room for the copy-on-write pair");
  if (partial && !bm->reserve_pages(1)) return budget_pressure(bm, 1);
  std::vector<int> child;
  child.reserve((size_t)(full + 1));
  for (long long i = 0; i < full; ++i) {
    const int b = parent[(size_t)i];
    bm->ref_request(b);
    child.push_back(b);
  }
  int ncow = 0;
  if (partial) {
    const int dst = bm->pop();
    cow_src[0] = parent[(size_t)full];
    cow_dst[0] = dst;
    child.push_back(dst);
    ncow = 1;
  }
  if (num_cow) *num_cow = ncow;
  bm->set_list(child_id, std::move(child));
  return RLSE_OK;
}

extern "C" int rlse_bm_block_table(const rlse_block_manager* bm, const char* request_id,
                                   int32_t* out_blocks, int capacity, int* num_out) {
  if (!bm || !request_id) return fail(RLSE_ERR_INVALID_VALUE, "bm_block_table: bad args");
  auto it = bm->allocations.find(request_id);
  if (it == bm->allocations.end())
    return fail(RLSE_ERR_UNKNOWN_REQUEST, "bm_block_table: unknown request '%s'", request_id);
  const std::vector<int>& v = it->second;
  if (num_out) *num_out = (int)v.size();
  if (out_blocks) {
    if (capacity < (int)v.size())
      return fail(RLSE_ERR_BUFFER_TOO_SMALL, "bm_block_table: capacity %d < %zu", capacity,
                  v.size());
    for (size_t i = 0; i < v.size(); ++i) out_blocks[i] = v[i];
  }
  return RLSE_OK;
}

extern "C" int rlse_bm_refcount(const rlse_block_manager* bm, int block) {
  if (!bm || block < 0 || block >= bm->total_blocks) return -1;
  return bm->refcount[block];
}

extern "C" int rlse_bm_stats(const rlse_block_manager* bm, rlse_cache_stats* out) {
  if (!bm || !out) return fail(RLSE_ERR_INVALID_VALUE, "bm_stats: bad args");
  const int total = bm->total_blocks;
  const int free_n = (int)bm->free_stack.size();
  const int allocated = total - free_n;
  const float utilization = total > 0 ? (float)allocated / (float)total : 0.0f;
  std::vector<char> is_free(total, 0);
  for (int b : bm->free_stack) is_free[b] = 1;
  int runs = 0;
  for (int i = 0; i < total; ++i)
    if (is_free[i] && (i == 0 || !is_free[i - 1])) ++runs;
  float frag = 0.0f;
  if (free_n > 0 && runs > 1) frag = ((float)runs - 1.0f) / (float)free_n;
  out->total_blocks = total;
  out->allocated_blocks = allocated;
  out->free_blocks = free_n;
  out->utilization = round3(utilization);
  out->fragmentation = round3(frag < 1.0f ? frag : 1.0f);
  return RLSE_OK;
}
