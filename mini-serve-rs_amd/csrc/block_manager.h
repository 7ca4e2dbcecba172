// Host block manager and tensor memory budget state, shared by the block
// manager, the memory budget and the prefix cache (host-only C++; see
// block_manager.cpp and memory_budget.cpp for the semantics).
#pragma once

#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "rlse_kv.h"

// Byte budget of TensorMemoryBudget (src/cache/tensor_memory.rs:41-125):
// three reserved classes, a headroom reserved at creation, the peak and the
// rejection count. Every update is all-or-nothing under the mutex, as the
// reference's Mutex<TensorMemoryStats>.
struct rlse_memory_budget {
  std::mutex mu;
  long long budget = 0, headroom = 0;
  long long active_kv = 0, execution = 0, prefix = 0;
  long long reserved = 0, available = 0, peak = 0, rejections = 0;
  struct Lease {
    long long active_kv, execution, prefix;
  };
  std::unordered_map<long long, Lease> leases;
  long long next_lease = 1;

  // Charges the three amounts if their sum fits the available bytes.
  bool try_charge(long long kv, long long ex, long long pf) {
    long long total = 0;
    if (kv < 0 || ex < 0 || pf < 0 || __builtin_add_overflow(kv, ex, &total) ||
        __builtin_add_overflow(total, pf, &total) || total > available)
      return false;
    active_kv += kv;
    execution += ex;
    prefix += pf;
    reserved += total;
    available -= total;
    if (reserved > peak) peak = reserved;
    return true;
  }
  void uncharge(long long kv, long long ex, long long pf) {
    active_kv -= kv;
    execution -= ex;
    prefix -= pf;
    reserved -= kv + ex + pf;
    available += kv + ex + pf;
  }
};

// Pages are charged to an attached budget by who holds them: a page held by
// at least one request is active KV, a page held only by prefix-cache chunks
// is retained prefix, a free page is not charged.
struct rlse_block_manager {
  int total_blocks;
  int block_size;
  std::vector<int> free_stack;
  std::vector<int> refcount;    // all holders: requests and prefix-cache chunks
  std::vector<int> cache_refs;  // holders that are prefix-cache chunks
  std::unordered_map<std::string, std::vector<int>> allocations;
  // Version of each request's list: a new value whenever the list is
  // replaced (allocate, fork into a child); appends keep it. A table row
  // built from (request, version) needs only the appended tail afterwards.
  std::unordered_map<std::string, unsigned long long> list_version;
  unsigned long long next_version = 0;
  rlse_memory_budget* budget = nullptr;
  long long page_bytes = 0;

  enum Class { kFree, kActive, kPrefix };
  Class cls(int b) const {
    return refcount[b] == 0 ? kFree : (refcount[b] > cache_refs[b] ? kActive : kPrefix);
  }
  // Moves the budget charge of page b from class `from` to its current class.
  void recharge(int b, Class from) {
    const Class to = cls(b);
    if (!budget || from == to) return;
    std::lock_guard<std::mutex> g(budget->mu);
    const long long kv = (from == kActive ? -page_bytes : 0) + (to == kActive ? page_bytes : 0);
    const long long pf = (from == kPrefix ? -page_bytes : 0) + (to == kPrefix ? page_bytes : 0);
    budget->active_kv += kv;
    budget->prefix += pf;
    budget->reserved += kv + pf;
    budget->available -= kv + pf;
    if (budget->reserved > budget->peak) budget->peak = budget->reserved;
  }
  // True when n more pages would fit now: enough free pages and, with a
  // budget, enough available bytes for them as active KV (a check only; an
  // allocation charges with reserve_pages).
  bool pages_fit(long long n) const {
    if (n > (long long)free_stack.size()) return false;
    if (!budget) return true;
    long long bytes = 0;
    if (__builtin_mul_overflow(n, page_bytes, &bytes)) return false;
    std::lock_guard<std::mutex> g(budget->mu);
    return bytes <= budget->available;
  }
  // Charges n pages as active KV in one step (all or nothing, so workers
  // sharing the budget cannot overdraw it); the caller then takes them with
  // pop(). Assumes n free pages.
  bool reserve_pages(long long n) {
    if (!budget) return true;
    long long bytes = 0;
    if (__builtin_mul_overflow(n, page_bytes, &bytes)) return false;
    std::lock_guard<std::mutex> g(budget->mu);
    return budget->try_charge(bytes, 0, 0);
  }
  void set_list(const std::string& id, std::vector<int>&& blocks) {
    allocations[id] = std::move(blocks);
    list_version[id] = ++next_version;
  }
  long long blocks_needed(long long tokens) const {
    if (tokens <= 0) return 1;
    return (tokens + block_size - 1) / block_size;
  }
  // A free page for a request, already charged by reserve_pages.
  int pop() {
    const int b = free_stack.back();
    free_stack.pop_back();
    refcount[b] = 1;
    cache_refs[b] = 0;
    return b;
  }
  void ref_request(int b) {
    const Class from = cls(b);
    ++refcount[b];
    recharge(b, from);
  }
  void ref_cache(int b) {
    const Class from = cls(b);
    ++refcount[b];
    ++cache_refs[b];
    recharge(b, from);
  }
  void unref_request(int b) {
    const Class from = cls(b);
    if (--refcount[b] == 0) free_stack.push_back(b);
    recharge(b, from);
  }
  void unref_cache(int b) {
    const Class from = cls(b);
    --cache_refs[b];
    if (--refcount[b] == 0) free_stack.push_back(b);
    recharge(b, from);
  }
};
