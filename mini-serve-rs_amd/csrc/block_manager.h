// Host block manager state, shared by the block manager and the prefix cache
// (both host-only C++; see block_manager.cpp for the semantics).
#pragma once

#include <string>
#include <unordered_map>
#include <vector>

#include "rlse_kv.h"

struct rlse_block_manager {
  int total_blocks;
  int block_size;
  std::vector<int> free_stack;
  std::vector<int> refcount;
  std::unordered_map<std::string, std::vector<int>> allocations;

  long long blocks_needed(long long tokens) const {
    if (tokens <= 0) return 1;
    return (tokens + block_size - 1) / block_size;
  }
  int pop() {
    const int b = free_stack.back();
    free_stack.pop_back();
    refcount[b] = 1;
    return b;
  }
  void unref(int b) {
    if (--refcount[b] == 0) free_stack.push_back(b);
  }
};
