// Prefix cache over refcounted pool pages: the successor of the reference's
// PrefixCache (src/cache/prefix_cache.rs:58-394).
//
// Kept from the reference, so lookups and eviction behave the same:
//   - a prompt is cut into chunks of chunk_size tokens, keyed by a chained
//     SHA-256: key_i = hex(sha256(key_{i-1} as ASCII hex || tokens of chunk i
//     as little-endian u32)), key_{-1} empty (compute_chunk_hashes, :98-124);
//   - lookup counts matching chunks from the start and stops at the first
//     miss, refreshing the LRU position of each match (:126-155);
//   - lookup_kv scans every chunk, refreshes each cached one and returns the
//     longest chunk that holds KV, with its logits only when that chunk ends
//     exactly at the end of the prompt (:157-196);
//   - insert adds metadata-only chunks; insert_kv stores KV for every chunk
//     boundary unless the chunk already holds KV (and logits, when logits are
//     offered); both evict the least recently used chunk while the cache is
//     full (:198-366);
//   - hit / miss / tokens-saved counters and the hit rate (:368-387).
// Changed for pages: a chunk holding KV keeps a reference on every page of
// its prefix (0 .. chunk_end) instead of a contiguous copy of the prefix, so
// inserting copies nothing and cached prefixes share pages with each other
// and with running requests. A restore (rlse_pc_fork) gives a new request
// those pages, copying only a trailing partial page. Pages return to the
// free list when their last holder -- request or chunk -- lets go.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <list>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "block_manager.h"

namespace rlse {
int fail(int code, const char* fmt, ...);
}
using rlse::fail;

namespace {

// ---------------------------------------------------------------------------
// SHA-256 (FIPS 180-4).
// ---------------------------------------------------------------------------
const uint32_t kSha256K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
    0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
    0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
    0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
    0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
    0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
    0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
    0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
    0xc67178f2};

class Sha256 {
 public:
  Sha256() {
    static const uint32_t init[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                     0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(h_, init, sizeof(h_));
  }
  void update(const uint8_t* p, size_t n) {
    for (size_t i = 0; i < n; ++i) {
      buf_[fill_++] = p[i];
      if (fill_ == 64) {
        block(buf_);
        fill_ = 0;
      }
    }
    bits_ += (uint64_t)n * 8;
  }
  std::string hex() {
    const uint64_t bits = bits_;
    const uint8_t one = 0x80, zero = 0;
    update(&one, 1);
    while (fill_ != 56) update(&zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(len, 8);
    static const char* digits = "0123456789abcdef";
    std::string out(64, '0');
    for (int i = 0; i < 8; ++i)
      for (int j = 0; j < 8; ++j) out[i * 8 + j] = digits[(h_[i] >> (28 - 4 * j)) & 15];
    return out;
  }

 private:
  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const uint8_t* p) {
    uint32_t w[64];
    for (int i = 0; i < 16; ++i)
      w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) |
             ((uint32_t)p[4 * i + 2] << 8) | (uint32_t)p[4 * i + 3];
    for (int i = 16; i < 64; ++i) {
      const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6],
             h = h_[7];
    for (int i = 0; i < 64; ++i) {
      const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
      const uint32_t ch = (e & f) ^ (~e & g);
      const uint32_t t1 = h + S1 + ch + kSha256K[i] + w[i];
      const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
      const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
      const uint32_t t2 = S0 + maj;
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    h_[0] += a;
    h_[1] += b;
    h_[2] += c;
    h_[3] += d;
    h_[4] += e;
    h_[5] += f;
    h_[6] += g;
    h_[7] += h;
  }
  uint32_t h_[8];
  uint8_t buf_[64];
  size_t fill_ = 0;
  uint64_t bits_ = 0;
};

// Chained keys of the whole chunks of tokens[0..n).
std::vector<std::string> chunk_keys(const uint32_t* tokens, long long n, int chunk_size) {
  std::vector<std::string> keys;
  const long long chunks = n / chunk_size;
  keys.reserve((size_t)chunks);
  std::string prev;
  for (long long i = 0; i < chunks; ++i) {
    Sha256 h;
    if (!prev.empty()) h.update(reinterpret_cast<const uint8_t*>(prev.data()), prev.size());
    for (int j = 0; j < chunk_size; ++j) {
      const uint32_t t = tokens[i * chunk_size + j];
      const uint8_t le[4] = {(uint8_t)t, (uint8_t)(t >> 8), (uint8_t)(t >> 16),
                             (uint8_t)(t >> 24)};
      h.update(le, 4);
    }
    prev = h.hex();
    keys.push_back(prev);
  }
  return keys;
}

struct Chunk {
  std::vector<uint32_t> tokens;  // the chunk's own tokens
  std::vector<int> pages;        // references on the prefix's pages (KV chunks)
  bool has_kv = false;
  bool has_logits = false;
  long long logits_handle = 0;   // caller's handle of the cached last logits
  std::list<std::string>::iterator lru;
};

}  // namespace

struct rlse_prefix_cache {
  rlse_block_manager* bm;
  int chunk_size;
  int max_chunks;
  std::unordered_map<std::string, Chunk> chunks;
  std::list<std::string> lru;  // front = least recently used
  long long hits = 0, misses = 0, tokens_saved = 0, kv_evictions = 0;

  void touch(Chunk& c) { lru.splice(lru.end(), lru, c.lru); }
  void drop(std::unordered_map<std::string, Chunk>::iterator it) {
    for (int p : it->second.pages) bm->unref_cache(p);
    lru.erase(it->second.lru);
    chunks.erase(it);
  }
  bool evict_oldest() {
    if (lru.empty()) return false;
    auto it = chunks.find(lru.front());
    if (it->second.has_kv) ++kv_evictions;
    drop(it);
    return true;
  }
  Chunk& add(const std::string& key, std::vector<uint32_t> tokens) {
    while ((int)chunks.size() >= max_chunks) evict_oldest();
    Chunk& c = chunks[key];
    c.tokens = std::move(tokens);
    lru.push_back(key);
    c.lru = std::prev(lru.end());
    return c;
  }
  long long held_pages() const {
    long long n = 0;
    for (const auto& kv : chunks) n += (long long)kv.second.pages.size();
    return n;
  }
};

static bool tokens_ok(const uint32_t* tokens, long long n) { return n == 0 || tokens != nullptr; }

extern "C" int rlse_pc_create(rlse_block_manager* bm, int chunk_size, int max_chunks,
                              rlse_prefix_cache** out) {
  if (!out) return fail(RLSE_ERR_INVALID_VALUE, "pc_create: null output");
  *out = nullptr;
  if (!bm || chunk_size <= 0 || max_chunks < 0 || chunk_size % bm->block_size != 0)
    return fail(RLSE_ERR_INVALID_VALUE,
                "pc_create: chunk_size %d must be a positive multiple of the block size",
                chunk_size);
  rlse_prefix_cache* pc = new (std::nothrow) rlse_prefix_cache;
  if (!pc) return fail(RLSE_ERR_INVALID_VALUE, "pc_create: out of memory");
  pc->bm = bm;
  pc->chunk_size = chunk_size;
  pc->max_chunks = max_chunks;
  *out = pc;
  return RLSE_OK;
}

extern "C" int rlse_pc_destroy(rlse_prefix_cache* pc) {
  if (!pc) return fail(RLSE_ERR_INVALID_VALUE, "pc_destroy: null");
  while (pc->evict_oldest()) {
  }
  delete pc;
  return RLSE_OK;
}

extern "C" int rlse_pc_chunk_hashes(const uint32_t* tokens, long long num_tokens, int chunk_size,
                                    char* out_hex, int capacity, int* num_chunks) {
  if (!tokens_ok(tokens, num_tokens) || num_tokens < 0 || chunk_size <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "pc_chunk_hashes: bad arguments");
  const std::vector<std::string> keys = chunk_keys(tokens, num_tokens, chunk_size);
  if (num_chunks) *num_chunks = (int)keys.size();
  if (out_hex) {
    if (capacity < (int)keys.size())
      return fail(RLSE_ERR_BUFFER_TOO_SMALL, "pc_chunk_hashes: capacity %d < %zu", capacity,
                  keys.size());
    for (size_t i = 0; i < keys.size(); ++i) memcpy(out_hex + 65 * i, keys[i].c_str(), 65);
  }
  return RLSE_OK;
}

extern "C" int rlse_pc_lookup(rlse_prefix_cache* pc, const uint32_t* tokens, long long num_tokens,
                              long long* matched_tokens) {
  if (!pc || !tokens_ok(tokens, num_tokens) || num_tokens < 0 || !matched_tokens)
    return fail(RLSE_ERR_INVALID_VALUE, "pc_lookup: bad arguments");
  long long matched = 0;
  for (const std::string& key : chunk_keys(tokens, num_tokens, pc->chunk_size)) {
    auto it = pc->chunks.find(key);
    if (it == pc->chunks.end()) break;
    ++matched;
    pc->touch(it->second);
  }
  *matched_tokens = matched * pc->chunk_size;
  return RLSE_OK;
}

extern "C" int rlse_pc_insert(rlse_prefix_cache* pc, const uint32_t* tokens,
                              long long num_tokens) {
  if (!pc || !tokens_ok(tokens, num_tokens) || num_tokens < 0)
    return fail(RLSE_ERR_INVALID_VALUE, "pc_insert: bad arguments");
  if (pc->max_chunks == 0) return RLSE_OK;
  const std::vector<std::string> keys = chunk_keys(tokens, num_tokens, pc->chunk_size);
  for (size_t i = 0; i < keys.size(); ++i) {
    if (pc->chunks.count(keys[i])) continue;
    pc->add(keys[i], std::vector<uint32_t>(tokens + i * pc->chunk_size,
                                           tokens + (i + 1) * pc->chunk_size));
  }
  return RLSE_OK;
}

extern "C" int rlse_pc_insert_kv(rlse_prefix_cache* pc, const uint32_t* tokens,
                                 long long num_tokens, const char* request_id, int has_logits,
                                 long long logits_handle) {
  if (!pc || !tokens_ok(tokens, num_tokens) || num_tokens < 0 || !request_id)
    return fail(RLSE_ERR_INVALID_VALUE, "pc_insert_kv: bad arguments");
  if (pc->max_chunks == 0) return RLSE_OK;
  auto rit = pc->bm->allocations.find(request_id);
  if (rit == pc->bm->allocations.end())
    return fail(RLSE_ERR_UNKNOWN_REQUEST, "pc_insert_kv: unknown request '%s'", request_id);
  const std::vector<std::string> keys = chunk_keys(tokens, num_tokens, pc->chunk_size);
  const int pages_per_chunk = pc->chunk_size / pc->bm->block_size;
  if ((long long)rit->second.size() < (long long)keys.size() * pages_per_chunk)
    return fail(RLSE_ERR_INVALID_VALUE,
                "pc_insert_kv: request '%s' holds %zu pages, %zu chunks need %lld", request_id,
                rit->second.size(), keys.size(), (long long)keys.size() * pages_per_chunk);
  for (size_t i = 0; i < keys.size(); ++i) {
    const long long chunk_end = (long long)(i + 1) * pc->chunk_size;
    const bool offer_logits = has_logits && chunk_end == num_tokens;
    auto it = pc->chunks.find(keys[i]);
    if (it != pc->chunks.end() && it->second.has_kv && (!offer_logits || it->second.has_logits))
      continue;
    // Replace an older metadata-only chunk, or one lacking logits.
    if (it != pc->chunks.end()) pc->drop(it);
    // The request's pages may be released by the eviction below; take the
    // chunk's references first.
    const std::vector<int>& req = pc->bm->allocations[request_id];
    std::vector<int> pages(req.begin(), req.begin() + (size_t)((i + 1) * pages_per_chunk));
    for (int p : pages) pc->bm->ref_cache(p);
    Chunk& c = pc->add(keys[i], std::vector<uint32_t>(tokens + i * pc->chunk_size,
                                                      tokens + (i + 1) * pc->chunk_size));
    c.pages = std::move(pages);
    c.has_kv = true;
    c.has_logits = offer_logits;
    c.logits_handle = offer_logits ? logits_handle : 0;
  }
  return RLSE_OK;
}

// The longest cached chunk with KV among tokens' chunks (refreshing every
// cached chunk met), or keys.end().
static const std::string* longest_kv(rlse_prefix_cache* pc, const std::vector<std::string>& keys,
                                     long long* end_tokens) {
  const std::string* best = nullptr;
  *end_tokens = 0;
  for (size_t i = 0; i < keys.size(); ++i) {
    auto it = pc->chunks.find(keys[i]);
    if (it == pc->chunks.end()) continue;  // a longer chunk may still be cached
    if (it->second.has_kv) {
      best = &it->first;
      *end_tokens = (long long)(i + 1) * pc->chunk_size;
    }
    pc->touch(it->second);
  }
  return best;
}

extern "C" int rlse_pc_lookup_kv(rlse_prefix_cache* pc, const uint32_t* tokens,
                                 long long num_tokens, long long* matched_tokens, int* has_logits,
                                 long long* logits_handle) {
  if (!pc || !tokens_ok(tokens, num_tokens) || num_tokens < 0 || !matched_tokens)
    return fail(RLSE_ERR_INVALID_VALUE, "pc_lookup_kv: bad arguments");
  long long end = 0;
  const std::string* key = longest_kv(pc, chunk_keys(tokens, num_tokens, pc->chunk_size), &end);
  *matched_tokens = end;
  const bool logits = key && end == num_tokens && pc->chunks[*key].has_logits;
  if (has_logits) *has_logits = logits ? 1 : 0;
  if (logits_handle) *logits_handle = logits ? pc->chunks[*key].logits_handle : 0;
  return RLSE_OK;
}

extern "C" int rlse_pc_fork(rlse_prefix_cache* pc, const uint32_t* tokens, long long num_tokens,
                            long long restore_tokens, const char* child_id, int32_t* cow_src,
                            int32_t* cow_dst, int cow_capacity, int* num_cow) {
  if (!pc || !tokens_ok(tokens, num_tokens) || num_tokens < 0 || !child_id || restore_tokens < 0)
    return fail(RLSE_ERR_INVALID_VALUE, "pc_fork: bad arguments");
  rlse_block_manager* bm = pc->bm;
  auto cit = bm->allocations.find(child_id);
  if (cit != bm->allocations.end() && !cit->second.empty())
    return fail(RLSE_ERR_INVALID_VALUE, "pc_fork: child '%s' already holds blocks", child_id);
  long long end = 0;
  const std::string* key = longest_kv(pc, chunk_keys(tokens, num_tokens, pc->chunk_size), &end);
  if (!key || restore_tokens > end)
    return fail(RLSE_ERR_INVALID_VALUE,
                "pc_fork: %lld tokens requested, the cache holds KV for %lld of this prompt",
                restore_tokens, end);
  const std::vector<int>& pages = pc->chunks[*key].pages;
  const long long full = restore_tokens / bm->block_size;
  const bool partial = restore_tokens % bm->block_size != 0;
  if (partial && bm->free_stack.empty())
    return fail(RLSE_ERR_CACHE_PRESSURE,
                "KV cache pressure: no free block for the copy-on-write of a partial block");
  if (partial && (!cow_src || !cow_dst || cow_capacity < 1))
    return fail(RLSE_ERR_BUFFER_TOO_SMALL, "pc_fork: no room for the copy-on-write pair");
  if (partial && !bm->reserve_pages(1)) {
    rlse_mb_record_rejection(bm->budget);
    return fail(RLSE_ERR_CACHE_PRESSURE,
                "Tensor memory budget exhausted: no room for the copy-on-write page");
  }
  std::vector<int> child;
  child.reserve((size_t)(full + 1));
  for (long long i = 0; i < full; ++i) {
    bm->ref_request(pages[(size_t)i]);
    child.push_back(pages[(size_t)i]);
  }
  int ncow = 0;
  if (partial) {
    const int dst = bm->pop();
    cow_src[0] = pages[(size_t)full];
    cow_dst[0] = dst;
    child.push_back(dst);
    ncow = 1;
  }
  if (num_cow) *num_cow = ncow;
  bm->set_list(child_id, std::move(child));
  return RLSE_OK;
}

extern "C" int rlse_pc_reclaim(rlse_prefix_cache* pc, int min_free_blocks, int* evicted) {
  if (!pc || min_free_blocks < 0) return fail(RLSE_ERR_INVALID_VALUE, "pc_reclaim: bad arguments");
  int n = 0;
  while (!pc->bm->pages_fit(min_free_blocks) && pc->evict_oldest()) ++n;
  if (evicted) *evicted = n;
  if ((int)pc->bm->free_stack.size() < min_free_blocks)
    return fail(RLSE_ERR_CACHE_PRESSURE,
                "KV cache pressure: %zu free blocks after evicting every cached prefix, %d needed",
                pc->bm->free_stack.size(), min_free_blocks);
  if (!pc->bm->pages_fit(min_free_blocks))
    return fail(RLSE_ERR_CACHE_PRESSURE,
                "Tensor memory budget exhausted: %d pages do not fit after evicting every cached "
                "prefix",
                min_free_blocks);
  return RLSE_OK;
}

extern "C" int rlse_pc_reserve_memory(rlse_prefix_cache* pc, long long active_kv_bytes,
                                      long long execution_bytes, long long prefix_bytes,
                                      long long* lease) {
  if (!pc || !lease) return fail(RLSE_ERR_INVALID_VALUE, "pc_reserve_memory: bad arguments");
  rlse_memory_budget* mb = pc->bm->budget;
  if (!mb)
    return fail(RLSE_ERR_INVALID_VALUE, "pc_reserve_memory: the block manager has no budget");
  for (;;) {
    if (rlse_mb_try_reserve(mb, active_kv_bytes, execution_bytes, prefix_bytes, lease) == RLSE_OK)
      return RLSE_OK;
    if (!pc->evict_oldest()) {
      rlse_mb_record_rejection(mb);
      return fail(RLSE_ERR_CACHE_PRESSURE, "Tensor memory budget exhausted");
    }
  }
}

extern "C" int rlse_pc_clear(rlse_prefix_cache* pc) {
  if (!pc) return fail(RLSE_ERR_INVALID_VALUE, "pc_clear: null");
  while (pc->evict_oldest()) {
  }
  return RLSE_OK;
}

extern "C" int rlse_pc_record_reuse(rlse_prefix_cache* pc, long long skipped_tokens) {
  if (!pc || skipped_tokens < 0) return fail(RLSE_ERR_INVALID_VALUE, "pc_record_reuse: bad args");
  if (skipped_tokens == 0) {
    ++pc->misses;
  } else {
    ++pc->hits;
    pc->tokens_saved += skipped_tokens;
  }
  return RLSE_OK;
}

extern "C" int rlse_pc_stats(const rlse_prefix_cache* pc, rlse_prefix_stats* out) {
  if (!pc || !out) return fail(RLSE_ERR_INVALID_VALUE, "pc_stats: bad arguments");
  out->hits = pc->hits;
  out->misses = pc->misses;
  out->tokens_saved = pc->tokens_saved;
  out->kv_evictions = pc->kv_evictions;
  out->chunks = (long long)pc->chunks.size();
  out->held_pages = pc->held_pages();
  const long long total = pc->hits + pc->misses;
  out->hit_rate = total > 0 ? ((float)pc->hits / (float)total) * 100.0f : 0.0f;
  return RLSE_OK;
}
