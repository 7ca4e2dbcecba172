// Tensor memory budget with page-based KV charges: the successor of the
// reference's TensorMemoryBudget (src/cache/tensor_memory.rs:1-125) and of
// CandleBackend::memory_charge (src/backends/candle.rs:241-282).
//
// Kept from the reference, so an admission path sees the same accounting:
//   - a budget with a headroom reserved at creation, refused unless
//     0 <= headroom < budget (tensor_memory.rs:48-67);
//   - three reserved classes (active KV, execution, retained prefix), the
//     peak of the reserved bytes and a rejection count (:28-39);
//   - try_reserve is all-or-nothing and refuses a charge whose total overflows
//     (:72-90); a lease gives its bytes back when released (:105-117);
//   - memory_charge's checked products and its token-limit check.
// Changed for paged KV: the reference charges every request its whole
// contiguous capacity, 2*layers*Hkv*d*(prompt+max_tokens)*bytes, up front.
// Here a block manager with an attached budget charges each page as it
// leaves the free stack -- active KV while a request holds it, retained
// prefix while only prefix-cache chunks hold it -- and uncharges it when its
// last holder lets go, so a request's KV charge follows the pages it
// actually holds and a prefix shared by many requests is charged once. The
// execution estimate drops the reference's KV-sized staging allowance: pages
// are written in place, with no contiguous staging copy.
#include <limits.h>

#include <new>

#include "block_manager.h"

namespace rlse {
int fail(int code, const char* fmt, ...);
}
using rlse::fail;

extern "C" int rlse_mb_create(long long budget_bytes, long long headroom_bytes,
                              rlse_memory_budget** out) {
  if (!out) return fail(RLSE_ERR_INVALID_VALUE, "mb_create: null output");
  *out = nullptr;
  if (budget_bytes <= 0 || headroom_bytes < 0 || headroom_bytes >= budget_bytes)
    return fail(RLSE_ERR_INVALID_VALUE,
                "tensor memory budget must be positive and greater than execution headroom");
  rlse_memory_budget* mb = new (std::nothrow) rlse_memory_budget;
  if (!mb) return fail(RLSE_ERR_INVALID_VALUE, "mb_create: out of memory");
  mb->budget = budget_bytes;
  mb->headroom = headroom_bytes;
  mb->reserved = headroom_bytes;
  mb->available = budget_bytes - headroom_bytes;
  mb->peak = headroom_bytes;
  *out = mb;
  return RLSE_OK;
}

extern "C" int rlse_mb_destroy(rlse_memory_budget* mb) {
  if (!mb) return fail(RLSE_ERR_INVALID_VALUE, "mb_destroy: null");
  delete mb;
  return RLSE_OK;
}

extern "C" int rlse_mb_stats(rlse_memory_budget* mb, rlse_memory_stats* out) {
  if (!mb || !out) return fail(RLSE_ERR_INVALID_VALUE, "mb_stats: bad arguments");
  std::lock_guard<std::mutex> g(mb->mu);
  out->budget_bytes = mb->budget;
  out->headroom_bytes = mb->headroom;
  out->active_kv_reserved_bytes = mb->active_kv;
  out->execution_reserved_bytes = mb->execution;
  out->prefix_retained_bytes = mb->prefix;
  out->reserved_bytes = mb->reserved;
  out->available_bytes = mb->available;
  out->peak_reserved_bytes = mb->peak;
  out->rejections = mb->rejections;
  return RLSE_OK;
}

extern "C" int rlse_mb_try_reserve(rlse_memory_budget* mb, long long active_kv_bytes,
                                   long long execution_bytes, long long prefix_bytes,
                                   long long* lease) {
  if (!mb || !lease || active_kv_bytes < 0 || execution_bytes < 0 || prefix_bytes < 0)
    return fail(RLSE_ERR_INVALID_VALUE, "mb_try_reserve: bad arguments");
  *lease = 0;
  std::lock_guard<std::mutex> g(mb->mu);
  if (!mb->try_charge(active_kv_bytes, execution_bytes, prefix_bytes))
    return fail(RLSE_ERR_CACHE_PRESSURE, "Tensor memory budget exhausted");
  const long long id = mb->next_lease++;
  mb->leases[id] = {active_kv_bytes, execution_bytes, prefix_bytes};
  *lease = id;
  return RLSE_OK;
}

extern "C" int rlse_mb_release(rlse_memory_budget* mb, long long lease) {
  if (!mb) return fail(RLSE_ERR_INVALID_VALUE, "mb_release: null");
  std::lock_guard<std::mutex> g(mb->mu);
  auto it = mb->leases.find(lease);
  if (it == mb->leases.end())
    return fail(RLSE_ERR_INVALID_VALUE, "mb_release: unknown lease %lld", lease);
  mb->uncharge(it->second.active_kv, it->second.execution, it->second.prefix);
  mb->leases.erase(it);
  return RLSE_OK;
}

extern "C" int rlse_mb_record_rejection(rlse_memory_budget* mb) {
  if (!mb) return fail(RLSE_ERR_INVALID_VALUE, "mb_record_rejection: null");
  std::lock_guard<std::mutex> g(mb->mu);
  ++mb->rejections;
  return RLSE_OK;
}

extern "C" int rlse_bm_attach_budget(rlse_block_manager* bm, rlse_memory_budget* mb,
                                     long long page_bytes) {
  if (!bm || (mb && page_bytes <= 0))
    return fail(RLSE_ERR_INVALID_VALUE, "bm_attach_budget: bad arguments");
  // Charges of the pages held now, by class.
  long long active = 0, prefix = 0;
  for (int b = 0; b < bm->total_blocks; ++b) {
    const auto c = bm->cls(b);
    active += c == rlse_block_manager::kActive;
    prefix += c == rlse_block_manager::kPrefix;
  }
  if (mb) {
    long long kv = 0, pf = 0;
    if (__builtin_mul_overflow(active, page_bytes, &kv) ||
        __builtin_mul_overflow(prefix, page_bytes, &pf))
      return fail(RLSE_ERR_CACHE_PRESSURE, "bm_attach_budget: page charges overflow");
    std::lock_guard<std::mutex> g(mb->mu);
    if (!mb->try_charge(kv, 0, pf))
      return fail(RLSE_ERR_CACHE_PRESSURE,
                  "Tensor memory budget exhausted: the %lld held pages do not fit",
                  active + prefix);
  }
  if (bm->budget) {
    std::lock_guard<std::mutex> g(bm->budget->mu);
    bm->budget->uncharge(active * bm->page_bytes, 0, prefix * bm->page_bytes);
  }
  bm->budget = mb;
  bm->page_bytes = mb ? page_bytes : 0;
  return RLSE_OK;
}

namespace {
// Checked product and sum of non-negative terms (false on overflow).
bool product(std::initializer_list<long long> v, long long* out) {
  long long acc = 1;
  for (long long x : v)
    if (x < 0 || __builtin_mul_overflow(acc, x, &acc)) return false;
  *out = acc;
  return true;
}
}  // namespace

extern "C" int rlse_memory_charge(const rlse_model_shape* s, long long prompt_tokens,
                                  long long max_tokens, long long* kv_bytes,
                                  long long* execution_bytes, long long* page_bytes) {
  if (!s || s->num_layers <= 0 || s->num_heads <= 0 || s->num_kv_heads <= 0 ||
      s->head_dim <= 0 || s->hidden_size <= 0 || s->intermediate_size <= 0 ||
      s->vocab_size <= 0 || s->dtype_bytes <= 0 || s->context_length <= 0 || s->block_size <= 0)
    return fail(RLSE_ERR_INVALID_VALUE, "memory_charge: bad model shape");
  long long total = 0;
  if (prompt_tokens < 0 || max_tokens < 0 ||
      __builtin_add_overflow(prompt_tokens, max_tokens, &total))
    return fail(RLSE_ERR_CACHE_PRESSURE, "Tensor memory estimate overflows usize");
  if (prompt_tokens == 0 || max_tokens == 0 || total > s->context_length)
    return fail(RLSE_ERR_TOKEN_LIMIT, "Request exceeds model context or has zero tokens");
  const long long B = s->dtype_bytes, B4 = B > 4 ? B : 4;
  const long long pages = (total + s->block_size - 1) / s->block_size;
  long long page = 0, kv = 0, attention = 0, hidden = 0, mlp = 0, decode = 0, logits = 0;
  bool ok = product({2, s->num_layers, s->num_kv_heads, s->head_dim, s->block_size, B}, &page) &&
            product({pages, page}, &kv) &&
            product({8, s->num_heads, prompt_tokens, total, B4}, &attention) &&
            product({16, s->hidden_size, prompt_tokens, B}, &hidden) &&
            product({8, s->intermediate_size, prompt_tokens, B}, &mlp) &&
            product({8, s->num_heads, total, s->head_dim, B}, &decode) &&
            product({16, s->vocab_size, B4}, &logits);
  long long ex = 0;
  for (long long term : {attention, hidden, mlp, decode, logits})
    ok = ok && !__builtin_add_overflow(ex, term, &ex);
  if (!ok) return fail(RLSE_ERR_CACHE_PRESSURE, "Tensor memory estimate overflows usize");
  if (kv_bytes) *kv_bytes = kv;
  if (execution_bytes) *execution_bytes = ex;
  if (page_bytes) *page_bytes = page;
  return RLSE_OK;
}
