// C ABI over the host-side page state (declarations and reference citations
// in include/inferno_host.h).  Every entry point catches the state's
// contract errors and reports them through ifr_last_error().
#include <limits.h>
#include <string.h>

#include <new>

#include "../../include/inferno_hip.h"
#include "../../include/inferno_host.h"
#include "host_state.hpp"

namespace ifr {
int32_t abi_fail(int32_t code, const char* msg);  // api.hip
int32_t abi_ok();
}  // namespace ifr

using ifr::host::ContractError;
using ifr::host::PageAccountant;
using ifr::host::PoolSpec;
using ifr::host::Scheduler;
using ifr::host::SlotRegistry;

namespace {

// The opaque handle types of the header stay incomplete; a handle is the
// address of the C++ object.
PageAccountant* acc(ifr_pages* p) { return reinterpret_cast<PageAccountant*>(p); }
const PageAccountant* acc(const ifr_pages* p) {
  return reinterpret_cast<const PageAccountant*>(p);
}
SlotRegistry* reg(ifr_registry* r) { return reinterpret_cast<SlotRegistry*>(r); }
const SlotRegistry* reg(const ifr_registry* r) { return reinterpret_cast<const SlotRegistry*>(r); }
Scheduler* sch(ifr_scheduler* s) { return reinterpret_cast<Scheduler*>(s); }
const Scheduler* sch(const ifr_scheduler* s) { return reinterpret_cast<const Scheduler*>(s); }
ifr_pages* handle(PageAccountant* p) { return reinterpret_cast<ifr_pages*>(p); }
ifr_registry* handle(SlotRegistry* r) { return reinterpret_cast<ifr_registry*>(r); }
ifr_scheduler* handle(Scheduler* s) { return reinterpret_cast<ifr_scheduler*>(s); }

std::vector<PoolSpec> read_specs(const int64_t* specs, int64_t num_pools) {
  ifr::host::require(num_pools >= 0 && (num_pools == 0 || specs != nullptr),
                     "pool_specs must hold num_pools x 3 values");
  std::vector<PoolSpec> out;
  for (int64_t p = 0; p < num_pools; ++p)
    out.push_back(PoolSpec{specs[3 * p], specs[3 * p + 1], specs[3 * p + 2]});
  return out;
}

void need_ptr(const void* p, const char* what) {
  if (!p) throw ContractError(std::string(what) + " is null");
}

// Runs `body` and maps exceptions to status codes.
template <class F>
int32_t guarded(F&& body) {
  try {
    body();
    return ifr::abi_ok();
  } catch (const ContractError& e) {
    return ifr::abi_fail(IFR_EINVAL, e.what());
  } catch (const std::out_of_range& e) {
    return ifr::abi_fail(IFR_EINVAL, "index out of range");
  } catch (const std::bad_alloc&) {
    return ifr::abi_fail(IFR_ESPACE, "host allocation failed");
  } catch (const std::exception& e) {
    return ifr::abi_fail(IFR_EINVAL, e.what());
  }
}

template <class F>
int64_t guarded_query(F&& body) {
  int64_t out = IFR_QUERY_ERROR;
  int32_t st = guarded([&] { out = body(); });
  return st == IFR_OK ? out : IFR_QUERY_ERROR;
}

}  // namespace

extern "C" {

// ---- prefix hash ----------------------------------------------------------

uint64_t ifr_splitmix64(uint64_t x) { return ifr::host::splitmix64(x); }

uint64_t ifr_hash_token_block(const int32_t* tokens, int64_t start, int64_t count) {
  if (!tokens || start < 0 || count < 0) return 0;
  return ifr::host::hash_token_block(tokens + start, count);
}

uint64_t ifr_chain_link(uint64_t prev, uint64_t block_hash) {
  return ifr::host::chain_link(prev, block_hash);
}

int64_t ifr_refresh_chain(uint64_t* chain, int64_t chain_len, int64_t chain_cap,
                          const int32_t* tokens, int64_t num_tokens, int64_t ppp) {
  if (ppp <= 0 || num_tokens < 0 || chain_len < 0 || chain_len > chain_cap ||
      (num_tokens > 0 && !tokens) || (chain_cap > 0 && !chain))
    return ifr::abi_fail(IFR_EINVAL, "refresh_chain: bad arguments");
  const int64_t sealed = num_tokens / ppp;
  if (sealed > chain_cap) return ifr::abi_fail(IFR_ESPACE, "refresh_chain: chain_cap too small");
  std::vector<uint64_t> v(chain, chain + chain_len);
  ifr::host::refresh_chain(v, tokens, num_tokens, ppp);
  if (!v.empty()) memcpy(chain, v.data(), v.size() * sizeof(uint64_t));
  ifr::abi_ok();
  return static_cast<int64_t>(v.size());
}

int64_t ifr_hashed_prefix_len(int64_t ppp, const int32_t* a, int64_t na, const uint64_t* ac,
                              int64_t nac, const int32_t* b, int64_t nb, const uint64_t* bc,
                              int64_t nbc) {
  if (ppp <= 0 || na < 0 || nb < 0 || nac < 0 || nbc < 0 || (na && !a) || (nb && !b) ||
      (nac && !ac) || (nbc && !bc) || nac > na / ppp || nbc > nb / ppp) {
    ifr::abi_fail(IFR_EINVAL, "hashed_prefix_len: bad arguments (chains longer than sealed pages?)");
    return IFR_QUERY_ERROR;
  }
  ifr::abi_ok();
  return ifr::host::hashed_prefix_len(ppp, a, na, ac, nac, b, nb, bc, nbc);
}

// ---- page accountant ------------------------------------------------------

int32_t ifr_pages_create(int64_t max_seqs, const int64_t* pool_specs, int64_t num_pools,
                         ifr_pages** out) {
  return guarded([&] {
    need_ptr(out, "out");
    *out = nullptr;
    auto* p = new PageAccountant(max_seqs, read_specs(pool_specs, num_pools));
    *out = handle(p);
  });
}

void ifr_pages_destroy(ifr_pages* pages) { delete acc(pages); }

int32_t ifr_pages_admit(ifr_pages* pages, int64_t* seq_id) {
  return guarded([&] {
    need_ptr(pages, "pages");
    need_ptr(seq_id, "seq_id");
    *seq_id = acc(pages)->admit();
  });
}

int32_t ifr_pages_release(ifr_pages* pages, int64_t seq_id) {
  return guarded([&] {
    need_ptr(pages, "pages");
    acc(pages)->release(seq_id);
  });
}

int32_t ifr_pages_share(ifr_pages* pages, int64_t pool, int64_t src_seq, int64_t dst_seq,
                        int64_t ordinal) {
  return guarded([&] {
    need_ptr(pages, "pages");
    acc(pages)->share(pool, src_seq, dst_seq, ordinal);
  });
}

int32_t ifr_pages_truncate(ifr_pages* pages, int64_t seq_id, int64_t last_keep_ordinal) {
  return guarded([&] {
    need_ptr(pages, "pages");
    ifr::host::require(seq_id >= 0 && seq_id < acc(pages)->max_seqs(),
                       "truncate: sequence out of range");
    acc(pages)->truncate(seq_id, last_keep_ordinal);
  });
}

int32_t ifr_pages_replace_with_private(ifr_pages* pages, int64_t pool, int64_t seq_id,
                                       int64_t ordinal, int64_t* fresh) {
  return guarded([&] {
    need_ptr(pages, "pages");
    need_ptr(fresh, "fresh");
    *fresh = acc(pages)->replace_with_private(pool, seq_id, ordinal);
  });
}

int32_t ifr_pages_pages_needed(const ifr_pages* pages, int64_t seq_id, int64_t last_ordinal,
                               int64_t* need) {
  return guarded([&] {
    need_ptr(pages, "pages");
    need_ptr(need, "need");
    const PageAccountant* a = acc(pages);
    std::vector<int64_t> v(need, need + a->pool_count());
    a->pages_needed(seq_id, last_ordinal, v);
    memcpy(need, v.data(), v.size() * sizeof(int64_t));
  });
}

int32_t ifr_pages_fits(const ifr_pages* pages, const int64_t* need, int64_t* result) {
  return guarded([&] {
    need_ptr(pages, "pages");
    need_ptr(need, "need");
    need_ptr(result, "result");
    const PageAccountant* a = acc(pages);
    *result = a->fits(std::vector<int64_t>(need, need + a->pool_count())) ? 1 : 0;
  });
}

int32_t ifr_pages_reserve(ifr_pages* pages, int64_t seq_id, int64_t last_ordinal,
                          int64_t* result) {
  return guarded([&] {
    need_ptr(pages, "pages");
    need_ptr(result, "result");
    *result = acc(pages)->reserve(seq_id, last_ordinal) ? 1 : 0;
  });
}

int32_t ifr_pages_retain_page(ifr_pages* pages, int64_t pool, int64_t page) {
  return guarded([&] {
    need_ptr(pages, "pages");
    acc(pages)->retain_page(pool, page);
  });
}

int32_t ifr_pages_release_page(ifr_pages* pages, int64_t pool, int64_t page) {
  return guarded([&] {
    need_ptr(pages, "pages");
    acc(pages)->release_page(pool, page);
  });
}

int64_t ifr_pages_query(const ifr_pages* pages, int64_t what, int64_t a, int64_t b, int64_t c) {
  return guarded_query([&]() -> int64_t {
    need_ptr(pages, "pages");
    const PageAccountant* pa = acc(pages);
    switch (what) {
      case IFR_PQ_POOL_COUNT: return pa->pool_count();
      case IFR_PQ_MAX_SEQS: return pa->max_seqs();
      case IFR_PQ_AVAILABLE: return pa->pool_available(a);
      case IFR_PQ_FIXED_PAGES: return pa->pool_fixed_pages(a);
      case IFR_PQ_POOL_PAGES: return pa->pool(a).spec.num_pages;
      case IFR_PQ_SEQ_LIMIT: return pa->pool(a).spec.max_pages_per_seq;
      case IFR_PQ_PAGE_INDEX: return pa->page_index(a, b, c);
      case IFR_PQ_PAGE_HOLDS:
        ifr::host::require(b >= 0 && b < pa->pool(a).spec.num_pages, "page out of range");
        return pa->page_holds(a, b);
      case IFR_PQ_FREEABLE:
        ifr::host::require(b >= 0 && b < pa->max_seqs(), "sequence out of range");
        return pa->freeable_pages(a, b);
      case IFR_PQ_ACTIVE:
        ifr::host::require(a >= 0 && a < pa->max_seqs(), "sequence out of range");
        return pa->active(a) ? 1 : 0;
      default: throw ContractError("unknown page query");
    }
  });
}

int32_t ifr_pages_export(const ifr_pages* pages, int64_t pool, int32_t* table, int32_t* holds,
                         int32_t* free_stack, int64_t* free_len) {
  return guarded([&] {
    need_ptr(pages, "pages");
    const auto& pl = acc(pages)->pool(pool);
    if (table) memcpy(table, pl.table.data(), pl.table.size() * sizeof(int32_t));
    const auto& h = pl.pages.hold_counts();
    if (holds) memcpy(holds, h.data(), h.size() * sizeof(int32_t));
    const auto& f = pl.pages.free_stack();
    if (free_stack && !f.empty()) memcpy(free_stack, f.data(), f.size() * sizeof(int32_t));
    if (free_len) *free_len = static_cast<int64_t>(f.size());
  });
}

// ---- slot registry ----------------------------------------------------------

int32_t ifr_registry_create(int64_t ppp, int64_t max_seqs, ifr_registry** out) {
  return guarded([&] {
    need_ptr(out, "out");
    *out = nullptr;
    *out = handle(new SlotRegistry(ppp, max_seqs));
  });
}

void ifr_registry_destroy(ifr_registry* r) { delete reg(r); }

int32_t ifr_registry_open(ifr_registry* r, int64_t seq_id, int64_t owner, uint64_t now) {
  return guarded([&] {
    need_ptr(r, "registry");
    reg(r)->open(seq_id, owner, now);
  });
}

int32_t ifr_registry_adopt(ifr_registry* r, int64_t seq_id, int64_t owner, uint64_t now) {
  return guarded([&] {
    need_ptr(r, "registry");
    reg(r)->adopt(seq_id, owner, now);
  });
}

int32_t ifr_registry_extend(ifr_registry* r, int64_t seq_id, const int32_t* source,
                            int64_t source_len, int64_t start, int64_t base_pos, int64_t count,
                            uint64_t now) {
  return guarded([&] {
    need_ptr(r, "registry");
    if (count > 0) need_ptr(source, "source");
    reg(r)->extend(seq_id, source, source_len, start, base_pos, count, now);
  });
}

int32_t ifr_registry_seed(ifr_registry* r, int64_t seq_id, const int32_t* source,
                          int64_t source_len, int64_t count, uint64_t now) {
  return guarded([&] {
    need_ptr(r, "registry");
    if (source_len > 0) need_ptr(source, "source");
    reg(r)->seed(seq_id, source, source_len, count, now);
  });
}

int32_t ifr_registry_set_warm(ifr_registry* r, int64_t seq_id) {
  return guarded([&] {
    need_ptr(r, "registry");
    reg(r)->set_warm(seq_id);
  });
}

int32_t ifr_registry_close(ifr_registry* r, int64_t seq_id) {
  return guarded([&] {
    need_ptr(r, "registry");
    reg(r)->close(seq_id);
  });
}

int64_t ifr_registry_prefix_len(const ifr_registry* r, int64_t seq_id, const int32_t* tokens,
                                int64_t num_tokens, const uint64_t* chain, int64_t chain_len) {
  return guarded_query([&]() -> int64_t {
    need_ptr(r, "registry");
    ifr::host::require(num_tokens >= 0 && chain_len >= 0 &&
                           chain_len <= num_tokens / reg(r)->ppp(),
                       "prefix_len: chain longer than the sealed pages of tokens");
    if (num_tokens > 0) need_ptr(tokens, "tokens");
    if (chain_len > 0) need_ptr(chain, "chain");
    return reg(r)->prefix_len(seq_id, tokens, num_tokens, chain, chain_len);
  });
}

int64_t ifr_registry_exact_prefix_len(const ifr_registry* r, int64_t seq_id,
                                      const int32_t* tokens, int64_t num_tokens) {
  return guarded_query([&]() -> int64_t {
    need_ptr(r, "registry");
    ifr::host::require(num_tokens >= 0, "num_tokens must be >= 0");
    if (num_tokens > 0) need_ptr(tokens, "tokens");
    return reg(r)->exact_prefix_len(seq_id, tokens, num_tokens);
  });
}

int64_t ifr_registry_lru_victim(const ifr_registry* r) {
  return guarded_query([&]() -> int64_t {
    need_ptr(r, "registry");
    return reg(r)->lru_victim();
  });
}

int64_t ifr_registry_query(const ifr_registry* r, int64_t what, int64_t s) {
  return guarded_query([&]() -> int64_t {
    need_ptr(r, "registry");
    const SlotRegistry* g = reg(r);
    switch (what) {
      case IFR_RQ_LENGTH: return g->length(s);
      case IFR_RQ_OWNER: return g->owner_of(s);
      case IFR_RQ_RESIDENT: return g->is_resident(s) ? 1 : 0;
      case IFR_RQ_LAST_USED: return static_cast<int64_t>(g->last_used(s));
      case IFR_RQ_CHAIN_LEN: return static_cast<int64_t>(g->chain(s).size());
      case IFR_RQ_MAX_SEQS: return g->max_seqs();
      case IFR_RQ_PPP: return g->ppp();
      default: throw ContractError("unknown registry query");
    }
  });
}

int32_t ifr_registry_export(const ifr_registry* r, int64_t s, int32_t* tokens,
                            int64_t tokens_cap, uint64_t* chain, int64_t chain_cap) {
  if (!r) return ifr::abi_fail(IFR_EINVAL, "registry is null");
  const SlotRegistry* g = reg(r);
  if (s < 0 || s >= g->max_seqs()) return ifr::abi_fail(IFR_EINVAL, "sequence out of range");
  const auto& t = g->tokens(s);
  const auto& c = g->chain(s);
  if (tokens) {
    if (static_cast<int64_t>(t.size()) > tokens_cap)
      return ifr::abi_fail(IFR_ESPACE, "tokens_cap too small");
    if (!t.empty()) memcpy(tokens, t.data(), t.size() * sizeof(int32_t));
  }
  if (chain) {
    if (static_cast<int64_t>(c.size()) > chain_cap)
      return ifr::abi_fail(IFR_ESPACE, "chain_cap too small");
    if (!c.empty()) memcpy(chain, c.data(), c.size() * sizeof(uint64_t));
  }
  return ifr::abi_ok();
}

// ---- scheduler ----------------------------------------------------------------

int32_t ifr_scheduler_create(int64_t ppp, int64_t max_seqs, int64_t max_slots,
                             int64_t max_step_tokens, const int64_t* pool_specs,
                             int64_t num_pools, int64_t step_budget, const int32_t* stop_tokens,
                             int64_t num_stop_tokens, int64_t decode_band, ifr_scheduler** out) {
  return guarded([&] {
    need_ptr(out, "out");
    *out = nullptr;
    ifr::host::require(num_stop_tokens >= 0 && (num_stop_tokens == 0 || stop_tokens),
                       "stop_tokens must hold num_stop_tokens values");
    std::vector<int32_t> stops(stop_tokens, stop_tokens + num_stop_tokens);
    auto* s = new Scheduler(ppp, max_seqs, max_slots, max_step_tokens,
                            read_specs(pool_specs, num_pools), step_budget, std::move(stops),
                            decode_band);
    *out = handle(s);
  });
}

void ifr_scheduler_destroy(ifr_scheduler* s) { delete sch(s); }

ifr_pages* ifr_scheduler_pages(ifr_scheduler* s) {
  return s ? handle(&sch(s)->pages()) : nullptr;
}

ifr_registry* ifr_scheduler_registry(ifr_scheduler* s) {
  return s ? handle(&sch(s)->registry()) : nullptr;
}

int32_t ifr_scheduler_submit(ifr_scheduler* s, const int32_t* tokens, int64_t num_tokens,
                             int64_t max_new_tokens, int64_t no_share, int64_t* request_id) {
  return guarded([&] {
    need_ptr(s, "scheduler");
    need_ptr(request_id, "request_id");
    if (num_tokens > 0) need_ptr(tokens, "tokens");
    *request_id = sch(s)->submit(tokens, num_tokens, max_new_tokens, no_share != 0);
  });
}

int32_t ifr_scheduler_cancel(ifr_scheduler* s, int64_t rid) {
  return guarded([&] {
    need_ptr(s, "scheduler");
    sch(s)->cancel(rid);
  });
}

int32_t ifr_scheduler_retire(ifr_scheduler* s, int64_t rid, int64_t* result) {
  return guarded([&] {
    need_ptr(s, "scheduler");
    need_ptr(result, "result");
    *result = sch(s)->retire(rid) ? 1 : 0;
  });
}

int32_t ifr_scheduler_evict_warm(ifr_scheduler* s, int64_t* result) {
  return guarded([&] {
    need_ptr(s, "scheduler");
    need_ptr(result, "result");
    *result = sch(s)->evict_warm() ? 1 : 0;
  });
}

int32_t ifr_scheduler_build_schedule(ifr_scheduler* s, uint64_t now, int64_t* built) {
  return guarded([&] {
    need_ptr(s, "scheduler");
    need_ptr(built, "built");
    *built = sch(s)->build_schedule(now) ? 1 : 0;
  });
}

int32_t ifr_scheduler_absorb(ifr_scheduler* s, const int32_t* emitted, int64_t num_emitted,
                             uint64_t now) {
  return guarded([&] {
    need_ptr(s, "scheduler");
    if (num_emitted > 0) need_ptr(emitted, "emitted");
    sch(s)->absorb(emitted, num_emitted, now);
  });
}

int32_t ifr_scheduler_discard_step(ifr_scheduler* s) {
  return guarded([&] {
    need_ptr(s, "scheduler");
    sch(s)->discard_step();
  });
}

int64_t ifr_scheduler_query(const ifr_scheduler* s, int64_t what, int64_t arg) {
  return guarded_query([&]() -> int64_t {
    need_ptr(s, "scheduler");
    const Scheduler* c = sch(s);
    const auto& sc = c->schedule();
    switch (what) {
      case IFR_SQ_PENDING_WORK: return c->pending_work() ? 1 : 0;
      case IFR_SQ_FULLY_CANCELLED: return c->fully_cancelled() ? 1 : 0;
      case IFR_SQ_NUM_SLOTS: return static_cast<int64_t>(sc.slots.size());
      case IFR_SQ_NUM_TOKENS: return static_cast<int64_t>(sc.tokens.size());
      case IFR_SQ_NUM_COPIES: return static_cast<int64_t>(sc.copies.size());
      case IFR_SQ_PREFILL_TOKENS: return sc.prefill_tokens;
      case IFR_SQ_DECODE_TOKENS: return sc.decode_tokens;
      case IFR_SQ_NUM_REQUESTS: return c->request_count();
      case IFR_SQ_NUM_PENDING: return static_cast<int64_t>(c->pending().size());
      case IFR_SQ_RING_CAPACITY: return c->ring_capacity();
      case IFR_SQ_SEQ_CEILING: return c->seq_ceiling();
      case IFR_SQ_RING_FLOOR: return c->ring_floor(arg);
      case IFR_SQ_REQ_SEQ_ID: return c->request(arg).seq_id;
      case IFR_SQ_REQ_DONE: return c->request(arg).done ? 1 : 0;
      case IFR_SQ_REQ_LIVE: return c->request(arg).live ? 1 : 0;
      case IFR_SQ_REQ_CANCELLED: return c->request(arg).cancelled ? 1 : 0;
      case IFR_SQ_REQ_NUM_TOKENS: return static_cast<int64_t>(c->request(arg).tokens.size());
      case IFR_SQ_REQ_NUM_GENERATED:
        return static_cast<int64_t>(c->request(arg).generated.size());
      case IFR_SQ_PPP: return c->ppp();
      case IFR_SQ_SHARED_WRITES: return c->shared_write_violations();
      case IFR_SQ_UNSHARABLE_SHARED: return c->unsharable_violations();
      default: throw ContractError("unknown scheduler query");
    }
  });
}

int32_t ifr_scheduler_export_schedule(const ifr_scheduler* s, int64_t* slots, int64_t slots_cap,
                                      int32_t* tokens, int64_t tokens_cap, int64_t* copies,
                                      int64_t copies_cap) {
  if (!s) return ifr::abi_fail(IFR_EINVAL, "scheduler is null");
  const auto& sc = sch(s)->schedule();
  // Every capacity is checked before anything is written.
  if (slots && static_cast<int64_t>(sc.slots.size()) > slots_cap)
    return ifr::abi_fail(IFR_ESPACE, "slots_cap too small");
  if (tokens && static_cast<int64_t>(sc.tokens.size()) > tokens_cap)
    return ifr::abi_fail(IFR_ESPACE, "tokens_cap too small");
  if (copies && static_cast<int64_t>(sc.copies.size()) > copies_cap)
    return ifr::abi_fail(IFR_ESPACE, "copies_cap too small");
  if (slots) {
    for (size_t k = 0; k < sc.slots.size(); ++k) {
      const auto& sl = sc.slots[k];
      int64_t* o = slots + 6 * k;
      o[0] = sl.seq_id;
      o[1] = sl.request_id;
      o[2] = sl.base_pos;
      o[3] = sl.n_tokens;
      o[4] = sl.prompt_len;
      o[5] = sl.emit ? 1 : 0;
    }
  }
  if (tokens && !sc.tokens.empty())
    memcpy(tokens, sc.tokens.data(), sc.tokens.size() * sizeof(int32_t));
  if (copies) {
    for (size_t k = 0; k < sc.copies.size(); ++k) {
      const auto& c = sc.copies[k];
      int64_t* o = copies + 5 * k;
      o[0] = c.pool;
      o[1] = c.src_page;
      o[2] = c.dst_page;
      o[3] = c.pos_start;
      o[4] = c.pos_count;
    }
  }
  return ifr::abi_ok();
}

int32_t ifr_scheduler_export_request(const ifr_scheduler* s, int64_t rid, int32_t* tokens,
                                     int64_t tokens_cap, int32_t* generated,
                                     int64_t generated_cap) {
  if (!s) return ifr::abi_fail(IFR_EINVAL, "scheduler is null");
  const Scheduler* c = sch(s);
  if (rid < 0 || rid >= c->request_count())
    return ifr::abi_fail(IFR_EINVAL, "request id out of range");
  const auto& r = c->request(rid);
  if (tokens) {
    if (static_cast<int64_t>(r.tokens.size()) > tokens_cap)
      return ifr::abi_fail(IFR_ESPACE, "tokens_cap too small");
    if (!r.tokens.empty()) memcpy(tokens, r.tokens.data(), r.tokens.size() * sizeof(int32_t));
  }
  if (generated) {
    if (static_cast<int64_t>(r.generated.size()) > generated_cap)
      return ifr::abi_fail(IFR_ESPACE, "generated_cap too small");
    if (!r.generated.empty())
      memcpy(generated, r.generated.data(), r.generated.size() * sizeof(int32_t));
  }
  return ifr::abi_ok();
}

int32_t ifr_scheduler_export_pending(const ifr_scheduler* s, int64_t* out, int64_t cap,
                                     int64_t* count) {
  if (!s) return ifr::abi_fail(IFR_EINVAL, "scheduler is null");
  const auto& p = sch(s)->pending();
  if (count) *count = static_cast<int64_t>(p.size());
  if (out) {
    if (static_cast<int64_t>(p.size()) > cap)
      return ifr::abi_fail(IFR_ESPACE, "cap too small");
    if (!p.empty()) memcpy(out, p.data(), p.size() * sizeof(int64_t));
  }
  return ifr::abi_ok();
}

// ---- kv_policy ------------------------------------------------------------------

int32_t ifr_bind_pool_run_table(const ifr_scheduler* s, int64_t pool, int64_t page_len,
                                int64_t pos_shard, int32_t* runs, int64_t runs_cap,
                                int32_t* base_rows, int64_t rows_cap, int64_t* num_runs,
                                int64_t* num_rows) {
  if (!s || !runs || !base_rows || !num_runs || !num_rows)
    return ifr::abi_fail(IFR_EINVAL, "bind_pool_run_table: null argument");
  if (page_len <= 0 || pos_shard <= 0 || page_len % pos_shard != 0)
    return ifr::abi_fail(IFR_EINVAL, "bind_pool_run_table: page_len must be a positive "
                                     "multiple of pos_shard");
  const Scheduler* c = sch(s);
  const PageAccountant& pa = c->pages();
  if (pool < 0 || pool >= pa.pool_count())
    return ifr::abi_fail(IFR_EINVAL, "bind_pool_run_table: pool out of range");
  const auto& pl = pa.pool(pool);
  const int64_t rpp = page_len / pos_shard;
  const auto& slots = c->schedule().slots;
  if (static_cast<int64_t>(slots.size()) > runs_cap)
    return ifr::abi_fail(IFR_ESPACE, "bind_pool_run_table: runs_cap too small");
  int64_t buf_start = 0, nr = 0;
  for (size_t i = 0; i < slots.size(); ++i) {
    const auto& sl = slots[i];
    const int64_t ordinals = pl.ring() ? pl.spec.fixed_pages_per_seq
                                       : (sl.base_pos + sl.n_tokens - 1) / page_len + 1;
    if (ordinals > pl.spec.max_pages_per_seq)
      return ifr::abi_fail(IFR_EINVAL, "bind_pool_run_table: slot reaches past the per-sequence "
                                       "page bound (page_len differs from the scheduler's?)");
    if (nr + ordinals > rows_cap)
      return ifr::abi_fail(IFR_ESPACE, "bind_pool_run_table: rows_cap too small");
    int32_t* run = runs + 4 * i;
    run[0] = static_cast<int32_t>(buf_start);
    run[1] = static_cast<int32_t>(sl.base_pos);
    run[2] = static_cast<int32_t>(nr);
    run[3] = static_cast<int32_t>(ordinals);
    for (int64_t o = 0; o < ordinals; ++o) {
      const int64_t page = pl.page_index(sl.seq_id, o);
      if (page < 0) return ifr::abi_fail(IFR_EINVAL, "run references unmapped page");
      base_rows[nr++] = static_cast<int32_t>(page * rpp);
    }
    buf_start += sl.n_tokens;
  }
  *num_runs = static_cast<int64_t>(slots.size());
  *num_rows = nr;
  return ifr::abi_ok();
}

int32_t ifr_prefix_copy_jobs(const int64_t* copies, int64_t num_copies, const int64_t* mirrors,
                             const int64_t* components, int64_t num_pools, int64_t* jobs,
                             int64_t jobs_cap, int64_t* num_jobs) {
  if ((num_copies > 0 && !copies) || !mirrors || !components || !num_jobs || num_pools <= 0 ||
      num_copies < 0)
    return ifr::abi_fail(IFR_EINVAL, "prefix_copy_jobs: null or empty argument");
  // Offsets of each pool's components in the flat component list.
  std::vector<int64_t> comp_off(num_pools + 1, 0);
  for (int64_t p = 0; p < num_pools; ++p) {
    const int64_t* m = mirrors + 6 * p;
    if (m[0] <= 0 || m[1] <= 0 || m[0] % m[1] != 0 || m[4] < 0 || m[5] < 0)
      return ifr::abi_fail(IFR_EINVAL, "prefix_copy_jobs: bad mirror");
    comp_off[p + 1] = comp_off[p] + m[5];
  }
  int64_t n = 0;
  for (int64_t k = 0; k < num_copies; ++k) {
    const int64_t* cp = copies + 5 * k;
    const int64_t pool = cp[0];
    if (pool < 0 || pool >= num_pools)
      return ifr::abi_fail(IFR_EINVAL, "prefix_copy_jobs: copy names an unknown pool");
    const int64_t* m = mirrors + 6 * pool;
    const int64_t page_len = m[0], pos_shard = m[1], region_off = m[2], stride = m[3];
    const int64_t layers = m[4];
    const int64_t rpp = page_len / pos_shard;
    const int64_t row_start = cp[3] / pos_shard;
    const int64_t row_end = (cp[3] + cp[4] + pos_shard - 1) / pos_shard;
    const int64_t rows = row_end - row_start;
    for (int64_t l = 0; l < layers; ++l) {
      const int64_t base = region_off + l * stride;
      for (int64_t c = comp_off[pool]; c < comp_off[pool + 1]; ++c) {
        const int64_t offset = components[2 * c], row_bytes = components[2 * c + 1];
        if (jobs) {
          if (n >= jobs_cap) return ifr::abi_fail(IFR_ESPACE, "prefix_copy_jobs: jobs_cap too small");
          int64_t* j = jobs + 3 * n;
          j[0] = base + offset + (cp[1] * rpp + row_start) * row_bytes;
          j[1] = base + offset + (cp[2] * rpp + row_start) * row_bytes;
          j[2] = rows * row_bytes;
        }
        ++n;
      }
    }
  }
  *num_jobs = n;
  return ifr::abi_ok();
}

}  // extern "C"
