// Host-side page state: implementation (declarations in host_state.hpp).
#include "host_state.hpp"

#include <algorithm>

namespace ifr {
namespace host {

namespace {
// Floor division for the non-negative position arithmetic of the scheduler
// (kept exact also should an operand ever be negative).
inline int64_t fdiv(int64_t a, int64_t b) {
  int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}
}  // namespace

// ---- PageAllocator (paging.mojo:16-58) -------------------------------------

PageAllocator::PageAllocator(int64_t num_pages) {
  require(num_pages >= 0 && num_pages < (int64_t{1} << 31), "page pool size out of range");
  free_.resize(num_pages);
  // Stack bottom holds the highest page, so acquire() returns 0, 1, 2, ...
  for (int64_t i = 0; i < num_pages; ++i) free_[i] = static_cast<int32_t>(num_pages - 1 - i);
  holds_.assign(num_pages, 0);
}

int64_t PageAllocator::acquire() {
  if (free_.empty()) return -1;
  int32_t page = free_.back();
  free_.pop_back();
  holds_[page] = 1;
  return page;
}

void PageAllocator::retain(int64_t page) {
  require(page >= 0 && page < size(), "page allocator: page out of range");
  require(holds_[page] > 0, "page allocator: retain of an unheld page");
  ++holds_[page];
}

void PageAllocator::release(int64_t page) {
  require(page >= 0 && page < size(), "page allocator: page out of range");
  require(holds_[page] > 0, "page allocator: release of an unheld page");
  if (--holds_[page] == 0) free_.push_back(static_cast<int32_t>(page));
}

// ---- PagePool / PageAccountant (paging.mojo:61-242) ------------------------

PagePool::PagePool(const PoolSpec& s, int64_t max_seqs) : spec(s), pages(s.num_pages) {
  require(s.fixed_pages_per_seq >= 0 && s.max_pages_per_seq > 0 &&
              s.fixed_pages_per_seq <= s.max_pages_per_seq,
          "pool spec: need 0 <= fixed_pages_per_seq <= max_pages_per_seq, max > 0");
  table.assign(max_seqs * s.max_pages_per_seq, -1);
}

int64_t PagePool::entry(int64_t seq, int64_t ordinal) const {
  require(ordinal >= 0 && ordinal < spec.max_pages_per_seq,
          "page table: ordinal beyond per-sequence bound");
  require(seq >= 0 && seq * spec.max_pages_per_seq < static_cast<int64_t>(table.size()),
          "page table: sequence out of range");
  return seq * spec.max_pages_per_seq + ordinal;
}

PageAccountant::PageAccountant(int64_t max_seqs, const std::vector<PoolSpec>& pools)
    : max_seqs_(max_seqs) {
  require(max_seqs > 0, "accountant: max_seqs must be positive");
  for (const auto& s : pools) pools_.emplace_back(s, max_seqs);
  active_.assign(max_seqs, 0);
}

const PagePool& PageAccountant::pool(int64_t p) const {
  require(p >= 0 && p < pool_count(), "accountant: pool out of range");
  return pools_[p];
}
PagePool& PageAccountant::pool(int64_t p) {
  require(p >= 0 && p < pool_count(), "accountant: pool out of range");
  return pools_[p];
}

int64_t PageAccountant::freeable_pages(int64_t p, int64_t seq) const {
  const PagePool& pl = pool(p);
  int64_t n = 0;
  for (int64_t o = 0; o < pl.spec.max_pages_per_seq; ++o) {
    int64_t page = pl.page_index(seq, o);
    if (page >= 0 && pl.pages.holds(page) == 1) ++n;
  }
  return n;
}

int64_t PageAccountant::admit() {
  for (int64_t s = 0; s < max_seqs_; ++s) {
    if (active_[s]) continue;
    // The first free sequence either gets every pool's ring pages or the
    // admission fails outright.
    for (const auto& pl : pools_)
      if (pl.spec.fixed_pages_per_seq > pl.pages.available()) return -1;
    for (auto& pl : pools_)
      for (int64_t o = 0; o < pl.spec.fixed_pages_per_seq; ++o) pl.map(s, o, pl.pages.acquire());
    active_[s] = 1;
    return s;
  }
  return -1;
}

void PageAccountant::release(int64_t seq) {
  require(seq >= 0 && seq < max_seqs_, "accountant: sequence out of range");
  if (!active_[seq]) return;
  for (auto& pl : pools_) {
    for (int64_t o = 0; o < pl.spec.max_pages_per_seq; ++o) {
      int64_t page = pl.page_index(seq, o);
      if (page >= 0) {
        pl.pages.release(page);
        pl.map(seq, o, -1);
      }
    }
  }
  active_[seq] = 0;
}

void PageAccountant::share(int64_t p, int64_t src_seq, int64_t dst_seq, int64_t ordinal) {
  PagePool& pl = pool(p);
  int64_t page = pl.page_index(src_seq, ordinal);
  require(page >= 0, "share: source ordinal is unmapped");
  require(pl.page_index(dst_seq, ordinal) < 0, "share: destination ordinal already mapped");
  pl.pages.retain(page);
  pl.map(dst_seq, ordinal, page);
}

void PageAccountant::truncate(int64_t seq, int64_t last_keep) {
  for (auto& pl : pools_) {
    if (pl.ring()) continue;
    for (int64_t o = std::max<int64_t>(last_keep + 1, 0); o < pl.spec.max_pages_per_seq; ++o) {
      int64_t page = pl.page_index(seq, o);
      if (page >= 0) {
        pl.pages.release(page);
        pl.map(seq, o, -1);
      }
    }
  }
}

int64_t PageAccountant::replace_with_private(int64_t p, int64_t seq, int64_t ordinal) {
  PagePool& pl = pool(p);
  int64_t fresh = pl.pages.acquire();
  if (fresh < 0) return -1;
  int64_t old = pl.page_index(seq, ordinal);
  require(old >= 0, "replace_with_private: ordinal is unmapped");
  pl.pages.release(old);
  pl.map(seq, ordinal, fresh);
  return fresh;
}

void PageAccountant::pages_needed(int64_t seq, int64_t last_ordinal,
                                  std::vector<int64_t>& need) const {
  require(static_cast<int64_t>(need.size()) >= pool_count(), "pages_needed: need too short");
  for (int64_t p = 0; p < pool_count(); ++p) {
    const PagePool& pl = pools_[p];
    if (pl.ring()) continue;
    for (int64_t o = 0; o <= last_ordinal; ++o)
      if (pl.page_index(seq, o) < 0) ++need[p];
  }
}

bool PageAccountant::fits(const std::vector<int64_t>& need) const {
  for (int64_t p = 0; p < pool_count(); ++p)
    if (need[p] > pools_[p].pages.available()) return false;
  return true;
}

bool PageAccountant::reserve(int64_t seq, int64_t last_ordinal) {
  for (auto& pl : pools_) {
    if (pl.ring()) continue;
    for (int64_t o = 0; o <= last_ordinal; ++o) {
      if (pl.page_index(seq, o) >= 0) continue;
      int64_t page = pl.pages.acquire();
      if (page < 0) return false;
      pl.map(seq, o, page);
    }
  }
  return true;
}

// ---- prefix hash (prefix_hash.mojo:22-97) -----------------------------------

uint64_t splitmix64(uint64_t x) {  // simd_math/sampling_rng.mojo:11-19
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

namespace {
inline uint32_t rotl32(uint32_t x, int b) { return (x << b) | (x >> (32 - b)); }
}  // namespace

uint64_t hash_token_block(const int32_t* tokens, int64_t count) {
  // Each of the 16 lanes absorbs every 16th token of the whole 16-token
  // groups with MurmurHash3's block step; the lanes, the count and the tail
  // tokens are then folded through SplitMix64.
  uint32_t lanes[kTokenLanes] = {0};
  int64_t i = 0;
  for (; i + kTokenLanes <= count; i += kTokenLanes) {
    for (int j = 0; j < kTokenLanes; ++j) {
      uint32_t m = static_cast<uint32_t>(tokens[i + j]) * 0xCC9E2D51u;
      m = rotl32(m, 15) * 0x1B873593u;
      uint32_t x = lanes[j] ^ m;
      lanes[j] = rotl32(x, 13) * 5u + 0xE6546B64u;
    }
  }
  uint64_t acc = splitmix64(static_cast<uint64_t>(count));
  for (int j = 0; j < kTokenLanes; ++j)
    acc = splitmix64(acc ^ ((static_cast<uint64_t>(j) << 32) | lanes[j]));
  for (; i < count; ++i) acc = splitmix64(acc ^ static_cast<uint32_t>(tokens[i]));
  return acc;
}

void refresh_chain(std::vector<uint64_t>& chain, const int32_t* tokens, int64_t n,
                   int64_t ppp) {
  const size_t sealed = static_cast<size_t>(n / ppp);
  if (chain.size() > sealed) chain.resize(sealed);
  while (chain.size() < sealed) {
    const size_t o = chain.size();
    const uint64_t prev = o > 0 ? chain[o - 1] : kChainSeed;
    chain.push_back(chain_link(prev, hash_token_block(tokens + o * ppp, ppp)));
  }
}

int64_t first_mismatch(const int32_t* a, const int32_t* b, int64_t start, int64_t limit) {
  for (int64_t i = start; i < limit; ++i)
    if (a[i] != b[i]) return i;
  return limit;
}

int64_t hashed_prefix_len(int64_t ppp, const int32_t* a, int64_t na, const uint64_t* ac,
                          int64_t nac, const int32_t* b, int64_t nb, const uint64_t* bc,
                          int64_t nbc) {
  const int64_t pages = std::min(nac, nbc);
  int64_t matched = 0;
  while (matched < pages && ac[matched] == bc[matched]) ++matched;
  const int64_t n = std::min(na, nb);
  const int64_t base = matched * ppp;
  return first_mismatch(a, b, base, std::min(n, base + ppp));
}

// ---- SlotRegistry (slot_registry.mojo:6-107) --------------------------------

SlotRegistry::SlotRegistry(int64_t ppp, int64_t max_seqs) : ppp_(ppp), max_seqs_(max_seqs) {
  require(ppp > 0, "slot registry: positions_per_page must be positive");
  require(max_seqs > 0, "slot registry: max_seqs must be positive");
  resident_.assign(max_seqs, 0);
  owner_.assign(max_seqs, -1);
  last_used_.assign(max_seqs, 0);
  tokens_.resize(max_seqs);
  chains_.resize(max_seqs);
}

void SlotRegistry::check_seq(int64_t s) const {
  require(s >= 0 && s < max_seqs_, "slot registry: sequence out of range");
}

void SlotRegistry::open(int64_t s, int64_t owner, uint64_t now) {
  check_seq(s);
  resident_[s] = 1;
  owner_[s] = owner;
  last_used_[s] = now;
  tokens_[s].clear();
  chains_[s].clear();
}

void SlotRegistry::adopt(int64_t s, int64_t owner, uint64_t now) {
  check_seq(s);
  owner_[s] = owner;
  last_used_[s] = now;
}

void SlotRegistry::extend(int64_t s, const int32_t* src, int64_t n_src, int64_t start,
                          int64_t base_pos, int64_t count, uint64_t now) {
  check_seq(s);
  auto& toks = tokens_[s];
  require(base_pos <= static_cast<int64_t>(toks.size()),
          "slot registry: extend would leave a position gap");
  require(start >= 0 && count >= 0 && start + count <= n_src,
          "slot registry: extend reads past the source");
  // Positions already in the history are skipped, so a re-fed token (the
  // last prompt token of a fully matched request) is not duplicated.
  for (int64_t t = 0; t < count; ++t) {
    if (base_pos + t < static_cast<int64_t>(toks.size())) continue;
    toks.push_back(src[start + t]);
  }
  refresh_chain(chains_[s], toks.data(), static_cast<int64_t>(toks.size()), ppp_);
  last_used_[s] = now;
}

void SlotRegistry::seed(int64_t s, const int32_t* src, int64_t n_src, int64_t count,
                        uint64_t now) {
  check_seq(s);
  require(count >= 0 && count <= n_src, "slot registry: seed reads past the source");
  auto& toks = tokens_[s];
  const int64_t same = first_mismatch(toks.data(), src, 0,
                                      std::min<int64_t>(static_cast<int64_t>(toks.size()), n_src));
  const size_t keep = static_cast<size_t>(std::min(same, count) / ppp_);
  if (chains_[s].size() > keep) chains_[s].resize(keep);
  toks.assign(src, src + count);
  refresh_chain(chains_[s], toks.data(), count, ppp_);
  last_used_[s] = now;
}

void SlotRegistry::close(int64_t s) {
  check_seq(s);
  resident_[s] = 0;
  owner_[s] = -1;
  tokens_[s].clear();
  chains_[s].clear();
}

int64_t SlotRegistry::prefix_len(int64_t s, const int32_t* in, int64_t n_in,
                                 const uint64_t* in_chain, int64_t n_chain) const {
  check_seq(s);
  const auto& toks = tokens_[s];
  const auto& ch = chains_[s];
  return hashed_prefix_len(ppp_, toks.data(), static_cast<int64_t>(toks.size()), ch.data(),
                           static_cast<int64_t>(ch.size()), in, n_in, in_chain, n_chain);
}

int64_t SlotRegistry::exact_prefix_len(int64_t s, const int32_t* in, int64_t n_in) const {
  check_seq(s);
  const auto& toks = tokens_[s];
  return first_mismatch(toks.data(), in, 0,
                        std::min<int64_t>(static_cast<int64_t>(toks.size()), n_in));
}

int64_t SlotRegistry::lru_victim() const {
  int64_t victim = -1;
  uint64_t oldest = 0;
  for (int64_t s = 0; s < max_seqs_; ++s) {
    if (!resident_[s] || owner_[s] >= 0) continue;
    if (victim < 0 || last_used_[s] < oldest) {
      victim = s;
      oldest = last_used_[s];
    }
  }
  return victim;
}

// ---- Scheduler (scheduler.mojo:61-780) --------------------------------------

Scheduler::Scheduler(int64_t ppp, int64_t max_seqs, int64_t max_slots, int64_t max_step_tokens,
                     const std::vector<PoolSpec>& pools, int64_t step_budget,
                     std::vector<int32_t> stop_tokens, int64_t decode_band)
    : ppp_(ppp),
      pages_(max_seqs, pools),
      registry_(ppp, max_seqs),
      need_(pools.size(), 0),
      max_slots_(max_slots),
      step_budget_(std::min(step_budget, max_step_tokens)),
      decode_band_(decode_band),
      stop_tokens_(std::move(stop_tokens)) {
  require(max_slots > 0 && max_step_tokens > 0, "scheduler: max_slots and max_step_tokens > 0");
  // Ring capacity: the shortest ring window in positions.  Sequence
  // ceiling: the fewest positions a growing pool can map for one sequence.
  ring_capacity_ = int64_t{1} << 62;
  seq_ceiling_ = int64_t{1} << 62;
  for (const auto& s : pools) {
    if (s.fixed_pages_per_seq > 0) {
      ring_capacity_ = std::min(ring_capacity_, s.fixed_pages_per_seq * ppp);
    } else {
      seq_ceiling_ = std::min(seq_ceiling_, std::min(s.max_pages_per_seq, s.num_pages) * ppp);
    }
  }
  ring_floor_.assign(max_seqs, 0);
  reuse_dirty_.assign(max_seqs, 0);
  unsharable_.assign(max_seqs, 0);
}

const Request& Scheduler::request(int64_t rid) const {
  require(rid >= 0 && rid < request_count(), "scheduler: request id out of range");
  return requests_[rid];
}

bool Scheduler::is_stop_token(int32_t t) const {
  return std::find(stop_tokens_.begin(), stop_tokens_.end(), t) != stop_tokens_.end();
}

int64_t Scheduler::submit(const int32_t* tokens, int64_t n, int64_t max_new_tokens,
                          bool no_share) {
  if (n <= 0 || n > seq_ceiling_) return -1;
  Request r;
  r.tokens.assign(tokens, tokens + n);
  r.max_new_tokens = max_new_tokens;
  r.no_share = no_share;
  refresh_chain(r.chain, r.tokens.data(), n, ppp_);
  int64_t rid;
  if (!free_slots_.empty()) {
    rid = free_slots_.back();
    free_slots_.pop_back();
    requests_[rid] = std::move(r);
  } else {
    rid = request_count();
    requests_.push_back(std::move(r));
  }
  pending_.push_back(rid);
  return rid;
}

void Scheduler::cancel(int64_t rid) {
  require(rid >= 0 && rid < request_count(), "scheduler: request id out of range");
  requests_[rid].cancelled = true;
}

bool Scheduler::retire(int64_t rid) {
  require(rid >= 0 && rid < request_count(), "scheduler: request id out of range");
  Request& r = requests_[rid];
  if (!r.live || !r.done) return false;
  r.live = false;
  r.tokens.clear();
  r.chain.clear();
  r.generated.clear();
  pending_.erase(std::remove(pending_.begin(), pending_.end(), rid), pending_.end());
  free_slots_.push_back(rid);
  return true;
}

bool Scheduler::pending_work() const {
  for (int64_t k : pending_)
    if (!requests_[k].done) return true;
  return false;
}

void Scheduler::evict(int64_t s) {
  pages_.release(s);
  registry_.close(s);
  unsharable_[s] = 0;
}

bool Scheduler::evict_warm() {
  int64_t victim = registry_.lru_victim();
  if (victim < 0) return false;
  evict(victim);
  return true;
}

bool Scheduler::evict_warm_for() {
  // Oldest warm sequence holding a sole-held page of a pool that is short.
  int64_t victim = -1;
  uint64_t oldest = 0;
  for (int64_t s = 0; s < registry_.max_seqs(); ++s) {
    if (!is_warm(s)) continue;
    bool frees = false;
    for (int64_t p = 0; p < pages_.pool_count(); ++p) {
      if (need_[p] <= pages_.pool_available(p)) continue;
      if (pages_.freeable_pages(p, s) > 0) frees = true;
    }
    if (!frees) continue;
    if (victim < 0 || registry_.last_used(s) < oldest) {
      victim = s;
      oldest = registry_.last_used(s);
    }
  }
  if (victim < 0) victim = chained_warm_victim();
  if (victim < 0) return false;
  evict(victim);
  return true;
}

int64_t Scheduler::chained_warm_victim() const {
  // Oldest warm sequence on a shared page whose every hold is warm: freeing
  // the whole chain eventually returns the page.
  int64_t victim = -1;
  uint64_t oldest = 0;
  for (int64_t p = 0; p < pages_.pool_count(); ++p) {
    if (need_[p] <= pages_.pool_available(p)) continue;
    const PagePool& pl = pages_.pool(p);
    std::vector<int64_t> warm_holds(pl.spec.num_pages, 0);
    for (int64_t s = 0; s < registry_.max_seqs(); ++s) {
      if (!is_warm(s)) continue;
      for (int64_t o = 0; o < pl.spec.max_pages_per_seq; ++o) {
        int64_t page = pl.page_index(s, o);
        if (page >= 0) ++warm_holds[page];
      }
    }
    for (int64_t s = 0; s < registry_.max_seqs(); ++s) {
      if (!is_warm(s)) continue;
      bool chained = false;
      for (int64_t o = 0; o < pl.spec.max_pages_per_seq; ++o) {
        int64_t page = pl.page_index(s, o);
        if (page < 0) continue;
        const int64_t h = pl.pages.holds(page);
        if (h > 1 && warm_holds[page] == h) chained = true;
      }
      if (!chained) continue;
      if (victim < 0 || registry_.last_used(s) < oldest) {
        victim = s;
        oldest = registry_.last_used(s);
      }
    }
  }
  return victim;
}

bool Scheduler::window_intact(int64_t s, int64_t lcp) const {
  // A match is usable only if the ring still holds the live window (the
  // last page of positions before lcp) that a resumed sequence attends to.
  const int64_t seq_len = registry_.length(s);
  if (lcp >= seq_len) return true;
  const int64_t live_start = std::max<int64_t>(lcp - ppp_, 0);
  const int64_t floor = std::max(ring_floor_[s], seq_len - ring_capacity_);
  return live_start >= floor;
}

void Scheduler::release_copy_pins() {
  for (const auto& pin : pins_) pages_.release_page(pin.first, pin.second);
  pins_.clear();
}

std::pair<int64_t, int64_t> Scheduler::best_reusable(int64_t rid, bool want_owned) const {
  const Request& r = requests_[rid];
  const int64_t nt = static_cast<int64_t>(r.tokens.size());
  const int64_t nc = static_cast<int64_t>(r.chain.size());
  int64_t best = -1, best_lcp = 0;
  for (int64_t s = 0; s < registry_.max_seqs(); ++s) {
    if (!registry_.is_resident(s) || unsharable_[s] || reuse_dirty_[s]) continue;
    if ((registry_.owner_of(s) >= 0) != want_owned) continue;
    const int64_t lcp = registry_.prefix_len(s, r.tokens.data(), nt, r.chain.data(), nc);
    if (lcp <= best_lcp) continue;
    if (!window_intact(s, lcp)) continue;
    best = s;
    best_lcp = lcp;
  }
  if (best >= 0) {
    // A hash collision can only overstate the match; the exact scan settles it.
    const int64_t exact = registry_.exact_prefix_len(best, r.tokens.data(), nt);
    if (exact < best_lcp) {
      best_lcp = exact;
      if (best_lcp == 0 || !window_intact(best, best_lcp)) return {-1, 0};
    }
  }
  return {best, best_lcp};
}

bool Scheduler::dirty_donor_exists(int64_t rid) const {
  const Request& r = requests_[rid];
  for (int64_t s = 0; s < registry_.max_seqs(); ++s) {
    if (!reuse_dirty_[s] || !registry_.is_resident(s)) continue;
    const int64_t lcp =
        registry_.prefix_len(s, r.tokens.data(), static_cast<int64_t>(r.tokens.size()),
                             r.chain.data(), static_cast<int64_t>(r.chain.size()));
    if (lcp < ppp_) continue;
    if (window_intact(s, lcp)) return true;
  }
  return false;
}

bool Scheduler::adopt_prefix(int64_t s, int64_t rid, int64_t lcp, uint64_t now) {
  Request& req = requests_[rid];
  const int64_t req_len = static_cast<int64_t>(req.tokens.size());
  const int64_t seq_len = registry_.length(s);
  int64_t take = lcp;
  const int64_t resume = take == req_len ? take - 1 : take;
  int64_t keep_last = fdiv(take - 1, ppp_);
  const int64_t private_ordinal = fdiv(resume, ppp_);
  // The page the request resumes writing into must be sole-held; a shared
  // one is replaced by a private copy of its kept rows.
  bool do_private = false;
  if (private_ordinal <= keep_last) {
    for (int64_t p = 0; p < pages_.pool_count(); ++p) {
      if (pages_.pool_fixed_pages(p) > 0) continue;
      if (pages_.page_holds(p, pages_.page_index(p, s, private_ordinal)) > 1) do_private = true;
    }
  }
  if (do_private) {
    clear_need();
    for (int64_t p = 0; p < pages_.pool_count(); ++p) {
      if (pages_.pool_fixed_pages(p) > 0) continue;
      if (pages_.page_holds(p, pages_.page_index(p, s, private_ordinal)) > 1) ++need_[p];
    }
    while (!pages_.fits(need_)) {
      if (evict_warm_for()) continue;
      // No room for the private page: take only the sealed pages before it.
      take = private_ordinal * ppp_;
      do_private = false;
      break;
    }
    if (!do_private) {
      if (take < 1) return false;
      keep_last = fdiv(take - 1, ppp_);
    }
  }
  registry_.adopt(s, rid, now);
  const int64_t copy_start = static_cast<int64_t>(reuse_copies_.size());
  int64_t trim = take;
  if (do_private) {
    const int64_t valid_rows = take - private_ordinal * ppp_;
    for (int64_t p = 0; p < pages_.pool_count(); ++p) {
      if (pages_.pool_fixed_pages(p) > 0) continue;
      const int64_t old_page = pages_.page_index(p, s, private_ordinal);
      if (pages_.page_holds(p, old_page) <= 1) continue;
      const int64_t fresh = pages_.replace_with_private(p, s, private_ordinal);
      require(fresh >= 0, "adopt: privatization page must fit");
      // The source stays pinned until the step's copies are issued.
      pages_.retain_page(p, old_page);
      pins_.emplace_back(p, old_page);
      reuse_copies_.push_back(PageCopy{p, old_page, fresh, 0, valid_rows});
    }
    trim = private_ordinal * ppp_;
  }
  if (take < seq_len) {
    const int64_t stale_floor = seq_len - ring_capacity_;
    if (stale_floor > ring_floor_[s]) ring_floor_[s] = stale_floor;
    pages_.truncate(s, keep_last);
    registry_.seed(s, req.tokens.data(), req_len, take, now);
  }
  reuse_.push_back(Reuse{s, true, trim, copy_start,
                         static_cast<int64_t>(reuse_copies_.size()) - copy_start});
  if (static_cast<int64_t>(reuse_copies_.size()) > copy_start ||
      (take == req_len && take % ppp_ == 0))
    reuse_dirty_[s] = 1;
  unsharable_[s] = req.no_share ? 1 : 0;
  req.seq_id = s;
  return true;
}

bool Scheduler::fork_prefix(int64_t donor, int64_t rid, int64_t lcp, uint64_t now) {
  Request& req = requests_[rid];
  const int64_t req_len = static_cast<int64_t>(req.tokens.size());
  const int64_t resume = lcp == req_len ? lcp - 1 : lcp;
  int64_t s = pages_.admit();
  if (s < 0) {
    if (!evict_warm()) return false;
    s = pages_.admit();
    if (s < 0) return false;
  }
  const int64_t sealed = fdiv(resume, ppp_);
  const int64_t last_ordinal = fdiv(lcp - 1, ppp_);
  for (int64_t p = 0; p < pages_.pool_count(); ++p) {
    if (pages_.pool_fixed_pages(p) > 0) continue;
    for (int64_t o = 0; o < sealed; ++o) pages_.share(p, donor, s, o);
  }
  for (;;) {
    clear_need();
    pages_.pages_needed(s, last_ordinal, need_);
    if (pages_.fits(need_)) break;
    if (!evict_warm_for()) {
      pages_.release(s);
      return false;
    }
  }
  if (!pages_.reserve(s, last_ordinal)) {
    pages_.release(s);
    return false;
  }
  const int64_t copy_start = static_cast<int64_t>(reuse_copies_.size());
  // Growing pools: copy the matched rows of the donor's partial page.
  const int64_t partial_rows = lcp - sealed * ppp_;
  if (partial_rows > 0) {
    for (int64_t p = 0; p < pages_.pool_count(); ++p) {
      if (pages_.pool_fixed_pages(p) > 0) continue;
      reuse_copies_.push_back(PageCopy{p, pages_.page_index(p, donor, sealed),
                                       pages_.page_index(p, s, sealed), 0, partial_rows});
    }
  }
  // Ring pools: copy the live window [lcp - ppp, lcp), one segment per page.
  const int64_t live_start = std::max<int64_t>(lcp - ppp_, 0);
  for (int64_t p = 0; p < pages_.pool_count(); ++p) {
    const int64_t ring_pages = pages_.pool_fixed_pages(p);
    if (ring_pages == 0) continue;
    for (int64_t a = live_start; a < lcp;) {
      const int64_t page_end = (fdiv(a, ppp_) + 1) * ppp_;
      const int64_t seg_end = std::min(lcp, page_end);
      const int64_t ring_slot = fdiv(a, ppp_) % ring_pages;
      reuse_copies_.push_back(PageCopy{p, pages_.page_index(p, donor, ring_slot),
                                       pages_.page_index(p, s, ring_slot), a % ppp_,
                                       seg_end - a});
      a = seg_end;
    }
  }
  registry_.open(s, rid, now);
  registry_.seed(s, req.tokens.data(), req_len, lcp, now);
  ring_floor_[s] = live_start;
  unsharable_[s] = req.no_share ? 1 : 0;
  req.seq_id = s;
  reuse_.push_back(Reuse{s, false, 0, copy_start,
                         static_cast<int64_t>(reuse_copies_.size()) - copy_start});
  reuse_dirty_[s] = 1;
  return true;
}

int64_t Scheduler::request_common_prefix(int64_t a, int64_t b) const {
  const Request& ra = requests_[a];
  const Request& rb = requests_[b];
  return hashed_prefix_len(ppp_, ra.tokens.data(), static_cast<int64_t>(ra.tokens.size()),
                           ra.chain.data(), static_cast<int64_t>(ra.chain.size()),
                           rb.tokens.data(), static_cast<int64_t>(rb.tokens.size()),
                           rb.chain.data(), static_cast<int64_t>(rb.chain.size()));
}

int64_t Scheduler::slot_base(int64_t rid) const {
  // A fully cached request still re-feeds its last token to get logits.
  const Request& r = requests_[rid];
  return std::min(registry_.length(r.seq_id), static_cast<int64_t>(r.tokens.size()) - 1);
}

int64_t Scheduler::admit_slot(int64_t rid, int64_t budget) {
  const Request& req = requests_[rid];
  const int64_t sid = req.seq_id;
  const int64_t n = static_cast<int64_t>(req.tokens.size());
  const int64_t base_pos = slot_base(rid);
  int64_t feed = std::min(n - base_pos, budget);
  // Stop one page past a prefix shared with a waiting request, so that the
  // waiting one can fork from sealed pages next step.
  for (int64_t j : pending_) {
    if (j == rid || requests_[j].seq_id >= 0) continue;
    const int64_t common = request_common_prefix(rid, j);
    if (common < ppp_) continue;
    const int64_t limit = common + ppp_ - base_pos;
    if (limit >= 1 && limit < feed) feed = limit;
  }
  const bool emit = base_pos + feed == n;
  schedule_.tokens.insert(schedule_.tokens.end(), req.tokens.begin() + base_pos,
                          req.tokens.begin() + base_pos + feed);
  const int64_t prompt_len = n - static_cast<int64_t>(req.generated.size());
  Slot slot{sid, rid, base_pos, feed, prompt_len, emit};
  schedule_.prefill_tokens += slot.prefill_count();
  schedule_.decode_tokens += slot.decode_count();
  schedule_.slots.push_back(slot);
  return budget - feed;
}

void Scheduler::preempt_last_slot(uint64_t now) {
  const Slot dropped = schedule_.slots.back();
  schedule_.slots.pop_back();
  schedule_.tokens.resize(schedule_.tokens.size() - dropped.n_tokens);
  schedule_.prefill_tokens -= dropped.prefill_count();
  schedule_.decode_tokens -= dropped.decode_count();
  const int64_t s = dropped.seq_id;
  const int64_t owner = registry_.owner_of(s);
  int64_t adopted_record = -1, fork_record = -1;
  for (int64_t k = 0; k < static_cast<int64_t>(reuse_.size()); ++k) {
    if (reuse_[k].seq_id != s) continue;
    if (reuse_[k].adopted)
      adopted_record = k;
    else
      fork_record = k;
    reuse_[k].seq_id = -1;
  }
  if (adopted_record >= 0) {
    const Request& o = requests_.at(owner);
    registry_.seed(s, o.tokens.data(), static_cast<int64_t>(o.tokens.size()),
                   reuse_[adopted_record].trim_len, now);
    registry_.set_warm(s);
  } else if (fork_record >= 0) {
    evict(s);
  } else {
    registry_.set_warm(s);
  }
  requests_.at(owner).seq_id = -1;
}

void Scheduler::unwind_prefix_reuse(uint64_t now) {
  for (const Reuse& r : reuse_) {
    const int64_t s = r.seq_id;
    if (s < 0) continue;
    const int64_t owner = registry_.owner_of(s);
    if (r.adopted) {
      if (owner >= 0) {
        Request& o = requests_[owner];
        o.seq_id = -1;
        registry_.seed(s, o.tokens.data(), static_cast<int64_t>(o.tokens.size()), r.trim_len,
                       now);
      }
      registry_.set_warm(s);
    } else {
      if (owner >= 0) requests_[owner].seq_id = -1;
      evict(s);
    }
  }
  reuse_.clear();
  reuse_copies_.clear();
  release_copy_pins();
}

bool Scheduler::build_schedule(uint64_t now) {
  // 1. Drop finished requests; cancelled ones demote their sequence to warm.
  {
    std::vector<int64_t> kept;
    kept.reserve(pending_.size());
    for (int64_t i : pending_) {
      Request& r = requests_[i];
      if (r.done) continue;
      if (r.cancelled) {
        r.done = true;
        if (r.seq_id >= 0) {
          registry_.set_warm(r.seq_id);
          r.seq_id = -1;
        }
        continue;
      }
      kept.push_back(i);
    }
    pending_.swap(kept);
  }
  reuse_.clear();
  reuse_copies_.clear();
  std::fill(reuse_dirty_.begin(), reuse_dirty_.end(), 0);

  // 2. Give every unattached request a sequence: adopt a warm prefix, fork
  //    an active one, or admit a fresh sequence.
  for (int64_t i : pending_) {
    Request& r = requests_[i];
    if (r.seq_id >= 0) continue;
    if (!r.no_share) {
      const auto warm = best_reusable(i, false);
      const auto active = best_reusable(i, true);
      const bool can_adopt = warm.first >= 0 && warm.second >= 1;
      const bool can_fork = active.first >= 0 && active.second >= ppp_;
      bool matched = false;
      if (can_adopt && (!can_fork || warm.second + ppp_ > active.second)) {
        matched = adopt_prefix(warm.first, i, warm.second, now);
        if (!matched && can_fork) matched = fork_prefix(active.first, i, active.second, now);
      } else if (can_fork) {
        matched = fork_prefix(active.first, i, active.second, now);
        if (!matched && can_adopt) matched = adopt_prefix(warm.first, i, warm.second, now);
      }
      if (matched) continue;
      if (dirty_donor_exists(i)) continue;  // retry once the donor settles
    }
    int64_t s = pages_.admit();
    if (s < 0) {
      if (!evict_warm()) continue;
      s = pages_.admit();
      if (s < 0) continue;
    }
    registry_.open(s, i, now);
    unsharable_[s] = r.no_share ? 1 : 0;
    ring_floor_[s] = 0;
    r.seq_id = s;
  }

  // 3. Slots: decodes first (one slot kept for a waiting prefill), then
  //    prefills, within the token budget.
  schedule_.clear();
  int64_t budget = step_budget_;
  bool prefill_waiting = false;
  for (int64_t i : pending_)
    if (requests_[i].seq_id >= 0 &&
        static_cast<int64_t>(requests_[i].tokens.size()) - slot_base(i) > decode_band_)
      prefill_waiting = true;
  const int64_t decode_cap = prefill_waiting ? max_slots_ - 1 : max_slots_;
  std::vector<uint8_t> slotted(pending_.size(), 0);
  for (size_t k = 0; k < pending_.size(); ++k) {
    const int64_t i = pending_[k];
    if (requests_[i].seq_id < 0) continue;
    if (static_cast<int64_t>(schedule_.slots.size()) >= decode_cap || budget < 1) break;
    if (static_cast<int64_t>(requests_[i].tokens.size()) - slot_base(i) > decode_band_) continue;
    budget = admit_slot(i, budget);
    slotted[k] = 1;
  }
  for (size_t k = 0; k < pending_.size(); ++k) {
    const int64_t i = pending_[k];
    if (slotted[k] || requests_[i].seq_id < 0) continue;
    if (static_cast<int64_t>(schedule_.slots.size()) >= max_slots_ || budget < 1) break;
    budget = admit_slot(i, budget);
  }

  // 4. Make the write ranges fit: evict warm caches, else preempt slots.
  while (!schedule_.slots.empty()) {
    clear_need();
    for (const Slot& sl : schedule_.slots)
      pages_.pages_needed(sl.seq_id, fdiv(sl.base_pos + sl.n_tokens - 1, ppp_), need_);
    if (pages_.fits(need_)) break;
    if (evict_warm_for()) continue;
    if (schedule_.slots.size() == 1) {
      unwind_prefix_reuse(now);
      return false;
    }
    preempt_last_slot(now);
  }
  if (schedule_.slots.empty()) {
    unwind_prefix_reuse(now);
    return false;
  }
  for (const Slot& sl : schedule_.slots) {
    if (!pages_.reserve(sl.seq_id, fdiv(sl.base_pos + sl.n_tokens - 1, ppp_))) {
      unwind_prefix_reuse(now);
      return false;
    }
  }
  // 5. The reference's debug-build invariants (scheduler.mojo:688-720):
  //    nothing writes into a shared page; an unsharable sequence holds no
  //    shared page.  Its release build runs on when they fail, and so does
  //    this one, counting each failure.  (A request whose whole prompt is
  //    cached re-feeds its last token; if a fork shared that page while the
  //    request waited for a slot, the write lands on the shared page with
  //    the rows it already holds.)
  for (const Slot& sl : schedule_.slots) {
    const int64_t first = fdiv(sl.base_pos, ppp_);
    const int64_t last = fdiv(sl.base_pos + sl.n_tokens - 1, ppp_);
    for (int64_t p = 0; p < pages_.pool_count(); ++p) {
      if (pages_.pool_fixed_pages(p) > 0) continue;
      for (int64_t o = first; o <= last; ++o)
        if (pages_.page_holds(p, pages_.page_index(p, sl.seq_id, o)) != 1)
          ++shared_write_violations_;
    }
  }
  for (const Slot& sl : schedule_.slots) {
    if (!unsharable_[sl.seq_id]) continue;
    const int64_t last = fdiv(sl.base_pos + sl.n_tokens - 1, ppp_);
    for (int64_t p = 0; p < pages_.pool_count(); ++p) {
      if (pages_.pool_fixed_pages(p) > 0) continue;
      for (int64_t o = 0; o <= last; ++o)
        if (pages_.page_holds(p, pages_.page_index(p, sl.seq_id, o)) != 1)
          ++unsharable_violations_;
    }
  }
  // 6. Copies of the reuse records that survived preemption.
  for (const Reuse& r : reuse_) {
    if (r.seq_id < 0) continue;
    schedule_.copies.insert(schedule_.copies.end(), reuse_copies_.begin() + r.copy_start,
                            reuse_copies_.begin() + r.copy_start + r.copy_count);
  }
  release_copy_pins();
  return true;
}

void Scheduler::absorb(const int32_t* emitted, int64_t n_emitted, uint64_t now) {
  int64_t want = 0;
  for (const Slot& sl : schedule_.slots) want += sl.emit ? 1 : 0;
  require(n_emitted >= want, "absorb: fewer sampled tokens than emitting slots");
  int64_t buf_start = 0, emit_idx = 0;
  const int64_t nt = static_cast<int64_t>(schedule_.tokens.size());
  for (const Slot& sl : schedule_.slots) {
    const int64_t rid = registry_.owner_of(sl.seq_id);
    registry_.extend(sl.seq_id, schedule_.tokens.data(), nt, buf_start, sl.base_pos,
                     sl.n_tokens, now);
    buf_start += sl.n_tokens;
    if (!sl.emit) continue;
    const int32_t token = emitted[emit_idx++];
    Request& req = requests_.at(rid);
    req.generated.push_back(token);
    req.tokens.push_back(token);
    refresh_chain(req.chain, req.tokens.data(), static_cast<int64_t>(req.tokens.size()), ppp_);
    if (is_stop_token(token) ||
        static_cast<int64_t>(req.generated.size()) >= req.max_new_tokens ||
        static_cast<int64_t>(req.tokens.size()) > seq_ceiling_) {
      req.done = true;
      registry_.set_warm(sl.seq_id);
    }
  }
}

void Scheduler::discard_step() {
  // The step's ring writes landed; positions they overwrote are gone.
  for (const Slot& sl : schedule_.slots) {
    const int64_t floor = sl.base_pos + sl.n_tokens - ring_capacity_;
    if (floor > ring_floor_[sl.seq_id]) ring_floor_[sl.seq_id] = floor;
  }
}

bool Scheduler::fully_cancelled() const {
  if (schedule_.slots.empty()) return false;
  for (const Slot& sl : schedule_.slots)
    if (!requests_[sl.request_id].cancelled) return false;
  return true;
}

}  // namespace host
}  // namespace ifr
