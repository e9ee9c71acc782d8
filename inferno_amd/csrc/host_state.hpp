// Host-side page state of the paged KV cache: page pools (allocator, page
// table, multi-pool accountant), the page-block prefix hash, the slot
// registry and the continuous-batching scheduler that produces each step's
// slots and copy-on-write page copies.  Plain C++ on the host thread that
// drives the GPU; the C ABI over it is in host_api.cpp.
//
// Reference: continuous_batching/{paging,prefix_hash,slot_registry,schedule,
// scheduler}.mojo and modeling/kv_policy.mojo.  Every decision that changes
// which page a position lands on (free-stack order, victim choice, tie
// breaks) follows the reference exactly, because the GPU kernels read the
// page tables this state produces.
#pragma once

#include <stdint.h>

#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace ifr {
namespace host {

// A violated contract (the reference's debug_assert / abort).  Caught at the
// C ABI and returned as IFR_EINVAL with the message.
struct ContractError : std::runtime_error {
  explicit ContractError(const std::string& m) : std::runtime_error(m) {}
};
inline void require(bool ok, const char* what) {
  if (!ok) throw ContractError(what);
}

struct PoolSpec {  // paging.mojo:1-5
  int64_t num_pages;
  int64_t fixed_pages_per_seq;  // > 0: ring pool, pages mapped at admission
  int64_t max_pages_per_seq;
};

// ---- pages ---------------------------------------------------------------

// LIFO free stack + per-page hold counts (paging.mojo:16-58).
class PageAllocator {
 public:
  explicit PageAllocator(int64_t num_pages);
  int64_t acquire();
  void retain(int64_t page);
  void release(int64_t page);
  int64_t holds(int64_t page) const { return holds_.at(page); }
  int64_t available() const { return static_cast<int64_t>(free_.size()); }
  int64_t size() const { return static_cast<int64_t>(holds_.size()); }
  const std::vector<int32_t>& free_stack() const { return free_; }
  const std::vector<int32_t>& hold_counts() const { return holds_; }

 private:
  std::vector<int32_t> free_;
  std::vector<int32_t> holds_;
};

// One pool: spec, pages, and the [max_seqs][max_pages_per_seq] table
// (paging.mojo:61-93).
struct PagePool {
  PoolSpec spec;
  PageAllocator pages;
  std::vector<int32_t> table;
  PagePool(const PoolSpec& s, int64_t max_seqs);
  int64_t entry(int64_t seq, int64_t ordinal) const;
  int64_t page_index(int64_t seq, int64_t ordinal) const { return table[entry(seq, ordinal)]; }
  void map(int64_t seq, int64_t ordinal, int64_t page) {
    table[entry(seq, ordinal)] = static_cast<int32_t>(page);
  }
  bool ring() const { return spec.fixed_pages_per_seq > 0; }
};

// Multi-pool accounting (paging.mojo:96-242).
class PageAccountant {
 public:
  PageAccountant(int64_t max_seqs, const std::vector<PoolSpec>& pools);

  int64_t max_seqs() const { return max_seqs_; }
  int64_t pool_count() const { return static_cast<int64_t>(pools_.size()); }
  const PagePool& pool(int64_t p) const;
  PagePool& pool(int64_t p);
  bool active(int64_t seq) const { return active_.at(seq) != 0; }

  int64_t page_index(int64_t p, int64_t seq, int64_t ordinal) const {
    return pool(p).page_index(seq, ordinal);
  }
  int64_t page_holds(int64_t p, int64_t page) const { return pool(p).pages.holds(page); }
  int64_t pool_available(int64_t p) const { return pool(p).pages.available(); }
  int64_t pool_fixed_pages(int64_t p) const { return pool(p).spec.fixed_pages_per_seq; }
  int64_t freeable_pages(int64_t p, int64_t seq) const;
  void retain_page(int64_t p, int64_t page) { pool(p).pages.retain(page); }
  void release_page(int64_t p, int64_t page) { pool(p).pages.release(page); }

  int64_t admit();
  void release(int64_t seq);
  void share(int64_t p, int64_t src_seq, int64_t dst_seq, int64_t ordinal);
  void truncate(int64_t seq, int64_t last_keep_ordinal);
  int64_t replace_with_private(int64_t p, int64_t seq, int64_t ordinal);
  void pages_needed(int64_t seq, int64_t last_ordinal, std::vector<int64_t>& need) const;
  bool fits(const std::vector<int64_t>& need) const;
  bool reserve(int64_t seq, int64_t last_ordinal);

 private:
  int64_t max_seqs_;
  std::vector<PagePool> pools_;
  std::vector<uint8_t> active_;
};

// ---- prefix hash (prefix_hash.mojo) ---------------------------------------

constexpr int kTokenLanes = 16;  // simd_width_of[DType.int32]() on AVX-512
constexpr uint64_t kChainSeed = 0x9AE16A3B2F90404Full;

uint64_t splitmix64(uint64_t x);
uint64_t hash_token_block(const int32_t* tokens, int64_t count);
inline uint64_t chain_link(uint64_t prev, uint64_t block_hash) {
  return splitmix64(prev ^ splitmix64(block_hash));
}
void refresh_chain(std::vector<uint64_t>& chain, const int32_t* tokens, int64_t n,
                   int64_t ppp);
int64_t first_mismatch(const int32_t* a, const int32_t* b, int64_t start, int64_t limit);
int64_t hashed_prefix_len(int64_t ppp, const int32_t* a, int64_t na, const uint64_t* ac,
                          int64_t nac, const int32_t* b, int64_t nb, const uint64_t* bc,
                          int64_t nbc);

// ---- slot registry (slot_registry.mojo) -----------------------------------

class SlotRegistry {
 public:
  SlotRegistry(int64_t ppp, int64_t max_seqs);
  int64_t ppp() const { return ppp_; }
  int64_t max_seqs() const { return max_seqs_; }
  int64_t length(int64_t s) const { return static_cast<int64_t>(tokens_.at(s).size()); }
  int64_t owner_of(int64_t s) const { return owner_.at(s); }
  bool is_resident(int64_t s) const { return resident_.at(s) != 0; }
  uint64_t last_used(int64_t s) const { return last_used_.at(s); }
  const std::vector<int32_t>& tokens(int64_t s) const { return tokens_.at(s); }
  const std::vector<uint64_t>& chain(int64_t s) const { return chains_.at(s); }

  void open(int64_t s, int64_t owner, uint64_t now);
  void adopt(int64_t s, int64_t owner, uint64_t now);
  void extend(int64_t s, const int32_t* src, int64_t n_src, int64_t start, int64_t base_pos,
              int64_t count, uint64_t now);
  void seed(int64_t s, const int32_t* src, int64_t n_src, int64_t count, uint64_t now);
  void set_warm(int64_t s) { owner_.at(s) = -1; }
  void close(int64_t s);
  int64_t prefix_len(int64_t s, const int32_t* in, int64_t n_in, const uint64_t* in_chain,
                     int64_t n_chain) const;
  int64_t exact_prefix_len(int64_t s, const int32_t* in, int64_t n_in) const;
  int64_t lru_victim() const;

 private:
  void check_seq(int64_t s) const;
  int64_t ppp_, max_seqs_;
  std::vector<uint8_t> resident_;
  std::vector<int64_t> owner_;
  std::vector<uint64_t> last_used_;
  std::vector<std::vector<int32_t>> tokens_;
  std::vector<std::vector<uint64_t>> chains_;
};

// ---- schedule (schedule.mojo) ----------------------------------------------

struct Slot {
  int64_t seq_id, request_id, base_pos, n_tokens, prompt_len;
  bool emit;
  int64_t prefill_count() const {
    int64_t pre = prompt_len - base_pos;
    if (pre < 0) return 0;
    return pre > n_tokens ? n_tokens : pre;
  }
  int64_t decode_count() const { return n_tokens - prefill_count(); }
};

struct PageCopy {
  int64_t pool, src_page, dst_page, pos_start, pos_count;
};

struct Schedule {
  std::vector<Slot> slots;
  std::vector<int32_t> tokens;
  std::vector<PageCopy> copies;
  int64_t prefill_tokens = 0, decode_tokens = 0;
  void clear() {
    slots.clear();
    tokens.clear();
    copies.clear();
    prefill_tokens = decode_tokens = 0;
  }
};

// ---- scheduler (scheduler.mojo) -------------------------------------------

struct Request {
  std::vector<int32_t> tokens;
  std::vector<uint64_t> chain;
  std::vector<int32_t> generated;
  int64_t max_new_tokens = 0;
  int64_t seq_id = -1;
  bool done = false, live = true, no_share = false, cancelled = false;
};

class Scheduler {
 public:
  Scheduler(int64_t ppp, int64_t max_seqs, int64_t max_slots, int64_t max_step_tokens,
            const std::vector<PoolSpec>& pools, int64_t step_budget,
            std::vector<int32_t> stop_tokens, int64_t decode_band);

  PageAccountant& pages() { return pages_; }
  const PageAccountant& pages() const { return pages_; }
  SlotRegistry& registry() { return registry_; }
  const SlotRegistry& registry() const { return registry_; }
  const Schedule& schedule() const { return schedule_; }
  const Request& request(int64_t rid) const;
  int64_t request_count() const { return static_cast<int64_t>(requests_.size()); }
  const std::vector<int64_t>& pending() const { return pending_; }
  int64_t ring_floor(int64_t s) const { return ring_floor_.at(s); }
  int64_t ring_capacity() const { return ring_capacity_; }
  int64_t seq_ceiling() const { return seq_ceiling_; }
  int64_t ppp() const { return ppp_; }
  int64_t shared_write_violations() const { return shared_write_violations_; }
  int64_t unsharable_violations() const { return unsharable_violations_; }

  int64_t submit(const int32_t* tokens, int64_t n, int64_t max_new_tokens, bool no_share);
  void cancel(int64_t rid);
  bool retire(int64_t rid);
  bool pending_work() const;
  bool evict_warm();
  bool build_schedule(uint64_t now);
  void absorb(const int32_t* emitted, int64_t n_emitted, uint64_t now);
  void discard_step();
  bool fully_cancelled() const;

 private:
  bool is_warm(int64_t s) const {
    return registry_.is_resident(s) && registry_.owner_of(s) < 0;
  }
  bool is_stop_token(int32_t t) const;
  void evict(int64_t s);
  bool evict_warm_for();
  int64_t chained_warm_victim() const;
  bool window_intact(int64_t s, int64_t lcp) const;
  void release_copy_pins();
  std::pair<int64_t, int64_t> best_reusable(int64_t rid, bool want_owned) const;
  bool dirty_donor_exists(int64_t rid) const;
  bool adopt_prefix(int64_t s, int64_t rid, int64_t lcp, uint64_t now);
  bool fork_prefix(int64_t donor, int64_t rid, int64_t lcp, uint64_t now);
  int64_t request_common_prefix(int64_t a, int64_t b) const;
  int64_t slot_base(int64_t rid) const;
  int64_t admit_slot(int64_t rid, int64_t budget);
  void preempt_last_slot(uint64_t now);
  void unwind_prefix_reuse(uint64_t now);
  void clear_need() {
    for (auto& n : need_) n = 0;
  }

  struct Reuse {
    int64_t seq_id;
    bool adopted;
    int64_t trim_len, copy_start, copy_count;
  };

  int64_t ppp_;
  PageAccountant pages_;
  SlotRegistry registry_;
  std::vector<Request> requests_;
  Schedule schedule_;
  std::vector<int64_t> need_;
  int64_t max_slots_, step_budget_, decode_band_;
  std::vector<int32_t> stop_tokens_;
  std::vector<int64_t> pending_, free_slots_;
  int64_t ring_capacity_, seq_ceiling_;
  std::vector<int64_t> ring_floor_;
  std::vector<Reuse> reuse_;
  std::vector<PageCopy> reuse_copies_;
  std::vector<std::pair<int64_t, int64_t>> pins_;
  std::vector<uint8_t> reuse_dirty_, unsharable_;
  int64_t shared_write_violations_ = 0, unsharable_violations_ = 0;
};

}  // namespace host
}  // namespace ifr
