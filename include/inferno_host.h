/*
 * inferno_host.h -- host-side page state of the paged KV cache, exported by
 * libinferno_hip.so next to the GPU path of inferno_hip.h.
 *
 * The reference keeps this state in Mojo on the host thread that drives the
 * attention kernels (continuous_batching/{paging,prefix_hash,slot_registry,
 * schedule,scheduler}.mojo, modeling/kv_policy.mojo).  It decides which page
 * every position lands on, which pages sequences share and which rows are
 * copied on write, so the GPU kernels' page tables come from here.  The C++
 * restatement follows the reference's free-stack order, victim choice and
 * tie breaks exactly, so a host that binds it gets the same page tables,
 * schedules and copies the reference computes.
 *
 * Objects: a page accountant, a slot registry and a scheduler are opaque
 * host objects created and destroyed through this ABI (like FILE*).  The
 * scheduler owns one accountant and one registry; ifr_scheduler_pages() and
 * ifr_scheduler_registry() lend them out for the read and write calls below
 * (never destroy a lent object).  Nothing here touches the GPU.
 *
 * Status: int32_t results are IFR_OK or a negative IFR_E* code (see
 * inferno_hip.h) with the message in ifr_last_error().  Query functions
 * returning int64_t return IFR_QUERY_ERROR on a bad argument.  A violated
 * reference contract (its debug_asserts, e.g. releasing an unheld page,
 * sharing onto a mapped ordinal) is IFR_EINVAL, never an abort.
 *
 * Pool specs cross as int64 [num_pools][3] = {num_pages, fixed_pages_per_seq,
 * max_pages_per_seq} (PagePoolSpec, paging.mojo:1-5).  Clocks ("now") are
 * caller-supplied monotonic values (the reference reads perf_counter_ns()),
 * which keeps LRU decisions reproducible.
 */
#ifndef INFERNO_HOST_H
#define INFERNO_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ifr_pages ifr_pages;          /* KVPageAccountant */
typedef struct ifr_registry ifr_registry;    /* SlotRegistry */
typedef struct ifr_scheduler ifr_scheduler;  /* ContinuousBatchScheduler */

#define IFR_QUERY_ERROR INT64_MIN

/* ---- prefix hash (continuous_batching/prefix_hash.mojo) ------------------ */
/* splitmix64 (simd_math/sampling_rng.mojo:11-19). */
uint64_t ifr_splitmix64(uint64_t x);
/* hash_token_block (prefix_hash.mojo:22-39): 16-lane MurmurHash3 block
 * mixing of tokens[start, start+count), folded through SplitMix64. */
uint64_t ifr_hash_token_block(const int32_t* tokens, int64_t start,
                              int64_t count);
/* chain_link (prefix_hash.mojo:42-44). */
uint64_t ifr_chain_link(uint64_t prev, uint64_t block_hash);
/* refresh_chain (prefix_hash.mojo:47-57): grows or trims chain[0,chain_len)
 * to num_tokens / ppp links; returns the new length, or a negative IFR_E*
 * code (IFR_ESPACE if chain_cap is too small). */
int64_t ifr_refresh_chain(uint64_t* chain, int64_t chain_len, int64_t chain_cap,
                          const int32_t* tokens, int64_t num_tokens,
                          int64_t ppp);
/* hashed_prefix_len (prefix_hash.mojo:86-97). */
int64_t ifr_hashed_prefix_len(int64_t ppp, const int32_t* a_tokens,
                              int64_t a_len, const uint64_t* a_chain,
                              int64_t a_chain_len, const int32_t* b_tokens,
                              int64_t b_len, const uint64_t* b_chain,
                              int64_t b_chain_len);

/* ---- page accountant (continuous_batching/paging.mojo:16-242) ------------ */
int32_t ifr_pages_create(int64_t max_seqs, const int64_t* pool_specs,
                         int64_t num_pools, ifr_pages** out);
void ifr_pages_destroy(ifr_pages* pages);
/* admit (paging.mojo:156-170): *seq_id = admitted sequence or -1. */
int32_t ifr_pages_admit(ifr_pages* pages, int64_t* seq_id);
/* release (:172-181), share (:183-191), truncate (:193-203). */
int32_t ifr_pages_release(ifr_pages* pages, int64_t seq_id);
int32_t ifr_pages_share(ifr_pages* pages, int64_t pool, int64_t src_seq,
                        int64_t dst_seq, int64_t ordinal);
int32_t ifr_pages_truncate(ifr_pages* pages, int64_t seq_id,
                           int64_t last_keep_ordinal);
/* replace_with_private (:205-215): *fresh = new page or -1. */
int32_t ifr_pages_replace_with_private(ifr_pages* pages, int64_t pool,
                                       int64_t seq_id, int64_t ordinal,
                                       int64_t* fresh);
/* pages_needed (:217-223): adds into need[num_pools]. */
int32_t ifr_pages_pages_needed(const ifr_pages* pages, int64_t seq_id,
                               int64_t last_ordinal, int64_t* need);
/* fits (:225-229) and reserve (:231-242): *result = 1 or 0. */
int32_t ifr_pages_fits(const ifr_pages* pages, const int64_t* need,
                       int64_t* result);
int32_t ifr_pages_reserve(ifr_pages* pages, int64_t seq_id,
                          int64_t last_ordinal, int64_t* result);
/* retain_page / release_page (:148-154). */
int32_t ifr_pages_retain_page(ifr_pages* pages, int64_t pool, int64_t page);
int32_t ifr_pages_release_page(ifr_pages* pages, int64_t pool, int64_t page);

enum {
  IFR_PQ_POOL_COUNT = 0,    /* ()                        */
  IFR_PQ_MAX_SEQS = 1,      /* ()                        */
  IFR_PQ_AVAILABLE = 2,     /* (pool)                    */
  IFR_PQ_FIXED_PAGES = 3,   /* (pool)                    */
  IFR_PQ_POOL_PAGES = 4,    /* (pool)                    */
  IFR_PQ_SEQ_LIMIT = 5,     /* (pool) max_pages_per_seq  */
  IFR_PQ_PAGE_INDEX = 6,    /* (pool, seq, ordinal)      */
  IFR_PQ_PAGE_HOLDS = 7,    /* (pool, page)              */
  IFR_PQ_FREEABLE = 8,      /* (pool, seq)               */
  IFR_PQ_ACTIVE = 9         /* (seq)                     */
};
int64_t ifr_pages_query(const ifr_pages* pages, int64_t what, int64_t a,
                        int64_t b, int64_t c);
/* Whole-pool state: table int32 [max_seqs][max_pages_per_seq], holds int32
 * [num_pages], free stack int32 [num_pages] bottom first (*free_len
 * entries).  Any output may be NULL. */
int32_t ifr_pages_export(const ifr_pages* pages, int64_t pool, int32_t* table,
                         int32_t* holds, int32_t* free_stack,
                         int64_t* free_len);

/* ---- slot registry (continuous_batching/slot_registry.mojo:6-107) -------- */
int32_t ifr_registry_create(int64_t ppp, int64_t max_seqs, ifr_registry** out);
void ifr_registry_destroy(ifr_registry* reg);
int32_t ifr_registry_open(ifr_registry* reg, int64_t seq_id, int64_t owner,
                          uint64_t now);
int32_t ifr_registry_adopt(ifr_registry* reg, int64_t seq_id, int64_t owner,
                           uint64_t now);
/* extend (:44-58): source[start, start+count) at positions base_pos... */
int32_t ifr_registry_extend(ifr_registry* reg, int64_t seq_id,
                            const int32_t* source, int64_t source_len,
                            int64_t start, int64_t base_pos, int64_t count,
                            uint64_t now);
/* seed (:60-72): history := source[0, count). */
int32_t ifr_registry_seed(ifr_registry* reg, int64_t seq_id,
                          const int32_t* source, int64_t source_len,
                          int64_t count, uint64_t now);
int32_t ifr_registry_set_warm(ifr_registry* reg, int64_t seq_id);
int32_t ifr_registry_close(ifr_registry* reg, int64_t seq_id);
/* prefix_len (:87-93), exact_prefix_len (:95-96), lru_victim (:98-107):
 * >= 0 (victim: -1 = none), IFR_QUERY_ERROR on a bad argument. */
int64_t ifr_registry_prefix_len(const ifr_registry* reg, int64_t seq_id,
                                const int32_t* tokens, int64_t num_tokens,
                                const uint64_t* chain, int64_t chain_len);
int64_t ifr_registry_exact_prefix_len(const ifr_registry* reg, int64_t seq_id,
                                      const int32_t* tokens,
                                      int64_t num_tokens);
int64_t ifr_registry_lru_victim(const ifr_registry* reg);
enum {
  IFR_RQ_LENGTH = 0,     /* (seq) */
  IFR_RQ_OWNER = 1,      /* (seq) */
  IFR_RQ_RESIDENT = 2,   /* (seq) */
  IFR_RQ_LAST_USED = 3,  /* (seq) */
  IFR_RQ_CHAIN_LEN = 4,  /* (seq) */
  IFR_RQ_MAX_SEQS = 5,   /* ()    */
  IFR_RQ_PPP = 6         /* ()    */
};
int64_t ifr_registry_query(const ifr_registry* reg, int64_t what,
                           int64_t seq_id);
/* History and chain of one sequence (IFR_ESPACE if a cap is too small;
 * either output may be NULL). */
int32_t ifr_registry_export(const ifr_registry* reg, int64_t seq_id,
                            int32_t* tokens, int64_t tokens_cap,
                            uint64_t* chain, int64_t chain_cap);

/* ---- scheduler (continuous_batching/scheduler.mojo:61-780) --------------- */
/* ContinuousBatchScheduler.__init__ (:82-128) for BatchGeometry
 * {max_seqs, max_slots, max_step_tokens, pools} and the stop-token list. */
int32_t ifr_scheduler_create(int64_t ppp, int64_t max_seqs, int64_t max_slots,
                             int64_t max_step_tokens,
                             const int64_t* pool_specs, int64_t num_pools,
                             int64_t step_budget, const int32_t* stop_tokens,
                             int64_t num_stop_tokens, int64_t decode_band,
                             ifr_scheduler** out);
void ifr_scheduler_destroy(ifr_scheduler* sched);
ifr_pages* ifr_scheduler_pages(ifr_scheduler* sched);
ifr_registry* ifr_scheduler_registry(ifr_scheduler* sched);
/* submit (:137-154): *request_id = id, or -1 when the prompt is empty or
 * longer than the sequence ceiling (the reference returns None). */
int32_t ifr_scheduler_submit(ifr_scheduler* sched, const int32_t* tokens,
                             int64_t num_tokens, int64_t max_new_tokens,
                             int64_t no_share, int64_t* request_id);
/* The request's CancelToken.cancel() (schedule.mojo:12-26). */
int32_t ifr_scheduler_cancel(ifr_scheduler* sched, int64_t request_id);
/* retire (:159-174), evict_warm (:182-189): *result = 1 or 0. */
int32_t ifr_scheduler_retire(ifr_scheduler* sched, int64_t request_id,
                             int64_t* result);
int32_t ifr_scheduler_evict_warm(ifr_scheduler* sched, int64_t* result);
/* build_schedule (:567-729): *built = 1 when a schedule with >= 1 slot is
 * ready for ifr_scheduler_export_schedule. */
int32_t ifr_scheduler_build_schedule(ifr_scheduler* sched, uint64_t now,
                                     int64_t* built);
/* absorb (:731-759): one sampled token per emitting slot, in slot order. */
int32_t ifr_scheduler_absorb(ifr_scheduler* sched, const int32_t* emitted,
                             int64_t num_emitted, uint64_t now);
/* discard_step (:761-768), for a fully cancelled step. */
int32_t ifr_scheduler_discard_step(ifr_scheduler* sched);
enum {
  IFR_SQ_PENDING_WORK = 0,     /* ()    */
  IFR_SQ_FULLY_CANCELLED = 1,  /* ()    */
  IFR_SQ_NUM_SLOTS = 2,        /* ()    */
  IFR_SQ_NUM_TOKENS = 3,       /* ()    */
  IFR_SQ_NUM_COPIES = 4,       /* ()    */
  IFR_SQ_PREFILL_TOKENS = 5,   /* ()    */
  IFR_SQ_DECODE_TOKENS = 6,    /* ()    */
  IFR_SQ_NUM_REQUESTS = 7,     /* ()    */
  IFR_SQ_NUM_PENDING = 8,      /* ()    */
  IFR_SQ_RING_CAPACITY = 9,    /* ()    */
  IFR_SQ_SEQ_CEILING = 10,     /* ()    */
  IFR_SQ_RING_FLOOR = 11,      /* (seq) */
  IFR_SQ_REQ_SEQ_ID = 12,      /* (rid) */
  IFR_SQ_REQ_DONE = 13,        /* (rid) */
  IFR_SQ_REQ_LIVE = 14,        /* (rid) */
  IFR_SQ_REQ_CANCELLED = 15,   /* (rid) */
  IFR_SQ_REQ_NUM_TOKENS = 16,  /* (rid) */
  IFR_SQ_REQ_NUM_GENERATED = 17, /* (rid) */
  IFR_SQ_PPP = 18,             /* ()    */
  /* How often the reference's debug-build schedule invariants
   * (scheduler.mojo:688-720) failed: a slot writing into a page another
   * sequence holds, an unsharable sequence holding a shared page.  Its
   * release build continues past them, and so does this library. */
  IFR_SQ_SHARED_WRITES = 19,   /* ()    */
  IFR_SQ_UNSHARABLE_SHARED = 20 /* ()   */
};
int64_t ifr_scheduler_query(const ifr_scheduler* sched, int64_t what,
                            int64_t arg);
/* The built schedule (schedule.mojo:29-90): slots int64 [n][6] = {seq_id,
 * request_id, base_pos, n_tokens, prompt_len, emit}, tokens int32 [sum of
 * n_tokens], copies int64 [m][5] = {pool, src_page, dst_page, pos_start,
 * pos_count}.  Sizes from IFR_SQ_NUM_*; the caps count rows (slots, copies)
 * and tokens; any output may be NULL.  IFR_ESPACE, with nothing written,
 * when a cap is below the schedule's count. */
int32_t ifr_scheduler_export_schedule(const ifr_scheduler* sched, int64_t* slots,
                                      int64_t slots_cap, int32_t* tokens,
                                      int64_t tokens_cap, int64_t* copies,
                                      int64_t copies_cap);
/* A request's tokens (prompt + generated) and generated tokens. */
int32_t ifr_scheduler_export_request(const ifr_scheduler* sched,
                                     int64_t request_id, int32_t* tokens,
                                     int64_t tokens_cap, int32_t* generated,
                                     int64_t generated_cap);
int32_t ifr_scheduler_export_pending(const ifr_scheduler* sched, int64_t* out,
                                     int64_t cap, int64_t* count);

/* ---- kv_policy (modeling/kv_policy.mojo) --------------------------------- */
/* bind_pool_run_table (kv_policy.mojo:99-123): the run table of the built
 * schedule for one pool, in the layout ifr_plan_attention() reads: runs int32
 * [num_slots][4] = {buf_start, base_pos, rows_off, page_count}, base_rows
 * int32 [...] = page * (page_len / pos_shard).  Ring pools list their fixed
 * pages; growing pools list ordinals 0..last_pos/page_len. */
int32_t ifr_bind_pool_run_table(const ifr_scheduler* sched, int64_t pool,
                                int64_t page_len, int64_t pos_shard,
                                int32_t* runs, int64_t runs_cap,
                                int32_t* base_rows, int64_t rows_cap,
                                int64_t* num_runs, int64_t* num_rows);
/* append_prefix_copy_jobs over a copy list (kv_policy.mojo:59-96): one byte
 * job per copy x layer x component, in the layout ifr_dispatch_copy_jobs()
 * reads.  copies int64 [num_copies][5] as exported above; mirrors int64
 * [num_pools][6] = {page_len, pos_shard, region_off, stride, layers,
 * num_components} (KVPoolMirror, :18-35); components int64 [sum][2] =
 * {offset, row_bytes}, pool after pool. */
int32_t ifr_prefix_copy_jobs(const int64_t* copies, int64_t num_copies,
                             const int64_t* mirrors,
                             const int64_t* components, int64_t num_pools,
                             int64_t* jobs, int64_t jobs_cap,
                             int64_t* num_jobs);

#ifdef __cplusplus
}
#endif

#endif /* INFERNO_HOST_H */
