// C ABI of libinferno_hip.so: argument validation, host-side planning (the
// reference dispatcher's routing and split plan), and kernel launches.
// Declarations and the reference interface each entry point replaces are in
// include/inferno_hip.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/inferno_hip.h"
#include "common.hpp"
#include "launch.hpp"

namespace {

thread_local std::string g_error;
thread_local int32_t g_status = IFR_OK;

int32_t fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  g_status = code;
  return code;
}

int32_t ok() {
  g_status = IFR_OK;
  return IFR_OK;
}

int32_t hip_fail(hipError_t err, const char* what) {
  return fail(IFR_EHIP, "%s: %s", what, hipGetErrorString(err));
}

#define IFR_HIP(call, what)                        \
  do {                                             \
    hipError_t e_ = (call);                        \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

inline hipStream_t as_stream(uint64_t s) {
  return reinterpret_cast<hipStream_t>(static_cast<uintptr_t>(s));
}

bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int64_t pow2_shift(int64_t value) {  // kernels/attention_ops.mojo:32-37
  int64_t shift = 0;
  while ((int64_t{1} << shift) < value) ++shift;
  return shift;
}

// ---- reference planning helpers -------------------------------------------

// worker_range (kernels/helpers.mojo:182-191).
void worker_range(int64_t total, int64_t nw, int64_t w, int64_t* s, int64_t* e) {
  const int64_t per = (total + nw - 1) / nw;
  int64_t start = w * per;
  int64_t end = std::min(start + per, total);
  if (start >= total) start = end = total;
  *s = start;
  *e = end;
}

// recommended_workers (kernels/helpers.mojo:206-219) with DISPATCH_BW_PRODUCT
// 2280 and PARALLEL_AMORTIZED_BYTES 1 MiB (kernels/dispatch_heuristics.mojo).
int64_t recommended_workers(int64_t data_bytes, int64_t capacity) {
  if (capacity <= 1) return capacity;
  if (data_bytes >= 1024 * 1024) return capacity;
  const int64_t target = data_bytes / 2280;
  int64_t n = 1;
  while ((n + 1) * (n + 1) <= target && n < capacity) ++n;
  return n;
}

int64_t sliding_valid_len(int64_t pos, int64_t window) {
  return pos + 1 >= window ? window : pos + 1;
}

// plan_run_splits (kernels/attention_ops.mojo:99-137).  The greedy step
// gives the next split to the run with the largest kv/n (first index wins
// ties); a max-heap keyed by that ratio and the index does the same in
// O(cap log runs).
void plan_run_splits(const std::vector<int64_t>& kv, int64_t cap,
                     int64_t min_split, std::vector<int64_t>& n_splits,
                     std::vector<int64_t>& split_base) {
  const size_t R = kv.size();
  n_splits.assign(R, 0);
  split_base.assign(R, 0);
  std::vector<int64_t> ceil_splits(R);
  int64_t remaining = cap;
  for (size_t i = 0; i < R; ++i) {
    ceil_splits[i] = kv[i] > 0 ? (kv[i] + min_split - 1) / min_split : 0;
    const int64_t seeded = (ceil_splits[i] > 0 && remaining > 0) ? 1 : 0;
    remaining -= seeded;
    n_splits[i] = seeded;
  }
  // heap entries: run index; ordering: larger kv/n first, then smaller index.
  auto better = [&](size_t a, size_t b) {  // true if a has lower priority
    const __int128 lhs = static_cast<__int128>(kv[b]) * n_splits[a];
    const __int128 rhs = static_cast<__int128>(kv[a]) * n_splits[b];
    if (lhs != rhs) return lhs > rhs;  // kv[b]/n[b] > kv[a]/n[a]
    return a > b;
  };
  std::vector<size_t> heap;
  for (size_t i = 0; i < R; ++i)
    if (n_splits[i] > 0 && n_splits[i] < ceil_splits[i]) heap.push_back(i);
  std::make_heap(heap.begin(), heap.end(), better);
  while (remaining > 0 && !heap.empty()) {
    std::pop_heap(heap.begin(), heap.end(), better);
    const size_t best = heap.back();
    heap.pop_back();
    n_splits[best] += 1;
    remaining -= 1;
    if (n_splits[best] < ceil_splits[best]) {
      heap.push_back(best);
      std::push_heap(heap.begin(), heap.end(), better);
    }
  }
  int64_t running = 0;
  for (size_t i = 0; i < R; ++i) {
    split_base[i] = running;
    running += n_splits[i];
  }
}

struct Geometry {
  int64_t shift, row_mask, page_mask;
};

int64_t plan_words(int64_t num_runs, int64_t num_rows, int64_t seq_len,
                   int64_t cap) {
  const int64_t items = std::max<int64_t>({cap, seq_len, 1});
  const int64_t units = std::max<int64_t>({seq_len, num_runs, 1});
  const int64_t qblocks = seq_len / ifr::kPrefillTokens + num_runs + 1;
  return ifr::kHdrWords + 4 * num_runs + num_rows + std::max<int64_t>(seq_len, 1) +
         ifr::kItemWords * items + ifr::kUnitWords * units + ifr::kQBlockWords * qblocks;
}

// Validates a host run table against the cache geometry and the positions
// the append and attention kernels will touch.
int32_t check_runs(const int32_t* runs, int64_t num_runs,
                   const int32_t* base_rows, int64_t num_rows, int64_t seq_len,
                   int64_t kind, int64_t window, const Geometry& g,
                   int64_t page_len, int64_t cache_rows) {
  if (num_runs <= 0) return fail(IFR_EINVAL, "num_runs must be positive");
  if (!runs || !base_rows) return fail(IFR_EINVAL, "null run table");
  if (runs[0] != 0) return fail(IFR_EINVAL, "runs[0].buf_start must be 0");
  for (int64_t i = 0; i < num_runs; ++i) {
    const int64_t buf_start = runs[4 * i], base_pos = runs[4 * i + 1];
    const int64_t rows_off = runs[4 * i + 2], page_count = runs[4 * i + 3];
    const int64_t next = i + 1 < num_runs ? runs[4 * (i + 1)] : seq_len;
    if (buf_start < 0 || next < buf_start || buf_start >= seq_len)
      return fail(IFR_EINVAL, "run %lld: buf_start %lld out of order or range",
                  (long long)i, (long long)buf_start);
    if (base_pos < 0) return fail(IFR_EINVAL, "run %lld: negative base_pos", (long long)i);
    if (rows_off < 0 || page_count < 0 || rows_off + page_count > num_rows)
      return fail(IFR_EINVAL, "run %lld: rows [%lld, +%lld) outside base_rows[%lld]",
                  (long long)i, (long long)rows_off, (long long)page_count,
                  (long long)num_rows);
    // Every run carries at least one token (a schedule slot feeds >= 1,
    // modeling/kv_policy.mojo:105-123): the seq_len == 1 route plans run 0
    // and the batched route one run per token, so an empty run would be
    // planned over rows that belong to no token of the step.
    const int64_t n_tok = next - buf_start;
    if (n_tok <= 0)
      return fail(IFR_EINVAL, "run %lld holds no token (buf_start %lld, next run at %lld)",
                  (long long)i, (long long)buf_start, (long long)next);
    const int64_t hi_pos = base_pos + n_tok - 1;
    if (hi_pos > INT32_MAX / 2) return fail(IFR_EINVAL, "run %lld: position overflow", (long long)i);
    int64_t lo_pos = 0;
    if (kind == 0) lo_pos = std::max<int64_t>(0, base_pos - window + 1);
    // Page ordinals the kernels index: (p >> shift) & page_mask, p in [lo, hi].
    int64_t need;
    if (g.page_mask < 0) {
      need = (hi_pos >> g.shift) + 1;
    } else if ((hi_pos >> g.shift) - (lo_pos >> g.shift) >= g.page_mask) {
      need = g.page_mask + 1;
    } else {
      need = 0;
      for (int64_t p = lo_pos >> g.shift; p <= (hi_pos >> g.shift); ++p)
        need = std::max(need, (p & g.page_mask) + 1);
    }
    if (need > page_count)
      return fail(IFR_EINVAL, "run %lld needs %lld pages, has %lld", (long long)i,
                  (long long)need, (long long)page_count);
    for (int64_t j = 0; j < need; ++j) {
      const int64_t row = base_rows[rows_off + j];
      if (row < 0 || row + page_len > cache_rows)
        return fail(IFR_EINVAL, "run %lld page %lld: base row %lld outside cache of %lld rows",
                    (long long)i, (long long)j, (long long)row, (long long)cache_rows);
    }
  }
  return IFR_OK;
}

int32_t geometry(int64_t kind, int64_t cache_size, int64_t page_len,
                 Geometry* g) {
  if (!is_pow2(page_len)) return fail(IFR_EINVAL, "page_len %lld is not a power of two", (long long)page_len);
  g->shift = pow2_shift(page_len);
  g->row_mask = page_len - 1;
  if (kind == 0) {
    const int64_t ring = cache_size / page_len;
    if (cache_size % page_len != 0 || !is_pow2(ring))
      return fail(IFR_EINVAL, "cache_size/page_len must be a power of two");
    g->page_mask = ring - 1;
  } else if (kind == 1) {
    g->page_mask = -1;
  } else {
    return fail(IFR_EINVAL, "kind must be 0 (sliding) or 1 (full)");
  }
  return IFR_OK;
}

// The reference dispatcher's routing (kernels/attention_dispatch_kernels.mojo:
// 36-160 sliding, 163-299 full, degree 1) written into a plan image.
int32_t plan_impl(int32_t* img, int64_t img_words, const int32_t* runs,
                  int64_t num_runs, const int32_t* base_rows, int64_t num_rows,
                  int64_t seq_len, int64_t kind, int64_t window,
                  int64_t cache_size, int64_t page_len, int64_t cache_rows,
                  int64_t cap, int64_t kv_row_bytes, int64_t* info) {
  using namespace ifr;
  if (!img || !info) return fail(IFR_EINVAL, "null image or info");
  if (seq_len <= 0) return fail(IFR_EINVAL, "seq_len must be positive");
  if (cap < 1) return fail(IFR_EINVAL, "cap must be >= 1");
  if (kind == 0 && window <= 0) return fail(IFR_EINVAL, "window must be positive");
  if (kv_row_bytes <= 0) return fail(IFR_EINVAL, "kv_row_bytes must be positive");
  if (cache_rows <= 0) return fail(IFR_EINVAL, "cache_rows must be positive");
  Geometry g;
  int32_t st = geometry(kind, cache_size, page_len, &g);
  if (st) return st;
  st = check_runs(runs, num_runs, base_rows, num_rows, seq_len, kind, window, g,
                  page_len, cache_rows);
  if (st) return st;
  const int64_t need = plan_words(num_runs, num_rows, seq_len, cap);
  if (need > img_words)
    return fail(IFR_ESPACE, "plan image needs %lld bytes, have %lld",
                (long long)(need * 4), (long long)(img_words * 4));
  if (need > INT32_MAX) return fail(IFR_EINVAL, "plan too large");

  const bool sliding = kind == 0;
  int64_t max_pos = 0;  // highest token position of the step
  for (int64_t i = 0; i < num_runs; ++i) {
    const int64_t next = i + 1 < num_runs ? runs[4 * (i + 1)] : seq_len;
    if (next > runs[4 * i]) max_pos = std::max<int64_t>(max_pos, runs[4 * i + 1] + next - 1 - runs[4 * i]);
  }
  int32_t* hdr = img;
  memset(hdr, 0, sizeof(int32_t) * kHdrWords);
  int64_t off = kHdrWords;
  // Items first, at the fixed offset the decode kernels read them from;
  // the region is sized for the most items a plan of this shape can have.
  static_assert(kItemsOff == kHdrWords, "items follow the header");
  int32_t* items = img + off;
  hdr[kHdrOffItems] = static_cast<int32_t>(off);
  off += kItemWords * std::max<int64_t>({cap, seq_len, 1});
  hdr[kHdrOffRuns] = static_cast<int32_t>(off);
  memcpy(img + off, runs, sizeof(int32_t) * 4 * num_runs);
  off += 4 * num_runs;
  hdr[kHdrOffRows] = static_cast<int32_t>(off);
  memcpy(img + off, base_rows, sizeof(int32_t) * num_rows);
  off += num_rows;
  hdr[kHdrOffTokRun] = static_cast<int32_t>(off);
  {
    int64_t r = 0;
    for (int64_t t = 0; t < seq_len; ++t) {
      while (r + 1 < num_runs && t >= runs[4 * (r + 1)]) ++r;
      img[off + t] = static_cast<int32_t>(r);
    }
  }
  off += seq_len;
  int64_t n_items = 0, n_units = 0, n_stripes = 0;
  int32_t mode = IFR_PLAN_SPLIT_MERGE;
  auto put_item = [&](int64_t q_row, int64_t run, int64_t start_pos,
                      int64_t start, int64_t end, int64_t stripe) {
    int32_t* it = items + n_items * kItemWords;
    it[0] = static_cast<int32_t>(q_row);
    it[1] = static_cast<int32_t>(run);
    it[2] = static_cast<int32_t>(start_pos);
    it[3] = static_cast<int32_t>(start);
    it[4] = static_cast<int32_t>(end);
    it[5] = static_cast<int32_t>(stripe);
    // The run's row table as a word offset into the image, so a kernel
    // reaches its pages in two dependent loads (item, rows).
    it[6] = hdr[kHdrOffRows] + runs[4 * run + 2];
    it[7] = 0;
    ++n_items;
  };
  std::vector<int64_t> unit_buf;  // out_row, stripe_base, n_stripes

  if (seq_len == 1) {
    const int64_t base_pos = runs[1];
    const int64_t valid = sliding ? sliding_valid_len(base_pos, window) : base_pos + 1;
    if (valid > 0) {
      const int64_t start_pos = sliding ? base_pos - valid + 1 : 0;
      int64_t nw = recommended_workers(valid * kv_row_bytes, cap);
      if (nw <= 0) nw = cap;
      nw = std::min(std::min(nw, cap), valid);
      for (int64_t w = 0; w < nw; ++w) {
        int64_t s, e;
        worker_range(valid, nw, w, &s, &e);
        put_item(0, 0, start_pos, s, e, w);
      }
      unit_buf.insert(unit_buf.end(), {0, 0, nw});
      n_stripes = nw;
    }
  } else if (num_runs == seq_len && num_runs > 1 && num_runs < cap) {
    std::vector<int64_t> kv(num_runs), ns, sb;
    for (int64_t i = 0; i < num_runs; ++i) {
      const int64_t p = runs[4 * i + 1];
      kv[i] = sliding ? sliding_valid_len(p, window) : p + 1;
    }
    plan_run_splits(kv, cap, ifr::kTile, ns, sb);
    for (int64_t i = 0; i < num_runs; ++i) {
      const int64_t start_pos = sliding ? runs[4 * i + 1] - kv[i] + 1 : 0;
      for (int64_t s = 0; s < ns[i]; ++s) {
        int64_t a, b;
        worker_range(kv[i], ns[i], s, &a, &b);
        put_item(runs[4 * i], i, start_pos, a, b, sb[i] + s);
      }
      unit_buf.insert(unit_buf.end(), {runs[4 * i], sb[i], ns[i]});
      n_stripes += ns[i];
    }
    // Longest items first: workgroups are dispatched in item order as
    // earlier ones finish, so this is a longest-processing-time schedule
    // over the CUs (each item names its own stripe; the order changes no
    // result).
    std::vector<std::array<int32_t, kItemWords>> recs(n_items);
    for (int64_t i = 0; i < n_items; ++i)
      std::copy(items + i * kItemWords, items + (i + 1) * kItemWords, recs[i].begin());
    std::stable_sort(recs.begin(), recs.end(), [](const auto& x, const auto& y) {
      return x[4] - x[3] > y[4] - y[3];
    });
    for (int64_t i = 0; i < n_items; ++i)
      std::copy(recs[i].begin(), recs[i].end(), items + i * kItemWords);
  } else {
    // Token-partitioned prefill kernels (kernels/flash_attention_prefill.mojo).
    mode = sliding ? IFR_PLAN_TOKEN_DIRECT : IFR_PLAN_TOKEN_MERGE;
    int64_t r = 0;
    for (int64_t t = 0; t < seq_len; ++t) {
      while (r + 1 < num_runs && t >= runs[4 * (r + 1)]) ++r;
      const int64_t abs_pos = runs[4 * r + 1] + (t - runs[4 * r]);
      int64_t lo = 0, hi = abs_pos + 1;
      if (sliding) lo = std::max<int64_t>(0, abs_pos - window + 1);
      put_item(t, r, 0, lo, hi, t);
      unit_buf.insert(unit_buf.end(), {t, t, 1});
    }
    n_stripes = seq_len;
  }
  hdr[kHdrOffUnits] = static_cast<int32_t>(off);
  n_units = static_cast<int64_t>(unit_buf.size() / 3);
  for (int64_t u = 0; u < n_units; ++u) {
    int32_t* un = img + off + u * kUnitWords;
    un[0] = static_cast<int32_t>(unit_buf[3 * u]);
    un[1] = static_cast<int32_t>(unit_buf[3 * u + 1]);
    un[2] = static_cast<int32_t>(unit_buf[3 * u + 2]);
    un[3] = 0;
  }
  off += n_units * kUnitWords;
  // Query blocks for the MFMA prefill (token plans of full attention).
  hdr[kHdrOffQBlocks] = static_cast<int32_t>(off);
  int64_t n_qblocks = 0;
  // The full-attention kernels hold a window of the run's page table in LDS
  // and take runs of any length; the sliding kernel holds the whole ring, so
  // the ring must fit.
  const bool mfma_tables_fit = !sliding || g.page_mask + 1 <= kPrefillLdsPages;
  if ((mode == IFR_PLAN_TOKEN_MERGE || mode == IFR_PLAN_TOKEN_DIRECT) && mfma_tables_fit) {
    std::vector<std::array<int64_t, 4>> qbs;
    for (int64_t r = 0; r < num_runs; ++r) {
      const int64_t b = runs[4 * r], e = r + 1 < num_runs ? runs[4 * (r + 1)] : seq_len;
      for (int64_t t = b; t < e; t += kPrefillTokens) {
        const int64_t n = std::min<int64_t>(kPrefillTokens, e - t);
        qbs.push_back({r, t, n, runs[4 * r + 1] + (t + n - 1 - b) + 1});
      }
    }
    // Run-major order: the blocks of one run start together and walk its
    // keys in step, so each XCD's L2 serves a key tile to all of them.
    // Runs with the longest key range first, and inside a run the longest
    // query block first, to even out the tail.
    std::vector<int64_t> run_top(num_runs, 0);
    for (const auto& qb : qbs) run_top[qb[0]] = std::max(run_top[qb[0]], qb[3]);
    std::stable_sort(qbs.begin(), qbs.end(),
                     [&](const std::array<int64_t, 4>& a, const std::array<int64_t, 4>& b) {
                       if (run_top[a[0]] != run_top[b[0]]) return run_top[a[0]] > run_top[b[0]];
                       if (a[0] != b[0]) return a[0] < b[0];
                       return a[3] > b[3];
                     });
    for (const auto& qb : qbs) {
      int32_t* w = img + off + n_qblocks * kQBlockWords;
      for (int i = 0; i < 4; ++i) w[i] = static_cast<int32_t>(qb[i]);
      ++n_qblocks;
    }
  }
  off += n_qblocks * kQBlockWords;
  hdr[kHdrNumQBlocks] = static_cast<int32_t>(n_qblocks);
  hdr[kHdrMagic] = kPlanMagic;
  hdr[kHdrNumRuns] = static_cast<int32_t>(num_runs);
  hdr[kHdrNumRows] = static_cast<int32_t>(num_rows);
  hdr[kHdrSeqLen] = static_cast<int32_t>(seq_len);
  hdr[kHdrNumItems] = static_cast<int32_t>(n_items);
  hdr[kHdrNumUnits] = static_cast<int32_t>(n_units);
  hdr[kHdrMode] = mode;
  hdr[kHdrNumStripes] = static_cast<int32_t>(n_stripes);
  hdr[kHdrTotalWords] = static_cast<int32_t>(off);
  info[0] = n_items;
  info[1] = n_units;
  info[2] = mode;
  info[3] = n_stripes;
  info[4] = off * 4;
  info[5] = seq_len;
  info[6] = num_runs;
  info[7] = g.shift;
  info[8] = g.row_mask;
  info[9] = g.page_mask;
  info[10] = cache_rows;
  info[11] = kind;
  info[12] = window;
  info[13] = max_pos;
  info[14] = n_qblocks;
  info[15] = 0;
  return ok();
}

int32_t check_info(const int64_t* info) {
  if (!info) return fail(IFR_EINVAL, "null info");
  if (info[0] < 0 || info[1] < 0 || info[0] > INT32_MAX || info[1] > INT32_MAX ||
      info[2] < 0 || info[2] > 2 || info[5] <= 0 || info[7] < 0 || info[7] > 30)
    return fail(IFR_EINVAL, "info does not describe a plan");
  return IFR_OK;
}

// The kernels index the cache with the geometry the plan was validated for;
// any other geometry could reach rows outside the cache.
int32_t check_geometry(const int64_t* info, int64_t shift, int64_t row_mask,
                       int64_t page_mask) {
  if (shift != info[7] || row_mask != info[8] || page_mask != info[9])
    return fail(IFR_EINVAL,
                "page geometry (shift %lld, row_mask %lld, page_mask %lld) differs from the "
                "plan's (%lld, %lld, %lld)",
                (long long)shift, (long long)row_mask, (long long)page_mask,
                (long long)info[7], (long long)info[8], (long long)info[9]);
  return IFR_OK;
}

int32_t check_attention_shapes(int64_t num_q, int64_t num_kv, int64_t head_dim,
                               int64_t partial_stride, int64_t kv_stride,
                               int64_t elt_bytes) {
  if (num_q <= 0 || num_kv <= 0 || num_q % num_kv != 0)
    return fail(IFR_EINVAL, "num_q must be a positive multiple of num_kv");
  if (num_q > 64) return fail(IFR_EUNSUPPORTED, "num_q > 64");
  if (!ifr::attention_shape_supported(static_cast<int>(head_dim),
                                      static_cast<int>(num_q / num_kv)))
    return fail(IFR_EUNSUPPORTED, "head_dim %lld with gqa %lld is not compiled",
                (long long)head_dim, (long long)(num_q / num_kv));
  if (kv_stride < num_kv * head_dim || (kv_stride * elt_bytes) % 16 != 0)
    return fail(IFR_EINVAL, "kv_stride must cover num_kv*head_dim and keep rows 16-byte aligned");
  if (partial_stride < num_q * head_dim + 2 * num_q || partial_stride % 4 != 0)
    return fail(IFR_EINVAL, "partial_stride too small or not a multiple of 4");
  return IFR_OK;
}

}  // namespace

namespace ifr {
// Status plumbing shared with the host-state entry points (host_api.cpp), so
// that ifr_last_error() reports every entry point's failure.
int32_t abi_fail(int32_t code, const char* msg) { return fail(code, "%s", msg); }
int32_t abi_ok() { return ok(); }
}  // namespace ifr

extern "C" {

int32_t ifr_abi_version(void) { return IFR_ABI_VERSION; }

int32_t ifr_last_error(char* buf, int64_t len) {
  if (buf && len > 0) {
    const size_t n = std::min<size_t>(static_cast<size_t>(len - 1), g_error.size());
    memcpy(buf, g_error.data(), n);
    buf[n] = '\0';
  }
  return g_status;
}

int32_t ifr_device_count(int64_t* out) {
  if (!out) return fail(IFR_EINVAL, "null out");
  int n = 0;
  IFR_HIP(hipGetDeviceCount(&n), "hipGetDeviceCount");
  *out = n;
  return ok();
}

int32_t ifr_set_device(int64_t device) {
  IFR_HIP(hipSetDevice(static_cast<int>(device)), "hipSetDevice");
  return ok();
}

int32_t ifr_malloc(void** out, int64_t bytes) {
  if (!out || bytes <= 0) return fail(IFR_EINVAL, "bad malloc arguments");
  IFR_HIP(hipMalloc(out, static_cast<size_t>(bytes)), "hipMalloc");
  return ok();
}

int32_t ifr_free(void* ptr) {
  IFR_HIP(hipFree(ptr), "hipFree");
  return ok();
}

int32_t ifr_host_alloc(void** out, int64_t bytes) {
  if (!out || bytes <= 0) return fail(IFR_EINVAL, "bad host alloc arguments");
  IFR_HIP(hipHostMalloc(out, static_cast<size_t>(bytes), hipHostMallocDefault),
          "hipHostMalloc");
  return ok();
}

int32_t ifr_host_free(void* ptr) {
  IFR_HIP(hipHostFree(ptr), "hipHostFree");
  return ok();
}

int32_t ifr_memcpy_h2d(void* dst, const void* src, int64_t bytes, uint64_t stream) {
  if (bytes < 0) return fail(IFR_EINVAL, "negative size");
  if (bytes == 0) return ok();
  IFR_HIP(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyHostToDevice,
                         as_stream(stream)), "hipMemcpyAsync H2D");
  return ok();
}

int32_t ifr_memcpy_d2h(void* dst, const void* src, int64_t bytes, uint64_t stream) {
  if (bytes < 0) return fail(IFR_EINVAL, "negative size");
  if (bytes == 0) return ok();
  IFR_HIP(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDeviceToHost,
                         as_stream(stream)), "hipMemcpyAsync D2H");
  return ok();
}

int32_t ifr_memcpy_d2d(void* dst, const void* src, int64_t bytes, uint64_t stream) {
  if (bytes < 0) return fail(IFR_EINVAL, "negative size");
  if (bytes == 0) return ok();
  IFR_HIP(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDeviceToDevice,
                         as_stream(stream)), "hipMemcpyAsync D2D");
  return ok();
}

int32_t ifr_memset(void* dst, int32_t value, int64_t bytes, uint64_t stream) {
  if (bytes < 0) return fail(IFR_EINVAL, "negative size");
  if (bytes == 0) return ok();
  IFR_HIP(hipMemsetAsync(dst, value, static_cast<size_t>(bytes), as_stream(stream)),
          "hipMemsetAsync");
  return ok();
}

int32_t ifr_stream_create(uint64_t* out) {
  if (!out) return fail(IFR_EINVAL, "null out");
  hipStream_t s;
  IFR_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  *out = static_cast<uint64_t>(reinterpret_cast<uintptr_t>(s));
  return ok();
}

int32_t ifr_stream_destroy(uint64_t stream) {
  IFR_HIP(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
  return ok();
}

int32_t ifr_stream_sync(uint64_t stream) {
  IFR_HIP(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
  return ok();
}

int32_t ifr_fill_normal_bf16(void* dst, int64_t n, uint64_t seed,
                             int64_t outlier_every, float outlier_scale,
                             uint64_t stream) {
  if (n < 0 || (n > 0 && !dst)) return fail(IFR_EINVAL, "bad fill arguments");
  IFR_HIP(ifr::launch_fill_normal_bf16(dst, n, seed, outlier_every, outlier_scale,
                                       as_stream(stream)), "fill_normal_bf16");
  return ok();
}

int64_t ifr_flash_partial_stride(int64_t num_q, int64_t head_dim) {
  return ((num_q * head_dim + 2 * num_q) * 4 + 63) / 64 * 16;
}

int64_t ifr_plan_bytes(int64_t num_runs, int64_t num_rows, int64_t seq_len,
                       int64_t cap) {
  if (num_runs < 0 || num_rows < 0 || seq_len < 0 || cap < 0) return -1;
  return 4 * plan_words(num_runs, num_rows, seq_len, cap);
}

int32_t ifr_plan_attention(void* image, int64_t image_bytes,
                           const int32_t* runs, int64_t num_runs,
                           const int32_t* base_rows, int64_t num_rows,
                           int64_t seq_len, int64_t kind, int64_t window,
                           int64_t cache_size, int64_t page_len,
                           int64_t cache_rows, int64_t cap,
                           int64_t kv_row_bytes, int64_t* info) {
  return plan_impl(static_cast<int32_t*>(image), image_bytes / 4, runs,
                   num_runs, base_rows, num_rows, seq_len, kind, window,
                   cache_size, page_len, cache_rows, cap, kv_row_bytes, info);
}

int32_t ifr_rope_cache_write(const void* image_dev, const int64_t* info,
                             void* q, const void* k_src, const void* v_src,
                             void* k_cache, void* v_cache,
                             const float* cos_table, const float* sin_table,
                             int64_t num_q, int64_t num_kv,
                             int64_t page_shift, int64_t row_mask,
                             int64_t page_mask, int64_t seq_len, int64_t half,
                             int64_t pair_stride, int64_t head_dim,
                             uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  if (seq_len != info[5]) return fail(IFR_EINVAL, "seq_len differs from the plan");
  if (!image_dev || !q || !k_src || !v_src || !k_cache || !v_cache || !cos_table || !sin_table)
    return fail(IFR_EINVAL, "null pointer");
  if (num_q <= 0 || num_kv <= 0 || head_dim <= 0 || half <= 0 || half > pair_stride ||
      pair_stride + half > head_dim)
    return fail(IFR_EINVAL, "bad rope geometry");
  st = check_geometry(info, page_shift, row_mask, page_mask);
  if (st) return st;
  ifr::PagedGeom g{static_cast<int>(page_shift), static_cast<int>(row_mask),
                   static_cast<int>(page_mask)};
  IFR_HIP(ifr::launch_rope_cache_write(static_cast<const int32_t*>(image_dev),
                                       static_cast<int>(seq_len), q, k_src, v_src,
                                       k_cache, v_cache, cos_table, sin_table,
                                       static_cast<int>(num_q), static_cast<int>(num_kv),
                                       g, static_cast<int>(half),
                                       static_cast<int>(pair_stride),
                                       static_cast<int>(head_dim), as_stream(stream)),
          "rope_cache_write");
  return ok();
}

int32_t ifr_rms_norm_qkv_heads(void* q, void* k, void* v, const void* q_weight,
                               const void* k_weight, int64_t num_q, int64_t num_kv,
                               int64_t seq_len, int64_t head_dim, float sqrt_n, float n_eps,
                               uint64_t stream) {
  if (!q || !k || !v || !q_weight || !k_weight) return fail(IFR_EINVAL, "null pointer");
  if (!aligned(q, 4) || !aligned(k, 4) || !aligned(v, 4))
    return fail(IFR_EINVAL, "q, k and v must be 4-byte aligned");
  if (num_q <= 0 || num_kv <= 0 || seq_len < 0)
    return fail(IFR_EINVAL, "need num_q, num_kv > 0 and seq_len >= 0");
  if (head_dim < 32 || head_dim > 1024 || head_dim % 32 != 0)
    return fail(IFR_EINVAL, "head_dim must be a multiple of 32 in [32, 1024]");
  IFR_HIP(ifr::launch_rms_norm_qkv(q, k, v, q_weight, k_weight, static_cast<int>(seq_len),
                                   static_cast<int>(num_q), static_cast<int>(num_kv),
                                   static_cast<int>(head_dim), sqrt_n, n_eps,
                                   as_stream(stream)),
          "rms_norm_qkv_heads");
  return ok();
}

int32_t ifr_rms_norm_rope_cache_write(const void* image_dev, const int64_t* info, void* q,
                                      const void* k_src, const void* v_src, void* k_cache,
                                      void* v_cache, const void* q_weight,
                                      const void* k_weight, const float* cos_table,
                                      const float* sin_table, int64_t num_q, int64_t num_kv,
                                      int64_t page_shift, int64_t row_mask, int64_t page_mask,
                                      int64_t seq_len, int64_t half, int64_t pair_stride,
                                      int64_t head_dim, float sqrt_n, float n_eps,
                                      uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  if (seq_len != info[5]) return fail(IFR_EINVAL, "seq_len differs from the plan");
  if (!image_dev || !q || !k_src || !v_src || !k_cache || !v_cache || !cos_table ||
      !sin_table || !q_weight || !k_weight)
    return fail(IFR_EINVAL, "null pointer");
  if (!aligned(q, 4) || !aligned(k_src, 4) || !aligned(v_src, 4))
    return fail(IFR_EINVAL, "q, k_src and v_src must be 4-byte aligned");
  if (num_q <= 0 || num_kv <= 0) return fail(IFR_EINVAL, "need num_q, num_kv > 0");
  if (head_dim < 32 || head_dim > 1024 || head_dim % 32 != 0)
    return fail(IFR_EINVAL, "head_dim must be a multiple of 32 in [32, 1024]");
  if (half <= 0 || half > pair_stride || pair_stride + half > head_dim)
    return fail(IFR_EINVAL, "bad rope geometry");
  st = check_geometry(info, page_shift, row_mask, page_mask);
  if (st) return st;
  ifr::PagedGeom g{static_cast<int>(page_shift), static_cast<int>(row_mask),
                   static_cast<int>(page_mask)};
  IFR_HIP(ifr::launch_rms_rope_cache_write(
              static_cast<const int32_t*>(image_dev), static_cast<int>(seq_len), q, k_src,
              v_src, k_cache, v_cache, q_weight, k_weight, cos_table, sin_table,
              static_cast<int>(num_q), static_cast<int>(num_kv), g, static_cast<int>(half),
              static_cast<int>(pair_stride), static_cast<int>(head_dim), sqrt_n, n_eps,
              as_stream(stream)),
          "rms_norm_rope_cache_write");
  return ok();
}

}  // extern "C"

namespace {
// Which MFMA prefill kernel, if any, runs a bf16 plan: token plans with
// query blocks at the shapes the kernels are built for (full attention at
// head_dim 256 / GQA 2 and 512 / GQA 8, sliding windows at 256 / GQA 2).
enum class PrefillRoute { kNone, kFull256, kWide512, kSliding256 };
PrefillRoute bf16_prefill_route(const int64_t* info, int64_t num_q, int64_t num_kv,
                                int64_t head_dim, int64_t page_mask) {
  if (info[14] <= 0) return PrefillRoute::kNone;
  if (info[2] == IFR_PLAN_TOKEN_MERGE && page_mask < 0) {
    if (head_dim == 256 && num_q == 2 * num_kv) return PrefillRoute::kFull256;
    if (head_dim == 512 && num_q == 8 * num_kv) return PrefillRoute::kWide512;
  }
  if (info[2] == IFR_PLAN_TOKEN_DIRECT && page_mask >= 0 && head_dim == 256 &&
      num_q == 2 * num_kv)
    return PrefillRoute::kSliding256;
  return PrefillRoute::kNone;
}
}  // namespace

extern "C" {

int32_t ifr_attention_bf16(const void* image_dev, const int64_t* info,
                           const void* q, const void* k_base,
                           const void* v_base, void* output, void* partials,
                           int64_t partials_bytes, int64_t num_q,
                           int64_t num_kv, int64_t head_dim,
                           int64_t partial_stride, int64_t kv_stride,
                           int64_t page_len, int64_t page_mask,
                           uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  st = check_attention_shapes(num_q, num_kv, head_dim, partial_stride, kv_stride, 2);
  if (st) return st;
  if (!image_dev || !q || !k_base || !v_base || !output || !partials)
    return fail(IFR_EINVAL, "null pointer");
  if (!aligned(q, 16) || !aligned(k_base, 16) || !aligned(v_base, 16) ||
      !aligned(output, 16) || !aligned(partials, 16))
    return fail(IFR_EINVAL, "q, k_base, v_base, output and partials must be 16-byte aligned");
  if (!is_pow2(page_len)) return fail(IFR_EINVAL, "page_len must be a power of two");
  st = check_geometry(info, pow2_shift(page_len), page_len - 1, page_mask);
  if (st) return st;
  ifr::PagedGeom g{static_cast<int>(pow2_shift(page_len)), static_cast<int>(page_len - 1),
                   static_cast<int>(page_mask)};
  const PrefillRoute route = bf16_prefill_route(info, num_q, num_kv, head_dim, page_mask);
  // The MFMA prefill routes finalise in-kernel and write no partials.
  if (route == PrefillRoute::kNone && partials_bytes < info[3] * partial_stride * 4)
    return fail(IFR_ESPACE, "partials need %lld bytes", (long long)(info[3] * partial_stride * 4));
  if (route == PrefillRoute::kFull256) {
    // Prefill chunk of full attention: MFMA query blocks, finalised in-kernel.
    IFR_HIP(ifr::launch_prefill_full_mfma(static_cast<const int32_t*>(image_dev),
                                          static_cast<int>(info[14]), q, k_base, v_base,
                                          output, static_cast<int>(num_q),
                                          static_cast<int>(num_kv), kv_stride, g,
                                          as_stream(stream)),
            "prefill_full_mfma");
    return ok();
  }
  if (route == PrefillRoute::kWide512) {
    // The same at Gemma-4's full-attention shape (head_dim 512, GQA 8).
    IFR_HIP(ifr::launch_prefill_wide_mfma(static_cast<const int32_t*>(image_dev),
                                          static_cast<int>(info[14]), q, k_base, v_base,
                                          output, static_cast<int>(num_q),
                                          static_cast<int>(num_kv), kv_stride, g,
                                          as_stream(stream)),
            "prefill_wide_mfma");
    return ok();
  }
  if (route == PrefillRoute::kSliding256) {
    // Prefill chunk of a sliding-window layer: MFMA query blocks.
    IFR_HIP(ifr::launch_prefill_sliding_mfma(static_cast<const int32_t*>(image_dev),
                                             static_cast<int>(info[14]), q, k_base, v_base,
                                             output, static_cast<int>(num_q),
                                             static_cast<int>(num_kv), kv_stride, g,
                                             static_cast<int>(info[12]), as_stream(stream)),
            "prefill_sliding_mfma");
    return ok();
  }
  IFR_HIP(ifr::launch_attention_bf16(static_cast<const int32_t*>(image_dev),
                                     static_cast<int>(info[0]), static_cast<int>(info[1]),
                                     static_cast<int>(info[2]), q, k_base, v_base, output,
                                     static_cast<float*>(partials), partial_stride,
                                     static_cast<int>(num_q), static_cast<int>(num_kv),
                                     static_cast<int>(head_dim), kv_stride, g,
                                     as_stream(stream)),
          "attention_bf16");
  return ok();
}

}  // extern "C"

// ---- the no-allocation variant of ifr_attention_bf16 --------------------------
// The partials live in a file-scope device array instead of a caller buffer.
// `scratch` names a host-side stand-in in host code; the array's device
// address, which differs per GPU, comes from hipGetSymbolAddress once per
// device (with that device current) and is the only form passed to kernels.
namespace {
constexpr int64_t kStaticScratchBytes = IFR_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxScratchDevices] = {};

int32_t static_scratch(void** out) {
  int dev = 0;
  IFR_HIP(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(IFR_EUNSUPPORTED, "device %d is beyond the %d devices with a static scratch",
                dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    IFR_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) return fail(IFR_EHIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return IFR_OK;
}
}  // namespace

extern "C" {

int32_t ifr_attention_bf16_noalloc(const void* image_dev, const int64_t* info, const void* q,
                                   const void* k_base, const void* v_base, void* output,
                                   int64_t num_q, int64_t num_kv, int64_t head_dim,
                                   int64_t kv_stride, int64_t page_len, int64_t page_mask,
                                   uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  if (num_q <= 0 || head_dim <= 0 || num_q > 64 || head_dim > 4096)
    return fail(IFR_EINVAL, "bad num_q or head_dim");
  const int64_t ps = ifr_flash_partial_stride(num_q, head_dim);
  // The MFMA prefill routes write no partials, so their chunks need no scratch.
  const bool mfma = bf16_prefill_route(info, num_q, num_kv, head_dim, page_mask) !=
                    PrefillRoute::kNone;
  const int64_t need = mfma ? 0 : info[3] * ps * 4;
  if (need > kStaticScratchBytes)
    return fail(IFR_ESPACE,
                "the plan's %lld partial stripes need %lld bytes; the static scratch holds %lld",
                (long long)info[3], (long long)need, (long long)kStaticScratchBytes);
  void* p = nullptr;
  st = static_scratch(&p);
  if (st) return st;
  return ifr_attention_bf16(image_dev, info, q, k_base, v_base, output, p, kStaticScratchBytes,
                            num_q, num_kv, head_dim, ps, kv_stride, page_len, page_mask,
                            stream);
}

int32_t ifr_flash_partials_bf16(const void* image_dev, const int64_t* info,
                                const void* q, const void* k_base, const void* v_base,
                                void* partials, int64_t partials_bytes, int64_t num_q,
                                int64_t num_kv, int64_t head_dim, int64_t partial_stride,
                                int64_t kv_stride, int64_t page_len, int64_t page_mask,
                                uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  st = check_attention_shapes(num_q, num_kv, head_dim, partial_stride, kv_stride, 2);
  if (st) return st;
  if (!image_dev || !q || !k_base || !v_base || !partials)
    return fail(IFR_EINVAL, "null pointer");
  if (!aligned(q, 16) || !aligned(k_base, 16) || !aligned(v_base, 16) || !aligned(partials, 16))
    return fail(IFR_EINVAL, "q, k_base, v_base and partials must be 16-byte aligned");
  if (!is_pow2(page_len)) return fail(IFR_EINVAL, "page_len must be a power of two");
  st = check_geometry(info, pow2_shift(page_len), page_len - 1, page_mask);
  if (st) return st;
  if (partials_bytes < info[3] * partial_stride * 4)
    return fail(IFR_ESPACE, "partials need %lld bytes", (long long)(info[3] * partial_stride * 4));
  ifr::PagedGeom g{static_cast<int>(pow2_shift(page_len)), static_cast<int>(page_len - 1),
                   static_cast<int>(page_mask)};
  IFR_HIP(ifr::launch_partials_bf16(static_cast<const int32_t*>(image_dev),
                                    static_cast<int>(info[0]), q, k_base, v_base,
                                    static_cast<float*>(partials), partial_stride,
                                    static_cast<int>(num_q), static_cast<int>(num_kv),
                                    static_cast<int>(head_dim), kv_stride, g,
                                    as_stream(stream)),
          "flash_partials_bf16");
  return ok();
}

int32_t ifr_merge_flash_partials(const void* image_dev, const int64_t* info,
                                 const void* partials, int64_t partials_bytes,
                                 void* output, int64_t num_q, int64_t head_dim,
                                 int64_t partial_stride, uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  if (!image_dev || !partials || !output) return fail(IFR_EINVAL, "null pointer");
  if (head_dim != 256 && head_dim != 512)
    return fail(IFR_EUNSUPPORTED, "merge is compiled for head_dim 256 and 512");
  if (num_q <= 0 || num_q > 64) return fail(IFR_EINVAL, "bad num_q");
  if (partial_stride < num_q * head_dim + 2 * num_q)
    return fail(IFR_EINVAL, "partial_stride too small");
  if (!aligned(output, 16) || !aligned(partials, 16))
    return fail(IFR_EINVAL, "output and partials must be 16-byte aligned");
  if (partials_bytes < info[3] * partial_stride * 4)
    return fail(IFR_ESPACE, "partials need %lld bytes", (long long)(info[3] * partial_stride * 4));
  IFR_HIP(ifr::launch_merge(static_cast<const int32_t*>(image_dev), static_cast<int>(info[1]),
                            static_cast<int>(info[3]), static_cast<int>(info[2]),
                            static_cast<const float*>(partials),
                            output, partial_stride, static_cast<int>(num_q),
                            static_cast<int>(head_dim), as_stream(stream)),
          "merge_flash_partials");
  return ok();
}

static int32_t dispatch_attention(int64_t kind, const void* q, const void* k_base,
                                  const void* v_base, void* output, void* partials,
                                  int64_t partials_bytes, const int32_t* runs,
                                  int64_t num_runs, const int32_t* base_rows,
                                  int64_t num_rows, int64_t num_q,
                                  int64_t partial_stride, int64_t kv_stride,
                                  int64_t seq_len, int64_t head_dim, int64_t gqa_ratio,
                                  int64_t window, int64_t cache_size, int64_t page_len,
                                  int64_t cache_rows, int64_t cap, void* ws_host,
                                  void* ws_dev, int64_t ws_bytes, uint64_t stream) {
  if (seq_len <= 0) return ok();  // the reference returns without work
  if (gqa_ratio <= 0 || num_q % gqa_ratio != 0)
    return fail(IFR_EINVAL, "num_q must be a multiple of gqa_ratio");
  if (!ws_host || !ws_dev) return fail(IFR_EINVAL, "null plan staging");
  int64_t info[16];
  int32_t st = plan_impl(static_cast<int32_t*>(ws_host), ws_bytes / 4, runs, num_runs,
                         base_rows, num_rows, seq_len, kind, window, cache_size,
                         page_len, cache_rows, cap, kv_stride * 2, info);
  if (st) return st;
  IFR_HIP(hipMemcpyAsync(ws_dev, ws_host, static_cast<size_t>(info[4]),
                         hipMemcpyHostToDevice, as_stream(stream)),
          "plan upload");
  const int64_t page_mask = kind == 0 ? cache_size / page_len - 1 : -1;
  return ifr_attention_bf16(ws_dev, info, q, k_base, v_base, output, partials,
                            partials_bytes, num_q, num_q / gqa_ratio, head_dim,
                            partial_stride, kv_stride, page_len, page_mask, stream);
}

int32_t ifr_dispatch_sliding_attention(
    const void* q, const void* k_base, const void* v_base, void* output,
    void* partials, int64_t partials_bytes, const int32_t* runs,
    int64_t num_runs, const int32_t* base_rows, int64_t num_rows,
    int64_t num_q, int64_t partial_stride, int64_t kv_stride, int64_t seq_len,
    int64_t head_dim, int64_t gqa_ratio, int64_t window, int64_t cache_size,
    int64_t page_len, int64_t cache_rows, int64_t cap, void* ws_host,
    void* ws_dev, int64_t ws_bytes, uint64_t stream) {
  return dispatch_attention(0, q, k_base, v_base, output, partials, partials_bytes,
                            runs, num_runs, base_rows, num_rows, num_q, partial_stride,
                            kv_stride, seq_len, head_dim, gqa_ratio, window, cache_size,
                            page_len, cache_rows, cap, ws_host, ws_dev, ws_bytes, stream);
}

int32_t ifr_dispatch_full_attention(
    const void* q, const void* k_base, const void* v_base, void* output,
    void* partials, int64_t partials_bytes, const int32_t* runs,
    int64_t num_runs, const int32_t* base_rows, int64_t num_rows,
    int64_t num_q, int64_t partial_stride, int64_t kv_stride, int64_t seq_len,
    int64_t head_dim, int64_t gqa_ratio, int64_t page_len, int64_t cache_rows,
    int64_t cap, void* ws_host, void* ws_dev, int64_t ws_bytes,
    uint64_t stream) {
  return dispatch_attention(1, q, k_base, v_base, output, partials, partials_bytes,
                            runs, num_runs, base_rows, num_rows, num_q, partial_stride,
                            kv_stride, seq_len, head_dim, gqa_ratio, 1, page_len,
                            page_len, cache_rows, cap, ws_host, ws_dev, ws_bytes, stream);
}

// ---- page copy and gather ---------------------------------------------------

static constexpr int64_t kCopyChunk = 64 * 1024;

int64_t ifr_copy_jobs_bytes(int64_t num_jobs, int64_t total_bytes) {
  if (num_jobs < 0 || total_bytes < 0) return -1;
  return 32 * (num_jobs + total_bytes / kCopyChunk + 1);
}

int32_t ifr_dispatch_copy_jobs(void* arena, const int64_t* jobs, int64_t num_jobs,
                               void* ws_host, void* ws_dev, int64_t ws_bytes,
                               uint64_t stream) {
  if (num_jobs <= 0) return ok();  // page_copy.mojo:72-74
  if (!arena || !jobs || !ws_host || !ws_dev) return fail(IFR_EINVAL, "null pointer");
  int64_t total = 0;
  for (int64_t i = 0; i < num_jobs; ++i) {
    const int64_t s = jobs[3 * i], d = jobs[3 * i + 1], n = jobs[3 * i + 2];
    if (s < 0 || d < 0 || n < 0) return fail(IFR_EINVAL, "job %lld has a negative field", (long long)i);
    if (n > 0 && ((s < d) ? (s + n > d) : (d + n > s)))
      return fail(IFR_EINVAL, "job %lld copies between overlapping ranges", (long long)i);
    total += n;
  }
  if (total == 0) return ok();
  int64_t* chunks = static_cast<int64_t*>(ws_host);
  int64_t nc = 0;
  const int64_t cap_chunks = ws_bytes / 32;
  for (int64_t i = 0; i < num_jobs; ++i) {
    for (int64_t o = 0; o < jobs[3 * i + 2]; o += kCopyChunk) {
      if (nc >= cap_chunks) return fail(IFR_ESPACE, "copy staging too small");
      chunks[4 * nc] = jobs[3 * i] + o;
      chunks[4 * nc + 1] = jobs[3 * i + 1] + o;
      chunks[4 * nc + 2] = std::min(kCopyChunk, jobs[3 * i + 2] - o);
      chunks[4 * nc + 3] = 0;
      ++nc;
    }
  }
  if (nc > INT32_MAX) return fail(IFR_EINVAL, "too many chunks");
  IFR_HIP(hipMemcpyAsync(ws_dev, ws_host, static_cast<size_t>(nc * 32),
                         hipMemcpyHostToDevice, as_stream(stream)),
          "copy job upload");
  IFR_HIP(ifr::launch_copy_chunks(arena, static_cast<const int64_t*>(ws_dev),
                                  static_cast<int>(nc), as_stream(stream)),
          "copy_chunks");
  return ok();
}

int32_t ifr_dispatch_gather_rows(const void* src, void* dst, const int32_t* rows,
                                 int64_t num_rows, int64_t cols, uint64_t stream) {
  if (num_rows <= 0) return ok();  // gather.mojo:42-43
  if (!src || !dst || !rows) return fail(IFR_EINVAL, "null pointer");
  if (cols <= 0 || cols > INT32_MAX) return fail(IFR_EINVAL, "bad cols");
  if ((cols & 7) == 0 && (!aligned(src, 16) || !aligned(dst, 16)))
    return fail(IFR_EINVAL, "src and dst must be 16-byte aligned");
  IFR_HIP(ifr::launch_gather_rows(src, dst, rows, static_cast<int>(num_rows),
                                  static_cast<int>(cols), as_stream(stream)),
          "gather_rows");
  return ok();
}

// ---- butterquant --------------------------------------------------------------

int32_t ifr_bq_attn_prep(const void* image_dev, const int64_t* info,
                         const void* q_src, const void* k_src, const void* v_src,
                         const void* q_norm, const void* k_norm, void* q_i8,
                         float* qi_bias, float* f_q, void* k_cache, float* k_scale,
                         void* v_cache, float* v_scale, const float* cos_table,
                         const float* sin_table, int64_t num_q, int64_t num_kv,
                         int64_t page_shift, int64_t row_mask, int64_t page_mask,
                         int64_t seq_len, int64_t head_dim, int64_t rope_half,
                         int64_t pair_stride, float sqrt_n, float n_eps,
                         uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  if (seq_len != info[5]) return fail(IFR_EINVAL, "seq_len differs from the plan");
  if (!image_dev || !q_src || !k_src || !v_src || !q_norm || !k_norm || !q_i8 || !qi_bias ||
      !f_q || !k_cache || !k_scale || !v_cache || !v_scale || !cos_table || !sin_table)
    return fail(IFR_EINVAL, "null pointer");
  if (head_dim != 256 && head_dim != 512)
    return fail(IFR_EUNSUPPORTED, "bq prep is compiled for head_dim 256 and 512");
  const int64_t epl = head_dim / 64;  // elements per lane of the prep kernel
  if (rope_half <= 0 || rope_half % epl != 0 || rope_half > pair_stride ||
      pair_stride + rope_half > head_dim || pair_stride % epl != 0)
    return fail(IFR_EINVAL, "bad rope geometry (rope_half and pair_stride must be multiples "
                "of head_dim/64)");
  if (num_q <= 0 || num_kv <= 0) return fail(IFR_EINVAL, "bad head counts");
  st = check_geometry(info, page_shift, row_mask, page_mask);
  if (st) return st;
  ifr::PagedGeom g{static_cast<int>(page_shift), static_cast<int>(row_mask),
                   static_cast<int>(page_mask)};
  IFR_HIP(ifr::launch_bq_attn_prep(static_cast<const int32_t*>(image_dev),
                                   static_cast<int>(seq_len), q_src, k_src, v_src, q_norm,
                                   k_norm, q_i8, qi_bias, f_q, k_cache, k_scale, v_cache,
                                   v_scale, cos_table, sin_table, static_cast<int>(num_q),
                                   static_cast<int>(num_kv), g, static_cast<int>(head_dim),
                                   static_cast<int>(rope_half),
                                   static_cast<int>(pair_stride), sqrt_n, n_eps,
                                   as_stream(stream)),
          "bq_attn_prep");
  return ok();
}

}  // extern "C"

namespace {
int32_t bq_attention(const void* image_dev, const int64_t* info, const void* q_i8,
                     const float* qi_bias, const float* f_q, const void* k_base,
                     const float* k_scale, const void* v_base, const float* v_scale,
                     void* output, void* partials, int64_t partials_bytes, int64_t num_q,
                     int64_t num_kv, int64_t head_dim, int64_t partial_stride,
                     int64_t kv_stride, int64_t page_len, int64_t page_mask,
                     uint64_t stream, void* o_i8, float* o_sa) {
  int32_t st = check_info(info);
  if (st) return st;
  st = check_attention_shapes(num_q, num_kv, head_dim, partial_stride, kv_stride, 1);
  if (st) return st;
  if (!((head_dim == 256 && num_q / num_kv == 2) || (head_dim == 512 && num_q / num_kv == 8)))
    return fail(IFR_EUNSUPPORTED,
                "bq attention is compiled for head_dim 256 with gqa 2 and head_dim 512 with gqa 8");
  if (!image_dev || !q_i8 || !qi_bias || !f_q || !k_base || !k_scale || !v_base ||
      !v_scale || !output || !partials)
    return fail(IFR_EINVAL, "null pointer");
  if (!aligned(q_i8, 16) || !aligned(k_base, 16) || !aligned(v_base, 16) ||
      !aligned(output, 16) || !aligned(partials, 16))
    return fail(IFR_EINVAL, "code, output and partial buffers must be 16-byte aligned");
  if (!is_pow2(page_len)) return fail(IFR_EINVAL, "page_len must be a power of two");
  st = check_geometry(info, pow2_shift(page_len), page_len - 1, page_mask);
  if (st) return st;
  if (partials_bytes < info[3] * partial_stride * 4)
    return fail(IFR_ESPACE, "partials need %lld bytes", (long long)(info[3] * partial_stride * 4));
  ifr::PagedGeom g{static_cast<int>(pow2_shift(page_len)), static_cast<int>(page_len - 1),
                   static_cast<int>(page_mask)};
  if (info[2] == IFR_PLAN_TOKEN_DIRECT && info[14] > 0 && head_dim == 256 &&
      num_q == 2 * num_kv && page_mask >= 0) {
    // Prefill chunk of a sliding-window layer: MFMA query blocks; the o_proj
    // block quant, if asked for, as its own pass over the finished rows.
    IFR_HIP(ifr::launch_prefill_sliding_mfma_bq(
                static_cast<const int32_t*>(image_dev), static_cast<int>(info[14]), q_i8,
                qi_bias, f_q, k_base, k_scale, v_base, v_scale, output,
                static_cast<int>(num_q), static_cast<int>(num_kv), kv_stride, g,
                static_cast<int>(info[12]), as_stream(stream)),
            "prefill_sliding_mfma_bq");
    if (o_i8)
      IFR_HIP(ifr::launch_bq_block_quant(output, o_i8, o_sa, num_q * head_dim,
                                         static_cast<int>(head_dim), info[5],
                                         as_stream(stream)),
              "bq_block_quant");
    return ok();
  }
  if (info[2] == IFR_PLAN_TOKEN_MERGE && info[14] > 0 && head_dim == 256 &&
      num_q == 2 * num_kv && page_mask < 0) {
    // Prefill chunk of a full-attention layer at head_dim 256 / GQA 2.
    IFR_HIP(ifr::launch_prefill_full_mfma_bq(
                static_cast<const int32_t*>(image_dev), static_cast<int>(info[14]), q_i8,
                qi_bias, f_q, k_base, k_scale, v_base, v_scale, output,
                static_cast<int>(num_q), static_cast<int>(num_kv), kv_stride, g,
                as_stream(stream)),
            "prefill_full_mfma_bq");
    if (o_i8)
      IFR_HIP(ifr::launch_bq_block_quant(output, o_i8, o_sa, num_q * head_dim,
                                         static_cast<int>(head_dim), info[5],
                                         as_stream(stream)),
              "bq_block_quant");
    return ok();
  }
  if (info[2] == IFR_PLAN_TOKEN_MERGE && info[14] > 0 && head_dim == 512 &&
      num_q == 8 * num_kv && page_mask < 0) {
    // Prefill chunk of a full-attention layer at head_dim 512 / GQA 8.
    IFR_HIP(ifr::launch_prefill_wide_mfma_bq(
                static_cast<const int32_t*>(image_dev), static_cast<int>(info[14]), q_i8,
                qi_bias, f_q, k_base, k_scale, v_base, v_scale, output,
                static_cast<int>(num_q), static_cast<int>(num_kv), kv_stride, g,
                as_stream(stream)),
            "prefill_wide_mfma_bq");
    if (o_i8)
      IFR_HIP(ifr::launch_bq_block_quant(output, o_i8, o_sa, num_q * head_dim,
                                         static_cast<int>(head_dim), info[5],
                                         as_stream(stream)),
              "bq_block_quant");
    return ok();
  }
  IFR_HIP(ifr::launch_bq_attention(static_cast<const int32_t*>(image_dev),
                                   static_cast<int>(info[0]), static_cast<int>(info[1]),
                                   static_cast<int>(info[2]), q_i8, qi_bias, f_q, k_base,
                                   k_scale, v_base, v_scale, output,
                                   static_cast<float*>(partials), partial_stride,
                                   static_cast<int>(num_q), static_cast<int>(num_kv),
                                   static_cast<int>(head_dim), kv_stride, g,
                                   as_stream(stream), static_cast<int8_t*>(o_i8), o_sa),
          "bq_attention");
  return ok();
}
}  // namespace

extern "C" {

int32_t ifr_bq_attention(const void* image_dev, const int64_t* info,
                         const void* q_i8, const float* qi_bias, const float* f_q,
                         const void* k_base, const float* k_scale, const void* v_base,
                         const float* v_scale, void* output, void* partials,
                         int64_t partials_bytes, int64_t num_q, int64_t num_kv,
                         int64_t head_dim, int64_t partial_stride, int64_t kv_stride,
                         int64_t page_len, int64_t page_mask, uint64_t stream) {
  return bq_attention(image_dev, info, q_i8, qi_bias, f_q, k_base, k_scale, v_base, v_scale,
                      output, partials, partials_bytes, num_q, num_kv, head_dim,
                      partial_stride, kv_stride, page_len, page_mask, stream, nullptr,
                      nullptr);
}

int32_t ifr_bq_attention_block_quant(const void* image_dev, const int64_t* info,
                                     const void* q_i8, const float* qi_bias,
                                     const float* f_q, const void* k_base,
                                     const float* k_scale, const void* v_base,
                                     const float* v_scale, void* output, void* partials,
                                     int64_t partials_bytes, int64_t num_q, int64_t num_kv,
                                     int64_t head_dim, int64_t partial_stride,
                                     int64_t kv_stride, int64_t page_len, int64_t page_mask,
                                     void* o_i8, float* o_sa, uint64_t stream) {
  if (!o_i8 || !o_sa) return fail(IFR_EINVAL, "null pointer");
  if (!aligned(o_i8, 16) || !aligned(o_sa, 4))
    return fail(IFR_EINVAL, "o_i8 must be 16-byte aligned, o_sa 4-byte aligned");
  return bq_attention(image_dev, info, q_i8, qi_bias, f_q, k_base, k_scale, v_base, v_scale,
                      output, partials, partials_bytes, num_q, num_kv, head_dim,
                      partial_stride, kv_stride, page_len, page_mask, stream, o_i8, o_sa);
}

int64_t ifr_index_scores_bytes(const int64_t* info, int64_t num_index_heads,
                               int64_t block_size) {
  if (check_info(info) != IFR_OK || num_index_heads <= 0 || block_size <= 0) return -1;
  return info[5] * num_index_heads * ifr::index_block_stride(info[13], block_size) * 4;
}

int32_t ifr_lightning_indexer(const void* image_dev, const int64_t* info, const void* index_q,
                              const void* index_k, int32_t* block_idx, float* scores,
                              int64_t scores_bytes, int64_t num_index_heads,
                              int64_t index_head_dim, int64_t block_size, int64_t topk_blocks,
                              int64_t local_blocks, int64_t init_blocks, float scale,
                              int64_t page_len, uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  if (info[11] != 1) return fail(IFR_EINVAL, "the indexer needs a full-attention plan");
  if (num_index_heads != 4 || index_head_dim != 128)
    return fail(IFR_EUNSUPPORTED, "the indexer is compiled for 4 index heads of dim 128");
  if (block_size <= 0 || block_size > (1 << 20))
    return fail(IFR_EINVAL, "block_size must be in [1, 2^20]");
  if (topk_blocks <= 0 || topk_blocks > 32) return fail(IFR_EINVAL, "topk_blocks must be in [1, 32]");
  if (local_blocks < 0 || init_blocks < 0) return fail(IFR_EINVAL, "negative forced blocks");
  if (!image_dev || !index_q || !index_k || !block_idx || !scores)
    return fail(IFR_EINVAL, "null pointer");
  if (!aligned(index_q, 16) || !aligned(index_k, 16) || !aligned(block_idx, 4) ||
      !aligned(scores, 4))
    return fail(IFR_EINVAL, "index_q and index_k must be 16-byte aligned");
  if (!is_pow2(page_len)) return fail(IFR_EINVAL, "page_len must be a power of two");
  st = check_geometry(info, pow2_shift(page_len), page_len - 1, -1);
  if (st) return st;
  const int64_t stride = ifr::index_block_stride(info[13], block_size);
  const int64_t need = info[5] * num_index_heads * stride * 4;
  if (scores_bytes < need)
    return fail(IFR_ESPACE, "scores need %lld bytes", (long long)need);
  IFR_HIP(ifr::launch_lightning_indexer(
              static_cast<const int32_t*>(image_dev), static_cast<int>(info[5]), index_q,
              index_k, block_idx, scores, static_cast<int>(stride),
              static_cast<int>(num_index_heads), static_cast<int>(index_head_dim),
              static_cast<int>(block_size), static_cast<int>(topk_blocks),
              static_cast<int>(local_blocks), static_cast<int>(init_blocks), scale,
              static_cast<int>(info[7]), static_cast<int>(info[8]), as_stream(stream)),
          "lightning_indexer");
  return ok();
}

int32_t ifr_block_sparse_attention(const void* image_dev, const int64_t* info, const void* q,
                                   const void* k_base, const void* v_base,
                                   const int32_t* block_idx, void* output, int64_t num_q,
                                   int64_t num_kv, int64_t head_dim, int64_t kv_stride,
                                   int64_t block_size, int64_t topk_blocks, int64_t page_len,
                                   uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  if (info[11] != 1) return fail(IFR_EINVAL, "sparse attention needs a full-attention plan");
  if (head_dim != 128 || num_kv <= 0 || num_q != 16 * num_kv || num_q > 1024)
    return fail(IFR_EUNSUPPORTED, "sparse attention is compiled for head_dim 128, gqa 16");
  if (kv_stride < num_kv * head_dim || kv_stride % 8 != 0)
    return fail(IFR_EINVAL, "kv_stride must cover num_kv heads and keep 16-byte rows");
  if (block_size <= 0 || block_size > (1 << 20) || block_size % 16 != 0)
    return fail(IFR_EINVAL, "block_size must be a multiple of 16 in [16, 2^20]");
  if (page_len < 16) return fail(IFR_EINVAL, "page_len must be at least 16");
  if (topk_blocks <= 0 || topk_blocks > (1 << 16)) return fail(IFR_EINVAL, "bad topk_blocks");
  if (!image_dev || !q || !k_base || !v_base || !block_idx || !output)
    return fail(IFR_EINVAL, "null pointer");
  if (!aligned(q, 16) || !aligned(k_base, 16) || !aligned(v_base, 16) || !aligned(output, 4) ||
      !aligned(block_idx, 4))
    return fail(IFR_EINVAL, "q, k and v must be 16-byte aligned");
  if (!is_pow2(page_len)) return fail(IFR_EINVAL, "page_len must be a power of two");
  st = check_geometry(info, pow2_shift(page_len), page_len - 1, -1);
  if (st) return st;
  IFR_HIP(ifr::launch_block_sparse_attention(
              static_cast<const int32_t*>(image_dev), static_cast<int>(info[5]), q, k_base,
              v_base, block_idx, output, kv_stride, static_cast<int>(num_q),
              static_cast<int>(num_kv), static_cast<int>(block_size),
              static_cast<int>(topk_blocks), static_cast<int>(info[7]),
              static_cast<int>(info[8]), as_stream(stream)),
          "block_sparse_attention");
  return ok();
}

}  // extern "C"

namespace {
// The decode route's (kv head, block slot) units and worker count:
// min(topk, causal blocks) slots per head, min(cap, units) workers.
void bq_sparse_decode_shape(const int64_t* info, int64_t num_kv, int64_t block_size,
                            int64_t topk, int64_t cap, int64_t* slots, int64_t* workers) {
  *slots = std::min<int64_t>(topk, info[13] / block_size + 1);
  *workers = std::min<int64_t>(cap, num_kv * *slots);
}
}  // namespace

extern "C" {

int64_t ifr_bq_sparse_partials_bytes(const int64_t* info, int64_t num_q, int64_t num_kv,
                                     int64_t head_dim, int64_t block_size,
                                     int64_t topk_blocks, int64_t cap) {
  if (check_info(info) != IFR_OK || num_kv <= 0 || block_size <= 0 || topk_blocks <= 0 ||
      cap < 1)
    return -1;
  if (info[5] != 1) return 0;
  int64_t slots, workers;
  bq_sparse_decode_shape(info, num_kv, block_size, topk_blocks, cap, &slots, &workers);
  return workers * ifr_flash_partial_stride(num_q, head_dim) * 4;
}

int32_t ifr_bq_block_sparse_attention(
    const void* image_dev, const int64_t* info, const void* q_i8, const float* qi_bias,
    const float* f_q, const void* k_base, const float* k_scale, const void* v_base,
    const float* v_scale, const int32_t* block_idx, void* output, void* partials,
    int64_t partials_bytes, int64_t num_q, int64_t num_kv, int64_t head_dim,
    int64_t kv_stride, int64_t block_size, int64_t topk_blocks, int64_t page_len,
    int64_t cap, uint64_t stream) {
  int32_t st = check_info(info);
  if (st) return st;
  if (info[11] != 1) return fail(IFR_EINVAL, "sparse attention needs a full-attention plan");
  if (head_dim != 128 || num_kv <= 0 || num_q != 16 * num_kv || num_q > 1024)
    return fail(IFR_EUNSUPPORTED, "bq sparse attention is compiled for head_dim 128, gqa 16");
  if (kv_stride < num_kv * head_dim || kv_stride % 16 != 0)
    return fail(IFR_EINVAL, "kv_stride must cover num_kv heads in 16-byte rows");
  if (block_size <= 0 || block_size > (1 << 20) || block_size % 16 != 0)
    return fail(IFR_EINVAL, "block_size must be a multiple of 16 in [16, 2^20]");
  if (page_len < 16) return fail(IFR_EINVAL, "page_len must be at least 16");
  if (topk_blocks <= 0 || topk_blocks > (1 << 16)) return fail(IFR_EINVAL, "bad topk_blocks");
  if (cap < 1 || cap > (1 << 20)) return fail(IFR_EINVAL, "cap must be in [1, 2^20]");
  if (!image_dev || !q_i8 || !qi_bias || !f_q || !k_base || !k_scale || !v_base || !v_scale ||
      !block_idx || !output)
    return fail(IFR_EINVAL, "null pointer");
  if (!aligned(q_i8, 16) || !aligned(k_base, 16) || !aligned(v_base, 16) ||
      !aligned(output, 8) || !aligned(block_idx, 4))
    return fail(IFR_EINVAL, "q, k and v codes must be 16-byte aligned");
  if (!is_pow2(page_len)) return fail(IFR_EINVAL, "page_len must be a power of two");
  st = check_geometry(info, pow2_shift(page_len), page_len - 1, -1);
  if (st) return st;
  const int64_t ps = ifr_flash_partial_stride(num_q, head_dim);
  int64_t slots = 0, workers = 1;
  if (info[5] == 1) {
    bq_sparse_decode_shape(info, num_kv, block_size, topk_blocks, cap, &slots, &workers);
    if (!partials || !aligned(partials, 16) || partials_bytes < workers * ps * 4)
      return fail(IFR_ESPACE, "partials need %lld bytes, 16-byte aligned",
                  (long long)(workers * ps * 4));
  }
  IFR_HIP(ifr::launch_bq_block_sparse_attention(
              static_cast<const int32_t*>(image_dev), static_cast<int>(info[5]), q_i8,
              qi_bias, f_q, k_base, k_scale, v_base, v_scale, block_idx, output,
              static_cast<float*>(partials), ps, kv_stride, static_cast<int>(num_q),
              static_cast<int>(num_kv), static_cast<int>(block_size),
              static_cast<int>(topk_blocks), static_cast<int>(slots),
              static_cast<int>(workers), static_cast<int>(info[7]),
              static_cast<int>(info[8]), as_stream(stream)),
          "bq_block_sparse_attention");
  return ok();
}

int64_t ifr_gemm_cols_workspace_bytes(int64_t rows, int64_t cols, int64_t seq_len) {
  if (rows <= 0 || cols <= 0 || seq_len < 0) return -1;
  return ifr::gemm_cols_workspace_bytes(seq_len, rows, cols);
}

int32_t ifr_dispatch_gemm_cols(const void* x, const void* weight, void* output, int64_t rows,
                               int64_t cols, int64_t seq_len, void* workspace,
                               int64_t workspace_bytes, uint64_t stream) {
  if (rows <= 0 || rows % 16 != 0 || rows > (int64_t{1} << 24))
    return fail(IFR_EINVAL, "rows must be a positive multiple of 16");
  if (cols <= 0 || cols % 128 != 0 || cols > (int64_t{1} << 24))
    return fail(IFR_EINVAL, "cols must be a positive multiple of 128");
  if (seq_len < 0 || seq_len > (int64_t{1} << 21))
    return fail(IFR_EINVAL, "seq_len must be in [0, 2^21]");
  if (seq_len == 0) return ok();
  if (!x || !weight || !output) return fail(IFR_EINVAL, "null pointer");
  if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(output, 16))
    return fail(IFR_EINVAL, "x, weight and output must be 16-byte aligned");
  const int64_t need = ifr::gemm_cols_workspace_bytes(seq_len, rows, cols);
  if (need > 0 && (!workspace || workspace_bytes < need || !aligned(workspace, 16)))
    return fail(IFR_ESPACE, "workspace needs %lld bytes, 16-byte aligned", (long long)need);
  IFR_HIP(ifr::launch_gemm_cols(x, weight, output, static_cast<float*>(workspace), seq_len,
                                rows, cols, as_stream(stream)),
          "gemm_cols");
  return ok();
}

int32_t ifr_bq_block_quant(const void* src, void* x_i8, float* x_sa, int64_t cols,
                           int64_t block, int64_t seq_len, uint64_t stream) {
  if (seq_len < 0) return fail(IFR_EINVAL, "seq_len must be >= 0");
  if (block <= 0 || block % 16 != 0 || block > (1 << 20))
    return fail(IFR_EINVAL, "block must be a positive multiple of 16 (the f32 SIMD width)");
  if (cols <= 0 || cols % block != 0) return fail(IFR_EINVAL, "cols must be block-aligned");
  if (seq_len == 0) return ok();
  if (!src || !x_i8 || !x_sa) return fail(IFR_EINVAL, "null pointer");
  if (seq_len > (int64_t{1} << 31) || seq_len * (cols / block) > (int64_t{1} << 32))
    return fail(IFR_EINVAL, "too many blocks for one launch");
  if (!aligned(src, 2) || !aligned(x_sa, 4))
    return fail(IFR_EINVAL, "src must be 2-byte aligned, x_sa 4-byte aligned");
  IFR_HIP(ifr::launch_bq_block_quant(src, x_i8, x_sa, cols, static_cast<int>(block),
                                     seq_len, as_stream(stream)),
          "bq_block_quant");
  return ok();
}

}  // extern "C"
