// Decode planning on the host (BatchDecodeWithPagedKVCacheWrapper.plan,
// src/models/llama.py:119-147): the shared-item and split partitions of
// pagedattn_decode_plan, the device-side partition set-up of
// pagedattn_decode_plan_device, and the plan queries.  Plain host C++ (no
// device code), so the planners can also be built and driven on a machine
// without a GPU, under the address and undefined-behaviour sanitizers.
#include <algorithm>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <queue>
#include <vector>

#include "plan_internal.h"

namespace pa {

// Waves the planner spreads the work over, per CU (one wave per SIMD keeps
// enough loads in flight with two register stages);
// PAGEDATTN_DECODE_WAVES_PER_CU overrides it.
static int decode_waves_per_cu() {
  if (const char* env = std::getenv("PAGEDATTN_DECODE_WAVES_PER_CU")) {
    const int v = std::atoi(env);
    if (v > 0) return v;
  }
  return 4;
}

// Page-equivalents charged per item by the balanced split (the cost of an
// item switch, measured: 6 gave the fastest TinyLlama B=256 step, 60.5 us
// against 63.7 us at 0); PAGEDATTN_DECODE_ITEM_COST overrides it.
static int decode_item_cost() {
  if (const char* env = std::getenv("PAGEDATTN_DECODE_ITEM_COST")) {
    const int v = std::atoi(env);
    if (v >= 0 && v <= 1024) return v;
  }
  return 6;
}

// Waves (KV heads) per head group: the largest of 4, 2, 1 that divides Hkv,
// so a page's K and V blocks are each read as one run of hg * 16 rows;
// PAGEDATTN_DECODE_HEAD_GROUP (1, 2 or 4) caps it.
static int decode_head_group(int hkv) {
  int cap = 4;
  if (const char* env = std::getenv("PAGEDATTN_DECODE_HEAD_GROUP")) {
    const int v = std::atoi(env);
    if (v == 1 || v == 2 || v == 4) cap = v;
  }
  int hg = 1;
  while (hg * 2 <= cap && hkv % (hg * 2) == 0) hg *= 2;
  return hg;
}

// Shared-item plans (decode_shared_kernel): PAGEDATTN_DECODE_SHARED=0 turns
// them off, =1 takes one whenever the items fit a workgroup's table; by
// default one is taken when its busiest CU holds at most
// PAGEDATTN_DECODE_SHARED_SLACK_KB KiB (default 96: what one CU streams in
// the 4-5 us that the split's merge launch costs) plus
// PAGEDATTN_DECODE_SHARED_SLACK_PCT percent of the mean (default 4: the
// split's partials and per-item restarts) more K/V than the mean.  Measured
// on the 70B-shaped e4m3 batch (D = 128, busiest CU 3.1 % over the mean):
// 214 us shared against 225 us split.
static int decode_shared_mode() {
  if (const char* env = std::getenv("PAGEDATTN_DECODE_SHARED")) {
    const int v = std::atoi(env);
    if (v == 0 || v == 1) return v;
  }
  return -1;
}
// Shared plans give wave w of a workgroup the chunks w, w + 4, w + 8, ...,
// so the output bits do not depend on timing (as FlashInfer's decode);
// PAGEDATTN_DECODE_DETERMINISTIC=0 lets the waves claim chunks in arrival
// order instead, which balances the waves of a workgroup but makes the last
// bits of the output vary from run to run.
static bool decode_deterministic() {
  const char* env = std::getenv("PAGEDATTN_DECODE_DETERMINISTIC");
  return !(env && std::atoi(env) == 0);
}

// XCDs of the device (MI355X: 8; the hardware deals workgroup w to XCD
// w mod 8).  PAGEDATTN_DECODE_XCD=0 lets the shared planner place a
// sequence's KV heads on any XCD (see plan_shared).
constexpr int kXcds = 8;
static bool shared_xcd_affine() {
  const char* env = std::getenv("PAGEDATTN_DECODE_XCD");
  return !(env && std::atoi(env) == 0);
}

static int64_t decode_shared_slack_bytes() {
  if (const char* env = std::getenv("PAGEDATTN_DECODE_SHARED_SLACK_KB")) {
    const int v = std::atoi(env);
    if (v >= 0) return (int64_t)v << 10;
  }
  return (int64_t)96 << 10;
}
static int decode_shared_slack_pct() {
  if (const char* env = std::getenv("PAGEDATTN_DECODE_SHARED_SLACK_PCT")) {
    const int v = std::atoi(env);
    if (v >= 0 && v <= 100) return v;
  }
  return 4;
}

// Shared-item partition: whole (sequence, KV head) items, longest first onto
// the least-loaded of `cus` workgroups, counted in chunks of
// kSharedStagePairs page pairs (the unit the kernel's waves take).  Then a
// bounded pass of moves and swaps lowers the busiest workgroups towards
// 4 ceil(mean / 4) chunks where the item sizes allow: the four waves take
// chunks w, w + 4, ..., so a workgroup of N chunks runs ceil(N / 4) rounds,
// and one chunk over a multiple of four costs a whole round.  (On the
// 70B-shaped e4m3 batch the busiest of 256 workgroups goes from 606 to about
// 590 chunks, 213 -> 210 us.)
// Returns false (and leaves the outputs unspecified) when some workgroup
// would hold more than kSharedMaxItems items or, unless forced, when the
// busiest workgroup exceeds the mean by more than the slack.
static bool plan_shared(const std::vector<int32_t>& npages, const int32_t* kv_indptr_host,
                        const int32_t* kv_last_page_len_host, int hkv, int d, int cus,
                        bool forced, std::vector<SharedItem>* items, int* n_wg_out) {
  const int batch = (int)npages.size();
  const int64_t n_all = (int64_t)batch * hkv;
  if (n_all == 0) return false;
  const int chunk_pages = 2 * kSharedStagePairs;
  auto chunks_of = [&](int32_t id) {
    const int32_t np = npages[id / hkv];
    return std::max<int32_t>(1, ((np + 1) / 2 + chunk_pages / 2 - 1) / (chunk_pages / 2));
  };
  std::vector<int32_t> ck((size_t)n_all);  // chunks of each item
  for (int64_t i = 0; i < n_all; ++i) ck[(size_t)i] = chunks_of((int32_t)i);
  // sequence-major item ids b hkv + h; longest first, ties in id order.  The
  // heads of a sequence share its key, so the sequences are sorted and each
  // expanded into its heads in order.
  std::vector<int32_t> seqs((size_t)batch);
  for (int b = 0; b < batch; ++b) seqs[(size_t)b] = b;
  std::stable_sort(seqs.begin(), seqs.end(),
                   [&](int32_t a, int32_t c) { return npages[a] > npages[c]; });
  std::vector<int32_t> order;
  order.reserve((size_t)n_all);
  for (int32_t b : seqs)
    for (int h = 0; h < hkv; ++h) order.push_back(b * hkv + h);
  const int n_wg = (int)std::min<int64_t>(std::max(cus, 1), n_all);
  // One partition: longest first (per XCD with `affine`), then the
  // refinement below.  Returns the chunks of its busiest workgroup.
  struct Part {
    std::vector<std::vector<int32_t>> per;
    std::vector<int64_t> load;
  };
  auto partition = [&](bool affine, Part* out) -> int64_t {
    std::vector<std::vector<int32_t>> per(n_wg);
    for (auto& list : per) list.reserve(kSharedMaxItems + 1);
    std::vector<int64_t> load(n_wg, 0);
    int64_t total = 0;
    // longest first onto the least-loaded workgroup among `wgs`
    auto lpt = [&](const std::vector<int32_t>& ids, const std::vector<int>& wgs) {
      std::priority_queue<std::pair<int64_t, int>, std::vector<std::pair<int64_t, int>>,
                          std::greater<std::pair<int64_t, int>>> heap;
      for (int w : wgs) heap.push({load[w], w});
      for (int32_t id : ids) {
        auto top = heap.top();
        heap.pop();
        per[top.second].push_back(id);
        top.first += ck[id];
        total += ck[id];
        load[top.second] = top.first;
        heap.push(top);
      }
    };
    if (affine) {
      // Workgroup w runs on XCD w mod 8.  The KV heads of one sequence share
      // its pages' scale line (e4m3 pools: [P, 2, Hkv] fp32, all heads of a
      // page in one 64-byte block), so the items of a sequence go to the
      // workgroups of one XCD, whose L2 then fetches each line once: whole
      // sequences longest first onto the least-loaded XCD, then each XCD's
      // items longest first onto its workgroups.
      std::vector<std::vector<int32_t>> xcd_ids(kXcds);
      std::vector<int64_t> xcd_load(kXcds, 0);
      for (size_t k = 0; k < order.size(); k += (size_t)hkv) {
        // `order` keeps a sequence's heads together (stable sort, ids b hkv + h)
        const int b = order[k] / hkv;
        int x = 0;
        for (int y = 1; y < kXcds; ++y)
          if (xcd_load[y] < xcd_load[x]) x = y;
        for (int h = 0; h < hkv; ++h) xcd_ids[x].push_back(b * hkv + h);
        xcd_load[x] += (int64_t)hkv * ck[(size_t)b * hkv];
      }
      for (int x = 0; x < kXcds; ++x) {
        std::vector<int> wgs;
        for (int w = x; w < n_wg; w += kXcds) wgs.push_back(w);
        lpt(xcd_ids[x], wgs);
      }
    } else {
      std::vector<int> wgs(n_wg);
      for (int w = 0; w < n_wg; ++w) wgs[w] = w;
      lpt(order, wgs);
    }
    // refinement: the busiest workgroup gives an item to another, or swaps an
    // item for a smaller one of another, whenever both end below its load
    // (partners tried from the least loaded up).  Every step lowers the
    // busiest load or the number of workgroups at it; it stops at the round
    // bound 4 ceil(mean / 4) (below it a workgroup's rounds cannot drop), when
    // no step helps, or after n_wg steps.  The partner order is kept sorted
    // by re-inserting the two workgroups a step changes.
    const int64_t lower = (total + n_wg - 1) / n_wg;
    const int64_t round_bound = 4 * ((lower + 3) / 4);
    auto lighter = [&](int x, int y) { return load[x] < load[y] || (load[x] == load[y] && x < y); };
    std::vector<int> by_load(n_wg);
    for (int v = 0; v < n_wg; ++v) by_load[v] = v;
    std::sort(by_load.begin(), by_load.end(), lighter);
    auto resort = [&](int x) {
      by_load.erase(std::find(by_load.begin(), by_load.end(), x));
      by_load.insert(std::lower_bound(by_load.begin(), by_load.end(), x, lighter), x);
    };
    auto by_size = [&](int32_t x, int32_t y) {
      return ck[x] > ck[y] || (ck[x] == ck[y] && x < y);
    };
    for (int iter = 0; iter < n_wg; ++iter) {
      const int w = by_load.back();
      const int64_t top = load[w];
      if (top <= round_bound) break;
      bool done = false;
      int partner = -1;
      // the busiest workgroup's items, largest first (every list is kept in
      // non-increasing chunk order: longest first from the LPT pass, by_size
      // after each step)
      for (size_t i = 0; i < per[w].size() && !done; ++i) {
        const int64_t a = ck[per[w][i]];
        for (int v : by_load) {
          if (v == w) continue;
          if (load[v] + 1 >= top) break;
          if ((int)per[v].size() < kSharedMaxItems && load[v] + a < top) {
            per[v].push_back(per[w][i]);
            per[w].erase(per[w].begin() + (long)i);
            load[v] += a;
            load[w] -= a;
            partner = v;
            done = true;
            break;
          }
          // a swap for a smaller item b of v needs a - b < top - load[v] (the
          // busiest side then drops by a - b > 0): the first item of v below a
          // is the largest such b, so if it does not fit, none does
          size_t j = 0;
          while (j < per[v].size() && ck[per[v][j]] >= a) ++j;
          if (j < per[v].size() && load[v] - ck[per[v][j]] + a < top) {
            const int64_t b = ck[per[v][j]];
            std::swap(per[w][i], per[v][j]);
            load[w] += b - a;
            load[v] += a - b;
            partner = v;
            done = true;
            break;
          }
        }
      }
      if (!done) break;
      std::sort(per[w].begin(), per[w].end(), by_size);
      std::sort(per[partner].begin(), per[partner].end(), by_size);
      resort(w);
      resort(partner);
    }
    out->per = std::move(per);
    out->load = std::move(load);
    int64_t mx = 0;
    for (int64_t l : out->load) mx = std::max(mx, l);
    return mx;
  };
  // The XCD-affine partition for 8 or more KV heads (a page's scales of all
  // heads fill its 64-byte block), unless it costs the busiest workgroup a
  // round of chunks (rounds of four: one per wave) over the unconstrained
  // one.  On the 70B-shaped e4m3 batch it takes the step's fetched bytes
  // from 1.032 to 1.003 times the algorithmic bytes, at the same speed; on
  // the 4-head TinyLlama batch (no scales) it measured 0.1 us slower.
  // (An affine partition at the round bound 4 ceil(mean / 4) cannot be
  // beaten, so the unconstrained one is then not built.)
  Part part;
  const bool can_affine = shared_xcd_affine() && n_wg % kXcds == 0 && n_wg >= kXcds && hkv >= 8;
  bool have = false;
  int64_t top_aff = 0;
  if (can_affine) {
    top_aff = partition(true, &part);
    bool fits = true;
    for (const auto& list : part.per) fits = fits && (int)list.size() <= kSharedMaxItems;
    int64_t sum = 0;
    for (int64_t l : part.load) sum += l;
    const int64_t bound = 4 * (((sum + n_wg - 1) / n_wg + 3) / 4);
    have = fits && top_aff <= bound;
    if (fits && !have) {
      Part free_part;
      const int64_t top_free = partition(false, &free_part);
      have = (top_aff + 3) / 4 <= (top_free + 3) / 4;
      if (!have) part = std::move(free_part);
      have = true;
    }
  }
  if (!have) partition(false, &part);
  std::vector<std::vector<int32_t>>& per = part.per;
  std::vector<int64_t>& load = part.load;
  // the kernel walks a workgroup's items in list order: longest first
  for (auto& list : per)
    std::stable_sort(list.begin(), list.end(), [&](int32_t a, int32_t c) {
      return npages[a / hkv] > npages[c / hkv] || (npages[a / hkv] == npages[c / hkv] && a < c);
    });
  // page loads for the slack rule
  for (int w = 0; w < n_wg; ++w) {
    load[w] = 0;
    for (int32_t id : per[w]) load[w] += std::max(1, npages[id / hkv]);
  }
  int64_t sum = 0, mx = 0;
  for (int w = 0; w < n_wg; ++w) {
    if ((int)per[w].size() > kSharedMaxItems) return false;
    sum += load[w];
    mx = std::max(mx, load[w]);
  }
  // K and V of one page of one KV head, counted at 16 bits per element
  const int64_t page_bytes = (int64_t)kPage * d * 2 * 2;
  // busiest - mean > slack + pct% of the mean, scaled by n_wg
  if (!forced && (mx * n_wg - sum) * page_bytes * 100 >
                     decode_shared_slack_bytes() * n_wg * 100 +
                         sum * page_bytes * decode_shared_slack_pct())
    return false;
  // fixed stride: workgroup w's items at [w kSharedMaxItems, ...), padded
  items->assign((size_t)n_wg * kSharedMaxItems, SharedItem{-1, 0, 0, 0, -1, 0, kPage, 0});
  for (int w = 0; w < n_wg; ++w) {
    int32_t chunk = 0;
    const int32_t cnt = (int32_t)per[w].size();
    SharedItem* at = items->data() + (size_t)w * kSharedMaxItems;
    for (int k = 0; k < kSharedMaxItems; ++k) at[k].wg_items = cnt;
    for (int k = 0; k < cnt; ++k) {
      const int32_t id = per[w][k];
      const int32_t np = npages[id / hkv];
      const int32_t nc = std::max<int32_t>(1, ((np + 1) / 2 + chunk_pages / 2 - 1) / (chunk_pages / 2));
      const int b = id / hkv;
      at[k] = SharedItem{b, id % hkv, chunk, nc, kv_indptr_host[b], np,
                         np > 0 ? kv_last_page_len_host[b] : kPage, cnt};
      chunk += nc;
    }
  }
  *n_wg_out = n_wg;
  return true;
}

// The device-side partition of a decode plan (pagedattn_decode_plan_device
// and pagedattn_decode_run_noalloc): shares of the (sequence, head group,
// page) stream for cus x waves-per-CU / hg head groups, split partials at
// `partials` (256-byte aligned, `bytes` long).
int setup_device_plan(const char* who, pagedattn_plan* plan, int32_t batch_size,
                             int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t page_size, int cus, char* partials, size_t bytes) {
  plan->mode = kPlanNone;
  if (batch_size < 0)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: batch_size %d < 0", who, batch_size);
  int rc = validate_heads(who, num_qo_heads, num_kv_heads, head_dim, page_size);
  if (rc) return rc;
  const int hg = decode_head_group(num_kv_heads);
  const int g = num_qo_heads / num_kv_heads;
  const int n_groups = std::max(1, cus * decode_waves_per_cu() / hg);
  const int n_slots = 2 * n_groups * hg;
  const size_t off_pl = ws_align(sizeof(float) * (size_t)n_slots * g * head_dim);
  const size_t end = ws_align(off_pl + sizeof(float) * (size_t)n_slots * g);
  if (end > bytes)
    return set_error(PAGEDATTN_ERR_WORKSPACE, "%s: needs %zu bytes of split partials, %zu "
                     "available", who, end, bytes);
  plan->implicit = true;
  plan->shared = false;
  plan->dev_table = false;
  plan->item_cost = decode_item_cost();
  plan->batch_size = batch_size;
  plan->hq = num_qo_heads;
  plan->hkv = num_kv_heads;
  plan->d = head_dim;
  plan->page_size = page_size;
  plan->n_items = n_groups;
  plan->hg_shift = hg == 4 ? 2 : hg == 2 ? 1 : 0;
  plan->n_merge = 0;
  plan->n_slots = n_slots;
  plan->split_pages = 0;
  plan->items_dev = nullptr;
  plan->wave_ptr_dev = nullptr;
  plan->merge_dev = nullptr;
  plan->partial_o = reinterpret_cast<float*>(partials);
  plan->partial_lse = reinterpret_cast<float*>(partials + off_pl);
  plan->total_pages = -1;
  plan->max_pages = -1;
  plan->mode = kPlanDecode;
  return PAGEDATTN_OK;
}

}  // namespace pa

using namespace pa;

extern "C" {

int pagedattn_decode_plan(pagedattn_plan* plan, const int32_t* kv_indptr_host,
                          const int32_t* kv_last_page_len_host,
                          int32_t batch_size, int32_t num_qo_heads,
                          int32_t num_kv_heads, int32_t head_dim,
                          int32_t page_size, int32_t split_pages,
                          void* workspace, size_t workspace_bytes,
                          void* stream) {
  const char* who = "decode_plan";
  if (!plan) return set_error(PAGEDATTN_ERR_INVALID, "%s: null plan", who);
  plan->mode = kPlanNone;
  if (batch_size < 0)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: batch_size %d < 0", who,
                     batch_size);
  int rc = validate_heads(who, num_qo_heads, num_kv_heads, head_dim, page_size);
  if (rc) return rc;
  if (!workspace || ((uintptr_t)workspace & (kWsAlign - 1)))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "%s: workspace must be a 256-byte aligned device buffer",
                     who);
  std::vector<int32_t> npages, kv_len;
  rc = validate_paged_metadata(who, kv_indptr_host, kv_last_page_len_host,
                               batch_size, page_size, &npages, &kv_len);
  if (rc) return rc;
  const int hkv = num_kv_heads;
  const int g = num_qo_heads / num_kv_heads;

  int64_t total = 0;
  int maxp = 0;
  for (int b = 0; b < batch_size; ++b) {
    total += npages[b];
    maxp = std::max(maxp, npages[b]);
  }
  int cus = device_cu_count();
  if (cus <= 0) cus = 256;
  plan->shared = false;
  plan->dev_table = false;

  if (split_pages == 0 && decode_shared_mode() != 0) {
    std::vector<SharedItem> sitems;
    int n_wg = 0;
    if (plan_shared(npages, kv_indptr_host, kv_last_page_len_host, hkv, head_dim, cus,
                    decode_shared_mode() == 1, &sitems, &n_wg)) {
      const size_t off_items = kWsHeader;
      const size_t end = ws_align(off_items + sizeof(SharedItem) * sitems.size());
      const size_t host_bytes = end - kWsHeader;
      plan->host.assign(host_bytes / sizeof(int32_t), 0);
      char* hb = reinterpret_cast<char*>(plan->host.data());
      std::memcpy(hb, sitems.data(), sizeof(SharedItem) * sitems.size());
      plan->workspace = workspace;
      plan->workspace_bytes = workspace_bytes;
      rc = upload_plan(plan, who, host_bytes, end, stream);
      if (rc) return rc;
      char* ws = static_cast<char*>(workspace);
      plan->implicit = false;
      plan->shared = true;
      plan->deterministic = decode_deterministic();
      plan->batch_size = batch_size;
      plan->hq = num_qo_heads;
      plan->hkv = num_kv_heads;
      plan->d = head_dim;
      plan->page_size = page_size;
      plan->n_items = n_wg;
      plan->hg_shift = 0;
      plan->n_merge = 0;
      plan->n_slots = 0;
      plan->split_pages = split_pages;
      plan->items_dev = ws + off_items;
      plan->wave_ptr_dev = nullptr;
      plan->merge_dev = nullptr;
      plan->partial_o = nullptr;
      plan->partial_lse = nullptr;
      plan->total_pages = total;
      plan->max_pages = maxp;
      plan->mode = kPlanDecode;
      return PAGEDATTN_OK;
    }
  }

  // work is planned per head group: hg KV heads walked together by hg waves
  const int hg = decode_head_group(hkv);
  const int hg_shift = hg == 4 ? 2 : hg == 2 ? 1 : 0;
  const int ngrp = hkv / hg;  // head groups per sequence
  const int64_t groups_max =
      std::max<int64_t>(1, (int64_t)cus * decode_waves_per_cu() / hg);

  // items, grouped per head group
  std::vector<DecodeItem> items;
  std::vector<int32_t> wave_ptr(1, 0);
  std::vector<int32_t> pieces((size_t)batch_size * ngrp, 0);
  auto make = [hg](int b, int hgrp, int lo, int hi) {
    return DecodeItem{b, hgrp * hg, lo, hi, -1, -1, 0, 0};
  };
  if (split_pages != 0) {
    // fixed chunks (split_pages > 0) or whole sequences (< 0), assigned
    // longest-first onto the least-loaded head group
    const int64_t chunk = split_pages > 0 ? ((int64_t)split_pages + 7) / 8 * 8 : INT32_MAX;
    // the item count first: the work list must fit the workspace before
    // anything is built
    int64_t n_all = 0;
    for (int b = 0; b < batch_size; ++b)
      n_all += ngrp * std::max<int64_t>(1, ((int64_t)npages[b] + chunk - 1) / chunk);
    if ((int64_t)sizeof(DecodeItem) * n_all > (int64_t)workspace_bytes)
      return set_error(PAGEDATTN_ERR_WORKSPACE,
                       "%s: %lld work items do not fit the %zu-byte workspace", who,
                       (long long)n_all, workspace_bytes);
    std::vector<DecodeItem> all;
    all.reserve((size_t)n_all);
    for (int b = 0; b < batch_size; ++b)
      for (int hgrp = 0; hgrp < ngrp; ++hgrp) {
        if (npages[b] == 0) {
          all.push_back(make(b, hgrp, 0, 0));
          pieces[(size_t)b * ngrp + hgrp]++;
          continue;
        }
        for (int lo = 0; lo < npages[b]; lo = npages[b] - lo > chunk ? lo + chunk : npages[b]) {
          all.push_back(make(b, hgrp, lo, (int)std::min<int64_t>(npages[b], (int64_t)lo + chunk)));
          pieces[(size_t)b * ngrp + hgrp]++;
        }
      }
    std::stable_sort(all.begin(), all.end(), [](const DecodeItem& a, const DecodeItem& c) {
      return a.page_hi - a.page_lo > c.page_hi - c.page_lo;
    });
    const int64_t nw = std::min<int64_t>(groups_max, std::max<size_t>(1, all.size()));
    std::vector<std::vector<int>> per_group(nw);
    std::priority_queue<std::pair<int64_t, int64_t>,
                        std::vector<std::pair<int64_t, int64_t>>,
                        std::greater<std::pair<int64_t, int64_t>>> heap;
    for (int64_t w = 0; w < nw; ++w) heap.push({0, w});
    for (size_t i = 0; i < all.size(); ++i) {
      auto top = heap.top();
      heap.pop();
      per_group[top.second].push_back((int)i);
      top.first += std::max(1, all[i].page_hi - all[i].page_lo);
      heap.push(top);
    }
    for (auto& lst : per_group) {
      for (int i : lst) items.push_back(all[i]);
      wave_ptr.push_back((int32_t)items.size());
    }
  } else {
    // balanced: the (sequence, head group, page) stream cut into equal
    // shares.  A share is counted in pages plus `cost` page-equivalents per
    // item it holds, since every item start waits for a fresh round trip of
    // loads: a share of several short pieces gets fewer pages and the groups
    // finish together.  Shares are contiguous, so only a group's first and
    // last items can be pieces of cut sequences.
    const int64_t cost = decode_item_cost();
    const int64_t est_items = (int64_t)batch_size * ngrp + groups_max;
    int64_t target = (total * ngrp + cost * est_items + groups_max - 1) / groups_max;
    target = std::max<int64_t>(4 + cost, (target + 1) / 2 * 2);
    for (;;) {
      items.clear();
      wave_ptr.assign(1, 0);
      std::fill(pieces.begin(), pieces.end(), 0);
      int64_t fill = 0;
      for (int b = 0; b < batch_size; ++b)
        for (int hgrp = 0; hgrp < ngrp; ++hgrp) {
          if (npages[b] == 0) {
            items.push_back(make(b, hgrp, 0, 0));
            pieces[(size_t)b * ngrp + hgrp]++;
            continue;
          }
          int lo = 0;
          while (lo < npages[b]) {
            if (fill > 0 && fill + cost >= target) {
              wave_ptr.push_back((int32_t)items.size());
              fill = 0;
            }
            const int take = (int)std::min<int64_t>(npages[b] - lo, target - fill - cost);
            items.push_back(make(b, hgrp, lo, lo + take));
            pieces[(size_t)b * ngrp + hgrp]++;
            lo += take;
            fill += take + cost;
            if (fill >= target) {
              wave_ptr.push_back((int32_t)items.size());
              fill = 0;
            }
          }
        }
      if (wave_ptr.back() != (int32_t)items.size())
        wave_ptr.push_back((int32_t)items.size());
      // the item charge can overshoot the estimate: never more shares than
      // head groups the launch keeps resident
      if ((int64_t)wave_ptr.size() - 1 <= groups_max || cost == 0) break;
      target += 2;
    }
  }

  // Partial slots and merge groups for (sequence, head group) pairs cut in
  // pieces: piece k of head h0 + i writes slot base + k * hg + i, and the
  // merge of (b, h0 + i) reads slots base + i + k * hg.
  std::vector<MergeItem> merges;
  std::vector<int32_t> first_merge((size_t)batch_size * ngrp, -1);
  std::vector<int32_t> base_slot((size_t)batch_size * ngrp, -1);
  int n_slots = 0;
  for (int b = 0; b < batch_size; ++b)
    for (int hgrp = 0; hgrp < ngrp; ++hgrp) {
      const int np = pieces[(size_t)b * ngrp + hgrp];
      if (np > 1) {
        first_merge[(size_t)b * ngrp + hgrp] = (int)merges.size();
        base_slot[(size_t)b * ngrp + hgrp] = n_slots;
        for (int i = 0; i < hg; ++i)
          merges.push_back(MergeItem{b, hgrp * hg + i, n_slots + i, np, hg});
        n_slots += np * hg;
      }
    }
  {
    std::vector<int32_t> next((size_t)batch_size * ngrp, 0);
    for (auto& it : items) {
      const size_t key = (size_t)it.b * ngrp + it.h / hg;
      if (first_merge[key] >= 0) {
        it.merge = first_merge[key];
        it.slot = base_slot[key] + hg * next[key]++;
      }
    }
  }

  const int n_items = (int)items.size();
  const int n_waves = (int)wave_ptr.size() - 1;
  const size_t n_merge = merges.size();
  const size_t off_items = kWsHeader;
  const size_t off_wave = ws_align(off_items + sizeof(DecodeItem) * n_items);
  const size_t off_merge = ws_align(off_wave + sizeof(int32_t) * (n_waves + 1));
  const size_t off_po = ws_align(off_merge + sizeof(MergeItem) * n_merge);
  const size_t off_pl =
      ws_align(off_po + sizeof(float) * (size_t)n_slots * g * head_dim);
  const size_t end = ws_align(off_pl + sizeof(float) * (size_t)n_slots * g);
  const size_t host_bytes = off_po - kWsHeader;

  plan->host.assign(host_bytes / sizeof(int32_t), 0);
  char* hb = reinterpret_cast<char*>(plan->host.data());
  if (n_items)
    std::memcpy(hb + (off_items - kWsHeader), items.data(), sizeof(DecodeItem) * n_items);
  std::memcpy(hb + (off_wave - kWsHeader), wave_ptr.data(), sizeof(int32_t) * (n_waves + 1));
  if (n_merge)
    std::memcpy(hb + (off_merge - kWsHeader), merges.data(), sizeof(MergeItem) * n_merge);

  plan->workspace = workspace;
  plan->workspace_bytes = workspace_bytes;
  rc = upload_plan(plan, who, host_bytes, end, stream);
  if (rc) return rc;

  char* ws = static_cast<char*>(workspace);
  plan->implicit = false;
  plan->batch_size = batch_size;
  plan->hq = num_qo_heads;
  plan->hkv = num_kv_heads;
  plan->d = head_dim;
  plan->page_size = page_size;
  plan->n_items = n_waves;
  plan->hg_shift = hg_shift;
  plan->n_merge = (int)n_merge;
  plan->n_slots = n_slots;
  plan->split_pages = split_pages;
  plan->items_dev = ws + off_items;
  plan->wave_ptr_dev = reinterpret_cast<const int32_t*>(ws + off_wave);
  plan->merge_dev = ws + off_merge;
  plan->partial_o = reinterpret_cast<float*>(ws + off_po);
  plan->partial_lse = reinterpret_cast<float*>(ws + off_pl);
  plan->total_pages = total;
  plan->max_pages = maxp;
  plan->mode = kPlanDecode;
  return PAGEDATTN_OK;
}

int pagedattn_decode_plan_kind(const pagedattn_plan* plan) {
  if (!plan || plan->mode != kPlanDecode) return 0;
  if (plan->implicit) return plan->shared ? PAGEDATTN_DECODE_DEVICE_SHARED : PAGEDATTN_DECODE_DEVICE;
  return plan->shared ? PAGEDATTN_DECODE_SHARED : PAGEDATTN_DECODE_SPLIT;
}

int pagedattn_decode_plan_device(pagedattn_plan* plan, int32_t batch_size,
                                 int32_t num_qo_heads, int32_t num_kv_heads,
                                 int32_t head_dim, int32_t page_size, void* workspace,
                                 size_t workspace_bytes) {
  const char* who = "decode_plan_device";
  if (!plan) return set_error(PAGEDATTN_ERR_INVALID, "%s: null plan", who);
  plan->mode = kPlanNone;
  if (!workspace || ((uintptr_t)workspace & (kWsAlign - 1)))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "%s: workspace must be a 256-byte aligned device buffer", who);
  int cus = device_cu_count();
  if (cus <= 0) cus = 256;
  if (workspace_bytes < kWsHeader)
    return set_error(PAGEDATTN_ERR_WORKSPACE, "%s: workspace smaller than its %zu-byte header",
                     who, kWsHeader);
  plan->host.clear();
  const int rc = setup_device_plan(who, plan, batch_size, num_qo_heads, num_kv_heads, head_dim,
                                   page_size, cus, static_cast<char*>(workspace) + kWsHeader,
                                   workspace_bytes - kWsHeader);
  if (rc) return rc;
  plan->workspace = workspace;
  plan->workspace_bytes = workspace_bytes;
  // Whole (sequence, KV head) items per CU workgroup, dealt on the device
  // (no partials, no merge launch), when the batch gives every workgroup 4
  // to kSharedMaxItems items: dealt in rounds of alternating direction, four
  // or more items per CU pair long items with short ones and balance the CUs
  // about as well as the host's longest-first assignment without knowing the
  // lengths here (busiest CU 1.3-2.7 % over the mean on the TinyLlama and
  // 70B-shaped batches; three items per CU leave 11-15 %).
  // PAGEDATTN_DECODE_SHARED=0 keeps the split partition.
  const int64_t n_all = (int64_t)batch_size * num_kv_heads;
  if (decode_shared_mode() != 0 && batch_size <= kDevSharedMaxBatch && n_all >= 4 * (int64_t)cus &&
      n_all <= (int64_t)kSharedMaxItems * cus) {
    plan->shared = true;
    plan->deterministic = decode_deterministic();
    plan->n_items = cus;  // workgroups
    plan->hg_shift = 0;
    plan->n_slots = 0;
    plan->partial_o = nullptr;
    plan->partial_lse = nullptr;
  }
  return PAGEDATTN_OK;
}

}  // extern "C"
