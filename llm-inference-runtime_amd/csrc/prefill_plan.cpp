// Prefill planning on the host (BatchPrefillWithPagedKVCacheWrapper.plan,
// src/models/llama.py:86-116): the q-tile work list of
// pagedattn_prefill_plan, and the fixed shapes of a device plan
// (pagedattn_prefill_plan_device), whose list prefill.hip's plan kernel
// builds at run time.  Plain host C++ (no device code), so the planner
// can also be built and driven on a machine without a GPU, under the
// address and undefined-behaviour sanitizers.
#include <algorithm>
#include <climits>
#include <cstdlib>
#include <vector>

#include "plan_internal.h"

namespace pa {

// Paired tiles (a q-tile of at most half a workgroup's rows, run for two KV
// heads by one workgroup) are planned by default; PAGEDATTN_PREFILL_PAIR=0
// plans every tile on its own.
static bool prefill_pairing() {
  const char* env = std::getenv("PAGEDATTN_PREFILL_PAIR");
  return !(env && std::atoi(env) == 0);
}

}  // namespace pa

using namespace pa;

extern "C" {

int pagedattn_prefill_plan(pagedattn_plan* plan, const int32_t* qo_indptr_host,
                           const int32_t* kv_indptr_host,
                           const int32_t* kv_last_page_len_host,
                           int32_t batch_size, int32_t num_qo_heads,
                           int32_t num_kv_heads, int32_t head_dim,
                           int32_t page_size, void* workspace,
                           size_t workspace_bytes, void* stream) {
  const char* who = "prefill_plan";
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
  if (batch_size > 0 && !qo_indptr_host)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null qo_indptr", who);
  std::vector<int32_t> npages, kv_len;
  rc = validate_paged_metadata(who, kv_indptr_host, kv_last_page_len_host,
                               batch_size, page_size, &npages, &kv_len);
  if (rc) return rc;
  if (batch_size > 0 && qo_indptr_host[0] < 0)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: qo_indptr[0] < 0", who);
  const int g = num_qo_heads / num_kv_heads;
  const int q_tile = kPrefillRows / g;
  const bool pair = prefill_pairing() && num_kv_heads % 2 == 0;
  // the q-tile count first: the work list must fit the workspace (and the
  // launch grid) before anything is built
  int64_t n_tiles = 0;
  for (int b = 0; b < batch_size; ++b) {
    const int64_t qo = (int64_t)qo_indptr_host[b + 1] - qo_indptr_host[b];
    if (qo < 0)
      return set_error(PAGEDATTN_ERR_INVALID,
                       "%s: qo_indptr is not monotone at %d", who, b);
    n_tiles += (qo + q_tile - 1) / q_tile;
  }
  if ((int64_t)sizeof(PrefillItem) * n_tiles > (int64_t)workspace_bytes ||
      n_tiles * num_kv_heads > INT32_MAX)
    return set_error(PAGEDATTN_ERR_WORKSPACE,
                     "%s: %lld q-tiles do not fit the %zu-byte workspace", who,
                     (long long)n_tiles, workspace_bytes);
  std::vector<PrefillItem> items;
  std::vector<int64_t> cost;
  items.reserve((size_t)n_tiles);
  cost.reserve((size_t)n_tiles);
  for (int b = 0; b < batch_size; ++b) {
    const int qo = qo_indptr_host[b + 1] - qo_indptr_host[b];  // >= 0, checked above
    for (int lo = 0; lo < qo; lo = qo - lo > q_tile ? lo + q_tile : qo) {
      const int hi = qo - lo > q_tile ? lo + q_tile : qo;
      // slot 1: a paired tile (kernels built without pairing -- e4m3 pools,
      // D = 64 -- run it like any other)
      const int flag = pair && (int64_t)(hi - lo) * g <= kPrefillRows / 2 ? 1 : -1;
      items.push_back(PrefillItem{b, lo, hi, flag});
      // kv tokens the tile's last row can see (causal)
      cost.push_back(std::max<int64_t>(
          0, std::min<int64_t>(kv_len[b], (int64_t)kv_len[b] - qo + hi)));
    }
  }
  // most expensive tiles first
  std::vector<int> order(items.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
  std::stable_sort(order.begin(), order.end(),
                   [&](int a, int c) { return cost[a] > cost[c]; });
  const size_t host_bytes = sizeof(PrefillItem) * items.size();
  plan->host.assign((host_bytes + 3) / 4, 0);
  auto* dst = reinterpret_cast<PrefillItem*>(plan->host.data());
  // paired tiles alternate between the even and the odd head of each pair in
  // list order, so the two XCDs that hold a head pair's workgroups share them
  int n_paired = 0;
  for (size_t i = 0; i < order.size(); ++i) {
    dst[i] = items[order[i]];
    if (dst[i].slot > 0) dst[i].slot = 1 + (n_paired++ & 1);
  }
  plan->workspace = workspace;
  plan->workspace_bytes = workspace_bytes;
  rc = upload_plan(plan, who, host_bytes, ws_align(kWsHeader + host_bytes),
                   stream);
  if (rc) return rc;
  plan->batch_size = batch_size;
  plan->hq = num_qo_heads;
  plan->hkv = num_kv_heads;
  plan->d = head_dim;
  plan->page_size = page_size;
  plan->n_items = (int)items.size();
  plan->n_merge = 0;
  plan->n_slots = 0;
  plan->q_tile = q_tile;
  plan->total_qo =
      batch_size > 0 ? (int64_t)qo_indptr_host[batch_size] - qo_indptr_host[0] : 0;
  plan->items_dev = static_cast<char*>(workspace) + kWsHeader;
  plan->implicit = false;
  plan->shared = false;
  plan->dev_table = false;
  plan->mode = kPlanPrefill;
  return PAGEDATTN_OK;
}

int pagedattn_prefill_plan_device(pagedattn_plan* plan, int32_t batch_size,
                                  int32_t num_qo_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t page_size, int64_t max_qo_tokens,
                                  void* workspace, size_t workspace_bytes) {
  const char* who = "prefill_plan_device";
  if (!plan) return set_error(PAGEDATTN_ERR_INVALID, "%s: null plan", who);
  plan->mode = kPlanNone;
  if (batch_size < 0 || batch_size > kPrefillDevMaxBatch)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: batch_size %d outside [0, %d]", who,
                     batch_size, kPrefillDevMaxBatch);
  if (max_qo_tokens < 0)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: max_qo_tokens %lld < 0", who,
                     (long long)max_qo_tokens);
  int rc = validate_heads(who, num_qo_heads, num_kv_heads, head_dim, page_size);
  if (rc) return rc;
  if (!workspace || ((uintptr_t)workspace & (kWsAlign - 1)))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "%s: workspace must be a 256-byte aligned device buffer", who);
  const int g = num_qo_heads / num_kv_heads;
  const int q_tile = kPrefillRows / g;
  // every sequence may end in a partial tile
  const int64_t cap = (max_qo_tokens + q_tile - 1) / q_tile + batch_size;
  if ((int64_t)sizeof(PrefillItem) * cap > (int64_t)workspace_bytes - (int64_t)kWsHeader ||
      cap * num_kv_heads > INT32_MAX)
    return set_error(PAGEDATTN_ERR_WORKSPACE,
                     "%s: %lld q-tiles do not fit the %zu-byte workspace", who,
                     (long long)cap, workspace_bytes);
  plan->host.clear();
  plan->workspace = workspace;
  plan->workspace_bytes = workspace_bytes;
  plan->implicit = true;
  plan->shared = false;
  plan->dev_table = false;
  plan->prefill_pair = prefill_pairing() && num_kv_heads % 2 == 0;
  plan->batch_size = batch_size;
  plan->hq = num_qo_heads;
  plan->hkv = num_kv_heads;
  plan->d = head_dim;
  plan->page_size = page_size;
  plan->n_items = (int)cap;
  plan->n_merge = 0;
  plan->n_slots = 0;
  plan->q_tile = q_tile;
  plan->total_qo = max_qo_tokens;
  plan->items_dev = static_cast<char*>(workspace) + kWsHeader;
  plan->mode = kPlanPrefill;
  return PAGEDATTN_OK;
}

}  // extern "C"
