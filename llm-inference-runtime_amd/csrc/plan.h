// Host plan object shared by the planner (plan.cpp) and the run launchers
// (decode.hip, prefill.hip).  The plan is the work partition that
// BatchDecode/BatchPrefillWithPagedKVCacheWrapper.begin_forward builds in the
// reference (src/models/llama.py:86-147); the device copy of its work list
// lives in the caller's workspace.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "common.h"

namespace pa {

enum PlanMode { kPlanNone = 0, kPlanDecode = 1, kPlanPrefill = 2 };

// One decode work item, processed by one head group of hg waves: pages
// [page_lo, page_hi) of sequence b for KV heads [h, h + hg), one wave per KV
// head and all its query heads.  slot < 0 means the item covers the whole
// sequence and writes the final output; otherwise wave i writes split
// partials to `slot + i` and the item takes part in merge group `merge`.
struct DecodeItem {
  int32_t b, h, page_lo, page_hi, slot, merge, pad0, pad1;
};

// Split-KV merge group: (sequence b, KV head h) owns the partial slots
// slot0 + k * stride, k in [0, nslots).
struct MergeItem {
  int32_t b, h, slot0, nslots, stride;
};

// One prefill work item: query tokens [q_lo, q_hi) of sequence b (relative to
// qo_indptr[b]) for one KV head and all its query heads.  slot 1 or 2 flags a
// paired tile (at most half a workgroup's rows), run for both KV heads of
// each head pair by the pair's even (1) or odd (2) head's workgroup; the
// planners alternate the two so that paired work lands on both XCDs of a
// pair.  slot -1: an ordinary tile.
struct PrefillItem {
  int32_t b, q_lo, q_hi, slot;
};

// One item of a shared-item decode plan (decode_shared_kernel): sequence b,
// KV head h, its page pairs being chunks [chunk_lo, chunk_lo + n_chunks) of
// the workgroup's chunk sequence; the sequence's pages are kv_indices
// [ind_lo, ind_lo + npages), the last holding `last` tokens (the planned
// metadata, which the run's is, as with FlashInfer's plan and run: the
// kernel then reads no kv_indptr / kv_last_page_len before its first page
// ids).  Workgroup w's items are entries [w kSharedMaxItems, (w + 1)
// kSharedMaxItems) of the list, each carrying the workgroup's item count in
// wg_items (entries past it are padding), so the kernel's first load is its
// items themselves.
struct SharedItem {
  int32_t b, h, chunk_lo, n_chunks, ind_lo, npages, last, wg_items;
};

// Shared-item decode geometry the planner sizes its partition by: items per
// workgroup (the kernel's LDS table) and page pairs per chunk (one register
// stage).
constexpr int kSharedMaxItems = 8;
constexpr int kSharedStagePairs = 1;
// Sequences a device-planned shared-item decode ranks in every workgroup's
// prologue (B compares per sequence).
constexpr int kDevSharedMaxBatch = 512;

// Prefill geometry: 8 waves per workgroup (two per SIMD) share every K/V tile
// loaded into LDS, which halves the global-to-LDS traffic per MFMA against 4
// waves; each wave owns kPrefillRB blocks of 32 query rows.
constexpr int kPrefillWaves = 8;
constexpr int kPrefillRB = 1;
constexpr int kPrefillRows = kPrefillWaves * 32 * kPrefillRB;
// Device-planned prefill: sequences a plan may hold (the plan kernel's
// workgroup scans four per thread) and q-tiles it orders longest first
// (one rank each per thread; beyond this the tiles keep sequence order).
constexpr int kPrefillDevMaxBatch = 4096;
constexpr int kPrefillDevSortMax = 1024;

// Workspace layout: [0, kWsHeader) is reserved for the caller's device flags
// (the Python shim keeps the append error counter at offset 0).
constexpr size_t kWsHeader = 256;
constexpr size_t kWsAlign = 256;

inline size_t ws_align(size_t x) { return (x + kWsAlign - 1) & ~(kWsAlign - 1); }

}  // namespace pa

struct pagedattn_plan {
  int mode = pa::kPlanNone;
  int batch_size = 0, hq = 0, hkv = 0, d = 0, page_size = 0;
  // n_items = head groups (decode) or work items (prefill)
  int n_items = 0, n_merge = 0, n_slots = 0, split_pages = 0;
  // decode: log2 of the waves (KV heads) per head group
  int hg_shift = 0;
  // decode: the partition is made on the device at run time from kv_indptr
  // (n_items = number of shares); no work list in the workspace.
  // prefill: the q-tile list is built on the device at run time from
  // qo_indptr (n_items = its capacity)
  bool implicit = false;
  // decode, implicit: page-equivalents charged per (sequence, head group)
  // segment by the device-side split
  int item_cost = 0;
  // decode: whole (sequence, KV head) items shared by the waves of one
  // workgroup per CU (n_items = workgroups; no split partials, no merge)
  bool shared = false;
  // decode, shared: fixed chunk assignment (output bits independent of timing)
  bool deterministic = false;
  // decode, implicit and shared: the items were dealt into the workspace by
  // pagedattn_decode_plan_device_update (items_dev, the host plan's layout)
  // and the runs read them there instead of dealing in their prologue.
  // prefill, implicit: pagedattn_prefill_plan_device_update built the q-tile
  // list and the runs launch no plan kernel of their own
  bool dev_table = false;
  // prefill: query tokens per tile (rows = tokens * hq/hkv)
  int q_tile = 0;
  // prefill: tiles of at most half a workgroup's rows run as KV-head pairs
  // (device plans apply it at run time; host plans flag their items)
  bool prefill_pair = false;
  int64_t total_qo = 0;
  // device pointers into the workspace
  void* items_dev = nullptr;
  const int32_t* wave_ptr_dev = nullptr;  // decode: items of head group w
  void* merge_dev = nullptr;
  float* partial_o = nullptr;
  float* partial_lse = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  // host staging of the work lists (kept until the next plan so the async
  // copy never reads freed memory)
  std::vector<int32_t> host;
  // statistics for the Python shim / tests
  int64_t total_pages = 0;
  int max_pages = 0;
};
