// Internal planner helpers (plan.cpp).
#pragma once

#include <vector>

#include "plan.h"

namespace pa {

// Checks indptr monotonicity and 1 <= last_page_len <= page_size for every
// non-empty sequence; returns pages and kv lengths per sequence.
int validate_paged_metadata(const char* who, const int32_t* kv_indptr_host,
                            const int32_t* kv_last_page_len_host,
                            int32_t batch_size, int32_t page_size,
                            std::vector<int32_t>* npages,
                            std::vector<int32_t>* kv_len);

// Checks the head shape the kernels support.
int validate_heads(const char* who, int32_t hq, int32_t hkv, int32_t d,
                   int32_t page_size);

// Copies plan->host (host_bytes) to workspace + kWsHeader on `stream` after
// checking that total_bytes (measured from the workspace start) fit.
int upload_plan(pagedattn_plan* plan, const char* who, size_t host_bytes,
                size_t total_bytes, void* stream);

// The device-side partition of a decode plan (pagedattn_decode_plan_device
// and pagedattn_decode_run_noalloc): shares of the (sequence, head group,
// page) stream for cus x waves-per-CU / hg head groups, split partials at
// `partials` (256-byte aligned, `bytes` long).  Host only, allocates nothing.
int setup_device_plan(const char* who, pagedattn_plan* plan, int32_t batch_size,
                      int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                      int32_t page_size, int cus, char* partials, size_t bytes);

}  // namespace pa
