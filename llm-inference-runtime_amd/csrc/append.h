// Page-append arguments and checks shared by the kernels that write new K/V
// rows into the pool (misc.hip: plain and RoPE-fused appends; kvwrite.hip:
// the e4m3 running-amax append).
#pragma once

#include "common.h"

namespace pa {

struct AppendArgs {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sn, k_sh, v_sn, v_sh;
  const int32_t* batch_indices;
  const int32_t* positions;
  int32_t nnz;
  void* cache;
  const float* scales;
  int32_t num_pages;
  const int32_t* kv_indices;
  int32_t num_indices;
  const int32_t* kv_indptr;
  int32_t batch_size, hkv, d;
  int32_t* err;
};

__device__ __forceinline__ int64_t append_target_page(const AppendArgs& a,
                                                      int j, int* slot) {
  const int b = a.batch_indices[j];
  const int pos = a.positions[j];
  if (b < 0 || b >= a.batch_size || pos < 0) return -1;
  const int lo = a.kv_indptr[b];
  const int hi = a.kv_indptr[b + 1];
  const int it = lo + pos / kPage;
  if (it < lo || it >= hi || it >= a.num_indices) return -1;
  const int page = a.kv_indices[it];
  if (page < 0 || page >= a.num_pages) return -1;
  *slot = pos % kPage;
  return page;
}

// Validation and argument packing shared by the append entry points.
// Returns PAGEDATTN_OK with *a filled, or an error; *empty is set when there
// is nothing to do (nnz == 0).
int append_setup(const char* who, const void* append_key, const void* append_value,
                 int64_t k_stride_n, int64_t k_stride_h, int64_t v_stride_n,
                 int64_t v_stride_h, int32_t src_dtype, const int32_t* batch_indices,
                 const int32_t* positions, int32_t nnz, void* paged_kv_cache,
                 int32_t cache_dtype, const float* kv_scales, int32_t num_pages,
                 const int32_t* kv_indices, int32_t num_indices, const int32_t* kv_indptr,
                 int32_t batch_size, int32_t num_kv_heads, int32_t head_dim,
                 int32_t page_size, int32_t* error_flag, AppendArgs* a, bool* empty);

}  // namespace pa
