// Host planner helpers: metadata validation and the upload of a work list
// into the caller's workspace.  The decode / prefill partitioners are in
// decode_plan.cpp and prefill_plan.cpp.
#include <climits>
#include <cstring>

#include "plan_internal.h"

namespace pa {

int validate_paged_metadata(const char* who, const int32_t* kv_indptr_host,
                            const int32_t* kv_last_page_len_host,
                            int32_t batch_size, int32_t page_size,
                            std::vector<int32_t>* npages,
                            std::vector<int32_t>* kv_len) {
  if (!kv_indptr_host || (batch_size > 0 && !kv_last_page_len_host))
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null metadata pointer", who);
  if (kv_indptr_host[0] < 0)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: kv_indptr[0] = %d < 0", who,
                     kv_indptr_host[0]);
  npages->resize(batch_size);
  kv_len->resize(batch_size);
  for (int b = 0; b < batch_size; ++b) {
    const int np = kv_indptr_host[b + 1] - kv_indptr_host[b];
    if (np < 0)
      return set_error(PAGEDATTN_ERR_INVALID,
                       "%s: kv_indptr is not monotone at %d (%d -> %d)", who, b,
                       kv_indptr_host[b], kv_indptr_host[b + 1]);
    const int last = kv_last_page_len_host[b];
    if (np > 0 && (last < 1 || last > page_size))
      return set_error(PAGEDATTN_ERR_INVALID,
                       "%s: kv_last_page_len[%d] = %d outside [1, %d]", who, b,
                       last, page_size);
    // kv lengths are int32 in the kernels
    const int64_t len = np > 0 ? (int64_t)(np - 1) * page_size + last : 0;
    if (len > INT32_MAX)
      return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                       "%s: sequence %d holds %lld tokens (at most %d)", who, b,
                       (long long)len, INT32_MAX);
    (*npages)[b] = np;
    (*kv_len)[b] = (int32_t)len;
  }
  return PAGEDATTN_OK;
}

int validate_heads(const char* who, int32_t hq, int32_t hkv, int32_t d,
                   int32_t page_size) {
  if (page_size != kPage)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: page_size %d not supported (16)", who, page_size);
  if (d != 64 && d != 128)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: head_dim %d not supported (64 or 128)", who, d);
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0)
    return set_error(PAGEDATTN_ERR_INVALID,
                     "%s: num_qo_heads %d must be a positive multiple of "
                     "num_kv_heads %d",
                     who, hq, hkv);
  const int g = hq / hkv;
  if (g > 16 || (g & (g - 1)))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: group size %d (num_qo_heads / num_kv_heads) must be a "
                     "power of two <= 16",
                     who, g);
  return PAGEDATTN_OK;
}

int upload_plan(pagedattn_plan* plan, const char* who, size_t host_bytes,
                size_t total_bytes, void* stream) {
  if (total_bytes > plan->workspace_bytes)
    return set_error(PAGEDATTN_ERR_WORKSPACE,
                     "%s: plan needs %zu workspace bytes, %zu available", who,
                     total_bytes, plan->workspace_bytes);
  if (host_bytes == 0) return PAGEDATTN_OK;
  hipError_t e = hipMemcpyAsync(static_cast<char*>(plan->workspace) + kWsHeader,
                                plan->host.data(), host_bytes,
                                hipMemcpyHostToDevice, (hipStream_t)stream);
  if (e != hipSuccess)
    return set_error(PAGEDATTN_ERR_HIP, "%s: work-list upload failed: %s", who,
                     hipGetErrorString(e));
  return PAGEDATTN_OK;
}

}  // namespace pa

extern "C" {

pagedattn_plan* pagedattn_plan_create(void) { return new pagedattn_plan(); }

void pagedattn_plan_destroy(pagedattn_plan* plan) { delete plan; }

}  // extern "C"
