// placeholder until the MFMA prefill kernel lands
#include "plan_internal.h"
using namespace pa;
extern "C" {
int pagedattn_prefill_plan(pagedattn_plan* plan, const int32_t*, const int32_t*, const int32_t*, int32_t, int32_t, int32_t, int32_t, int32_t, void*, size_t, void*) {
  if (plan) plan->mode = kPlanNone;
  return set_error(PAGEDATTN_ERR_UNSUPPORTED, "prefill_plan: not built yet");
}
int pagedattn_prefill_run(const pagedattn_plan*, const void*, int64_t, int64_t, int32_t, const int32_t*, const void*, int32_t, const float*, int32_t, const int32_t*, int32_t, const int32_t*, const int32_t*, void*, float*, int32_t, float, void*) {
  return set_error(PAGEDATTN_ERR_UNSUPPORTED, "prefill_run: not built yet");
}
}
