// Drives the host planners of libpagedattn (pagedattn_decode_plan,
// pagedattn_decode_plan_device, pagedattn_prefill_plan, and the metadata
// validation they share) with randomized and malformed metadata, built with
// the address and undefined-behaviour sanitizers (Makefile next to this
// file).  The metadata is what the engine's callers build
// (src/engine/runtime/step_executor.py:98-165, 204-243) plus what a bad
// caller could pass: non-monotone or negative indptr, last_page_len outside
// [1, 16], lengths near INT32_MAX, bad head shapes, short or misaligned
// workspaces.  Every call must return a documented status with a message; a
// sanitizer report aborts the run.  On a machine without a GPU the planners
// run up to the work-list upload, which then fails with PAGEDATTN_ERR_HIP.
//
//   plan_fuzz <iterations> <seed>
#include <cinttypes>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "pagedattn.h"

namespace {

std::mt19937_64 rng;

int64_t uni(int64_t lo, int64_t hi) {  // inclusive
  return std::uniform_int_distribution<int64_t>(lo, hi)(rng);
}
bool coin(double p) { return std::uniform_real_distribution<double>(0, 1)(rng) < p; }

struct Meta {
  std::vector<int32_t> indptr, last, qo;
  int32_t batch = 0;
  bool valid = true;  // the metadata satisfies every documented rule
};

// kv_indptr / kv_last_page_len (and qo_indptr) of `batch` sequences; with
// probability `bad` one rule is broken.
Meta make_meta(double bad) {
  Meta m;
  m.batch = (int32_t)(coin(0.05) ? 0 : uni(1, coin(0.1) ? 1200 : 64));
  const int max_pages = coin(0.2) ? 9000 : 80;
  m.indptr.resize(m.batch + 1);
  m.last.resize(m.batch);
  m.qo.resize(m.batch + 1);
  m.indptr[0] = coin(0.3) ? (int32_t)uni(0, 5000) : 0;
  m.qo[0] = coin(0.3) ? (int32_t)uni(0, 5000) : 0;
  for (int b = 0; b < m.batch; ++b) {
    const int np = coin(0.05) ? 0 : (int)uni(1, max_pages);
    m.indptr[b + 1] = m.indptr[b] + np;
    m.last[b] = (int32_t)uni(1, 16);
    const int kv = np > 0 ? (np - 1) * 16 + m.last[b] : 0;
    m.qo[b + 1] = m.qo[b] + (int32_t)(kv > 0 ? uni(1, std::min(kv, 600)) : uni(0, 3));
  }
  if (m.batch > 0 && coin(bad)) {
    m.valid = false;
    const int b = (int)uni(0, m.batch - 1);
    switch (uni(0, 9)) {
      case 0: m.indptr[0] = -(int32_t)uni(1, INT_MAX); break;
      case 1: m.indptr[b + 1] = m.indptr[b] - (int32_t)uni(1, 100); break;  // not monotone
      case 2: m.last[b] = (int32_t)uni(17, INT_MAX); m.indptr[b + 1] = m.indptr[b] + 1; break;
      case 3: m.last[b] = -(int32_t)uni(0, INT_MAX); m.indptr[b + 1] = m.indptr[b] + 1; break;
      case 4:  // a sequence longer than INT32_MAX tokens
        m.indptr[b + 1] = m.indptr[b] + (int32_t)uni(134217728, INT_MAX / 2);
        for (int c = b + 1; c < m.batch; ++c) m.indptr[c + 1] = m.indptr[b + 1];
        break;
      case 5: m.indptr[m.batch] = INT_MAX; break;
      case 6: m.qo[b + 1] = m.qo[b] - (int32_t)uni(1, INT_MAX / 2); break;
      case 7: m.qo[b + 1] = INT_MIN + (int32_t)uni(0, 10); break;
      case 8: m.qo[0] = -(int32_t)uni(1, 1000); break;
      default:  // a huge chunk: qo near INT32_MAX
        m.qo[b + 1] = m.qo[b] + (int32_t)uni(INT_MAX / 4, INT_MAX / 2);
        for (int c = b + 1; c < m.batch; ++c) m.qo[c + 1] = m.qo[b + 1];
        break;
    }
  }
  return m;
}

const char* kEnv[] = {"PAGEDATTN_DECODE_SHARED", "PAGEDATTN_DECODE_DETERMINISTIC",
                      "PAGEDATTN_DECODE_HEAD_GROUP", "PAGEDATTN_DECODE_ITEM_COST",
                      "PAGEDATTN_DECODE_WAVES_PER_CU", "PAGEDATTN_DECODE_SHARED_SLACK_KB",
                      "PAGEDATTN_DECODE_SHARED_SLACK_PCT",
                      "PAGEDATTN_PREFILL_PAIR"};

void shuffle_env() {
  for (const char* e : kEnv) {
    if (coin(0.6)) {
      unsetenv(e);
      continue;
    }
    const long v = coin(0.2) ? (long)uni(-5, 2000) : (long)uni(0, 12);
    setenv(e, std::to_string(v).c_str(), 1);
  }
}

int failures = 0;

void check(const char* what, int rc, const Meta& m, bool args_valid, int64_t iter) {
  const char* msg = pagedattn_last_error();
  const bool known = rc >= PAGEDATTN_OK && rc <= PAGEDATTN_ERR_PLAN;
  bool ok = known && (rc == PAGEDATTN_OK || (msg && msg[0]));
  // valid metadata and arguments may only fail at the upload (no GPU here)
  // or on the workspace size
  if (ok && m.valid && args_valid && rc != PAGEDATTN_OK && rc != PAGEDATTN_ERR_HIP &&
      rc != PAGEDATTN_ERR_WORKSPACE)
    ok = false;
  if (!ok) {
    ++failures;
    std::fprintf(stderr, "iteration %" PRId64 ": %s returned %d (%s) on %s metadata, batch %d\n",
                 iter, what, rc, msg ? msg : "(null)", m.valid ? "valid" : "invalid", m.batch);
  }
}

}  // namespace

int main(int argc, char** argv) {
  const int64_t iters = argc > 1 ? std::atoll(argv[1]) : 2000;
  rng.seed(argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 1);
  // a 256-byte aligned stand-in for the device workspace, as large as the
  // engine's (128 MiB): the planners only compare sizes against it; the
  // work-list upload (failing without a GPU) is the only access
  const size_t ws_bytes = (size_t)128 << 20;
  char* ws = static_cast<char*>(std::aligned_alloc(256, ws_bytes));
  if (!ws) return 2;
  const int hq_kv[][2] = {{32, 4}, {32, 8}, {64, 8}, {8, 8}, {16, 1}, {4, 2}};
  for (int64_t it = 0; it < iters; ++it) {
    shuffle_env();
    Meta m = make_meta(0.3);
    int hq = 32, hkv = 8, d = coin(0.5) ? 64 : 128, page = 16;
    const int pick = (int)uni(0, 5);
    hq = hq_kv[pick][0];
    hkv = hq_kv[pick][1];
    bool args_valid = true;
    if (coin(0.08)) {  // an unsupported or invalid shape
      args_valid = false;
      switch (uni(0, 4)) {
        case 0: d = (int)uni(-10, 300); break;
        case 1: hq = (int)uni(-4, 70); break;
        case 2: hkv = (int)uni(-4, 70); break;
        case 3: page = (int)uni(-4, 64); break;
        default: hq = 96; hkv = 3; break;  // group size 32
      }
      if (d == 64 || d == 128) args_valid = page == 16 && hq > 0 && hkv > 0 && hq % hkv == 0 &&
                                            hq / hkv <= 16 && ((hq / hkv) & (hq / hkv - 1)) == 0;
    }
    void* w = ws;
    size_t wb = coin(0.1) ? (size_t)uni(0, 4096) : ws_bytes;
    if (coin(0.03)) {
      w = ws + 8;  // misaligned
      args_valid = false;
    }
    if (coin(0.02)) {
      w = nullptr;
      args_valid = false;
    }
    const int32_t batch = coin(0.02) ? -(int32_t)uni(1, 5) : m.batch;
    if (batch < 0) args_valid = false;
    pagedattn_plan* plan = pagedattn_plan_create();
    switch (uni(0, 2)) {
      case 0: {
        static const int splits[] = {0, 0, -1, 8, 256, 3, 1000, INT_MAX, INT_MIN};
        const int split = splits[uni(0, 8)];
        const int rc = pagedattn_decode_plan(plan, m.indptr.data(), m.last.data(), batch, hq,
                                             hkv, d, page, split, w, wb, nullptr);
        check("decode_plan", rc, m, args_valid, it);
        break;
      }
      case 1: {
        const int rc = pagedattn_decode_plan_device(plan, batch, hq, hkv, d, page, w, wb);
        Meta any = m;
        any.valid = true;  // the device plan reads no metadata on the host
        check("decode_plan_device", rc, any, args_valid, it);
        break;
      }
      default: {
        const int rc = pagedattn_prefill_plan(plan, m.qo.data(), m.indptr.data(), m.last.data(),
                                              batch, hq, hkv, d, page, w, wb, nullptr);
        check("prefill_plan", rc, m, args_valid, it);
        break;
      }
    }
    pagedattn_plan_destroy(plan);
    if (failures > 0) break;  // stop at the first finding
  }
  std::free(ws);
  std::printf("plan_fuzz: %" PRId64 " iterations, %d failures\n", iters, failures);
  return failures ? 1 : 0;
}
