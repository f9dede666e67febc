// Device-side paged metadata: what the engine's step executor builds in
// Python lists and uploads every step (src/engine/runtime/step_executor.py:
// 98-165 for a chunked-prefill step, :204-234 for a decode step) and what
// build_batch_indices_positions derives after a device-to-host sync
// (src/models/llama.py:70-83), built on the GPU from a fixed-capacity block
// table and the sequence lengths.  No host round trip, fixed launch shapes,
// no memsets: the whole step can be captured in a HIP graph.
//
// Per sequence b with kv length L (tokens in the cache after this step's
// appends, including them) and n new tokens:
//   pages   = ceil(L / 16), the table cut to the pages in use (the reference
//             decode step passes the whole table, step_executor.py:209, which
//             overstates kv_len by a page whenever L % 16 == 0)
//   last    = L % 16, or 16
//   tokens  = positions L - n .. L - 1 (decode: one token, row b)
#include <algorithm>

#include "common.h"

namespace pa {

struct MetaArgs {
  const int32_t* tables;
  int64_t stride;
  int32_t max_pages;
  const int32_t* kv_lens;
  const int32_t* new_lens;  // null: decode, one new token per sequence
  int32_t batch;
  int32_t* qo_indptr;
  int32_t* kv_indptr;
  int32_t* kv_indices;
  int32_t indices_cap;
  int32_t* last;
  int32_t* bi;
  int32_t* pos;
  int32_t tokens_cap;
  int32_t* err;
};

constexpr int kMetaThreads = 1024;

__device__ __forceinline__ int seq_pages(const MetaArgs& a, int L) {
  const int np = L > 0 ? (L + kPage - 1) / kPage : 0;
  return min(np, a.max_pages);
}

__device__ __forceinline__ int seq_new_tokens(const MetaArgs& a, int b, int L) {
  if (!a.new_lens) return 1;
  return min(max(a.new_lens[b], 0), max(L, 0));
}

// Whether some of sequence b's outputs fall past a capacity (or behind an
// offset that overflowed int32): decided from its offsets, so the sequence
// is counted once whatever the grid.
__device__ __forceinline__ bool seq_dropped(const MetaArgs& a, int off, int np, int qo, int nt) {
  const bool pages = np > 0 && (off < 0 || (int64_t)off + np > a.indices_cap);
  const bool toks = a.new_lens && nt > 0 && (qo < 0 || (int64_t)qo + nt > a.tokens_cap);
  return pages || toks;
}

// One workgroup: page and token offsets of every sequence, last page
// lengths, and (decode) the token -> sequence / position rows.
__global__ void __launch_bounds__(kMetaThreads) meta_scan_kernel(MetaArgs a) {
  __shared__ int red[2][kMetaThreads / kWave];
  int run_pages = 0, run_tokens = 0;
  int clipped = 0;
  for (int base = 0; base < a.batch; base += kMetaThreads) {
    const int b = base + (int)threadIdx.x;
    const int L = b < a.batch ? a.kv_lens[b] : 0;
    const int full = L > 0 ? (L + kPage - 1) / kPage : 0;
    const int np = b < a.batch ? seq_pages(a, L) : 0;
    const int nt = b < a.batch ? seq_new_tokens(a, b, L) : 0;
    clipped += full > np ? 1 : 0;
    int tot_p, tot_t;
    const int ep = block_excl_scan<kMetaThreads>(np, &tot_p, red[0]);
    const int et = block_excl_scan<kMetaThreads>(nt, &tot_t, red[1]);
    if (b < a.batch) {
      a.kv_indptr[b] = run_pages + ep;
      if (a.qo_indptr) a.qo_indptr[b] = run_tokens + et;
      a.last[b] = L > 0 ? (L - 1) % kPage + 1 : kPage;
      if (!a.new_lens) {
        a.bi[b] = b;
        a.pos[b] = L - 1;
      }
    }
    run_pages += tot_p;
    run_tokens += tot_t;
  }
  if (clipped > 0 && a.err) atomicAdd(a.err, clipped);
  if (threadIdx.x == 0) {
    a.kv_indptr[a.batch] = run_pages;
    if (a.qo_indptr) a.qo_indptr[a.batch] = run_tokens;
  }
}

// Grid (x, b): the page ids of sequence b copied out of its table row, and
// (prefill) its new tokens' sequence / position rows.  Entries past the
// output capacities (or behind offsets that overflowed int32) are dropped;
// the sequence is counted once.
__global__ void __launch_bounds__(256) meta_fill_kernel(MetaArgs a) {
  const int b = blockIdx.y;
  const int L = a.kv_lens[b];
  const int np = seq_pages(a, L);
  const int off = a.kv_indptr[b];
  const int step = gridDim.x * blockDim.x;
  const int first = blockIdx.x * blockDim.x + threadIdx.x;
  const int32_t* row = a.tables + (int64_t)b * a.stride;
  for (int i = first; i < np; i += step)
    if (off >= 0 && (int64_t)off + i < a.indices_cap) a.kv_indices[off + i] = row[i];
  const int nt = seq_new_tokens(a, b, L);
  const int qo = a.new_lens ? a.qo_indptr[b] : 0;
  if (a.new_lens) {
    for (int j = first; j < nt; j += step) {
      const int64_t t = (int64_t)qo + j;
      if (qo >= 0 && t < a.tokens_cap) {
        a.bi[t] = b;
        a.pos[t] = L - nt + j;
      }
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0 && a.err && seq_dropped(a, off, np, qo, nt))
    atomicAdd(a.err, 1);
}

// Batches up to kMetaFuseMax sequences: one launch, grid (x, b).  Every
// workgroup of sequence b sums the page and token counts of the sequences
// before it itself (at most kMetaFuseMax loads per workgroup), so no
// workgroup waits for another; then it writes what the scan and the fill
// kernels write for b.  A clipped row, and a sequence some of whose outputs
// were dropped, are each counted once per sequence (as the two-launch path
// counts them).
constexpr int kMetaFuseMax = 1024;
constexpr int kMetaFuseThreads = 256;

__global__ void __launch_bounds__(kMetaFuseThreads) meta_fused_kernel(MetaArgs a) {
  __shared__ int red[2][kMetaFuseThreads / kWave];
  const int b = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  int sp = 0, st = 0;
  for (int i = (int)threadIdx.x; i < b; i += kMetaFuseThreads) {
    const int Li = a.kv_lens[i];
    sp += seq_pages(a, Li);
    st += seq_new_tokens(a, i, Li);
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    sp += __shfl_xor(sp, o);
    st += __shfl_xor(st, o);
  }
  if (lane == 0) {
    red[0][wave] = sp;
    red[1][wave] = st;
  }
  __syncthreads();
  int off = 0, qo = 0;
#pragma unroll
  for (int w = 0; w < kMetaFuseThreads / kWave; ++w) {
    off += red[0][w];
    qo += red[1][w];
  }
  const int L = a.kv_lens[b];
  const int np = seq_pages(a, L);
  const int nt = seq_new_tokens(a, b, L);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    a.kv_indptr[b] = off;
    if (a.qo_indptr) a.qo_indptr[b] = qo;
    a.last[b] = L > 0 ? (L - 1) % kPage + 1 : kPage;
    if (!a.new_lens) {
      a.bi[b] = b;
      a.pos[b] = L - 1;
    }
    if (b == a.batch - 1) {
      a.kv_indptr[a.batch] = off + np;
      if (a.qo_indptr) a.qo_indptr[a.batch] = qo + nt;
    }
    const int full = L > 0 ? (L + kPage - 1) / kPage : 0;
    if (full > np && a.err) atomicAdd(a.err, 1);
  }
  const int step = gridDim.x * blockDim.x;
  const int first = blockIdx.x * blockDim.x + threadIdx.x;
  const int32_t* row = a.tables + (int64_t)b * a.stride;
  for (int i = first; i < np; i += step)
    if (off >= 0 && (int64_t)off + i < a.indices_cap) a.kv_indices[off + i] = row[i];
  if (a.new_lens) {
    for (int j = first; j < nt; j += step) {
      const int64_t t = (int64_t)qo + j;
      if (qo >= 0 && t < a.tokens_cap) {
        a.bi[t] = b;
        a.pos[t] = L - nt + j;
      }
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0 && a.err && seq_dropped(a, off, np, qo, nt))
    atomicAdd(a.err, 1);
}

}  // namespace pa

using namespace pa;

extern "C" {

int pagedattn_build_paged_metadata(const int32_t* block_tables, int64_t table_stride,
                                   int32_t max_pages, const int32_t* kv_lens,
                                   const int32_t* new_lens, int32_t batch_size,
                                   int32_t* qo_indptr, int32_t* kv_indptr, int32_t* kv_indices,
                                   int32_t indices_capacity, int32_t* kv_last_page_len,
                                   int32_t* batch_indices, int32_t* positions,
                                   int32_t tokens_capacity, int32_t* error_flag, void* stream) {
  const char* who = "build_paged_metadata";
  if (batch_size < 0 || max_pages < 0 || table_stride < max_pages || indices_capacity < 0 ||
      tokens_capacity < 0)
    return set_error(PAGEDATTN_ERR_INVALID,
                     "%s: bad sizes batch=%d max_pages=%d stride=%lld capacities=%d/%d", who,
                     batch_size, max_pages, (long long)table_stride, indices_capacity,
                     tokens_capacity);
  if (!kv_indptr || (batch_size > 0 && (!kv_lens || !kv_last_page_len || !batch_indices ||
                                        !positions || (max_pages > 0 && !block_tables) ||
                                        (indices_capacity > 0 && !kv_indices))))
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null pointer", who);
  if (new_lens && !qo_indptr)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: a prefill step (new_lens) needs qo_indptr",
                     who);
  if (!new_lens && tokens_capacity < batch_size)
    return set_error(PAGEDATTN_ERR_INVALID,
                     "%s: a decode step writes one token row per sequence (%d > capacity %d)",
                     who, batch_size, tokens_capacity);
  if (batch_size > 65535)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: batch_size %d above 65535", who,
                     batch_size);
  MetaArgs a{block_tables, table_stride, max_pages, kv_lens, new_lens, batch_size,
             qo_indptr, kv_indptr, kv_indices, indices_capacity, kv_last_page_len,
             batch_indices, positions, tokens_capacity, error_flag};
  hipStream_t s = (hipStream_t)stream;
  const unsigned gx = (unsigned)std::max(1, std::min(64, (max_pages + 255) / 256));
  if (batch_size > 0 && batch_size <= kMetaFuseMax) {
    hipLaunchKernelGGL(meta_fused_kernel, dim3(gx, batch_size), dim3(kMetaFuseThreads), 0, s,
                       a);
    return check_launch(who);
  }
  hipLaunchKernelGGL(meta_scan_kernel, dim3(1), dim3(kMetaThreads), 0, s, a);
  int rc = check_launch(who);
  if (rc || batch_size == 0) return rc;
  hipLaunchKernelGGL(meta_fill_kernel, dim3(gx, batch_size), dim3(256), 0, s, a);
  return check_launch(who);
}

}  // extern "C"
