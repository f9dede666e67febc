// KV write path of an engine that owns its pages:
//  * e4m3 page append that keeps each (page, K|V, kv-head) scale a running
//    amax while the page fills (power-of-two scales, so growing a scale
//    re-encodes the rows already in the page by an exact exponent shift);
//  * copy-on-write page fork: copy the valid rows of shared pages to fresh
//    pages across every layer of the pool (todo.md:17-19 of the reference
//    asks for it before a sequence appends to a shared partial block).
// Both are HBM-bound byte movers; neither reads a byte twice from HBM.
#include <algorithm>

#include "append.h"

namespace pa {

// ----------------------------------------------------------------------------
// Smallest power of two s with 448 * s >= amax (0 when amax is 0, never below
// 2^-126).  amax = m * 2^e with m in [0.5, 1) and 448 = 0.875 * 2^9, so
// s = 2^(e - 9 + [m > 0.875]).
__device__ __forceinline__ float pow2_scale_of(float amax) {
  if (!(amax > 0.f)) return 0.f;
  int e;
  const float m = frexpf(amax, &e);
  const int ex = max(e - 9 + (m > 0.875f ? 1 : 0), -126);
  return ldexpf(1.f, ex);
}

// Eight e4m3 bytes -> fp32 (exact).
__device__ __forceinline__ void e4m3x8_to_f32(u32x2 q, float (&f)[8]) {
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)q[w], false);
    const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)q[w], true);
    f[4 * w + 0] = lo[0];
    f[4 * w + 1] = lo[1];
    f[4 * w + 2] = hi[0];
    f[4 * w + 3] = hi[1];
  }
}

__device__ __forceinline__ u32x2 f32x8_to_e4m3(const float (&f)[8]) {
  u32x2 o;
  o[0] = f32_to_e4m3x4(f[0], f[1], f[2], f[3]);
  o[1] = f32_to_e4m3x4(f[4], f[5], f[6], f[7]);
  return o;
}

// Token t starts a run: the tokens of one sequence that land in one page,
// consecutive and in position order.  t starts one unless it continues
// t - 1 (same sequence, next position, not the first slot of a page).
__device__ __forceinline__ bool starts_run(const AppendArgs& a, int t) {
  if (t <= 0 || t >= a.nnz) return true;
  const int b0 = a.batch_indices[t - 1];
  const int b1 = a.batch_indices[t];
  const int p0 = a.positions[t - 1];
  const int p1 = a.positions[t];
  return !(b0 == b1 && (int64_t)p1 == (int64_t)p0 + 1 && (p1 % kPage) != 0);
}

constexpr int kAmaxMaxD = 256;  // head_dim limit

// One run's (page, K|V, head) block, worked by the lanes of `width` lanes
// (a power of two, a multiple of L = D/8): lane chunk gl of rows
// row0, row0 + step, ... (NR rows at most).  Per run:
//   s_old = scale if the run starts past slot 0, else 0
//   s_new = max(s_old, pow2_scale(amax of the run's rows))
//   s_new > s_old: rows [0, slot0) <- e4m3(decode(row) * (s_old / s_new))
//   run rows <- e4m3(clamp(x * (1 / s_new), +-448))   (zero codes when s_new
//   is 0; 1 / s_new is exact, s_new being a power of two in [2^-126, 2^127])
template <bool IS_BF16, int NR>
__device__ __forceinline__ void amax_run(const AppendArgs& a, float* __restrict__ scales,
                                         const uint16_t* src, int64_t sn, int t0, int n,
                                         int kind, int h, int gl, int row0, int step,
                                         int width, bool leader) {
  // every load in flight at once: rows past the run repeat its last row,
  // which leaves the amax unchanged and is never written
  u32x4 x[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const int j = min(row0 + k * step, n - 1);
    x[k] = *reinterpret_cast<const u32x4*>(src + (int64_t)(t0 + j) * sn + 8 * gl);
  }
  float amax = 0.f;
#pragma unroll
  for (int k = 0; k < NR; ++k) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      amax = fmaxf(amax, fabsf(h2f<IS_BF16>((uint16_t)(x[k][e] & 0xffffu))));
      amax = fmaxf(amax, fabsf(h2f<IS_BF16>((uint16_t)(x[k][e] >> 16))));
    }
  }
  for (int off = width >> 1; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  int slot0 = 0;
  const int64_t page = append_target_page(a, t0, &slot0);
  if (page < 0) {
    if (leader && kind == 0 && h == 0 && a.err) atomicAdd(a.err, n);
    return;
  }
  const int64_t sidx = (page * 2 + kind) * a.hkv + h;
  const float s_old = slot0 > 0 ? scales[sidx] : 0.f;
  const float s_new = fmaxf(s_old, pow2_scale_of(amax));
  uint8_t* blk = static_cast<uint8_t*>(a.cache) + sidx * kPage * (int64_t)a.d;
  if (slot0 > 0 && s_new > s_old) {
    const float ratio = s_old / s_new;
    for (int row = row0; row < slot0; row += step) {
      uint8_t* q = blk + (int64_t)row * a.d + 8 * gl;
      float f[8];
      e4m3x8_to_f32(*reinterpret_cast<const u32x2*>(q), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = fminf(fmaxf(f[e] * ratio, -448.f), 448.f);
      *reinterpret_cast<u32x2*>(q) = f32x8_to_e4m3(f);
    }
  }
  const float inv = s_new > 0.f ? 1.f / s_new : 0.f;
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const int j = row0 + k * step;
    if (j >= n) continue;
    u32x2 o = {0u, 0u};
    if (s_new > 0.f) {
      float f[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = h2f<IS_BF16>((uint16_t)(x[k][e] & 0xffffu));
        f[2 * e + 1] = h2f<IS_BF16>((uint16_t)(x[k][e] >> 16));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = fminf(fmaxf(f[e] * inv, -448.f), 448.f);
      o = f32x8_to_e4m3(f);
    }
    *reinterpret_cast<u32x2*>(blk + (int64_t)(slot0 + j) * a.d + 8 * gl) = o;
  }
  if (leader) scales[sidx] = s_new;
}

// One wave per (block of `blk` <= 16 tokens, K|V, kv-head), four waves to a
// workgroup.  Lanes test 32 tokens for run starts (a run is at most 16
// tokens, so every run that starts in the block ends inside the window).
// Lane groups of L = D/8 lanes hold one 8-element chunk of a row per lane;
// ngroups = 64 / L groups to a wave.
//   RPL == 0 (decode-like steps, blk = min(16, ngroups), about one token per
//     run): the runs starting in the block go round-robin to the groups, one
//     run's 16 rows per group;
//   RPL > 0 (prefill chunks, blk = 16, about one run per block): the whole
//     wave works one run at a time, group g taking rows g, g + ngroups, ...
//     (RPL = 16 / ngroups rows per lane).
template <bool IS_BF16, int RPL>
__global__ void __launch_bounds__(256)
    append_e4m3_amax_kernel(AppendArgs a, float* __restrict__ scales, int nblk) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int kh_count = 2 * a.hkv;
  if (w >= ((int64_t)a.nnz + nblk - 1) / nblk * kh_count) return;
  const int t_blk = uniform((int)(w / kh_count)) * nblk;
  const int kind = uniform((int)(w % kh_count)) / a.hkv;
  const int h = uniform((int)(w % kh_count)) % a.hkv;
  const int L = a.d >> 3;       // lanes per row
  const int ngroups = kWave / L;
  const int grp = lane / L;
  const int gl = lane % L;      // chunk of the row this lane moves
  const uint64_t starts = __builtin_amdgcn_ballot_w64(lane < 32 && starts_run(a, t_blk + lane));
  const uint32_t in_blk = (uint32_t)starts & ((1u << nblk) - 1u);
  const int n_runs = __builtin_popcount(in_blk);
  const uint16_t* src = kind ? a.v + (int64_t)h * a.v_sh : a.k + (int64_t)h * a.k_sh;
  const int64_t sn = kind ? a.v_sn : a.k_sn;
  // the r-th run start of the block, and the run's length
  auto run_of = [&](int r, int* t0, int* n) {
    uint32_t m = in_blk;
    for (int i = 0; i < r; ++i) m &= m - 1;
    const int i0 = __builtin_ctz(m);
    const uint64_t after = (starts >> (i0 + 1)) | (1ull << (31 - i0));
    *t0 = t_blk + i0;
    *n = min((int)__builtin_ctzll(after) + 1, a.nnz - *t0);
  };
  if constexpr (RPL == 0) {
    for (int r0 = 0; r0 < n_runs; r0 += ngroups) {
      const int r = r0 + grp;
      if (r >= n_runs) continue;
      int t0, n;
      run_of(r, &t0, &n);
      if (t0 >= a.nnz) continue;
      amax_run<IS_BF16, kPage>(a, scales, src, sn, t0, n, kind, h, gl, 0, 1, L, gl == 0);
    }
  } else {
    for (int r = 0; r < n_runs; ++r) {
      int t0, n;
      run_of(r, &t0, &n);
      if (t0 >= a.nnz) continue;
      amax_run<IS_BF16, RPL>(a, scales, src, sn, t0, n, kind, h, gl, grp, ngroups, kWave,
                             lane == 0);
    }
  }
}

// ----------------------------------------------------------------------------
// Copy-on-write fork.  One wave per (fork, layer, K|V, kv-head) block: rows
// [0, n) of the block are one contiguous run of n * row_bytes bytes, copied
// 16 bytes per lane.
struct ForkArgs {
  uint8_t* pool;
  float* scales;  // [L, P, 2, Hkv] or null
  const int32_t* src;
  const int32_t* dst;
  const int32_t* valid;  // rows to copy per fork, or null for whole pages
  int32_t n_forks, num_layers, num_pages, hkv, row_bytes;
  int64_t layer_bytes;
  int32_t* err;
};

__global__ void __launch_bounds__(256) fork_pages_kernel(ForkArgs f) {
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & (kWave - 1);
  const int blocks = 2 * f.hkv;  // (K|V, head) blocks per page
  const int64_t per_fork = (int64_t)f.num_layers * blocks;
  const int64_t w = (int64_t)blockIdx.x * 4 + wave;
  if (w >= (int64_t)f.n_forks * per_fork) return;
  const int fi = uniform((int)(w / per_fork));
  const int rem = uniform((int)(w % per_fork));
  const int l = rem / blocks;
  const int kh = rem % blocks;
  const int s = uniform(load_invariant(f.src + fi));
  const int d = uniform(load_invariant(f.dst + fi));
  const int n = f.valid ? uniform(load_invariant(f.valid + fi)) : kPage;
  if (s < 0 || s >= f.num_pages || d < 0 || d >= f.num_pages || n < 0 || n > kPage) {
    if (rem == 0 && lane == 0 && f.err) atomicAdd(f.err, 1);
    return;
  }
  if (s == d) return;
  const int64_t blk_bytes = (int64_t)kPage * f.row_bytes;
  const uint8_t* from = f.pool + l * f.layer_bytes + ((int64_t)s * blocks + kh) * blk_bytes;
  uint8_t* to = f.pool + l * f.layer_bytes + ((int64_t)d * blocks + kh) * blk_bytes;
  const int n16 = n * f.row_bytes / 16;
  for (int c = lane; c < n16; c += kWave)
    reinterpret_cast<u32x4*>(to)[c] = reinterpret_cast<const u32x4*>(from)[c];
  if (f.scales && lane == 0) {
    const int64_t per_layer = (int64_t)f.num_pages * blocks;
    f.scales[l * per_layer + (int64_t)d * blocks + kh] =
        f.scales[l * per_layer + (int64_t)s * blocks + kh];
  }
}

}  // namespace pa

using namespace pa;

extern "C" {

int pagedattn_append_paged_kv_cache_e4m3_amax(
    const void* append_key, const void* append_value, int64_t k_stride_n,
    int64_t k_stride_h, int64_t v_stride_n, int64_t v_stride_h, int32_t src_dtype,
    const int32_t* batch_indices, const int32_t* positions, int32_t nnz,
    void* paged_kv_cache, float* kv_scales, int32_t num_pages, const int32_t* kv_indices,
    int32_t num_indices, const int32_t* kv_indptr, int32_t batch_size,
    int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int32_t* error_flag,
    void* stream) {
  const char* who = "append_paged_kv_cache_e4m3_amax";
  // one 8-element chunk per lane, a row on a power-of-two group of lanes
  if (head_dim > kAmaxMaxD || head_dim < 8 || (head_dim & (head_dim - 1)))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: head_dim %d must be a power of two in [8, %d]", who, head_dim,
                     kAmaxMaxD);
  AppendArgs a;
  bool empty = false;
  int rc = append_setup(who, append_key, append_value, k_stride_n, k_stride_h, v_stride_n,
                        v_stride_h, src_dtype, batch_indices, positions, nnz, paged_kv_cache,
                        PAGEDATTN_E4M3, kv_scales, num_pages, kv_indices, num_indices,
                        kv_indptr, batch_size, num_kv_heads, head_dim, page_size, error_flag,
                        &a, &empty);
  if (rc || empty) return rc;
  // decode-like steps (under 4 new tokens per sequence on average): one run
  // per lane group; else 16-token blocks, each worked by the whole wave
  const int ngroups = 64 / (head_dim / 8);
  const bool per_group = (int64_t)nnz < 4 * (int64_t)std::max(batch_size, 1);
  const int blk = per_group ? std::min(ngroups, 16) : 16;
  const int rpl = std::max(1, 16 / ngroups);
  const int64_t waves = ((int64_t)nnz + blk - 1) / blk * 2 * num_kv_heads;
  if ((waves + 3) / 4 > INT32_MAX)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: %d tokens x %d heads is too many", who,
                     nnz, num_kv_heads);
  const dim3 grid((unsigned)((waves + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  const bool bf16 = src_dtype == PAGEDATTN_BF16;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, a, kv_scales, blk);
  };
  if (per_group) launch(bf16 ? append_e4m3_amax_kernel<true, 0> : append_e4m3_amax_kernel<false, 0>);
  else if (rpl == 8) launch(bf16 ? append_e4m3_amax_kernel<true, 8> : append_e4m3_amax_kernel<false, 8>);
  else if (rpl == 4) launch(bf16 ? append_e4m3_amax_kernel<true, 4> : append_e4m3_amax_kernel<false, 4>);
  else if (rpl == 2) launch(bf16 ? append_e4m3_amax_kernel<true, 2> : append_e4m3_amax_kernel<false, 2>);
  else launch(bf16 ? append_e4m3_amax_kernel<true, 1> : append_e4m3_amax_kernel<false, 1>);
  return check_launch(who);
}

int pagedattn_fork_pages(void* kv_pool, int32_t pool_dtype, int32_t num_layers,
                         int32_t num_pages, int32_t num_kv_heads, int32_t head_dim,
                         int32_t page_size, float* kv_scales, const int32_t* src_pages,
                         const int32_t* dst_pages, const int32_t* valid_tokens,
                         int32_t num_forks, int32_t* error_flag, void* stream) {
  const char* who = "fork_pages";
  if (page_size != kPage)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: page_size %d not supported (16)", who,
                     page_size);
  int esz = 0;
  if (pool_dtype == PAGEDATTN_BF16 || pool_dtype == PAGEDATTN_F16) esz = 2;
  if (pool_dtype == PAGEDATTN_E4M3) esz = 1;
  if (!esz)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: pool dtype %d not supported", who,
                     pool_dtype);
  if (num_forks < 0 || num_layers <= 0 || num_pages < 0 || num_kv_heads <= 0 ||
      head_dim <= 0 || (head_dim * esz) % 16)
    return set_error(PAGEDATTN_ERR_INVALID,
                     "%s: bad shape forks=%d layers=%d pages=%d hkv=%d d=%d (rows must be "
                     "a multiple of 16 bytes)",
                     who, num_forks, num_layers, num_pages, num_kv_heads, head_dim);
  if (pool_dtype == PAGEDATTN_E4M3 && !kv_scales)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: an e4m3 pool needs kv_scales", who);
  if (num_forks == 0 || num_pages == 0) return PAGEDATTN_OK;
  if (!kv_pool || !src_pages || !dst_pages || !aligned16(kv_pool))
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null or misaligned pointer", who);
  const int64_t waves = (int64_t)num_forks * num_layers * 2 * num_kv_heads;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks > INT32_MAX)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: too many forks x layers x heads", who);
  ForkArgs f;
  f.pool = static_cast<uint8_t*>(kv_pool);
  f.scales = kv_scales;
  f.src = src_pages;
  f.dst = dst_pages;
  f.valid = valid_tokens;
  f.n_forks = num_forks;
  f.num_layers = num_layers;
  f.num_pages = num_pages;
  f.hkv = num_kv_heads;
  f.row_bytes = head_dim * esz;
  f.layer_bytes = (int64_t)num_pages * 2 * num_kv_heads * kPage * f.row_bytes;
  f.err = error_flag;
  hipLaunchKernelGGL(fork_pages_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, f);
  return check_launch(who);
}

}  // extern "C"
