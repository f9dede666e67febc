// KV write path of an engine that owns its pages:
//  * e4m3 page append that keeps each (page, K|V, kv-head) scale a running
//    amax while the page fills (power-of-two scales, so growing a scale
//    re-encodes the rows already in the page by an exact exponent shift);
//  * copy-on-write page fork: copy the valid rows of shared pages to fresh
//    pages across every layer of the pool (todo.md:17-19 of the reference
//    asks for it before a sequence appends to a shared partial block).
// Both are HBM-bound byte movers; neither reads a byte twice from HBM.
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

// Token t continues token t - 1 inside one page: same sequence, next
// position, not the first slot of a page.
__device__ __forceinline__ bool continues_run(const AppendArgs& a, int t) {
  const int b0 = load_invariant(a.batch_indices + t - 1);
  const int b1 = load_invariant(a.batch_indices + t);
  const int p0 = load_invariant(a.positions + t - 1);
  const int p1 = load_invariant(a.positions + t);
  return b0 == b1 && (int64_t)p1 == (int64_t)p0 + 1 && (p1 % kPage) != 0;
}

constexpr int kAmaxMaxD = 256;                             // head_dim limit
constexpr int kAmaxChunks = kPage * (kAmaxMaxD / 8) / kWave;  // 8-element chunks per lane

// One wave per (token, K|V, kv-head).  The wave of the first token of a run
// (tokens of one sequence that land in one page, in position order) owns the
// run's (page, K|V, head) block; every other wave exits at once.
//   s_old = scale if the run starts past slot 0, else 0
//   s_new = max(s_old, pow2_scale(amax of the run's rows))
//   s_new > s_old: rows [0, slot0) <- e4m3(decode(row) * (s_old / s_new))
//   run rows <- e4m3(clamp(x / s_new, +-448))   (zero codes when s_new == 0)
template <bool IS_BF16>
__global__ void __launch_bounds__(256)
    append_e4m3_amax_kernel(AppendArgs a, float* __restrict__ scales) {
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & (kWave - 1);
  const int units = 2 * a.hkv;
  const int64_t w = (int64_t)blockIdx.x * 4 + wave;
  if (w >= (int64_t)a.nnz * units) return;
  const int t0 = uniform((int)(w / units));
  const int kind = uniform((int)((w % units) / a.hkv));
  const int h = uniform((int)(w % a.hkv));
  if (t0 > 0 && continues_run(a, t0)) return;
  int t1 = t0 + 1;
  while (t1 < a.nnz && t1 - t0 < kPage && continues_run(a, t1)) ++t1;
  const int n = t1 - t0;
  int slot0 = 0;
  const int64_t page = append_target_page(a, t0, &slot0);
  if (page < 0) {
    if (lane == 0 && kind == 0 && h == 0 && a.err) atomicAdd(a.err, n);
    return;
  }
  const int cpr = a.d >> 3;  // 8-element chunks per row
  const int n_new = n * cpr;
  const uint16_t* src = kind ? a.v + (int64_t)h * a.v_sh : a.k + (int64_t)h * a.k_sh;
  const int64_t sn = kind ? a.v_sn : a.k_sn;

  u32x4 x[kAmaxChunks];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < kAmaxChunks; ++i) {
    const int c = lane + kWave * i;
    x[i] = u32x4{0u, 0u, 0u, 0u};
    if (c < n_new) {
      const int row = c / cpr;
      x[i] = *reinterpret_cast<const u32x4*>(src + (int64_t)(t0 + row) * sn + 8 * (c % cpr));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        amax = fmaxf(amax, fabsf(h2f<IS_BF16>((uint16_t)(x[i][e] & 0xffffu))));
        amax = fmaxf(amax, fabsf(h2f<IS_BF16>((uint16_t)(x[i][e] >> 16))));
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));

  const int64_t sidx = (page * 2 + kind) * a.hkv + h;
  const float s_old = slot0 > 0 ? scales[sidx] : 0.f;
  const float s_new = fmaxf(s_old, pow2_scale_of(amax));
  uint8_t* blk = static_cast<uint8_t*>(a.cache) + sidx * kPage * (int64_t)a.d;

  if (slot0 > 0 && s_new > s_old) {
    const float r = s_old / s_new;
    for (int c = lane; c < slot0 * cpr; c += kWave) {
      float f[8];
      e4m3x8_to_f32(*reinterpret_cast<const u32x2*>(blk + 8 * c), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = fminf(fmaxf(f[e] * r, -448.f), 448.f);
      *reinterpret_cast<u32x2*>(blk + 8 * c) = f32x8_to_e4m3(f);
    }
  }
#pragma unroll
  for (int i = 0; i < kAmaxChunks; ++i) {
    const int c = lane + kWave * i;
    if (c >= n_new) continue;
    u32x2 o = {0u, 0u};
    if (s_new > 0.f) {
      float f[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = h2f<IS_BF16>((uint16_t)(x[i][e] & 0xffffu));
        f[2 * e + 1] = h2f<IS_BF16>((uint16_t)(x[i][e] >> 16));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = fminf(fmaxf(f[e] / s_new, -448.f), 448.f);
      o = f32x8_to_e4m3(f);
    }
    *reinterpret_cast<u32x2*>(blk + (int64_t)slot0 * a.d + 8 * c) = o;
  }
  if (lane == 0) scales[sidx] = s_new;
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
  if (head_dim > kAmaxMaxD)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: head_dim %d above %d", who, head_dim,
                     kAmaxMaxD);
  AppendArgs a;
  bool empty = false;
  int rc = append_setup(who, append_key, append_value, k_stride_n, k_stride_h, v_stride_n,
                        v_stride_h, src_dtype, batch_indices, positions, nnz, paged_kv_cache,
                        PAGEDATTN_E4M3, kv_scales, num_pages, kv_indices, num_indices,
                        kv_indptr, batch_size, num_kv_heads, head_dim, page_size, error_flag,
                        &a, &empty);
  if (rc || empty) return rc;
  const int64_t waves = (int64_t)nnz * 2 * num_kv_heads;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks > INT32_MAX)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: %lld tokens x heads is too many", who,
                     (long long)waves);
  hipStream_t s = (hipStream_t)stream;
  if (src_dtype == PAGEDATTN_BF16)
    hipLaunchKernelGGL(append_e4m3_amax_kernel<true>, dim3((unsigned)blocks), dim3(256), 0,
                       s, a, kv_scales);
  else
    hipLaunchKernelGGL(append_e4m3_amax_kernel<false>, dim3((unsigned)blocks), dim3(256), 0,
                       s, a, kv_scales);
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
