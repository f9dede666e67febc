// Small kernels of the path: batch index / position expansion, RoPE, page
// append (bf16/fp16 copy or e4m3 quantise), fp8 pool builder, HBM copy.
// All are HBM- or latency-bound; none reads a byte twice.
#include <cmath>

#include "append.h"

namespace pa {

// ----------------------------------------------------------------------------
// get_batch_indices_positions (src/models/llama.py:70-83).  One workgroup per
// sequence walks its append range, so the expansion is a single coalesced
// write per token without a search over indptr.
__global__ void __launch_bounds__(256)
    batch_indices_positions_kernel(const int32_t* __restrict__ append_indptr,
                                   const int32_t* __restrict__ seq_lens,
                                   int32_t nnz, int32_t* __restrict__ out_bi,
                                   int32_t* __restrict__ out_pos) {
  const int b = blockIdx.x;
  const int start = append_indptr[b];
  const int end = append_indptr[b + 1];
  const int len = end - start;
  const int base = seq_lens[b] - len;
  const int lo = start < 0 ? 0 : start;
  const int hi = end > nnz ? nnz : end;
  for (int j = lo + (int)threadIdx.x; j < hi; j += blockDim.x) {
    out_bi[j] = b;
    out_pos[j] = base + (j - start);
  }
}

// ----------------------------------------------------------------------------
// RoPE in place on strided q and k (src/models/llama.py:175-182).  One thread
// per (token, rotation pair) computes sin/cos once and rotates that pair in
// every q and k head, so the transcendental cost is paid once per token and
// frequency rather than once per head.  The angle (pos / scale) * inv_freq is
// formed and reduced modulo 2 pi in fp64 (cheap on CDNA4), so positions up
// to 128K keep full fp32 accuracy in sin/cos; the rotation itself is fp32.
template <bool IS_BF16>
__global__ void __launch_bounds__(256)
    rope_kernel(uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                const int32_t* __restrict__ pos_ids, int32_t nnz, int32_t hq,
                int32_t hkv, int32_t rotary_dim, int64_t q_sn, int64_t q_sh,
                int64_t k_sn, int64_t k_sh, int32_t interleave,
                double inv_rope_scale, double log2_theta) {
  const int half = rotary_dim >> 1;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)nnz * half) return;
  const int j = (int)(t / half);
  const int i = (int)(t % half);
  float s, c;
  rope_cos_sin(pos_ids[j], i, rotary_dim, inv_rope_scale, log2_theta, &c, &s);
  const int i0 = interleave ? 2 * i : i;
  const int i1 = interleave ? 2 * i + 1 : i + half;
  for (int h = 0; h < hq + hkv; ++h) {
    uint16_t* x = h < hq ? q + (int64_t)j * q_sn + (int64_t)h * q_sh
                         : k + (int64_t)j * k_sn + (int64_t)(h - hq) * k_sh;
    float y0, y1;
    rope_rotate(h2f<IS_BF16>(x[i0]), h2f<IS_BF16>(x[i1]), c, s, &y0, &y1);
    x[i0] = f2h<IS_BF16>(y0);
    x[i1] = f2h<IS_BF16>(y1);
  }
}

// ----------------------------------------------------------------------------
// Writes one 8-element chunk of a K (kind 0) or V (kind 1) row of head h to
// slot `slot` of `page`.  e4m3 pools: quantised with the page's fixed scale
// (quant8_e4m3); a clamped chunk is counted in a.err[1].
template <bool IS_BF16, bool TO_FP8>
__device__ __forceinline__ void store_chunk(const AppendArgs& a, int64_t page, int slot,
                                            int kind, int h, int d0, u32x4 x) {
  const int64_t dst_elem =
      (((page * 2 + kind) * a.hkv + h) * kPage + slot) * (int64_t)a.d + d0;
  if constexpr (!TO_FP8) {
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.cache) + dst_elem) = x;
  } else {
    const float scale = a.scales[(page * 2 + kind) * a.hkv + h];
    bool clamped = false;
    const u32x2 o = quant8_e4m3<IS_BF16>(x, scale, &clamped);
    *reinterpret_cast<u32x2*>(static_cast<uint8_t*>(a.cache) + dst_elem) = o;
    count_lanes(a.err ? a.err + 1 : nullptr, clamped);
  }
}

// append_paged_kv_cache (src/models/llama.py:188-210), HND pool.  One thread
// moves one 16-byte chunk (8 elements) of one head of K or V, so a wave
// writes whole 128/256-byte page rows.  Metadata outside its ranges skips the
// token and bumps err[0] instead of faulting (once per token); e4m3 chunks
// whose values were clamped bump err[1] once per chunk.
template <bool FP8_IS_BF16_SRC, bool TO_FP8>
__global__ void __launch_bounds__(256) append_kernel(AppendArgs a) {
  const int chunks = a.d >> 3;  // 8 elements per chunk
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.nnz * 2 * a.hkv * chunks;
  if (t >= total) return;
  const int c = (int)(t % chunks);
  const int h = (int)((t / chunks) % a.hkv);
  const int kind = (int)((t / ((int64_t)chunks * a.hkv)) & 1);
  const int j = (int)(t / ((int64_t)chunks * a.hkv * 2));
  int slot = 0;
  const int64_t page = append_target_page(a, j, &slot);
  if (page < 0) {
    count_lanes(a.err, c == 0 && h == 0 && kind == 0);
    return;
  }
  const uint16_t* src = kind ? a.v + (int64_t)j * a.v_sn + (int64_t)h * a.v_sh
                             : a.k + (int64_t)j * a.k_sn + (int64_t)h * a.k_sh;
  store_chunk<FP8_IS_BF16_SRC, TO_FP8>(a, page, slot, kind, h, c * 8,
                                       *reinterpret_cast<const u32x4*>(src + c * 8));
}

// ----------------------------------------------------------------------------
// RoPE + append in one launch: what apply_rope_pos_ids_inplace
// (src/models/llama.py:175-182, non-interleaved, full head) followed by
// append_paged_kv_cache (:188-210) do.  Threads [0, nnz * D/16) own (token,
// frequency chunk of 8): sin/cos once, then every q head rotated in place and
// every k head rotated in place and written to its page slot.  The remaining
// threads copy the V rows, one 16-byte chunk each.
struct RopeAppendArgs {
  AppendArgs a;
  uint16_t* q;
  int64_t q_sn, q_sh;
  int32_t hq;
  double inv_scale, log2_theta;
};

template <bool IS_BF16, bool TO_FP8>
__global__ void __launch_bounds__(256) rope_append_kernel(RopeAppendArgs r) {
  const AppendArgs& a = r.a;
  const int d = a.d;
  const int nrot = d >> 4;  // frequency chunks of 8 per token
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n_rot = (int64_t)a.nnz * nrot;
  if (t < n_rot) {
    const int j = (int)(t / nrot);
    const int c = (int)(t % nrot);
    float cs[8], sn[8];
    const int pos = a.positions[j];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      rope_cos_sin(pos, 8 * c + e, d, r.inv_scale, r.log2_theta, &cs[e], &sn[e]);
    for (int h = 0; h < r.hq; ++h) {
      uint16_t* x = r.q + (int64_t)j * r.q_sn + (int64_t)h * r.q_sh;
      u32x4 lo = *reinterpret_cast<const u32x4*>(x + 8 * c);
      u32x4 hi = *reinterpret_cast<const u32x4*>(x + 8 * c + d / 2);
      rope8<IS_BF16>(lo, hi, cs, sn);
      *reinterpret_cast<u32x4*>(x + 8 * c) = lo;
      *reinterpret_cast<u32x4*>(x + 8 * c + d / 2) = hi;
    }
    int slot = 0;
    const int64_t page = append_target_page(a, j, &slot);
    count_lanes(a.err, page < 0 && c == 0);
    for (int h = 0; h < a.hkv; ++h) {
      uint16_t* x = const_cast<uint16_t*>(a.k) + (int64_t)j * a.k_sn + (int64_t)h * a.k_sh;
      u32x4 lo = *reinterpret_cast<const u32x4*>(x + 8 * c);
      u32x4 hi = *reinterpret_cast<const u32x4*>(x + 8 * c + d / 2);
      rope8<IS_BF16>(lo, hi, cs, sn);
      *reinterpret_cast<u32x4*>(x + 8 * c) = lo;
      *reinterpret_cast<u32x4*>(x + 8 * c + d / 2) = hi;
      if (page >= 0) {
        store_chunk<IS_BF16, TO_FP8>(a, page, slot, 0, h, 8 * c, lo);
        store_chunk<IS_BF16, TO_FP8>(a, page, slot, 0, h, 8 * c + d / 2, hi);
      }
    }
    return;
  }
  const int chunks = d >> 3;
  const int64_t u = t - n_rot;
  if (u >= (int64_t)a.nnz * a.hkv * chunks) return;
  const int c = (int)(u % chunks);
  const int h = (int)((u / chunks) % a.hkv);
  const int j = (int)(u / ((int64_t)chunks * a.hkv));
  int slot = 0;
  const int64_t page = append_target_page(a, j, &slot);
  if (page < 0) return;
  const u32x4 x = *reinterpret_cast<const u32x4*>(a.v + (int64_t)j * a.v_sn +
                                                  (int64_t)h * a.v_sh + 8 * c);
  store_chunk<IS_BF16, TO_FP8>(a, page, slot, 1, h, 8 * c, x);
}

// ----------------------------------------------------------------------------
// fp8 pool builder: one workgroup per (page, K|V, head) block of 16 x D
// elements; amax through an LDS tree, then quantise the block it still holds
// in registers.
template <bool IS_BF16>
__global__ void __launch_bounds__(256)
    quantize_pages_kernel(const uint16_t* __restrict__ src,
                          uint8_t* __restrict__ dst,
                          float* __restrict__ scales, int32_t block_elems) {
  __shared__ float red[256 / kWave];
  const int64_t blk = blockIdx.x;
  const uint16_t* s = src + blk * block_elems;
  uint8_t* o = dst + blk * block_elems;
  // block_elems = 16 * D <= 2048 = 256 threads x 8 elements
  const int e0 = threadIdx.x * 8;
  const bool active = e0 < block_elems;
  float f[8];
  float amax = 0.f;
  if (active) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(s + e0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = h2f<IS_BF16>((uint16_t)(x[e] & 0xffffu));
      f[2 * e + 1] = h2f<IS_BF16>((uint16_t)(x[e] >> 16));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < 256 / kWave; ++w) amax = fmaxf(amax, red[w]);
  float scale = amax / 448.f;
  if (!(scale > 0.f)) scale = 1.f;
  if (threadIdx.x == 0) scales[blk] = scale;
  if (active) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = fminf(fmaxf(f[e] / scale, -448.f), 448.f);
    u32x2 w;
    w[0] = f32_to_e4m3x4(f[0], f[1], f[2], f[3]);
    w[1] = f32_to_e4m3x4(f[4], f[5], f[6], f[7]);
    *reinterpret_cast<u32x2*>(o + e0) = w;
  }
}

// ----------------------------------------------------------------------------
// plain 16-byte streaming copy, grid-stride
__global__ void __launch_bounds__(256)
    copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += stride)
    dst[i] = src[i];
}

// plain streaming read, grid-stride, 16 bytes per thread and step: each
// workgroup XOR-reduces what it read and writes one dword to sink[blockIdx],
// so the kernel's HBM traffic is the read plus a few KiB of writes
__global__ void __launch_bounds__(256)
    read_kernel(const u32x4* __restrict__ src, int64_t n16, uint32_t* __restrict__ sink) {
  __shared__ uint32_t red[256 / kWave];
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  uint32_t x = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const u32x4 v = src[i];
    x ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x ^= __shfl_xor(x, off);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < 256 / kWave; ++w) r ^= red[w];
    sink[blockIdx.x] = r;
  }
}

}  // namespace pa

using namespace pa;

extern "C" {

int pagedattn_get_batch_indices_positions(const int32_t* append_indptr,
                                          const int32_t* seq_lens,
                                          int32_t batch_size, int32_t nnz,
                                          int32_t* batch_indices,
                                          int32_t* positions, void* stream) {
  if (batch_size < 0 || nnz < 0)
    return set_error(PAGEDATTN_ERR_INVALID,
                     "get_batch_indices_positions: negative batch_size (%d) or "
                     "nnz (%d)",
                     batch_size, nnz);
  if (batch_size == 0 || nnz == 0) return PAGEDATTN_OK;
  if (!append_indptr || !seq_lens || !batch_indices || !positions)
    return set_error(PAGEDATTN_ERR_INVALID,
                     "get_batch_indices_positions: null pointer");
  hipLaunchKernelGGL(batch_indices_positions_kernel, dim3(batch_size),
                     dim3(256), 0, (hipStream_t)stream, append_indptr, seq_lens,
                     nnz, batch_indices, positions);
  return check_launch("get_batch_indices_positions");
}

int pagedattn_apply_rope_pos_ids_inplace(
    void* q, void* k, const int32_t* pos_ids, int32_t nnz,
    int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t rotary_dim, int64_t q_stride_n, int64_t q_stride_h,
    int64_t k_stride_n, int64_t k_stride_h, int32_t interleave,
    float rope_scale, float rope_theta, int32_t dtype, void* stream) {
  if (dtype != PAGEDATTN_BF16 && dtype != PAGEDATTN_F16)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "apply_rope_pos_ids_inplace: dtype %d not supported "
                     "(float16 or bfloat16)",
                     dtype);
  if (nnz < 0 || num_qo_heads < 0 || num_kv_heads < 0 || head_dim <= 0)
    return set_error(PAGEDATTN_ERR_INVALID,
                     "apply_rope_pos_ids_inplace: bad shape nnz=%d hq=%d "
                     "hkv=%d d=%d",
                     nnz, num_qo_heads, num_kv_heads, head_dim);
  if (rotary_dim <= 0) rotary_dim = head_dim;
  if (rotary_dim > head_dim || (rotary_dim & 1))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "apply_rope_pos_ids_inplace: rotary_dim %d must be even "
                     "and <= head_dim %d",
                     rotary_dim, head_dim);
  if (!(rope_scale > 0.f) || !(rope_theta > 0.f))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "apply_rope_pos_ids_inplace: rope_scale and rope_theta "
                     "must be positive");
  if (nnz == 0 || num_qo_heads + num_kv_heads == 0) return PAGEDATTN_OK;
  if (!pos_ids || (num_qo_heads && !q) || (num_kv_heads && !k))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "apply_rope_pos_ids_inplace: null pointer");
  const int64_t threads = (int64_t)nnz * (rotary_dim / 2);
  const dim3 grid((unsigned)((threads + 255) / 256));
  const double inv_scale = 1.0 / (double)rope_scale;
  const double log2_theta = std::log2((double)rope_theta);
  if (dtype == PAGEDATTN_BF16)
    hipLaunchKernelGGL(rope_kernel<true>, grid, dim3(256), 0,
                       (hipStream_t)stream, (uint16_t*)q, (uint16_t*)k, pos_ids,
                       nnz, num_qo_heads, num_kv_heads, rotary_dim, q_stride_n,
                       q_stride_h, k_stride_n, k_stride_h, interleave,
                       inv_scale, log2_theta);
  else
    hipLaunchKernelGGL(rope_kernel<false>, grid, dim3(256), 0,
                       (hipStream_t)stream, (uint16_t*)q, (uint16_t*)k, pos_ids,
                       nnz, num_qo_heads, num_kv_heads, rotary_dim, q_stride_n,
                       q_stride_h, k_stride_n, k_stride_h, interleave,
                       inv_scale, log2_theta);
  return check_launch("apply_rope_pos_ids_inplace");
}

}  // extern "C"

namespace pa {

int append_setup(const char* who, const void* append_key, const void* append_value,
                 int64_t k_stride_n, int64_t k_stride_h, int64_t v_stride_n,
                 int64_t v_stride_h, int32_t src_dtype, const int32_t* batch_indices,
                 const int32_t* positions, int32_t nnz, void* paged_kv_cache,
                 int32_t cache_dtype, const float* kv_scales, int32_t num_pages,
                 const int32_t* kv_indices, int32_t num_indices, const int32_t* kv_indptr,
                 int32_t batch_size, int32_t num_kv_heads, int32_t head_dim,
                 int32_t page_size, int32_t* error_flag, AppendArgs* a, bool* empty) {
  *empty = false;
  if (page_size != kPage)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: page_size %d not supported (16)", who,
                     page_size);
  if (src_dtype != PAGEDATTN_BF16 && src_dtype != PAGEDATTN_F16)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: source dtype %d not supported", who,
                     src_dtype);
  if (cache_dtype != src_dtype && cache_dtype != PAGEDATTN_E4M3)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: cache dtype %d must equal the source dtype %d or be e4m3", who,
                     cache_dtype, src_dtype);
  if (cache_dtype == PAGEDATTN_E4M3 && !kv_scales)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: e4m3 cache needs kv_scales", who);
  if (nnz < 0 || batch_size < 0 || num_pages < 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      (head_dim & 7))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "%s: bad shape nnz=%d batch=%d pages=%d hkv=%d d=%d (d must be a "
                     "multiple of 8)",
                     who, nnz, batch_size, num_pages, num_kv_heads, head_dim);
  if ((k_stride_n & 7) || (k_stride_h & 7) || (v_stride_n & 7) || (v_stride_h & 7) ||
      !aligned16(append_key) || !aligned16(append_value) || !aligned16(paged_kv_cache))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: k/v/cache must be 16-byte aligned with strides that are "
                     "multiples of 8 elements",
                     who);
  if (nnz == 0) {
    *empty = true;
    return PAGEDATTN_OK;
  }
  if (!append_key || !append_value || !batch_indices || !positions || !paged_kv_cache ||
      !kv_indices || !kv_indptr)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null pointer", who);
  a->k = (const uint16_t*)append_key;
  a->v = (const uint16_t*)append_value;
  a->k_sn = k_stride_n;
  a->k_sh = k_stride_h;
  a->v_sn = v_stride_n;
  a->v_sh = v_stride_h;
  a->batch_indices = batch_indices;
  a->positions = positions;
  a->nnz = nnz;
  a->cache = paged_kv_cache;
  a->scales = kv_scales;
  a->num_pages = num_pages;
  a->kv_indices = kv_indices;
  a->num_indices = num_indices;
  a->kv_indptr = kv_indptr;
  a->batch_size = batch_size;
  a->hkv = num_kv_heads;
  a->d = head_dim;
  a->err = error_flag;
  return PAGEDATTN_OK;
}

}  // namespace pa

extern "C" {

int pagedattn_append_paged_kv_cache(
    const void* append_key, const void* append_value, int64_t k_stride_n,
    int64_t k_stride_h, int64_t v_stride_n, int64_t v_stride_h,
    int32_t src_dtype, const int32_t* batch_indices, const int32_t* positions,
    int32_t nnz, void* paged_kv_cache, int32_t cache_dtype,
    const float* kv_scales, int32_t num_pages, const int32_t* kv_indices,
    int32_t num_indices, const int32_t* kv_indptr,
    const int32_t* kv_last_page_len, int32_t batch_size, int32_t num_kv_heads,
    int32_t head_dim, int32_t page_size, int32_t* error_flag, void* stream) {
  (void)kv_last_page_len;  // not used for addressing, as in the reference
  AppendArgs a;
  bool empty = false;
  int rc = append_setup("append_paged_kv_cache", append_key, append_value, k_stride_n,
                        k_stride_h, v_stride_n, v_stride_h, src_dtype, batch_indices,
                        positions, nnz, paged_kv_cache, cache_dtype, kv_scales, num_pages,
                        kv_indices, num_indices, kv_indptr, batch_size, num_kv_heads,
                        head_dim, page_size, error_flag, &a, &empty);
  if (rc || empty) return rc;
  const int64_t threads = (int64_t)nnz * 2 * num_kv_heads * (head_dim / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (cache_dtype != PAGEDATTN_E4M3)
    hipLaunchKernelGGL((append_kernel<true, false>), grid, dim3(256), 0, s, a);
  else if (src_dtype == PAGEDATTN_BF16)
    hipLaunchKernelGGL((append_kernel<true, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((append_kernel<false, true>), grid, dim3(256), 0, s, a);
  return check_launch("append_paged_kv_cache");
}

int pagedattn_rope_append_paged_kv_cache(
    void* q, int64_t q_stride_n, int64_t q_stride_h, int32_t num_qo_heads,
    void* append_key, const void* append_value, int64_t k_stride_n,
    int64_t k_stride_h, int64_t v_stride_n, int64_t v_stride_h,
    int32_t src_dtype, const int32_t* batch_indices, const int32_t* positions,
    int32_t nnz, float rope_scale, float rope_theta, void* paged_kv_cache,
    int32_t cache_dtype, const float* kv_scales, int32_t num_pages,
    const int32_t* kv_indices, int32_t num_indices, const int32_t* kv_indptr,
    int32_t batch_size, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
    int32_t* error_flag, void* stream) {
  const char* who = "rope_append_paged_kv_cache";
  if (!(rope_scale > 0.f) || !(rope_theta > 0.f))
    return set_error(PAGEDATTN_ERR_INVALID, "%s: rope_scale and rope_theta must be > 0",
                     who);
  if (num_qo_heads < 0 || (head_dim & 15))
    return set_error(PAGEDATTN_ERR_INVALID, "%s: bad shape hq=%d d=%d (d must be a "
                     "multiple of 16)", who, num_qo_heads, head_dim);
  if ((q_stride_n & 7) || (q_stride_h & 7) || !aligned16(q))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: q must be 16-byte aligned with strides that are multiples "
                     "of 8 elements", who);
  AppendArgs a;
  bool empty = false;
  int rc = append_setup(who, append_key, append_value, k_stride_n, k_stride_h, v_stride_n,
                        v_stride_h, src_dtype, batch_indices, positions, nnz, paged_kv_cache,
                        cache_dtype, kv_scales, num_pages, kv_indices, num_indices, kv_indptr,
                        batch_size, num_kv_heads, head_dim, page_size, error_flag, &a, &empty);
  if (rc || empty) return rc;
  if (num_qo_heads > 0 && !q)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null q", who);
  RopeAppendArgs r;
  r.a = a;
  r.q = static_cast<uint16_t*>(q);
  r.q_sn = q_stride_n;
  r.q_sh = q_stride_h;
  r.hq = num_qo_heads;
  r.inv_scale = 1.0 / (double)rope_scale;
  r.log2_theta = std::log2((double)rope_theta);
  const int64_t threads = (int64_t)nnz * (head_dim / 16) +
                          (int64_t)nnz * num_kv_heads * (head_dim / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  const bool bf16 = src_dtype == PAGEDATTN_BF16;
  if (cache_dtype != PAGEDATTN_E4M3) {
    if (bf16)
      hipLaunchKernelGGL((rope_append_kernel<true, false>), grid, dim3(256), 0, s, r);
    else
      hipLaunchKernelGGL((rope_append_kernel<false, false>), grid, dim3(256), 0, s, r);
  } else {
    if (bf16)
      hipLaunchKernelGGL((rope_append_kernel<true, true>), grid, dim3(256), 0, s, r);
    else
      hipLaunchKernelGGL((rope_append_kernel<false, true>), grid, dim3(256), 0, s, r);
  }
  return check_launch(who);
}

int pagedattn_quantize_pages_e4m3(const void* src_cache, int32_t src_dtype,
                                  void* dst_cache, float* scales,
                                  int32_t num_pages, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t page_size,
                                  void* stream) {
  if (page_size != kPage || (head_dim != 64 && head_dim != 128))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "quantize_pages_e4m3: page_size 16 and head_dim 64/128 "
                     "only (got %d, %d)",
                     page_size, head_dim);
  if (src_dtype != PAGEDATTN_BF16 && src_dtype != PAGEDATTN_F16)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "quantize_pages_e4m3: source dtype %d not supported",
                     src_dtype);
  if (num_pages < 0 || num_kv_heads <= 0)
    return set_error(PAGEDATTN_ERR_INVALID,
                     "quantize_pages_e4m3: bad shape pages=%d hkv=%d",
                     num_pages, num_kv_heads);
  if (num_pages == 0) return PAGEDATTN_OK;
  if (!src_cache || !dst_cache || !scales || !aligned16(src_cache) ||
      ((uintptr_t)dst_cache & 7))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "quantize_pages_e4m3: null or misaligned pointer");
  const int64_t blocks = (int64_t)num_pages * 2 * num_kv_heads;
  const int block_elems = kPage * head_dim;
  if (src_dtype == PAGEDATTN_BF16)
    hipLaunchKernelGGL(quantize_pages_kernel<true>, dim3((unsigned)blocks),
                       dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)src_cache, (uint8_t*)dst_cache, scales,
                       block_elems);
  else
    hipLaunchKernelGGL(quantize_pages_kernel<false>, dim3((unsigned)blocks),
                       dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)src_cache, (uint8_t*)dst_cache, scales,
                       block_elems);
  return check_launch("quantize_pages_e4m3");
}

int pagedattn_read_bytes(const void* src, size_t bytes, uint32_t* sink,
                         int32_t sink_entries, void* stream) {
  if ((bytes & 15) || !aligned16(src))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "read_bytes: size and pointer must be 16-byte aligned");
  if (bytes == 0) return PAGEDATTN_OK;
  if (!sink || sink_entries <= 0)
    return set_error(PAGEDATTN_ERR_INVALID, "read_bytes: null or empty sink");
  const int64_t n16 = (int64_t)(bytes / 16);
  int cus = device_cu_count();
  if (cus <= 0) cus = 256;
  int64_t blocks = (n16 + 255) / 256;
  if (blocks > (int64_t)cus * 8) blocks = (int64_t)cus * 8;
  if (blocks > sink_entries) blocks = sink_entries;
  hipLaunchKernelGGL(read_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const u32x4*)src, n16, sink);
  return check_launch("read_bytes");
}

int pagedattn_copy_bytes(void* dst, const void* src, size_t bytes,
                         void* stream) {
  if ((bytes & 15) || !aligned16(dst) || !aligned16(src))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "copy_bytes: size and pointers must be 16-byte aligned");
  if (bytes == 0) return PAGEDATTN_OK;
  const int64_t n16 = (int64_t)(bytes / 16);
  int cus = device_cu_count();
  if (cus <= 0) cus = 256;
  int64_t blocks = (n16 + 255) / 256;
  if (blocks > (int64_t)cus * 8) blocks = (int64_t)cus * 8;
  hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, (u32x4*)dst, (const u32x4*)src, n16);
  return check_launch("copy_bytes");
}

}  // extern "C"
