// Paged decode attention for gfx950 (BatchDecodeWithPagedKVCacheWrapper,
// src/models/llama.py:119-147 plan and :230-245 run).
//
// Work unit: (page range of one sequence, one KV head) for all g = Hq/Hkv
// query heads of that head's group, so each K/V byte is read from HBM once.
// A 256-thread workgroup runs 4 waves; wave w takes page pairs w, w+4, ...
// of its range and keeps its own online-softmax state, merged through LDS at
// the end of the range.
//
// Per page pair (32 tokens) one wave does:
//   S^T[32 tok x 16 heads] = K[tok x D] . Q^T      (v_mfma_f32_16x16x32, D/32 k-steps per page)
//   O^T[D x 16 heads]     += V^T[D x 32 tok] . P^T (D/16 MFMAs, K = the 32 tokens)
// Query heads occupy the MFMA N dimension (g <= 16, padded), tokens the
// M dimension of QK, so a lane's softmax values all belong to one head and the
// row max needs two cross-group shuffles only.
//
// Loads go through buffer resources sized to the valid tokens of each page:
// absent pages (num_records = 0) and slots past last_page_len read as zero
// without touching HBM, so the loop issues a fixed number of loads per pair
// and the compiler can keep the next pair's loads in flight while the
// current one is computed (two register stages, ping-pong).
//
// K rows are read as 16-byte (bf16/fp16) or 8-byte (e4m3) pieces in the
// MFMA A-operand layout (lane -> token row, 8 consecutive d).  V rows are
// read as W = D/16 consecutive d per lane (lane n owns d in [W n, W n + W)),
// which gives W PV tiles whose row m is d = W m + e; the 8 tokens a lane
// needs for one tile come from its own 8 loads, repacked with bit ops.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "plan_internal.h"

namespace pa {

struct DecodeParams {
  const DecodeItem* items;
  const int32_t* wg_ptr;  // [gridDim.x + 1]: items of workgroup x
  const uint16_t* q;
  int64_t q_sn, q_sh;
  const uint8_t* cache;
  const float* kv_scales;
  int32_t num_pages;
  const int32_t* kv_indices;
  int32_t num_indices;
  const int32_t* kv_indptr;
  const int32_t* last_page_len;
  uint16_t* out;
  float* lse;
  float* partial_o;
  float* partial_lse;
  int32_t hq, hkv, g;
  float scale_log2;  // sm_scale * log2(e)
};

template <int N>
struct RawT;
template <>
struct RawT<16> {
  using type = u32x4;
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r,
                                              uint32_t off) {
    return buf_load16(r, off);
  }
};
template <>
struct RawT<8> {
  using type = u32x2;
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r,
                                              uint32_t off) {
    return buf_load8(r, off);
  }
};
template <>
struct RawT<4> {
  using type = uint32_t;
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r,
                                              uint32_t off) {
    return buf_load4(r, off);
  }
};

template <typename T>
__device__ __forceinline__ uint32_t dword_of(const T& v, int i) {
  if constexpr (sizeof(T) == 4) {
    return v;
  } else {
    return v[i];
  }
}

// e4m3 -> 16-bit conversions through gfx950's scaled converters with a
// unit scale: every e4m3 value is exact in bf16 and fp16.  (Extracting the
// halves of v_cvt_pk_f32_fp8's fp32 pair instead is folded incorrectly by
// this compiler: element 1 is replaced by element 0.)
template <bool BF16, bool HI>
__device__ __forceinline__ uint32_t e4m3x2_to_16(uint32_t w) {
  if constexpr (BF16) {
    return __builtin_bit_cast(
        uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
  } else {
    return __builtin_bit_cast(
        uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
}

// 8 e4m3 bytes -> 8 sixteen-bit values (bf16 or fp16), exact.
template <bool BF16>
__device__ __forceinline__ u32x4 e4m3x8_to_16(uint32_t lo, uint32_t hi) {
  u32x4 r;
  r[0] = e4m3x2_to_16<BF16, false>(lo);
  r[1] = e4m3x2_to_16<BF16, true>(lo);
  r[2] = e4m3x2_to_16<BF16, false>(hi);
  r[3] = e4m3x2_to_16<BF16, true>(hi);
  return r;
}

// 4 e4m3 bytes -> 4 sixteen-bit values.
template <bool BF16>
__device__ __forceinline__ u32x2 e4m3x4_to_16(uint32_t w) {
  u32x2 r;
  r[0] = e4m3x2_to_16<BF16, false>(w);
  r[1] = e4m3x2_to_16<BF16, true>(w);
  return r;
}

template <bool BF16>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
        0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)f2h<BF16>(a) | ((uint32_t)f2h<BF16>(b) << 16);
}

// pages whose ids are staged in LDS at a time
constexpr int kSegPages = 1024;

template <int D, bool BF16, bool FP8>
struct DecodeTraits {
  static constexpr int ESZ = FP8 ? 1 : 2;
  static constexpr int KS = D / 32;          // QK k-steps per page
  static constexpr int W = D / 16;           // V elements per lane per token
  static constexpr int KB = 8 * ESZ;         // K bytes per lane per k-step
  static constexpr int VB = W * ESZ;         // V bytes per lane per token
  static constexpr int PAGE_BYTES = kPage * D * ESZ;
  using KRaw = typename RawT<KB>::type;
  using VRaw = typename RawT<VB>::type;
};

template <int D, bool BF16, bool FP8>
struct Stage {
  using Tr = DecodeTraits<D, BF16, FP8>;
  typename Tr::KRaw k[2][Tr::KS];
  typename Tr::VRaw v[8];
  int ntok[2];
  float kscale[2], vscale[2];
};

// Page ids of the current segment live in LDS (staged once per segment), so
// issuing a pair's loads costs one LDS read instead of a dependent HBM round
// trip for the page id.  sm_pages[i] < 0 marks an absent or invalid page.
template <int D, bool BF16, bool FP8>
__device__ __forceinline__ void load_pair(Stage<D, BF16, FP8>& st,
                                          const DecodeParams& p, int h,
                                          const int* sm_pages, int seg_lo,
                                          int seg_hi, int npages, int last,
                                          int pg0, int n, int G) {
  using Tr = DecodeTraits<D, BF16, FP8>;
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) {
    const int pg = pg0 + pi;
    int page = pg < seg_hi ? uniform(sm_pages[pg - seg_lo]) : -1;
    const int ntok = page < 0 ? 0 : (pg == npages - 1 ? last : kPage);
    page = page < 0 ? 0 : page;
    st.ntok[pi] = ntok;
    const uint8_t* kbase =
        p.cache + ((int64_t)page * 2 * p.hkv + h) * (int64_t)Tr::PAGE_BYTES;
    const uint8_t* vbase = kbase + (int64_t)p.hkv * Tr::PAGE_BYTES;
    const uint32_t bytes = (uint32_t)(ntok * D * Tr::ESZ);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, bytes);
#pragma unroll
    for (int ks = 0; ks < Tr::KS; ++ks)
      st.k[pi][ks] = RawT<Tr::KB>::load(
          rk, (uint32_t)((n * D + 32 * ks + 8 * G) * Tr::ESZ));
#pragma unroll
    for (int r = 0; r < 4; ++r)
      st.v[pi * 4 + r] = RawT<Tr::VB>::load(
          rv, (uint32_t)(((4 * G + r) * D + Tr::W * n) * Tr::ESZ));
    if constexpr (FP8) {
      const int64_t si = ((int64_t)page * 2) * p.hkv + h;
      st.kscale[pi] = ntok ? p.kv_scales[si] : 0.f;
      st.vscale[pi] = ntok ? p.kv_scales[si + p.hkv] : 0.f;
    }
  }
}

template <int D, bool BF16, bool FP8>
struct SoftmaxState {
  f32x4 o[D / 16];
  float m, l;
};

template <int D, bool BF16, bool FP8>
__device__ __forceinline__ void compute_pair(const Stage<D, BF16, FP8>& st,
                                             const u32x4 (&qf)[D / 32],
                                             SoftmaxState<D, BF16, FP8>& sm,
                                             float scale_log2, int G) {
  using Tr = DecodeTraits<D, BF16, FP8>;
  constexpr int W = Tr::W;
  // ---- S^T = K . Q^T for both pages
  f32x4 s4[2];
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < Tr::KS; ++ks) {
      u32x4 a;
      if constexpr (FP8) {
        a = e4m3x8_to_16<BF16>(st.k[pi][ks][0], st.k[pi][ks][1]);
      } else {
        a = st.k[pi][ks];
      }
      acc = mfma16<BF16>(a, qf[ks], acc);
    }
    s4[pi] = acc;
  }
  float s[8];
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) {
    const float c = FP8 ? scale_log2 * st.kscale[pi] : scale_log2;
#pragma unroll
    for (int r = 0; r < 4; ++r) s[pi * 4 + r] = s4[pi][r] * c;
  }
  if (st.ntok[0] < kPage || st.ntok[1] < kPage) {
#pragma unroll
    for (int pi = 0; pi < 2; ++pi)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (4 * G + r >= st.ntok[pi]) s[pi * 4 + r] = -INFINITY;
  }
  // ---- online softmax (all 8 values of a lane belong to its head)
  float mx = s[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) mx = fmaxf(mx, s[j]);
  mx = max_over_groups16(mx);
  const float m_new = fmaxf(sm.m, mx);
  const float m_use = m_new == -INFINITY ? 0.f : m_new;
  const float alpha = exp2f(sm.m - m_use);
  float pr[8];
  float psum = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pr[j] = exp2f(s[j] - m_use);
    psum += pr[j];
  }
  sm.l = sm.l * alpha + psum;
  sm.m = m_new;
#pragma unroll
  for (int e = 0; e < W; ++e) sm.o[e] *= alpha;
  if constexpr (FP8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) pr[j] *= st.vscale[j >> 2];
  }
  u32x4 pb;
#pragma unroll
  for (int i = 0; i < 4; ++i) pb[i] = pack2<BF16>(pr[2 * i], pr[2 * i + 1]);
  // ---- V rows as 16-bit values: lane holds W consecutive d per token
  uint32_t vw[8][W / 2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (FP8) {
      if constexpr (W == 8) {
        const u32x4 c = e4m3x8_to_16<BF16>(dword_of(st.v[j], 0),
                                           dword_of(st.v[j], 1));
#pragma unroll
        for (int i = 0; i < 4; ++i) vw[j][i] = c[i];
      } else {
        const u32x2 c = e4m3x4_to_16<BF16>(dword_of(st.v[j], 0));
        vw[j][0] = c[0];
        vw[j][1] = c[1];
      }
    } else {
#pragma unroll
      for (int i = 0; i < W / 2; ++i) vw[j][i] = dword_of(st.v[j], i);
    }
  }
  // ---- O^T += V^T . P^T, one MFMA per d offset e (tile rows d = W m + e)
#pragma unroll
  for (int e = 0; e < W; ++e) {
    u32x4 a;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t x0 = vw[2 * i][e >> 1];
      const uint32_t x1 = vw[2 * i + 1][e >> 1];
      a[i] = (e & 1) ? ((x0 >> 16) | (x1 & 0xffff0000u))
                     : ((x0 & 0xffffu) | (x1 << 16));
    }
    sm.o[e] = mfma16<BF16>(a, pb, sm.o[e]);
  }
}

template <int D, bool BF16, bool FP8>
__global__ void __launch_bounds__(256, 2) decode_kernel(DecodeParams p) {
  using Tr = DecodeTraits<D, BF16, FP8>;
  constexpr int W = Tr::W;
  constexpr int OPAD = D + 4;
  __shared__ float sm_o[4][16][OPAD];
  __shared__ float sm_m[4][16];
  __shared__ float sm_l[4][16];
  __shared__ int sm_pages[kSegPages];

  const int lane = threadIdx.x & 63;
  // wave-uniform by construction; readfirstlane tells the compiler, so page
  // indices are scalar loads and buffer descriptors stay in SGPRs
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15;
  const int G = lane >> 4;
  const int h = blockIdx.y;
  const int g = p.g;

  const int it_lo = p.wg_ptr[blockIdx.x];
  const int it_hi = p.wg_ptr[blockIdx.x + 1];
  for (int it = it_lo; it < it_hi; ++it) {
    const DecodeItem item = p.items[it];
    const int b = uniform(item.b);
    const int ind_lo = uniform(p.kv_indptr[b]);
    const int npages = max(0, uniform(p.kv_indptr[b + 1]) - ind_lo);
    const int last = min(max(uniform(p.last_page_len[b]), 1), kPage);
    const int page_lo = uniform(item.page_lo);
    const int page_hi = min(uniform(item.page_hi), npages);
    const int slot = uniform(item.slot);

    // Q fragments: lane (G, n) holds head n, d in [32 ks + 8 G, +8)
    u32x4 qf[D / 32];
    {
      const bool hv = n < g;
      const uint16_t* qrow =
          p.q + (int64_t)b * p.q_sn + (int64_t)(h * g + (hv ? n : 0)) * p.q_sh;
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) {
        u32x4 z = {0u, 0u, 0u, 0u};
        if (hv) z = *reinterpret_cast<const u32x4*>(qrow + 32 * ks + 8 * G);
        qf[ks] = z;
      }
    }

    SoftmaxState<D, BF16, FP8> sm;
#pragma unroll
    for (int e = 0; e < W; ++e) sm.o[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    sm.m = -INFINITY;
    sm.l = 0.f;

    // segments of at most kSegPages pages: stage their page ids in LDS, then
    // wave w takes page pairs w, w+4, ... of the segment
    for (int seg_lo = page_lo; seg_lo < page_hi; seg_lo += kSegPages) {
      const int seg_hi = min(page_hi, seg_lo + kSegPages);
      for (int t = threadIdx.x; t < seg_hi - seg_lo; t += 256) {
        const int idx = ind_lo + seg_lo + t;
        int page = -1;
        if (ind_lo >= 0 && idx < p.num_indices) page = p.kv_indices[idx];
        sm_pages[t] = (page >= 0 && page < p.num_pages) ? page : -1;
      }
      __syncthreads();
      const int n_pairs = (seg_hi - seg_lo + 1) >> 1;
      const int n_my = n_pairs > wave ? (n_pairs - wave + 3) >> 2 : 0;
      if (n_my > 0) {
        Stage<D, BF16, FP8> sa, sb;
        load_pair(sa, p, h, sm_pages, seg_lo, seg_hi, npages, last,
                  seg_lo + 2 * wave, n, G);
        for (int i = 0; i < n_my; i += 2) {
          load_pair(sb, p, h, sm_pages, seg_lo, seg_hi, npages, last,
                    seg_lo + 2 * (wave + 4 * (i + 1)), n, G);
          compute_pair(sa, qf, sm, p.scale_log2, G);
          if (i + 1 >= n_my) break;
          load_pair(sa, p, h, sm_pages, seg_lo, seg_hi, npages, last,
                    seg_lo + 2 * (wave + 4 * (i + 2)), n, G);
          compute_pair(sb, qf, sm, p.scale_log2, G);
        }
      }
      __syncthreads();  // sm_pages is rewritten by the next segment
    }
    const float l_tot = sum_over_groups16(sm.l);

    // ---- merge the four waves through LDS
#pragma unroll
    for (int e = 0; e < W; ++e)
#pragma unroll
      for (int r = 0; r < 4; ++r) sm_o[wave][n][W * (4 * G + r) + e] = sm.o[e][r];
    if (G == 0) {
      sm_m[wave][n] = sm.m;
      sm_l[wave][n] = l_tot;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < g * D; idx += 256) {
      const int hn = idx / D;
      const int dd = idx - hn * D;
      float M = sm_m[0][hn];
#pragma unroll
      for (int w = 1; w < 4; ++w) M = fmaxf(M, sm_m[w][hn]);
      float o = 0.f, lse2 = -INFINITY;
      if (M != -INFINITY) {
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float wt = exp2f(sm_m[w][hn] - M);
          num += wt * sm_o[w][hn][dd];
          den += wt * sm_l[w][hn];
        }
        o = num / den;
        lse2 = M + log2f(den);
      }
      const int head = h * g + hn;
      if (slot < 0) {
        p.out[((int64_t)b * p.hq + head) * D + dd] = f2h<BF16>(o);
        if (p.lse && dd == 0)
          p.lse[(int64_t)b * p.hq + head] = lse2 * 0.69314718055994531f;
      } else {
        p.partial_o[((int64_t)slot * p.hq + head) * D + dd] = o;
        if (dd == 0) p.partial_lse[(int64_t)slot * p.hq + head] = lse2;
      }
    }
    __syncthreads();
  }
}

// Split-KV merge: o = sum_c 2^(lse_c - M) o_c / sum_c 2^(lse_c - M),
// lse = M + log2(sum_c 2^(lse_c - M)) (base-2 partials, natural-log output).
template <bool BF16>
__global__ void __launch_bounds__(128)
    decode_merge_kernel(const MergeItem* __restrict__ merges,
                        const float* __restrict__ po,
                        const float* __restrict__ pl, uint16_t* __restrict__ out,
                        float* __restrict__ lse, int hq, int d) {
  const MergeItem mi = merges[blockIdx.x];
  const int head = blockIdx.y;
  float M = -INFINITY;
  for (int s = 0; s < mi.nslots; ++s)
    M = fmaxf(M, pl[(int64_t)(mi.slot0 + s) * hq + head]);
  float num = 0.f, den = 0.f;
  const int dd = threadIdx.x;
  if (M != -INFINITY) {
    for (int s = 0; s < mi.nslots; ++s) {
      const int64_t sh = (int64_t)(mi.slot0 + s) * hq + head;
      const float wt = exp2f(pl[sh] - M);
      den += wt;
      if (dd < d) num += wt * po[sh * d + dd];
    }
  }
  const float o = M != -INFINITY ? num / den : 0.f;
  if (dd < d) out[((int64_t)mi.b * hq + head) * d + dd] = f2h<BF16>(o);
  if (lse && dd == 0)
    lse[(int64_t)mi.b * hq + head] =
        M != -INFINITY ? (M + log2f(den)) * 0.69314718055994531f : -INFINITY;
}

// ----------------------------------------------------------------------------
// launch table
using DecodeFn = void (*)(DecodeParams);

template <int D, bool BF16, bool FP8>
DecodeFn decode_fn() {
  return decode_kernel<D, BF16, FP8>;
}

static DecodeFn pick_decode(int d, bool bf16, bool fp8) {
  if (d == 64) {
    if (bf16) return fp8 ? decode_fn<64, true, true>() : decode_fn<64, true, false>();
    return fp8 ? decode_fn<64, false, true>() : decode_fn<64, false, false>();
  }
  if (bf16) return fp8 ? decode_fn<128, true, true>() : decode_fn<128, true, false>();
  return fp8 ? decode_fn<128, false, true>() : decode_fn<128, false, false>();
}

// Resident decode workgroups per CU for the bf16 kernel of this head_dim
// (the planner's slot count); PAGEDATTN_DECODE_WGS_PER_CU overrides it.
static int decode_wgs_per_cu(int d) {
  if (const char* env = std::getenv("PAGEDATTN_DECODE_WGS_PER_CU")) {
    const int v = std::atoi(env);
    if (v > 0) return v;
  }
  static int cached[2] = {0, 0};
  int& c = cached[d == 128 ? 1 : 0];
  if (c == 0) {
    int nb = 0;
    DecodeFn fn = pick_decode(d, true, false);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &nb, reinterpret_cast<const void*>(fn), 256, 0) != hipSuccess ||
        nb <= 0)
      nb = 2;
    c = nb;
  }
  return c;
}

}  // namespace pa

using namespace pa;

extern "C" {

int pagedattn_decode_plan(pagedattn_plan* plan, const int32_t* kv_indptr_host,
                          const int32_t* kv_last_page_len_host,
                          int32_t batch_size, int32_t num_qo_heads,
                          int32_t num_kv_heads, int32_t head_dim,
                          int32_t page_size, int32_t split_pages,
                          void* workspace, size_t workspace_bytes,
                          void* stream) {
  const char* who = "decode_plan";
  if (!plan) return set_error(PAGEDATTN_ERR_INVALID, "%s: null plan", who);
  plan->mode = kPlanNone;
  if (batch_size < 0)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: batch_size %d < 0", who,
                     batch_size);
  int rc = validate_heads(who, num_qo_heads, num_kv_heads, head_dim, page_size);
  if (rc) return rc;
  if (!workspace || ((uintptr_t)workspace & (kWsAlign - 1)))
    return set_error(PAGEDATTN_ERR_INVALID,
                     "%s: workspace must be a 256-byte aligned device buffer",
                     who);
  std::vector<int32_t> npages, kv_len;
  rc = validate_paged_metadata(who, kv_indptr_host, kv_last_page_len_host,
                               batch_size, page_size, &npages, &kv_len);
  if (rc) return rc;

  int64_t total = 0;
  int maxp = 0;
  for (int b = 0; b < batch_size; ++b) {
    total += npages[b];
    maxp = std::max(maxp, npages[b]);
  }

  std::vector<DecodeItem> items;
  std::vector<int32_t> wg_ptr;
  items.reserve(batch_size * 2 + 16);
  // pieces per sequence, for slots / merges
  std::vector<int32_t> first_piece(batch_size, -1), n_pieces(batch_size, 0);
  auto add_piece = [&](int b, int lo, int hi) {
    if (first_piece[b] < 0) first_piece[b] = (int)items.size();
    n_pieces[b]++;
    items.push_back(DecodeItem{b, lo, hi, -1});
  };

  if (split_pages != 0) {
    // fixed chunks (split_pages > 0) or whole sequences (< 0): one item per
    // workgroup
    const int chunk =
        split_pages > 0 ? ((split_pages + 7) / 8) * 8 : std::max(1, maxp);
    for (int b = 0; b < batch_size; ++b) {
      if (npages[b] == 0) {
        add_piece(b, 0, 0);
        continue;
      }
      for (int lo = 0; lo < npages[b]; lo += chunk)
        add_piece(b, lo, std::min(npages[b], lo + chunk));
    }
    // longest first
    std::vector<int> order(items.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int c) {
      return items[a].page_hi - items[a].page_lo >
             items[c].page_hi - items[c].page_lo;
    });
    std::vector<DecodeItem> sorted(items.size());
    for (size_t i = 0; i < order.size(); ++i) sorted[i] = items[order[i]];
    // pieces of one sequence keep their relative order (first_piece stays a
    // valid "has pieces" marker; slots are assigned below by sequence)
    items.swap(sorted);
    wg_ptr.resize(items.size() + 1);
    for (size_t i = 0; i <= items.size(); ++i) wg_ptr[i] = (int32_t)i;
  } else {
    // balanced partition: every workgroup gets ~the same number of pages,
    // cutting sequences at workgroup boundaries
    int cus = device_cu_count();
    if (cus <= 0) cus = 256;
    const int64_t slots = (int64_t)cus * decode_wgs_per_cu(head_dim);
    const int64_t x_max = std::max<int64_t>(1, slots / num_kv_heads);
    int64_t target = (total + x_max - 1) / x_max;
    target = std::max<int64_t>(8, ((target + 7) / 8) * 8);
    int64_t fill = 0;
    wg_ptr.push_back(0);
    for (int b = 0; b < batch_size; ++b) {
      if (npages[b] == 0) {
        add_piece(b, 0, 0);
        continue;
      }
      int lo = 0;
      while (lo < npages[b]) {
        const int take = (int)std::min<int64_t>(npages[b] - lo, target - fill);
        add_piece(b, lo, lo + take);
        lo += take;
        fill += take;
        if (fill == target) {
          wg_ptr.push_back((int32_t)items.size());
          fill = 0;
        }
      }
    }
    if (wg_ptr.back() != (int32_t)items.size())
      wg_ptr.push_back((int32_t)items.size());
  }

  // slots for split sequences, merge items
  std::vector<MergeItem> merges;
  int n_slots = 0;
  {
    std::vector<int32_t> slot0(batch_size, -1);
    for (int b = 0; b < batch_size; ++b) {
      if (n_pieces[b] > 1) {
        slot0[b] = n_slots;
        merges.push_back(MergeItem{b, n_slots, n_pieces[b], 0});
        n_slots += n_pieces[b];
      }
    }
    std::vector<int32_t> next(batch_size, 0);
    for (auto& it : items)
      if (slot0[it.b] >= 0) it.slot = slot0[it.b] + next[it.b]++;
  }

  const int n_items = (int)items.size();
  const int n_wg = (int)wg_ptr.size() - 1;
  const size_t off_items = kWsHeader;
  const size_t off_wg = ws_align(off_items + sizeof(DecodeItem) * n_items);
  const size_t off_merge = ws_align(off_wg + sizeof(int32_t) * (n_wg + 1));
  const size_t off_po = ws_align(off_merge + sizeof(MergeItem) * merges.size());
  const size_t off_pl =
      ws_align(off_po + sizeof(float) * (size_t)n_slots * num_qo_heads * head_dim);
  const size_t end = ws_align(off_pl + sizeof(float) * (size_t)n_slots * num_qo_heads);
  const size_t host_bytes = off_po - kWsHeader;

  plan->host.assign(host_bytes / sizeof(int32_t), 0);
  char* hb = reinterpret_cast<char*>(plan->host.data());
  if (n_items)
    std::memcpy(hb + (off_items - kWsHeader), items.data(),
                sizeof(DecodeItem) * n_items);
  std::memcpy(hb + (off_wg - kWsHeader), wg_ptr.data(),
              sizeof(int32_t) * (n_wg + 1));
  if (!merges.empty())
    std::memcpy(hb + (off_merge - kWsHeader), merges.data(),
                sizeof(MergeItem) * merges.size());

  plan->workspace = workspace;
  plan->workspace_bytes = workspace_bytes;
  rc = upload_plan(plan, who, host_bytes, end, stream);
  if (rc) return rc;

  char* ws = static_cast<char*>(workspace);
  plan->batch_size = batch_size;
  plan->hq = num_qo_heads;
  plan->hkv = num_kv_heads;
  plan->d = head_dim;
  plan->page_size = page_size;
  plan->n_items = n_wg;  // workgroups along x
  plan->n_merge = (int)merges.size();
  plan->n_slots = n_slots;
  plan->split_pages = split_pages;
  plan->items_dev = ws + off_items;
  plan->merge_dev = ws + off_merge;
  plan->partial_o = reinterpret_cast<float*>(ws + off_po);
  plan->partial_lse = reinterpret_cast<float*>(ws + off_pl);
  plan->total_pages = total;
  plan->max_pages = maxp;
  plan->wg_ptr_dev = reinterpret_cast<const int32_t*>(ws + off_wg);
  plan->mode = kPlanDecode;
  return PAGEDATTN_OK;
}

int pagedattn_decode_run(const pagedattn_plan* plan, const void* q,
                         int64_t q_stride_n, int64_t q_stride_h,
                         int32_t q_dtype, const void* paged_kv_cache,
                         int32_t kv_dtype, const float* kv_scales,
                         int32_t num_pages, const int32_t* kv_indices,
                         int32_t num_indices, const int32_t* kv_indptr,
                         const int32_t* kv_last_page_len, void* out,
                         float* lse, float sm_scale, void* stream) {
  const char* who = "decode_run";
  if (!plan || plan->mode != kPlanDecode)
    return set_error(PAGEDATTN_ERR_PLAN, "%s: no decode plan (call plan first)",
                     who);
  if (q_dtype != PAGEDATTN_BF16 && q_dtype != PAGEDATTN_F16)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: q dtype %d not supported",
                     who, q_dtype);
  const bool fp8 = kv_dtype == PAGEDATTN_E4M3;
  if (!fp8 && kv_dtype != q_dtype)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: kv dtype %d must equal q dtype %d or be e4m3", who,
                     kv_dtype, q_dtype);
  if (fp8 && !kv_scales)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: e4m3 pool needs kv_scales",
                     who);
  if (plan->batch_size == 0) return PAGEDATTN_OK;
  if (!q || !paged_kv_cache || !kv_indices || !kv_indptr ||
      !kv_last_page_len || !out)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null pointer", who);
  if ((q_stride_n & 7) || (q_stride_h & 7) || !aligned16(q) ||
      !aligned16(paged_kv_cache))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: q and the pool must be 16-byte aligned with strides "
                     "that are multiples of 8 elements",
                     who);
  if (num_pages < 0)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: num_pages %d < 0", who,
                     num_pages);
  DecodeParams p;
  p.items = static_cast<const DecodeItem*>(plan->items_dev);
  p.wg_ptr = plan->wg_ptr_dev;
  p.q = static_cast<const uint16_t*>(q);
  p.q_sn = q_stride_n;
  p.q_sh = q_stride_h;
  p.cache = static_cast<const uint8_t*>(paged_kv_cache);
  p.kv_scales = kv_scales;
  p.num_pages = num_pages;
  p.kv_indices = kv_indices;
  p.num_indices = num_indices;
  p.kv_indptr = kv_indptr;
  p.last_page_len = kv_last_page_len;
  p.out = static_cast<uint16_t*>(out);
  p.lse = lse;
  p.partial_o = plan->partial_o;
  p.partial_lse = plan->partial_lse;
  p.hq = plan->hq;
  p.hkv = plan->hkv;
  p.g = plan->hq / plan->hkv;
  p.scale_log2 = sm_scale * 1.4426950408889634f;

  hipStream_t s = (hipStream_t)stream;
  const bool bf16 = q_dtype == PAGEDATTN_BF16;
  DecodeFn fn = pick_decode(plan->d, bf16, fp8);
  if (plan->n_items > 0) {
    hipLaunchKernelGGL(fn, dim3(plan->n_items, plan->hkv), dim3(256), 0, s, p);
    int rc = check_launch(who);
    if (rc) return rc;
  }
  if (plan->n_merge > 0) {
    const dim3 grid(plan->n_merge, plan->hq);
    const dim3 block(plan->d);
    if (bf16)
      hipLaunchKernelGGL(decode_merge_kernel<true>, grid, block, 0, s,
                         static_cast<const MergeItem*>(plan->merge_dev),
                         plan->partial_o, plan->partial_lse, p.out, lse,
                         plan->hq, plan->d);
    else
      hipLaunchKernelGGL(decode_merge_kernel<false>, grid, block, 0, s,
                         static_cast<const MergeItem*>(plan->merge_dev),
                         plan->partial_o, plan->partial_lse, p.out, lse,
                         plan->hq, plan->d);
    return check_launch("decode_run(merge)");
  }
  return PAGEDATTN_OK;
}

}  // extern "C"
