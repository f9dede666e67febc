// Paged decode attention for gfx950 (BatchDecodeWithPagedKVCacheWrapper,
// src/models/llama.py:119-147 plan and :230-245 run).
//
// Work unit: a head group of hg waves (hg KV heads, hg = 4, 2 or 1) owns a
// list of items; an item is (page range of one sequence, KV heads h0 ..
// h0 + hg - 1), wave i taking head h0 + i for all g = Hq/Hkv query heads of
// that head, so each K/V byte is read from HBM once and a page's K (then V)
// blocks of the group's heads are read as one contiguous run.  Waves are
// independent: no barriers, no cross-wave LDS merges, so one slow memory
// request stalls one wave only.  The host planner cuts the concatenated
// (sequence, head group, page) stream into equal shares per group (or
// assigns whole sequences / fixed chunks to the least-loaded group);
// sequences cut in pieces write split partials that a small merge launch
// combines.
//
// Per page pair (32 tokens) a wave does:
//   S^T[32 tok x 16 heads] = K[tok x D] . Q^T      (v_mfma_f32_16x16x32, D/32 k-steps per page)
//   O^T[D x 16 heads]     += V^T[D x 32 tok] . P^T (D/16 MFMAs, K = the 32 tokens)
// Query heads occupy the MFMA N dimension (g <= 16, padded), tokens the
// M dimension of QK, so a lane's softmax values all belong to one head and the
// row max needs two cross-group shuffles only.
//
// Loads go through buffer resources sized to the valid tokens of each page:
// absent pages (num_records = 0) and slots past last_page_len read as zero
// without touching HBM, so the loop issues a fixed number of loads per pair
// and the compiler keeps the next pair's loads in flight while the current
// one is computed (two register buffers of 16 KiB each, ping-pong).  Page
// ids are scalar loads issued one buffer ahead of their use.
//
// K rows are read as 16-byte (bf16/fp16) or 8-byte (e4m3) pieces in the
// MFMA A-operand layout (lane -> token row, 8 consecutive d).  V rows are
// read as W = D/16 consecutive d per lane (lane n owns d in [W n, W n + W)),
// which gives W PV tiles whose row m is d = W m + e; the 8 tokens a lane
// needs for one tile come from its own 8 loads, repacked with bit ops.
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <queue>
#include <vector>

#include "plan_internal.h"

namespace pa {

struct DecodeParams {
  const DecodeItem* items;
  const int32_t* wave_ptr;  // [n_groups + 1]: items of head group w
  int32_t n_groups, n_merge, n_slots, batch_size;
  int32_t hg_shift;  // log2(waves per head group), 0..2
  int32_t deterministic;  // shared plans: fixed chunk assignment
  int32_t item_cost;  // implicit partition: header units per segment
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
  float* partial_o;    // [n_slots, g, D]
  float* partial_lse;  // [n_slots, g] (base 2)
  int32_t hq, hkv, g;
  float scale_log2;  // sm_scale * log2(e)
  // fused append (decode_run_append only): row b of k_new / v_new
  // [B, Hkv, D] is sequence b's newest token, position kv_len_b - 1
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t k_sn, k_sh, v_sn, v_sh;
  // position of sequence b's new token: new_pos[b], or kv_len_b - 1 when
  // new_pos is null; the fused append writes it to page new_pos / 16, slot
  // new_pos % 16, and the fused RoPE rotates q and the new K row there
  const int32_t* new_pos;
  double rope_inv_scale, rope_log2_theta;
  // fused append: tokens skipped (position outside the sequence's pages or
  // an invalid page id) are counted at append_err[0], clamped e4m3 pieces at
  // append_err[1] (may be null)
  int32_t* append_err;
  // shared-item plans: slot waits that gave up (never in a consistent run)
  int32_t* fault_count;
};

template <int N>
struct RawT;
template <>
struct RawT<16> {
  using type = u32x4;
  template <int POLICY>
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return buf_load16<POLICY>(r, off);
  }
};
template <>
struct RawT<8> {
  using type = u32x2;
  template <int POLICY>
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return buf_load8<POLICY>(r, off);
  }
};
template <>
struct RawT<4> {
  using type = uint32_t;
  template <int POLICY>
  static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return buf_load4<POLICY>(r, off);
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

template <int D, bool BF16, bool FP8>
struct DecodeTraits {
  static constexpr int ESZ = FP8 ? 1 : 2;
  static constexpr int KS = D / 32;          // QK k-steps per page
  static constexpr int W = D / 16;           // V elements per lane per token
  static constexpr int KB = 8 * ESZ;         // K bytes per lane per k-step
  static constexpr int VB = W * ESZ;         // V bytes per lane per token
  static constexpr int PAGE_BYTES = kPage * D * ESZ;
  // page pairs per register buffer: 16 KiB of K/V per buffer, except e4m3
  // at D = 128, whose 8-KiB pairs convert to bf16 in registers: one pair per
  // buffer keeps the kernel at two waves per SIMD (230 registers) and ran
  // the 70B-shaped e4m3 batch in 279 us against 282 us with two
  static constexpr int NP =
      (FP8 && D == 128) ? 1 : ((kPage * D * ESZ * 2 * 2 >= 16384) ? 1 : 2);
  using KRaw = typename RawT<KB>::type;
  using VRaw = typename RawT<VB>::type;
  // Cache policy of the K/V loads.  16-bit pools stream (non-temporal); e4m3
  // pools load with the default policy.  Measured on the decode steps, with
  // pools rotated past the Infinity Cache: the 70B-shaped e4m3 batch takes
  // 225 us with the default policy against 276 us streamed, while the bf16
  // long-context and TinyLlama steps take 1946 / 66 us with it against
  // 1799 / 58 us streamed.
  static constexpr int KV_POLICY = FP8 ? kCachePolicyDefault : kCachePolicyStream;
};

template <int D, bool BF16, bool FP8>
struct Stage {
  using Tr = DecodeTraits<D, BF16, FP8>;
  typename Tr::KRaw k[2][Tr::KS];
  typename Tr::VRaw v[8];
  int ntok[2];
  float kscale[2], vscale[2];
};

// Page ids of a pair, fetched with scalar loads two pairs ahead of use
// (-1: absent or invalid page).
// Device-side decode partition (plans made with pagedattn_decode_plan_device):
// a virtual stream of (sequence, head group) segments in sequence-major
// order, segment (b, hgrp) being `cost` header units followed by the
// sequence's pages, cut into shares of `share` units (share >= 4 + cost and
// even, at most n_groups shares).  The headers charge each item start, as
// the host planner's balanced split does; with cost 0 the two partitions
// are the same.  Segment (b, hgrp) starts at
//   seg(b) + hgrp * (np_b + cost),
//   seg(b) = ngrp * (kv_indptr[b] - kv_indptr[0]) + cost * ngrp * b,
// and its page j sits at unit start + cost + j.
struct ImplicitSplit {
  int64_t stream, share;
  int base, ngrp, cost;
};

__device__ __forceinline__ ImplicitSplit implicit_split(const int32_t* kv_indptr, int batch,
                                                        int ngrp, int n_groups, int cost) {
  ImplicitSplit sp;
  sp.ngrp = ngrp;
  sp.cost = cost;
  sp.base = uniform(load_invariant(kv_indptr));
  const int top = uniform(load_invariant(kv_indptr + batch));
  sp.stream = (int64_t)ngrp * max(0, top - sp.base) + (int64_t)cost * ngrp * batch;
  int64_t t = (sp.stream + n_groups - 1) / n_groups;
  t = (t + 1) / 2 * 2;
  sp.share = max<int64_t>(4 + cost, t);
  return sp;
}

__device__ __forceinline__ int64_t seq_start(const ImplicitSplit& sp, int b, int ind_lo) {
  return (int64_t)sp.ngrp * (ind_lo - sp.base) + (int64_t)sp.cost * sp.ngrp * b;
}

// Largest b in [0, batch) whose segments start at or before unit x, by a
// 64-way search: each round every lane tests one candidate of the range and
// the ballot narrows it 64-fold.  Always ends (the range shrinks every
// round) and stays in [0, batch) whatever kv_indptr holds.
__device__ __forceinline__ int find_sequence(const int32_t* kv_indptr, int batch,
                                             const ImplicitSplit& sp, int64_t x, int lane) {
  int lo = 0, hi = batch;
  while (hi - lo > 1) {
    const int step = (hi - lo + kWave - 1) / kWave;
    const int c = lo + lane * step;
    bool ok = false;
    if (c < hi) ok = seq_start(sp, c, kv_indptr[c]) <= x;
    const int cnt = __builtin_popcountll(__builtin_amdgcn_ballot_w64(ok));
    const int nlo = lo + max(cnt - 1, 0) * step;
    hi = uniform(min(nlo + step, hi));
    lo = uniform(nlo);
  }
  return lo;
}

struct PairIds {
  int p0, p1;
};

__device__ __forceinline__ int page_id(const DecodeParams& p, int ind_lo,
                                       int pg, int page_hi) {
  int page = -1;
  if (pg < page_hi && ind_lo >= 0 && ind_lo + pg < p.num_indices)
    page = uniform(load_invariant(p.kv_indices + ind_lo + pg));
  return (page >= 0 && page < p.num_pages) ? page : -1;
}

__device__ __forceinline__ PairIds fetch_ids(const DecodeParams& p, int ind_lo,
                                             int pg0, int page_hi) {
  return PairIds{page_id(p, ind_lo, pg0, page_hi),
                 page_id(p, ind_lo, pg0 + 1, page_hi)};
}

template <int D, bool BF16, bool FP8>
__device__ __forceinline__ void load_pair(Stage<D, BF16, FP8>& st,
                                          const DecodeParams& p, int h,
                                          PairIds ids, int pg0, int npages,
                                          int last, int n, int G) {
  using Tr = DecodeTraits<D, BF16, FP8>;
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) {
    const int pg = pg0 + pi;
    int page = pi ? ids.p1 : ids.p0;
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
      st.k[pi][ks] = RawT<Tr::KB>::template load<Tr::KV_POLICY>(
          rk, (uint32_t)((n * D + 32 * ks + 8 * G) * Tr::ESZ));
#pragma unroll
    for (int r = 0; r < 4; ++r)
      st.v[pi * 4 + r] = RawT<Tr::VB>::template load<Tr::KV_POLICY>(
          rv, (uint32_t)(((4 * G + r) * D + Tr::W * n) * Tr::ESZ));
    if constexpr (FP8) {
      const int64_t si = ((int64_t)page * 2) * p.hkv + h;
      st.kscale[pi] = ntok ? load_invariant(p.kv_scales + si) : 0.f;
      st.vscale[pi] = ntok ? load_invariant(p.kv_scales + si + p.hkv) : 0.f;
    }
  }
}

constexpr float kDecodeRescaleSlack = 8.f;

template <int D, bool BF16, bool FP8>
struct SoftmaxState {
  f32x4 o[D / 16];
  float m, l;
};

// One call handles NPC page pairs (one register stage) as one online-softmax
// step: one cross-lane max and one rescale check for all of them, and their
// independent MFMA chains interleave.
template <int D, bool BF16, bool FP8, int NPC>
__device__ __forceinline__ void compute_pairs(const Stage<D, BF16, FP8> (&st)[NPC],
                                              const u32x4 (&qf)[D / 32],
                                              SoftmaxState<D, BF16, FP8>& sm,
                                              float scale_log2, int G, int n) {
  using Tr = DecodeTraits<D, BF16, FP8>;
  constexpr int W = Tr::W;
  constexpr int NS = NPC * 8;  // scores per lane
  // ---- S^T = K . Q^T for every page of the stage
  f32x4 s4[NPC][2];
#pragma unroll
  for (int k = 0; k < NPC; ++k)
#pragma unroll
    for (int pi = 0; pi < 2; ++pi) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < Tr::KS; ++ks) {
        const typename Tr::KRaw kr = st[k].k[pi][ks];
        u32x4 a;
        if constexpr (FP8) {
          a = e4m3x8_to_16<BF16>(kr[0], kr[1]);
        } else {
          a = kr;
        }
        acc = mfma16<BF16>(a, qf[ks], acc);
      }
      s4[k][pi] = acc;
    }
  float s[NS];
  bool partial = false;
#pragma unroll
  for (int k = 0; k < NPC; ++k)
#pragma unroll
    for (int pi = 0; pi < 2; ++pi) {
      const float c = FP8 ? scale_log2 * st[k].kscale[pi] : scale_log2;
#pragma unroll
      for (int r = 0; r < 4; ++r) s[k * 8 + pi * 4 + r] = s4[k][pi][r] * c;
      partial |= st[k].ntok[pi] < kPage;
    }
  if (partial) {
#pragma unroll
    for (int k = 0; k < NPC; ++k)
#pragma unroll
      for (int pi = 0; pi < 2; ++pi)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (4 * G + r >= st[k].ntok[pi]) s[k * 8 + pi * 4 + r] = -INFINITY;
  }
  // ---- online softmax (all values of a lane belong to its head), lazy:
  // the running max only moves, with a rescale of O and l, when a score
  // exceeds it by more than kDecodeRescaleSlack (log2 units), so P stays
  // <= 2^slack and most steps skip the rescale.  exp2 is the raw v_exp_f32.
  float mx = s[0];
#pragma unroll
  for (int j = 1; j < NS; ++j) mx = fmaxf(mx, s[j]);
  mx = max_over_groups16(mx);
  const bool grow = mx > sm.m + kDecodeRescaleSlack;
  if (__builtin_amdgcn_ballot_w64(grow)) {
    const float m_new = grow ? mx : sm.m;
    const float alpha = __builtin_amdgcn_exp2f(sm.m - m_new);
    sm.l *= alpha;
#pragma unroll
    for (int e = 0; e < W; ++e) sm.o[e] *= alpha;
    sm.m = m_new;
  }
  const float m_use = sm.m == -INFINITY ? 0.f : sm.m;
  float pr[NS];
  float psum = 0.f;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    pr[j] = __builtin_amdgcn_exp2f(s[j] - m_use);
    psum += pr[j];
  }
  sm.l += psum;
#pragma unroll
  for (int k = 0; k < NPC; ++k) {
    if constexpr (FP8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) pr[k * 8 + j] *= st[k].vscale[j >> 2];
    }
    u32x4 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = pack2<BF16>(pr[k * 8 + 2 * i], pr[k * 8 + 2 * i + 1]);
    // ---- V rows, tokens 2i and 2i+1 interleaved per d with one v_perm: the
    // MFMA operand of tile row d = W m + e holds (token 2i, token 2i+1) at d.
    constexpr int VWORDS = Tr::VB / 4;  // dwords of one token's V slice
    uint32_t vw[8][VWORDS];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const typename Tr::VRaw vr = st[k].v[j];
#pragma unroll
      for (int w = 0; w < VWORDS; ++w) vw[j][w] = dword_of(vr, w);
    }
    // ---- O^T += V^T . P^T, one MFMA per d offset e (tile rows d = W m + e)
    if constexpr (FP8) {
      // e4m3 bytes of d = e, e + 1 for tokens 2i, 2i+1 gathered into one
      // dword; one converter per d gives the bf16 pair directly
#pragma unroll
      for (int e = 0; e < W; e += 2) {
        u32x4 a0, a1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t t = __builtin_amdgcn_perm(vw[2 * i + 1][e >> 2], vw[2 * i][e >> 2],
                                                   (e & 2) ? 0x07030602u : 0x05010400u);
          a0[i] = e4m3x2_to_16<BF16, false>(t);
          a1[i] = e4m3x2_to_16<BF16, true>(t);
        }
        sm.o[e] = mfma16<BF16>(a0, pb, sm.o[e]);
        sm.o[e + 1] = mfma16<BF16>(a1, pb, sm.o[e + 1]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < W; ++e) {
        u32x4 a;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          a[i] = __builtin_amdgcn_perm(vw[2 * i + 1][e >> 1], vw[2 * i][e >> 1],
                                       (e & 1) ? 0x07060302u : 0x05040100u);
        sm.o[e] = mfma16<BF16>(a, pb, sm.o[e]);
      }
    }
  }
}

// Writes sequence b / head h's new row to slot `slot` of page `page` (the
// append of flashinfer.append_paged_kv_cache at position kv_len - 1).  Lanes
// [0, D/8) move the K row, lanes [32, 32 + D/8) the V row, 8 elements each.
// The same wave reads the page back later in program order (its own store
// to the same addresses comes first), so the attention sees the new row
// exactly as the pool holds it, with no patching of loaded registers.
// With ROPE the K row is rotated first (position `pos`): lane c < D/16 takes
// the chunk pair c, c + D/16 (elements i and i + D/2).
template <int D, bool BF16, bool FP8>
__device__ __forceinline__ void put_chunk(const DecodeParams& p, int h, int page, int slot,
                                          int is_v, int c, u32x4 x) {
  using Tr = DecodeTraits<D, BF16, FP8>;
  uint8_t* dst = const_cast<uint8_t*>(p.cache) +
                 (((int64_t)page * 2 + is_v) * p.hkv + h) * (int64_t)Tr::PAGE_BYTES +
                 ((int64_t)slot * D + 8 * c) * Tr::ESZ;
  if constexpr (FP8) {
    const float scale =
        load_invariant(p.kv_scales + ((int64_t)page * 2 + is_v) * p.hkv + h);
    bool clamped = false;
    const u32x2 q = quant8_e4m3<BF16>(x, scale, &clamped);
    *reinterpret_cast<u32x2*>(dst) = q;
    count_lanes(p.append_err ? p.append_err + 1 : nullptr, clamped);
  } else {
    *reinterpret_cast<u32x4*>(dst) = x;
  }
}

template <int D, bool BF16, bool FP8, bool ROPE>
__device__ __forceinline__ void fused_append(const DecodeParams& p, int b, int h,
                                             int page, int slot, int lane, int pos) {
  const int is_v = lane >> 5;
  const int c = lane & 31;
  if (c >= D / 8) return;
  const uint16_t* src =
      is_v ? p.v_new + (int64_t)b * p.v_sn + (int64_t)h * p.v_sh
           : p.k_new + (int64_t)b * p.k_sn + (int64_t)h * p.k_sh;
  if (ROPE && !is_v) {
    if (c >= D / 16) return;
    u32x4 lo = *reinterpret_cast<const u32x4*>(src + 8 * c);
    u32x4 hi = *reinterpret_cast<const u32x4*>(src + 8 * c + D / 2);
    float cs[8], sn[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      rope_cos_sin(pos, 8 * c + e, D, p.rope_inv_scale, p.rope_log2_theta, &cs[e], &sn[e]);
    rope8<BF16>(lo, hi, cs, sn);
    put_chunk<D, BF16, FP8>(p, h, page, slot, 0, c, lo);
    put_chunk<D, BF16, FP8>(p, h, page, slot, 0, c + D / 16, hi);
    return;
  }
  put_chunk<D, BF16, FP8>(p, h, page, slot, is_v, c,
                          *reinterpret_cast<const u32x4*>(src + 8 * c));
}

// Final normalisation of one softmax state of (sequence b, KV head h): the
// output rows (and lse) of its g query heads, or base-2 split partials at
// `slot` when slot >= 0.  Lane (G, n) owns d = W (4 G + r) + e of head n.
template <int D, bool BF16, bool FP8>
__device__ __forceinline__ void write_item_output(const DecodeParams& p, int b, int h, int slot,
                                                  const SoftmaxState<D, BF16, FP8>& sm, int G,
                                                  int n) {
  constexpr int W = DecodeTraits<D, BF16, FP8>::W;
  const int g = p.g;
  const float l_tot = sum_over_groups16(sm.l);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const float lse2 = l_tot > 0.f ? sm.m + log2f(l_tot) : -INFINITY;
  if (slot < 0) {
    if (n < g) {
      uint16_t* orow = p.out + ((int64_t)b * p.hq + h * g + n) * D;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint16_t* dst = orow + W * (4 * G + r);
        if constexpr (W == 8) {
          u32x4 w4;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            w4[i] = pack2<BF16>(sm.o[2 * i][r] * inv, sm.o[2 * i + 1][r] * inv);
          *reinterpret_cast<u32x4*>(dst) = w4;
        } else {
          u32x2 w2;
#pragma unroll
          for (int i = 0; i < 2; ++i)
            w2[i] = pack2<BF16>(sm.o[2 * i][r] * inv, sm.o[2 * i + 1][r] * inv);
          *reinterpret_cast<u32x2*>(dst) = w2;
        }
      }
      if (p.lse && G == 0)
        p.lse[(int64_t)b * p.hq + h * g + n] = lse2 * 0.69314718055994531f;
    }
  } else {
    if (n < g) {
      float* prow = p.partial_o + ((int64_t)slot * g + n) * D;
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int e = 0; e < W; ++e) prow[W * (4 * G + r) + e] = sm.o[e][r] * inv;
      if (G == 0) p.partial_lse[(int64_t)slot * g + n] = lse2;
    }
  }
}

template <int D, bool BF16, bool FP8, bool APPEND, bool ROPE, bool IMPLICIT>
__global__ void __launch_bounds__(256, 1) decode_kernel(DecodeParams p) {
  using Tr = DecodeTraits<D, BF16, FP8>;
  constexpr int W = Tr::W;
  const int lane = threadIdx.x & 63;
  // wave-uniform by construction; readfirstlane tells the compiler, so item
  // fields are scalar loads and buffer descriptors stay in SGPRs
  const int wave = uniform(threadIdx.x >> 6);
  // head group gw = the hg consecutive waves of a workgroup; wave wi of the
  // group takes KV head h0 + wi of every item, so the group reads each page's
  // K (then V) blocks of hg heads, one contiguous run, at the same time
  const int wi = wave & ((1 << p.hg_shift) - 1);
  const int gw = uniform(((int)blockIdx.x * 4 + wave) >> p.hg_shift);
  if (gw >= p.n_groups) return;
  const int n = lane & 15;
  const int G = lane >> 4;
  const int g = p.g;

  // one work item: pages [item_lo, item_hi) of sequence b for KV heads
  // h0 + [0, hg); slot0 >= 0: the item is one piece of a cut sequence and
  // writes split partials to slots slot0 + wi
  auto run_item = [&](const int b, const int h0, const int item_lo, const int item_hi,
                      const int slot0) {
    const int h = h0 + wi;
    const int slot = slot0 >= 0 ? slot0 + wi : -1;
    const int ind_lo = uniform(load_invariant(p.kv_indptr + b));
    const int npages = max(0, uniform(load_invariant(p.kv_indptr + b + 1)) - ind_lo);
    const int last = min(max(uniform(load_invariant(p.last_page_len + b)), 1), kPage);
    const int page_lo = max(0, item_lo);
    const int page_hi = min(item_hi, npages);

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
    int new_pos = npages > 0 ? (npages - 1) * kPage + last - 1 : -1;
    if constexpr (APPEND) {
      if (p.new_pos) new_pos = uniform(load_invariant(p.new_pos + b));
    }
    if constexpr (ROPE) {
      const int rope_at = new_pos;
      // d and d + D/2 sit in the same lane: fragments ks and ks + D/64
#pragma unroll
      for (int ks = 0; ks < D / 64; ++ks) {
        float cs[8], sn[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          rope_cos_sin(rope_at, 32 * ks + 8 * G + e, D, p.rope_inv_scale,
                       p.rope_log2_theta, &cs[e], &sn[e]);
        rope8<BF16>(qf[ks], qf[ks + D / 64], cs, sn);
      }
    }

    // the item that holds the new token's page also performs the append (a
    // position outside the sequence's pages is skipped, as the stand-alone
    // append skips it)
    const int new_slot = new_pos & (kPage - 1);
    if constexpr (APPEND) {
      const int pg = new_pos >= 0 ? new_pos / kPage : -1;
      bool skipped = false;
      if (pg >= 0 && pg < npages) {
        if (pg >= page_lo && pg < page_hi) {
          const int page = page_id(p, ind_lo, pg, npages);
          if (page >= 0) {
            fused_append<D, BF16, FP8, ROPE>(p, b, h, page, new_slot, lane, new_pos);
          } else {
            skipped = true;
          }
        }
      } else {
        // outside the sequence's pages: counted by its first piece
        skipped = npages > 0 && page_lo == 0;
      }
      count_lanes(p.append_err, skipped && h == 0 && lane == 0);
    }

    SoftmaxState<D, BF16, FP8> sm;
#pragma unroll
    for (int e = 0; e < W; ++e) sm.o[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    sm.m = -INFINITY;
    sm.l = 0.f;

    // Two register buffers (ping-pong) of NP page pairs each; page ids run
    // one buffer ahead of the loads.  NP = 2 for the 8-KiB pairs (D = 64
    // bf16/fp16, D = 128 e4m3) keeps 16 KiB per wave in flight.
    constexpr int NP = DecodeTraits<D, BF16, FP8>::NP;
    const int n_pairs = page_hi > page_lo ? (page_hi - page_lo + 1) >> 1 : 0;
    const int n_chunks = (n_pairs + NP - 1) / NP;
    auto fetch_chunk = [&](PairIds (&ids)[NP], int c) {
#pragma unroll
      for (int k = 0; k < NP; ++k)
        ids[k] = fetch_ids(p, ind_lo, page_lo + 2 * (NP * c + k), page_hi);
    };
    auto load_chunk = [&](Stage<D, BF16, FP8> (&st)[NP], const PairIds (&ids)[NP], int c) {
#pragma unroll
      for (int k = 0; k < NP; ++k)
        load_pair(st[k], p, h, ids[k], page_lo + 2 * (NP * c + k), npages, last, n, G);
    };
    // pairs past the end of the item were loaded as empty pages (no tokens,
    // zero data) and add nothing
    auto compute_chunk = [&](Stage<D, BF16, FP8> (&st)[NP], int c) {
      compute_pairs<D, BF16, FP8, NP>(st, qf, sm, p.scale_log2, G, n);
    };
    if (n_chunks > 0) {
      Stage<D, BF16, FP8> sa[NP], sb[NP];
      PairIds ida[NP], idb[NP];
      fetch_chunk(ida, 0);
      fetch_chunk(idb, 1);
      load_chunk(sa, ida, 0);
      for (int c = 0; c < n_chunks; c += 2) {
        fetch_chunk(ida, c + 2);
        load_chunk(sb, idb, c + 1);
        compute_chunk(sa, c);
        if (c + 1 >= n_chunks) break;
        fetch_chunk(idb, c + 3);
        load_chunk(sa, ida, c + 2);
        compute_chunk(sb, c + 1);
      }
    }

    write_item_output<D, BF16, FP8>(p, b, h, slot, sm, G, n);
  };

  if constexpr (!IMPLICIT) {
    const int it_lo = uniform(load_invariant(p.wave_ptr + gw));
    const int it_hi = uniform(load_invariant(p.wave_ptr + gw + 1));
    for (int it = it_lo; it < it_hi; ++it) {
      const int32_t* itp = reinterpret_cast<const int32_t*>(p.items + it);
      const int b = uniform(load_invariant(itp + 0));
      const int h0 = uniform(load_invariant(itp + 1));
      const int item_lo = uniform(load_invariant(itp + 2));
      const int item_hi = uniform(load_invariant(itp + 3));
      const int slot0 = uniform(load_invariant(itp + 4));
      const int merge = uniform(load_invariant(itp + 5));
      const int slot = slot0 >= 0 ? slot0 + wi : -1;
      // a work list that does not match this launch is skipped, never followed
      if (b < 0 || b >= p.batch_size || h0 < 0 || h0 + wi >= p.hkv ||
          slot >= p.n_slots || merge >= p.n_merge || (slot >= 0) != (merge >= 0))
        continue;
      run_item(b, h0, item_lo, item_hi, slot0);
    }
  } else {
    // Device-side partition, read from kv_indptr at run time: the virtual
    // stream of (sequence, head group) segments (implicit_split) is cut into
    // equal shares, share gw for head group gw.  A sequence cut by a share
    // boundary leaves at most two pieces in one share: one that continues
    // from the previous share (slot 2 gw) and one that starts at the
    // sequence's first page after the share's start (slot 2 gw + 1); a
    // share's only piece may be both kinds and uses slot 2 gw.
    const ImplicitSplit sp = implicit_split(p.kv_indptr, p.batch_size, p.hkv >> p.hg_shift,
                                            p.n_groups, p.item_cost);
    const int64_t start = (int64_t)gw * sp.share;
    if (start >= sp.stream) return;
    const int64_t end = min(start + sp.share, sp.stream);
    const int ngrp = sp.ngrp;
    int b = find_sequence(p.kv_indptr, p.batch_size, sp, start, lane);
    int ind_lo = uniform(load_invariant(p.kv_indptr + b));
    int np = uniform(load_invariant(p.kv_indptr + b + 1)) - ind_lo;
    int hgrp = np > 0 ? (int)min<int64_t>(ngrp, max<int64_t>(0, (start - seq_start(sp, b, ind_lo)) /
                                                                      (np + sp.cost)))
                      : ngrp;
    int64_t pos = start;
    while (pos < end) {
      if (hgrp >= ngrp) {
        if (++b >= p.batch_size) break;
        ind_lo = uniform(load_invariant(p.kv_indptr + b));
        np = uniform(load_invariant(p.kv_indptr + b + 1)) - ind_lo;
        hgrp = np > 0 ? 0 : ngrp;
        continue;
      }
      // unit of the segment's first page; segments only move further on
      const int64_t p0 = seq_start(sp, b, ind_lo) + (int64_t)hgrp * (np + sp.cost) + sp.cost;
      if (p0 >= end) break;
      const int64_t lo = max<int64_t>(0, pos - p0);
      const int64_t hi = min<int64_t>(np, end - p0);
      if (hi > lo) {
        const bool cut = lo > 0 || hi < np;
        const int slot0 = cut ? (2 * gw + ((lo == 0 && p0 > start) ? 1 : 0)) << p.hg_shift : -1;
        run_item(b, hgrp << p.hg_shift, (int)lo, (int)hi, slot0);
        pos = p0 + hi;
      }
      ++hgrp;
    }
  }
}

// ----------------------------------------------------------------------------
// Shared-item decode (plans of pagedattn_decode_plan whose whole (sequence,
// KV head) items balance over the CUs).  Workgroup w holds one CU, one wave
// per SIMD, and owns the items [wave_ptr[w], wave_ptr[w + 1]).  The chunks
// of its items (NP page pairs each, items in list order) form one sequence
// that the four waves take in turn (wave w: chunks w, w + 4, ...).  A wave
// keeps one softmax state: when it reaches a chunk of a later item it leaves
// its state for the earlier item in an LDS slot, and the wave that completes
// the item's chunk count merges the states left there, in wave order, and
// writes the output.  No sequence is
// cut across workgroups, so there are no split partials and no merge launch.

// Items whose states can wait in LDS at once: with the fixed chunk
// assignment a wave that runs ahead by more items than this waits for a slot
// to be merged (three at D = 128 keep the workgroup's LDS under 160 KiB).
template <int D>
constexpr int shared_slots() { return D == 64 ? 4 : 3; }
// Bound of the wait for a slot to be released (each round sleeps ~64 clocks);
// the wait always ends long before, since a slot only waits for items of
// lower index, whose waves never wait for it.  A wait that gives up counts
// in DecodeParams::fault_count and writes nothing.
constexpr int kSharedSpinLimit = 1 << 24;

template <int D>
struct SharedLds {
  int n_it;       // items of the workgroup
  int total;      // chunks of the workgroup's items
  int next;       // chunk counter (claims in arrival order)
  static constexpr int S = shared_slots<D>();
  int tag[S];   // item index the slot is open for
  int cnt[S];   // chunks accounted for by the states left in the slot
  int mask[S];  // waves whose states are in the slot
  int b[kSharedMaxItems], h[kSharedMaxItems], chunk_lo[kSharedMaxItems],
      n_chunks[kSharedMaxItems], ind_lo[kSharedMaxItems], npages[kSharedMaxItems],
      last[kSharedMaxItems], new_pos[kSharedMaxItems];
  u32x4 q[kSharedMaxItems][D / 32][kWave];  // Q B-operands (rotated with ROPE)
  struct State {
    f32x4 o[D / 16][kWave];
    float m[kWave], l[kWave];
  } st[S][4];
};

// A claimed chunk: item index in the workgroup's table (-1: none left) and
// its first page within the sequence.
struct ChunkRef {
  int item, pg0;
};

// Device-planned shared-item decode (DEV): the workgroup finds its items
// itself from kv_indptr.  The B * Hkv items (sequence, KV head) are ordered
// by the sequences' page counts, longest first (ties by index), heads in
// order, and dealt to the n_wg workgroups in rounds of n_wg, the direction
// alternating (round r gives workgroup w item r n_wg + w for even r, r n_wg +
// n_wg - 1 - w for odd r), which pairs long items with short ones much as
// the host planner's longest-first assignment does.  Every workgroup ranks
// all sequences in its prologue (B compares of one integer key per
// sequence, B <= kDevSharedMaxBatch), so no other launch and no host copy is
// involved.
// Fills L.b / h / chunk_lo / n_chunks of the workgroup's items; returns
// their number (uniform).
// The workgroups of the device deal are relabelled: workgroup w takes the
// items the alternating deal gives to position deal_pos(w), whose inverse
// sends each aligned group of 8 positions (the KV heads of a sequence, whose
// pages share a scale block) to workgroups of one XCD (workgroup w runs on
// XCD w mod 8).  Every workgroup's item list is one of the plain deal's, so
// the balance and the output bits are those of the plain deal.
__device__ __forceinline__ int deal_pos(int w, int nwg) {
  if (nwg % 8) return w;
  const int m = nwg / 8;
  return (w % m) * 8 + w / m;
}

template <int D>
__device__ __forceinline__ int dev_item_table(const DecodeParams& p, SharedLds<D>& L, int* ip,
                                              int* lastp, int* key) {
  const int B = p.batch_size, H = p.hkv, nwg = (int)gridDim.x;
  const int w = deal_pos((int)blockIdx.x, nwg);
  const int N = B * H;
  if (B <= 0 || B > kDevSharedMaxBatch || N > kSharedMaxItems * nwg) {
    // a launch the plan did not make (the host plan keeps both bounds)
    if (threadIdx.x == 0) count_lanes(p.fault_count, true);
    return 0;
  }
  int n_it = 0;
  for (int r = 0; r < kSharedMaxItems; ++r)
    if (r * nwg + ((r & 1) ? nwg - 1 - w : w) < N) n_it = r + 1;
  if (n_it == 0) return 0;
  for (int t = (int)threadIdx.x; t <= B; t += (int)blockDim.x) {
    ip[t] = load_invariant(p.kv_indptr + t);
    if (t < B) lastp[t] = load_invariant(p.last_page_len + t);
  }
  __syncthreads();
  // one distinct key per sequence, larger for more pages, then for a smaller
  // index (page counts capped at 2^21 for the key); -1 pads to a multiple of
  // 16, below every key.  A sequence's rank is the number of larger keys.
  constexpr int kKeyIdx = 1024;  // > kDevSharedMaxBatch
  const int B16 = (B + 15) & ~15;
  for (int t = (int)threadIdx.x; t < B16; t += (int)blockDim.x)
    key[t] = t < B ? min(max(0, ip[t + 1] - ip[t]), (1 << 21) - 1) * kKeyIdx + (kKeyIdx - 1 - t)
                   : -1;
  __syncthreads();
  for (int b = (int)threadIdx.x; b < B; b += (int)blockDim.x) {
    const int kb = key[b];
    int rank = 0;
    for (int j = 0; j < B16; j += 16) {
      const int4 v0 = *reinterpret_cast<const int4*>(key + j);
      const int4 v1 = *reinterpret_cast<const int4*>(key + j + 4);
      const int4 v2 = *reinterpret_cast<const int4*>(key + j + 8);
      const int4 v3 = *reinterpret_cast<const int4*>(key + j + 12);
      rank += (v0.x > kb) + (v0.y > kb) + (v0.z > kb) + (v0.w > kb);
      rank += (v1.x > kb) + (v1.y > kb) + (v1.z > kb) + (v1.w > kb);
      rank += (v2.x > kb) + (v2.y > kb) + (v2.z > kb) + (v2.w > kb);
      rank += (v3.x > kb) + (v3.y > kb) + (v3.z > kb) + (v3.w > kb);
    }
    for (int hh = 0; hh < H; ++hh) {
      const int i = rank * H + hh;
      const int r = i / nwg, pos = i - r * nwg;
      if (r < n_it && ((r & 1) ? nwg - 1 - pos : pos) == w) {
        L.b[r] = b;
        L.h[r] = hh;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int r = 0; r < n_it; ++r) {
      const int b = L.b[r];
      const int np = max(0, ip[b + 1] - ip[b]);
      const int nc = max(1, (np + 2 * kSharedStagePairs - 1) / (2 * kSharedStagePairs));
      L.chunk_lo[r] = acc;
      L.n_chunks[r] = nc;
      L.ind_lo[r] = ip[b];
      L.npages[r] = np;
      L.last[r] = lastp[b];
      acc += nc;
    }
  }
  __syncthreads();
  return n_it;
}

// The same deal as dev_item_table, made once for all the runs that share
// the metadata (pagedattn_decode_plan_device_update): one workgroup ranks the
// sequences and writes every workgroup's items, page ranges and chunk offsets
// in the host plan's layout, so the attention launches read their items as a
// host-planned shared run does (no ranking in their prologue).  Threads are
// sequences for the ranking and workgroups for the table.
struct SharedTableArgs {
  const int32_t* kv_indptr;
  const int32_t* last_page_len;
  int32_t batch_size, hkv, n_wg;
  SharedItem* items;  // n_wg * kSharedMaxItems entries
  int32_t* fault_count;
};

constexpr int kSharedTableThreads = 1024;

__global__ void __launch_bounds__(kSharedTableThreads) decode_shared_table_kernel(SharedTableArgs a) {
  static_assert(kDevSharedMaxBatch <= kSharedTableThreads, "one sequence per thread");
  __shared__ int ip[kDevSharedMaxBatch + 1];
  __shared__ int lastp[kDevSharedMaxBatch];
  __shared__ __attribute__((aligned(16))) int key[kDevSharedMaxBatch];
  __shared__ int order[kDevSharedMaxBatch];  // sequence of each rank
  const int t = (int)threadIdx.x;
  const int B = a.batch_size, H = a.hkv, nwg = a.n_wg;
  const int N = B * H;
  if (B <= 0 || B > kDevSharedMaxBatch || H <= 0 || N > kSharedMaxItems * nwg) {
    // a plan the entry point would not make: every workgroup gets no items
    for (int i = t; i < nwg * kSharedMaxItems; i += kSharedTableThreads)
      a.items[i] = SharedItem{-1, 0, 0, 0, -1, 0, kPage, 0};
    if (t == 0) count_lanes(a.fault_count, true);
    return;
  }
  for (int i = t; i <= B; i += kSharedTableThreads) {
    ip[i] = a.kv_indptr[i];
    if (i < B) lastp[i] = a.last_page_len[i];
  }
  __syncthreads();
  // keys and ranks as dev_item_table: more pages first, then smaller index
  constexpr int kKeyIdx = 1024;  // > kDevSharedMaxBatch
  const int B16 = (B + 15) & ~15;
  if (t < B16)
    key[t] = t < B ? min(max(0, ip[t + 1] - ip[t]), (1 << 21) - 1) * kKeyIdx + (kKeyIdx - 1 - t)
                   : -1;
  __syncthreads();
  if (t < B) {
    const int kb = key[t];
    int rank = 0;
    for (int j = 0; j < B16; j += 4) {
      const int4 v = *reinterpret_cast<const int4*>(key + j);
      rank += (v.x > kb) + (v.y > kb) + (v.z > kb) + (v.w > kb);
    }
    order[rank] = t;
  }
  __syncthreads();
  // workgroup wg's round-r item is item r nwg + w (r even) or
  // r nwg + nwg - 1 - w (r odd) of the rank order, heads in order, with
  // w = deal_pos(wg) as in the prologue's deal
  for (int wg = t; wg < nwg; wg += kSharedTableThreads) {
    const int w = deal_pos(wg, nwg);
    int n_it = 0;
    for (int r = 0; r < kSharedMaxItems; ++r)
      if (r * nwg + ((r & 1) ? nwg - 1 - w : w) < N) n_it = r + 1;
    int acc = 0;
    for (int r = 0; r < kSharedMaxItems; ++r) {
      SharedItem it{-1, 0, 0, 0, -1, 0, kPage, n_it};
      if (r < n_it) {
        const int i = r * nwg + ((r & 1) ? nwg - 1 - w : w);
        const int b = order[i / H];
        const int np = max(0, ip[b + 1] - ip[b]);
        const int nc = max(1, (np + 2 * kSharedStagePairs - 1) / (2 * kSharedStagePairs));
        it = SharedItem{b, i - (i / H) * H, acc, nc, ip[b], np, lastp[b], n_it};
        acc += nc;
      }
      a.items[(int64_t)wg * kSharedMaxItems + r] = it;
    }
  }
}

template <int D, bool BF16, bool FP8, bool APPEND, bool ROPE, bool DEV>
__global__ void __launch_bounds__(256, 1) decode_shared_kernel(DecodeParams p) {
  using Tr = DecodeTraits<D, BF16, FP8>;
  constexpr int W = Tr::W;
  // one page pair per register stage (not Tr::NP): the waves of a
  // workgroup then end within one pair of each other (TinyLlama B=256 step
  // 56.2 against 56.8 us with two pairs per stage, same runs)
  constexpr int NP = kSharedStagePairs;
  __shared__ SharedLds<D> L;
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n = lane & 15;
  const int G = lane >> 4;
  const int g = p.g;
  int n_it = 0;
  if constexpr (DEV) {
    __shared__ int dev_ip[kDevSharedMaxBatch + 1];
    __shared__ int dev_last[kDevSharedMaxBatch];
    __shared__ __attribute__((aligned(16))) int dev_key[kDevSharedMaxBatch];
    n_it = uniform(dev_item_table<D>(p, L, dev_ip, dev_last, dev_key));
    if (n_it == 0) return;  // uniform over the workgroup: no barrier is skipped by part of it
  }

  // ---- item table: thread t < n_it fills item t from the plan and the
  // metadata of this launch; an item that does not match the launch keeps
  // its chunks but reads and writes nothing (b = -1, no pages).  A host
  // plan's workgroup reads its kSharedMaxItems entries at once (fixed
  // stride), every entry carrying the workgroup's item count.
  {
    const int t = threadIdx.x;
    bool skipped = false;
    SharedItem it{-1, 0, 0, 0, -1, 0, kPage, 0};
    int cnt = n_it;
    if constexpr (DEV) {
      if (t < n_it)
        it = SharedItem{L.b[t], L.h[t], L.chunk_lo[t], L.n_chunks[t], L.ind_lo[t], L.npages[t],
                        L.last[t], n_it};
    } else {
      if (t < kSharedMaxItems) {
        it = reinterpret_cast<const SharedItem*>(p.items)[(int64_t)blockIdx.x * kSharedMaxItems + t];
        cnt = min(max(it.wg_items, 0), kSharedMaxItems);
        if (t == 0) L.n_it = cnt;
      }
    }
    if (t < cnt) {
      // the item's page range comes with it (the plan's metadata, or the
      // kv_indptr / kv_last_page_len this launch's prologue loaded)
      int b = it.b, h = it.h, ind_lo = 0, npages = 0, last = kPage, new_pos = -1;
      if (b < 0 || b >= p.batch_size || h < 0 || h >= p.hkv || it.ind_lo < 0) {
        b = -1;
      } else {
        ind_lo = it.ind_lo;
        npages = max(0, it.npages);
        last = min(max(it.last, 1), kPage);
        new_pos = npages > 0 ? (npages - 1) * kPage + last - 1 : -1;
        if (APPEND && p.new_pos) new_pos = load_invariant(p.new_pos + b);
        // a new token outside the sequence's pages is skipped (counted once
        // per sequence, by its KV head 0)
        const int pg = new_pos >= 0 ? new_pos / kPage : -1;
        skipped = APPEND && h == 0 && npages > 0 && !(pg >= 0 && pg < npages);
      }
      L.b[t] = b;
      L.h[t] = h;
      L.chunk_lo[t] = it.chunk_lo;
      L.n_chunks[t] = max(it.n_chunks, 0);
      L.ind_lo[t] = ind_lo;
      L.npages[t] = npages;
      L.last[t] = last;
      L.new_pos[t] = new_pos;
      if (t == cnt - 1) L.total = it.chunk_lo + max(it.n_chunks, 0);
    }
    if (t == 0) L.next = 0;
    if (t < SharedLds<D>::S) {
      L.tag[t] = t;
      L.cnt[t] = 0;
      L.mask[t] = 0;
    }
    if constexpr (APPEND) count_lanes(p.append_err, skipped);
  }
  __syncthreads();
  if constexpr (!DEV) {
    n_it = uniform(L.n_it);
    if (n_it == 0) return;  // uniform over the workgroup: no barrier is skipped by part of it
  }

  // the table in lanes: lane i < n_it holds item i's fields
  const int li = lane < n_it ? lane : 0;
  const int t_b = L.b[li], t_h = L.h[li], t_lo = L.chunk_lo[li], t_nc = L.n_chunks[li],
            t_ind = L.ind_lo[li], t_np = L.npages[li], t_last = L.last[li],
            t_pos = L.new_pos[li];
  const int total = uniform(L.total);
  auto field = [](int v, int i) { return __builtin_amdgcn_readlane(v, i); };

  // ---- Q of the wave's items (items wave and wave + 4), loaded before the
  // first K/V loads so that waiting for them never waits for K/V
  constexpr int QPW = kSharedMaxItems / 4;
  u32x4 qtmp[QPW][D / 32];
#pragma unroll
  for (int k = 0; k < QPW; ++k) {
    const int i = wave + 4 * k;
    const int b = i < n_it ? field(t_b, i) : -1;
    const int h = b >= 0 ? field(t_h, i) : 0;
    // unconditional loads (a padded head reads head 0's row and is zeroed
    // when the rows are stored), so no wait is placed right after them
    const bool hv = b >= 0 && n < g;
    const uint16_t* qrow =
        p.q + (int64_t)(b < 0 ? 0 : b) * p.q_sn + (int64_t)(h * g + (hv ? n : 0)) * p.q_sh;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
      qtmp[k][ks] = *reinterpret_cast<const u32x4*>(qrow + 32 * ks + 8 * G);
  }

  // with p.deterministic (the default) wave w takes chunks w, w + 4, w + 8,
  // ..., so the states merged per item (and the output bits) do not depend on
  // timing; otherwise chunks are claimed in arrival order through an LDS
  // counter, so a wave that streams more slowly takes fewer
  int next_chunk = wave;
  auto claim = [&]() -> ChunkRef {
    int c;
    if (p.deterministic) {
      c = next_chunk;
      next_chunk += 4;
    } else {
      c = 0;
      if (lane == 0)
        c = __hip_atomic_fetch_add(&L.next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      c = uniform(c);
    }
    if (c >= total) return ChunkRef{-1, 0};
    const int cnt = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < n_it && t_lo <= c));
    const int it = uniform(cnt > 0 ? cnt - 1 : 0);
    return ChunkRef{it, (c - field(t_lo, it)) * 2 * NP};
  };
  // no chunk left: page ids -1, so the loads below read nothing
  auto fetch = [&](PairIds (&ids)[NP], const ChunkRef& r) {
    const int it = max(r.item, 0);
    const int ind_lo = field(t_ind, it), np = r.item < 0 ? 0 : field(t_np, it);
#pragma unroll
    for (int k = 0; k < NP; ++k) ids[k] = fetch_ids(p, ind_lo, r.pg0 + 2 * k, np);
  };
  // loads are issued whether or not a chunk was claimed (an empty one reads
  // nothing), so every iteration issues the same number and the compiler's
  // wait for one stage never waits for the other
  auto load = [&](Stage<D, BF16, FP8> (&st)[NP], const PairIds (&ids)[NP], const ChunkRef& r) {
    const int it = max(r.item, 0);
    const int h = r.item < 0 ? 0 : field(t_h, it), np = field(t_np, it), last = field(t_last, it);
#pragma unroll
    for (int k = 0; k < NP; ++k) load_pair(st[k], p, h, ids[k], r.pg0 + 2 * k, np, last, n, G);
  };

  // Q operands into LDS (rotated with ROPE); lanes of padded heads store zeros
  auto store_q = [&]() {
#pragma unroll
    for (int k = 0; k < QPW; ++k) {
      const int i = wave + 4 * k;
      if (i < n_it) {
        if constexpr (ROPE) {
          const int rope_at = field(t_pos, i);
#pragma unroll
          for (int ks = 0; ks < D / 64; ++ks) {
            float cs[8], sn[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
              rope_cos_sin(rope_at, 32 * ks + 8 * G + e, D, p.rope_inv_scale,
                           p.rope_log2_theta, &cs[e], &sn[e]);
            rope8<BF16>(qtmp[k][ks], qtmp[k][ks + D / 64], cs, sn);
          }
        }
        const bool hv = field(t_b, i) >= 0 && n < g;
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
          const u32x4 z = {0u, 0u, 0u, 0u};
          L.q[i][ks][lane] = hv ? qtmp[k][ks] : z;
        }
      }
    }
  };

  // ---- appends: item i's new K/V rows are written to the pool before any
  // wave loads that page.  With the fixed chunk assignment the wave that
  // will load the chunk holding the new row writes it itself: its own store
  // precedes its load of those addresses in program order, so no wait and
  // no barrier is needed, and the first chunk's loads are issued before the
  // Q barrier.  With arrival-order claims any wave may load the page: the
  // item's wave writes the rows, waits for the stores, and the barrier
  // orders them before every wave's first K/V load.
  const bool det = p.deterministic != 0;
  auto append_item = [&](int i) {
    const int b = field(t_b, i), h = field(t_h, i), np = field(t_np, i), pos = field(t_pos, i);
    const int pg = pos >= 0 ? pos / kPage : -1;
    if (b < 0 || pg < 0 || pg >= np) return;
    const int page = page_id(p, field(t_ind, i), pg, np);
    if (page >= 0)
      fused_append<D, BF16, FP8, ROPE>(p, b, h, page, pos & (kPage - 1), lane, pos);
    else
      count_lanes(p.append_err, h == 0 && lane == 0);
  };
  if constexpr (APPEND) {
    if (det) {
      // chunk chunk_lo + pg / (2 NP) holds page pg of item i; wave (chunk
      // mod 4) claims it
      for (int i = 0; i < n_it; ++i) {
        const int pos = field(t_pos, i);
        const int pg = pos >= 0 ? pos / kPage : 0;
        if (((field(t_lo, i) + pg / (2 * NP)) & 3) == wave) append_item(i);
      }
    } else {
#pragma unroll
      for (int k = 0; k < QPW; ++k) {
        const int i = wave + 4 * k;
        if (i < n_it) append_item(i);
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the appended rows are in L2
      store_q();
      __syncthreads();
    }
  }

  Stage<D, BF16, FP8> sa[NP], sb[NP];
  PairIds ida[NP], idb[NP];
  ChunkRef ra = claim();
  fetch(ida, ra);
  ChunkRef rb = claim();
  fetch(idb, rb);
  load(sa, ida, ra);
  if (!APPEND || det) {
    store_q();
    __syncthreads();
  }

  SoftmaxState<D, BF16, FP8> sm;
  u32x4 qf[D / 32];
  int cur = -1, kcur = 0;

  // leaves the state of item i in its slot; the wave that completes the
  // item's chunk count merges every state there and writes the output
  auto flush = [&](int i, int k) {
    const int s = i % SharedLds<D>::S;
    // the acquire pairs with the release that reopened the slot, so the
    // previous item's resets and reads of the slot come before this write
    bool open = false;
    for (int spin = 0; spin < kSharedSpinLimit; ++spin) {
      const int tg = uniform(__hip_atomic_load(&L.tag[s], __ATOMIC_ACQUIRE,
                                               __HIP_MEMORY_SCOPE_WORKGROUP));
      if (tg == i) {
        open = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!open) {
      // never reached in a consistent run (a slot only waits for items of
      // lower index, whose waves never wait for it); leave the slot alone
      // and count the item as not written rather than corrupt another's state
      count_lanes(p.fault_count, lane == 0);
      return;
    }
    typename SharedLds<D>::State& mine = L.st[s][wave];
#pragma unroll
    for (int e = 0; e < W; ++e) mine.o[e][lane] = sm.o[e];
    mine.m[lane] = sm.m;
    mine.l[lane] = sm.l;
    int old = 0;
    if (lane == 0) {
      __hip_atomic_fetch_or(&L.mask[s], 1 << wave, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      old = __hip_atomic_fetch_add(&L.cnt[s], k, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    old = uniform(old);
    if (old + k != field(t_nc, i)) return;
    const int mask = uniform(__hip_atomic_load(&L.mask[s], __ATOMIC_ACQUIRE,
                                               __HIP_MEMORY_SCOPE_WORKGROUP));
    // every state in the slot (this wave's included), in wave order against
    // their common max, so the sum does not depend on which wave came last
    float M = -INFINITY;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2)
      if ((mask >> w2) & 1) M = fmaxf(M, L.st[s][w2].m[lane]);
    sm.m = M;
    sm.l = 0.f;
#pragma unroll
    for (int e = 0; e < W; ++e) sm.o[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        if (!((mask >> w2) & 1)) continue;
        const typename SharedLds<D>::State& o2 = L.st[s][w2];
        const float m2 = o2.m[lane];
        const float a2 = m2 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m2 - M);
        sm.l += o2.l[lane] * a2;
#pragma unroll
        for (int e = 0; e < W; ++e) sm.o[e] += o2.o[e][lane] * a2;
      }
    }
    const int b = field(t_b, i);
    if (b >= 0) write_item_output<D, BF16, FP8>(p, b, field(t_h, i), -1, sm, G, n);
    if (lane == 0) {
      __hip_atomic_store(&L.cnt[s], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_store(&L.mask[s], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_store(&L.tag[s], i + SharedLds<D>::S, __ATOMIC_RELEASE,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  auto compute = [&](Stage<D, BF16, FP8> (&st)[NP], const ChunkRef& r) {
    if (r.item != cur) {
      if (cur >= 0) flush(cur, kcur);
      cur = r.item;
      kcur = 0;
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) qf[ks] = L.q[cur][ks][lane];
#pragma unroll
      for (int e = 0; e < W; ++e) sm.o[e] = f32x4{0.f, 0.f, 0.f, 0.f};
      sm.m = -INFINITY;
      sm.l = 0.f;
    }
    compute_pairs<D, BF16, FP8, NP>(st, qf, sm, p.scale_log2, G, n);
    ++kcur;
  };

  // ---- chunks: two register stages, the next chunk's loads in flight while
  // the current one is computed, page ids one chunk further ahead
  while (ra.item >= 0) {
    load(sb, idb, rb);
    ChunkRef rc = claim();
    fetch(ida, rc);
    compute(sa, ra);
    if (rb.item < 0) break;
    load(sa, ida, rc);
    ChunkRef rd = claim();
    fetch(idb, rd);
    compute(sb, rb);
    ra = rc;
    rb = rd;
  }
  if (cur >= 0) flush(cur, kcur);
}

// Combine the base-2 partials of n pieces, slot_of(s) giving piece s's
// (slot * g + head) index: M = max lse, den = sum 2^(lse - M), num = sum
// 2^(lse - M) o[dd].  The lse and o of up to four pieces are loaded together,
// so the o loads do not wait for the max; later batches rescale the sums.
template <typename SlotOf>
__device__ __forceinline__ void merge_pieces(int n, SlotOf slot_of, const float* __restrict__ pl,
                                             const float* __restrict__ po, int d, int dd,
                                             float* M_out, float* num_out, float* den_out) {
  constexpr int kBatch = 4;
  float M = -INFINITY, num = 0.f, den = 0.f;
  for (int s0 = 0; s0 < n; s0 += kBatch) {
    float lv[kBatch], ov[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      lv[k] = -INFINITY;
      ov[k] = 0.f;
      if (s0 + k < n) {
        const int64_t sh = slot_of(s0 + k);
        lv[k] = pl[sh];
        if (dd < d) ov[k] = po[sh * d + dd];
      }
    }
    float Mb = M;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) Mb = fmaxf(Mb, lv[k]);
    if (Mb == -INFINITY) continue;
    const float r = M == -INFINITY ? 0.f : exp2f(M - Mb);
    num *= r;
    den *= r;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const float wt = lv[k] == -INFINITY ? 0.f : exp2f(lv[k] - Mb);
      den += wt;
      num += wt * ov[k];
    }
    M = Mb;
  }
  *M_out = M;
  *num_out = num;
  *den_out = den;
}

// Split-KV merge, one workgroup per (split group, query head):
// o = sum_c 2^(lse_c - M) o_c / sum_c 2^(lse_c - M),
// lse = M + log2(sum_c 2^(lse_c - M)) (base-2 partials, natural-log output).
// A separate launch: the kernel boundary orders the partial writes before
// these reads across the XCDs' L2 caches without per-item cache flushes.
template <bool BF16>
__global__ void __launch_bounds__(128)
    decode_merge_kernel(const MergeItem* __restrict__ merges,
                        const float* __restrict__ po,
                        const float* __restrict__ pl, uint16_t* __restrict__ out,
                        float* __restrict__ lse, int hq, int g, int d) {
  const MergeItem mi = merges[blockIdx.x];
  const int hn = blockIdx.y;  // query head within the group
  const int head = mi.h * g + hn;
  const int dd = threadIdx.x;
  float M, num, den;
  merge_pieces(mi.nslots, [&](int s) { return (int64_t)(mi.slot0 + s * mi.stride) * g + hn; },
               pl, po, d, dd, &M, &num, &den);
  if (dd < d)
    out[((int64_t)mi.b * hq + head) * d + dd] =
        f2h<BF16>(M != -INFINITY ? num / den : 0.f);
  if (lse && dd == 0)
    lse[(int64_t)mi.b * hq + head] =
        M != -INFINITY ? (M + log2f(den)) * 0.69314718055994531f : -INFINITY;
}

// Split-KV merge of a device-side partition, one workgroup per (sequence,
// KV head, query head of its group), one thread per d: the pieces of a cut (sequence, head group) segment sit in shares
// first..last; the piece in share w wrote slot (2 w + j) * hg + wi with j = 1
// only for the first share when the segment starts inside it.  Empty
// sequences get zero output and lse = -inf here (the attention launch has no
// item for them); uncut segments were written by the attention launch.
struct MergeImplicitArgs {
  const int32_t* kv_indptr;
  const float* po;
  const float* pl;
  uint16_t* out;
  float* lse;
  int32_t batch, hq, hkv, g, d, hg_shift, n_groups, item_cost;
};

template <bool BF16>
__global__ void __launch_bounds__(128) decode_merge_implicit_kernel(MergeImplicitArgs a) {
  const int b = blockIdx.x / a.hkv;
  const int h = blockIdx.x % a.hkv;
  const int hn = blockIdx.y;  // query head within the group
  const int dd = threadIdx.x;
  const int head = h * a.g + hn;
  const int ngrp = a.hkv >> a.hg_shift;
  const ImplicitSplit sp = implicit_split(a.kv_indptr, a.batch, ngrp, a.n_groups, a.item_cost);
  const int ind_lo = load_invariant(a.kv_indptr + b);
  const int np = load_invariant(a.kv_indptr + b + 1) - ind_lo;
  uint16_t* orow = a.out + ((int64_t)b * a.hq + head) * a.d;
  if (np <= 0) {
    if (dd < a.d) orow[dd] = f2h<BF16>(0.f);
    if (a.lse && dd == 0) a.lse[(int64_t)b * a.hq + head] = -INFINITY;
    return;
  }
  // unit of the segment's first page (implicit_split)
  const int64_t p0 =
      seq_start(sp, b, ind_lo) + (int64_t)(h >> a.hg_shift) * (np + sp.cost) + sp.cost;
  const int64_t first = p0 / sp.share;
  const int64_t last = (p0 + np - 1) / sp.share;
  if (p0 < 0 || first == last || last >= a.n_groups) return;
  const int wi = h & ((1 << a.hg_shift) - 1);
  auto slot_of = [&](int64_t w) {
    const int j = (w == first && p0 != w * sp.share) ? 1 : 0;
    return ((2 * w + j) << a.hg_shift) + wi;
  };
  float M, num, den;
  merge_pieces((int)(last - first + 1), [&](int s) { return slot_of(first + s) * a.g + hn; },
               a.pl, a.po, a.d, dd, &M, &num, &den);
  if (dd < a.d) orow[dd] = f2h<BF16>(M != -INFINITY ? num / den : 0.f);
  if (a.lse && dd == 0)
    a.lse[(int64_t)b * a.hq + head] =
        M != -INFINITY ? (M + log2f(den)) * 0.69314718055994531f : -INFINITY;
}

// ----------------------------------------------------------------------------
// launch table
using DecodeFn = void (*)(DecodeParams);

template <int D, bool BF16, bool FP8, bool IMPLICIT>
DecodeFn decode_fn(bool append, bool rope) {
  if (!append) return decode_kernel<D, BF16, FP8, false, false, IMPLICIT>;
  return rope ? decode_kernel<D, BF16, FP8, true, true, IMPLICIT>
              : decode_kernel<D, BF16, FP8, true, false, IMPLICIT>;
}

template <int D, bool IMPLICIT>
DecodeFn decode_fn_d(bool bf16, bool fp8, bool append, bool rope) {
  if (bf16)
    return fp8 ? decode_fn<D, true, true, IMPLICIT>(append, rope)
               : decode_fn<D, true, false, IMPLICIT>(append, rope);
  return fp8 ? decode_fn<D, false, true, IMPLICIT>(append, rope)
             : decode_fn<D, false, false, IMPLICIT>(append, rope);
}

template <int D, bool BF16, bool FP8, bool DEV>
DecodeFn decode_shared_fn(bool append, bool rope) {
  if (!append) return decode_shared_kernel<D, BF16, FP8, false, false, DEV>;
  return rope ? decode_shared_kernel<D, BF16, FP8, true, true, DEV>
              : decode_shared_kernel<D, BF16, FP8, true, false, DEV>;
}

template <int D, bool DEV>
DecodeFn decode_shared_fn_d(bool bf16, bool fp8, bool append, bool rope) {
  if (bf16)
    return fp8 ? decode_shared_fn<D, true, true, DEV>(append, rope)
               : decode_shared_fn<D, true, false, DEV>(append, rope);
  return fp8 ? decode_shared_fn<D, false, true, DEV>(append, rope)
             : decode_shared_fn<D, false, false, DEV>(append, rope);
}

static DecodeFn pick_decode_shared(int d, bool bf16, bool fp8, bool append, bool rope,
                                   bool dev) {
  if (dev)
    return d == 64 ? decode_shared_fn_d<64, true>(bf16, fp8, append, rope)
                   : decode_shared_fn_d<128, true>(bf16, fp8, append, rope);
  return d == 64 ? decode_shared_fn_d<64, false>(bf16, fp8, append, rope)
                 : decode_shared_fn_d<128, false>(bf16, fp8, append, rope);
}

static DecodeFn pick_decode(int d, bool bf16, bool fp8, bool append, bool rope, bool implicit) {
  if (d == 64)
    return implicit ? decode_fn_d<64, true>(bf16, fp8, append, rope)
                    : decode_fn_d<64, false>(bf16, fp8, append, rope);
  return implicit ? decode_fn_d<128, true>(bf16, fp8, append, rope)
                  : decode_fn_d<128, false>(bf16, fp8, append, rope);
}

}  // namespace pa

using namespace pa;


namespace pa {

struct AppendRows {
  const void* k;
  const void* v;
  int64_t k_sn, k_sh, v_sn, v_sh;
  int32_t dtype;
  bool rope;
  const int32_t* new_pos;
  double rope_inv_scale, rope_log2_theta;
  // fused append: tokens skipped (position outside the sequence's pages or
  // an invalid page id) are counted at append_err[0], clamped e4m3 pieces at
  // append_err[1] (may be null)
  int32_t* append_err;
};

static int decode_run_impl(const char* who, const pagedattn_plan* plan,
                           const void* q, int64_t q_stride_n,
                           int64_t q_stride_h, int32_t q_dtype,
                           const void* paged_kv_cache, int32_t kv_dtype,
                           const float* kv_scales, int32_t num_pages,
                           const int32_t* kv_indices, int32_t num_indices,
                           const int32_t* kv_indptr,
                           const int32_t* kv_last_page_len, void* out,
                           float* lse, float sm_scale, const AppendRows* app,
                           void* stream) {
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
  if (plan->batch_size == 0 || plan->n_items == 0) return PAGEDATTN_OK;
  if (!q || !paged_kv_cache || !kv_indices || !kv_indptr ||
      !kv_last_page_len || !out)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null pointer", who);
  if ((q_stride_n & 7) || (q_stride_h & 7) || !aligned16(q) ||
      !aligned16(paged_kv_cache) || !aligned16(out))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: q, out and the pool must be 16-byte aligned with "
                     "strides that are multiples of 8 elements",
                     who);
  if (num_pages < 0 || num_indices < 0)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: negative sizes", who);

  DecodeParams p;
  p.items = static_cast<const DecodeItem*>(plan->items_dev);
  p.wave_ptr = plan->wave_ptr_dev;
  p.n_groups = plan->n_items;
  p.hg_shift = plan->hg_shift;
  p.deterministic = plan->deterministic ? 1 : 0;
  p.item_cost = plan->item_cost;
  p.n_merge = plan->n_merge;
  p.n_slots = plan->n_slots;
  p.batch_size = plan->batch_size;
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
  p.k_new = app ? static_cast<const uint16_t*>(app->k) : nullptr;
  p.v_new = app ? static_cast<const uint16_t*>(app->v) : nullptr;
  p.k_sn = app ? app->k_sn : 0;
  p.k_sh = app ? app->k_sh : 0;
  p.v_sn = app ? app->v_sn : 0;
  p.v_sh = app ? app->v_sh : 0;
  p.new_pos = app ? app->new_pos : nullptr;
  p.rope_inv_scale = app ? app->rope_inv_scale : 1.0;
  p.rope_log2_theta = app ? app->rope_log2_theta : 0.0;
  p.append_err = app ? app->append_err : nullptr;
  // int32 2 of the workspace header (plan workspaces; noalloc runs have none)
  p.fault_count = plan->workspace ? static_cast<int32_t*>(plan->workspace) + 2 : nullptr;

  hipStream_t s = (hipStream_t)stream;
  const bool bf16 = q_dtype == PAGEDATTN_BF16;
  if (plan->shared) {
    // a device-planned shared plan (implicit) finds its items from kv_indptr,
    // unless pagedattn_decode_plan_device_update has dealt them into the
    // workspace (read as a host plan's)
    DecodeFn fn = pick_decode_shared(plan->d, bf16, fp8, app != nullptr, app && app->rope,
                                     plan->implicit && !plan->dev_table);
    if (!fn)
      return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: shared-item plan for D = %d", who,
                       plan->d);
    hipLaunchKernelGGL(fn, dim3(plan->n_items), dim3(256), 0, s, p);
    return check_launch(who);
  }
  DecodeFn fn = pick_decode(plan->d, bf16, fp8, app != nullptr, app && app->rope,
                            plan->implicit);
  const int blocks = ((plan->n_items << plan->hg_shift) + 3) / 4;
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), 0, s, p);
  int rc = check_launch(who);
  if (rc) return rc;
  if (plan->implicit) {
    MergeImplicitArgs m{kv_indptr, plan->partial_o, plan->partial_lse, p.out, lse,
                        plan->batch_size, plan->hq, plan->hkv, p.g, plan->d,
                        plan->hg_shift, plan->n_items, plan->item_cost};
    const dim3 grid((unsigned)((int64_t)plan->batch_size * plan->hkv), p.g);
    if (bf16)
      hipLaunchKernelGGL(decode_merge_implicit_kernel<true>, grid, dim3(plan->d), 0, s, m);
    else
      hipLaunchKernelGGL(decode_merge_implicit_kernel<false>, grid, dim3(plan->d), 0, s, m);
    return check_launch("decode_run(merge)");
  }
  if (plan->n_merge == 0) return rc;
  const dim3 grid(plan->n_merge, p.g);
  const MergeItem* merges = static_cast<const MergeItem*>(plan->merge_dev);
  if (bf16)
    hipLaunchKernelGGL(decode_merge_kernel<true>, grid, dim3(plan->d), 0, s, merges,
                       plan->partial_o, plan->partial_lse, p.out, lse, plan->hq, p.g,
                       plan->d);
  else
    hipLaunchKernelGGL(decode_merge_kernel<false>, grid, dim3(plan->d), 0, s, merges,
                       plan->partial_o, plan->partial_lse, p.out, lse, plan->hq, p.g,
                       plan->d);
  return check_launch("decode_run(merge)");
}

}  // namespace pa

extern "C" {

int pagedattn_decode_plan_device_update(pagedattn_plan* plan, const int32_t* kv_indptr,
                                        const int32_t* kv_last_page_len, void* stream) {
  const char* who = "decode_plan_device_update";
  if (!plan || plan->mode != kPlanDecode || !plan->implicit)
    return set_error(PAGEDATTN_ERR_PLAN, "%s: no device decode plan (call plan_device first)",
                     who);
  if (!plan->shared) return PAGEDATTN_OK;  // the split partition is made by every run
  if (!kv_indptr || !kv_last_page_len)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null pointer", who);
  const size_t bytes = sizeof(SharedItem) * (size_t)plan->n_items * kSharedMaxItems;
  if (!plan->workspace || plan->workspace_bytes < kWsHeader + bytes)
    return set_error(PAGEDATTN_ERR_WORKSPACE, "%s: the item table needs %zu bytes after the "
                     "workspace header", who, bytes);
  SharedTableArgs a{kv_indptr, kv_last_page_len, plan->batch_size, plan->hkv, plan->n_items,
                    reinterpret_cast<SharedItem*>(static_cast<char*>(plan->workspace) + kWsHeader),
                    static_cast<int32_t*>(plan->workspace) + 2};
  hipLaunchKernelGGL(decode_shared_table_kernel, dim3(1), dim3(kSharedTableThreads), 0,
                     (hipStream_t)stream, a);
  const int rc = check_launch(who);
  if (rc) return rc;
  plan->items_dev = a.items;
  plan->dev_table = true;
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
  return decode_run_impl("decode_run", plan, q, q_stride_n, q_stride_h, q_dtype,
                         paged_kv_cache, kv_dtype, kv_scales, num_pages,
                         kv_indices, num_indices, kv_indptr, kv_last_page_len,
                         out, lse, sm_scale, nullptr, stream);
}

int pagedattn_decode_run_append(
    const pagedattn_plan* plan, const void* q, int64_t q_stride_n,
    int64_t q_stride_h, int32_t q_dtype, const void* append_key,
    const void* append_value, int64_t k_stride_n, int64_t k_stride_h,
    int64_t v_stride_n, int64_t v_stride_h, void* paged_kv_cache,
    int32_t kv_dtype, const float* kv_scales, int32_t num_pages,
    const int32_t* kv_indices, int32_t num_indices, const int32_t* kv_indptr,
    const int32_t* kv_last_page_len, void* out, float* lse, float sm_scale,
    void* stream) {
  const char* who = "decode_run_append";
  if (!append_key || !append_value)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null append rows", who);
  if ((k_stride_n & 7) || (k_stride_h & 7) || (v_stride_n & 7) ||
      (v_stride_h & 7) || !aligned16(append_key) || !aligned16(append_value))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: append rows must be 16-byte aligned with strides that "
                     "are multiples of 8 elements",
                     who);
  // skipped tokens are counted in the int32 at byte 0 of the workspace,
  // clamped e4m3 pieces in the one at byte 4
  AppendRows app{append_key, append_value, k_stride_n, k_stride_h,
                 v_stride_n, v_stride_h, q_dtype, false, nullptr, 1.0, 0.0,
                 plan ? static_cast<int32_t*>(plan->workspace) : nullptr};
  return decode_run_impl(who, plan, q, q_stride_n, q_stride_h, q_dtype,
                         paged_kv_cache, kv_dtype, kv_scales, num_pages,
                         kv_indices, num_indices, kv_indptr, kv_last_page_len,
                         out, lse, sm_scale, &app, stream);
}

int pagedattn_decode_run_rope_append(
    const pagedattn_plan* plan, const void* q, int64_t q_stride_n,
    int64_t q_stride_h, int32_t q_dtype, const void* append_key,
    const void* append_value, int64_t k_stride_n, int64_t k_stride_h,
    int64_t v_stride_n, int64_t v_stride_h, const int32_t* positions,
    float rope_scale, float rope_theta, void* paged_kv_cache, int32_t kv_dtype,
    const float* kv_scales, int32_t num_pages, const int32_t* kv_indices,
    int32_t num_indices, const int32_t* kv_indptr,
    const int32_t* kv_last_page_len, void* out, float* lse, float sm_scale,
    void* stream) {
  const char* who = "decode_run_rope_append";
  if (!append_key || !append_value)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null append rows", who);
  if ((k_stride_n & 7) || (k_stride_h & 7) || (v_stride_n & 7) ||
      (v_stride_h & 7) || !aligned16(append_key) || !aligned16(append_value))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: append rows must be 16-byte aligned with strides that "
                     "are multiples of 8 elements",
                     who);
  if (!(rope_scale > 0.f) || !(rope_theta > 0.f))
    return set_error(PAGEDATTN_ERR_INVALID, "%s: rope_scale and rope_theta must be > 0",
                     who);
  AppendRows app{append_key, append_value, k_stride_n, k_stride_h, v_stride_n,
                 v_stride_h, q_dtype, true, positions, 1.0 / (double)rope_scale,
                 std::log2((double)rope_theta),
                 plan ? static_cast<int32_t*>(plan->workspace) : nullptr};
  return decode_run_impl(who, plan, q, q_stride_n, q_stride_h, q_dtype,
                         paged_kv_cache, kv_dtype, kv_scales, num_pages,
                         kv_indices, num_indices, kv_indptr, kv_last_page_len,
                         out, lse, sm_scale, &app, stream);
}

}  // extern "C"

// ----------------------------------------------------------------------------
// Decode without a plan object or workspace (pagedattn_decode_run_noalloc).
namespace pa {

// Split partials of pagedattn_decode_run_noalloc: one array per GPU, loaded
// with the code object and held until the process ends.  Host code never
// uses its name as an address: the per-device address comes from
// hipGetSymbolAddress.
static __device__ __align__(256) uint8_t scratch[PAGEDATTN_NOALLOC_SCRATCH_BYTES];

constexpr int kNoAllocMaxDevices = 64;
struct NoAllocDevice {
  char* scratch;  // device address of `scratch` on this GPU
  int cus;
};
static NoAllocDevice g_noalloc[kNoAllocMaxDevices];
static std::mutex g_noalloc_mu;

// Set-up on the current device, once: the address of its copy of the
// array and its CU count.  Allocates nothing.
static int noalloc_device(const char* who, NoAllocDevice* out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(PAGEDATTN_ERR_HIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: device %d (at most %d devices)", who, dev,
                     kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  NoAllocDevice& d = g_noalloc[dev];
  if (d.scratch == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return set_error(PAGEDATTN_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", who,
                       hipGetErrorString(e));
    int cus = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess || cus <= 0)
      return set_error(PAGEDATTN_ERR_HIP, "%s: CU count of device %d: %s", who, dev,
                       hipGetErrorString(e));
    d.cus = cus;
    d.scratch = static_cast<char*>(ptr);
  }
  *out = d;
  return PAGEDATTN_OK;
}

}  // namespace pa

extern "C" {

int pagedattn_decode_run_noalloc(int32_t batch_size, int32_t num_qo_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                 const void* q, int64_t q_stride_n, int64_t q_stride_h,
                                 int32_t q_dtype, const void* paged_kv_cache, int32_t kv_dtype,
                                 const float* kv_scales, int32_t num_pages,
                                 const int32_t* kv_indices, int32_t num_indices,
                                 const int32_t* kv_indptr, const int32_t* kv_last_page_len,
                                 void* out, float* lse, float sm_scale, void* stream) {
  const char* who = "decode_run_noalloc";
  NoAllocDevice dev;
  int rc = noalloc_device(who, &dev);
  if (rc) return rc;
  // a stack plan: its host staging vector stays empty, nothing is allocated
  pagedattn_plan plan;
  rc = setup_device_plan(who, &plan, batch_size, num_qo_heads, num_kv_heads, head_dim,
                         page_size, dev.cus, dev.scratch, PAGEDATTN_NOALLOC_SCRATCH_BYTES);
  if (rc) return rc;
  return decode_run_impl(who, &plan, q, q_stride_n, q_stride_h, q_dtype, paged_kv_cache,
                         kv_dtype, kv_scales, num_pages, kv_indices, num_indices, kv_indptr,
                         kv_last_page_len, out, lse, sm_scale, nullptr, stream);
}

}  // extern "C"
