// Ragged, paged, causal prefill attention for gfx950
// (BatchPrefillWithPagedKVCacheWrapper, src/models/llama.py:86-116 plan and
// :212-228 run).
//
// Work unit: a tile of ROWS query rows of one sequence and one KV head, where
// a row is (query token, query head of the group): rows are token-major with
// the g = Hq/Hkv heads of a token adjacent, so every K/V tile staged in LDS
// serves all heads of the group.  A 512-thread workgroup runs 8 waves (two
// per SIMD); wave w owns RB blocks of 32 rows.  The KV loop walks 64-token
// tiles (4 pages):
//
//   S^T[64 tok x 32 rows] = K[tok x D] . Q^T          v_mfma_f32_32x32x16_bf16
//   O^T[D x 32 rows]     += V^T[D x 64 tok] . P^T      (P stays in registers)
//
// The S^T accumulator layout (lane = row, 16 registers = tokens) is already
// the B-operand layout that PV needs once the token order inside each
// 16-token step is permuted the same way on both operands, so P never leaves
// registers; a lane's row max / sum need one cross-half exchange.  K and V
// tiles are staged row-major in LDS by direct-to-LDS buffer loads (e4m3:
// register loads converted to 16-bit on the way in) into unpadded rows whose
// 16-byte chunks are XOR-swizzled per row; the V^T operand is read with
// ds_read_b64_tr_b16, whose 16-lane groups return the transposed 4x16 block,
// so no transposing writes exist.  Loads use buffer resources sized to each
// page's valid tokens: absent pages and slots past last_page_len read as
// zero without touching memory.  Causal tiles entirely below the diagonal
// skip masking; tiles above the last row's diagonal are never visited.
#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <vector>

#include "plan_internal.h"

namespace pa {

struct PrefillParams {
  const PrefillItem* items;
  int32_t n_items, batch_size;
  const uint16_t* q;
  int64_t q_sn, q_sh;
  const int32_t* qo_indptr;
  const uint8_t* cache;
  const float* kv_scales;
  int32_t num_pages;
  const int32_t* kv_indices;
  int32_t num_indices;
  const int32_t* kv_indptr;
  const int32_t* last_page_len;
  uint16_t* out;  // [nnz, hq, D]
  float* lse;     // [nnz, hq] or null
  int32_t hq, hkv, g, causal;
  float scale_log2;
};

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <bool BF16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
        0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

template <bool BF16, bool HI>
__device__ __forceinline__ uint32_t e4m3x2_to16(uint32_t w) {
  if constexpr (BF16) {
    return __builtin_bit_cast(
        uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
  } else {
    return __builtin_bit_cast(
        uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
}


template <int D, bool BF16, bool FP8, int RB>
struct PrefillCfg {
  static constexpr int ESZ = FP8 ? 1 : 2;
  static constexpr int BN = 64;             // kv tokens per tile
  static constexpr int WAVES = kPrefillWaves;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int ROWS = WAVES * 32 * RB;  // rows per workgroup
  static constexpr int KS = D / 16;         // QK k-steps
  static constexpr int DT = D / 32;         // PV d tiles
  // LDS tiles are unpadded rows of ROWB bytes (16-bit elements) whose
  // 16-byte chunks are XOR-swizzled per row (see swz), so whole 1 KiB runs
  // can be written by direct-to-LDS loads and both read patterns below are
  // free of bank conflicts.
  static constexpr int ROWB = D * 2;
  static constexpr int TILEB = BN * ROWB;  // bytes of one K or V tile
  static constexpr int CHUNKS = BN * D / 8;   // 16-byte (bf16) chunks per tile
  static constexpr int CPT = CHUNKS / THREADS;  // chunks per thread
  static constexpr int PAGE_BYTES = kPage * D * ESZ;
  using Raw = typename std::conditional<FP8, u32x2, u32x4>::type;
};

// Chunk swizzle of LDS row r: chunk c of the row is stored at position
// c ^ swz(r).  LDS has 64 banks of 4 bytes, so a 16-byte position p of a
// 256-byte row covers banks 4p..4p+3.  D = 128 (16 chunks of 16 B per row):
//  * K operand reads (ds_read_b128; 16 lanes at a time read one chunk of 16
//    consecutive rows) need swz to be a bijection on r mod 16;
//  * V transpose reads (ds_read_b64_tr_b16; 32 lanes at a time read chunks
//    4i..4i+3 of 4 consecutive rows) need the 4 rows to put that chunk
//    quad in 4 different position quads, i.e. distinct swz(r) >> 2.
// Swapping the two 2-bit fields of r mod 16 does both: no bank conflicts for
// either read (measured with SQ_LDS_BANK_CONFLICT; the previous
// ((r & 7) << 1) | ((r >> 3) & 1) left the transpose reads 2-way
// conflicted, half their LDS cycles).  D = 64 (8 chunks, two rows per bank
// line, so a K read's 16 rows share 8 lines): bits 1-2 of r, and r1 ^ r3 on
// top, is conflict-free for both reads in a model of the bank mapping that
// reproduces the D = 128 measurements (the previous
// ((r & 3) << 1) | ((r >> 2) & 1) left the K reads 2-way conflicted there).
template <int D>
__device__ __forceinline__ int swz(int r) {
  if constexpr (D == 128) {
    return ((r & 3) << 2) | ((r >> 2) & 3);
  } else {
    return ((r >> 1) & 3) | ((((r >> 1) ^ (r >> 3)) & 1) << 2);
  }
}

template <int D>
__device__ __forceinline__ int lds_off(int r, int c) {
  return r * (D * 2) + ((c ^ swz<D>(r)) << 4);
}

// Registers staging one half (K rows or V rows) of an e4m3 K/V tile between
// its global loads and its converting LDS store.
template <int D, bool BF16, bool FP8, int RB>
struct HalfRegs {
  using C = PrefillCfg<D, BF16, FP8, RB>;
  // 16 e4m3 elements per lane and load where the tile divides evenly
  static constexpr bool WIDE = (C::CHUNKS / 2) % C::THREADS == 0;
  static constexpr int NL = WIDE ? C::CHUNKS / 2 / C::THREADS : C::CPT;
  typename std::conditional<WIDE, u32x4, u32x2>::type x[NL];
  float sc;  // lane j < 4 holds the scale of the tile's page j
};

// Page ids of tile `tile` as a vector load: lane j < 4 gets the id of the
// tile's page j (-1 past the sequence).  Issued a tile ahead of the K/V
// loads that use it, it is waited on with the in-order vector counter, so
// no K/V load ever waits for a page-id fetch.
__device__ __forceinline__ int fetch_page_ids(const PrefillParams& p,
                                              int ind_lo, int npages,
                                              int tile, int lane) {
  const int pg = tile * 4 + lane;
  int id = -1;
  if (lane < 4 && pg < npages && ind_lo >= 0 && ind_lo + pg < p.num_indices)
    id = p.kv_indices[ind_lo + pg];
  return id;
}

// Buffer resource of the K (V = false) or V block of tile page j, sized to
// its valid tokens: absent pages and slots past last_page_len read as zero.
template <int D, bool BF16, bool FP8, int RB, bool V>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(
    const PrefillParams& p, int h, int pid, int npages, int last, int tile,
    int j) {
  using C = PrefillCfg<D, BF16, FP8, RB>;
  int id = __builtin_amdgcn_readlane(pid, j);
  if (id >= p.num_pages) id = -1;
  const int pg = tile * 4 + j;
  const int ntok = id < 0 ? 0 : (pg == npages - 1 ? last : kPage);
  const uint8_t* base =
      p.cache + (((int64_t)(id < 0 ? 0 : id) * 2 + (V ? 1 : 0)) * p.hkv + h) *
                    (int64_t)C::PAGE_BYTES;
  return make_rsrc(base, (uint32_t)(ntok * D * C::ESZ));
}

// bf16/fp16 pools: direct-to-LDS loads of one half of a K/V tile by a group
// of NW waves.  Wave w's k-th load fills the 1 KiB block NW k + w of the tile
// (lane i -> bytes [16 i, 16 i + 16) of the block), so each lane fetches the
// global chunk that the swizzle puts at its position.
template <int D, bool BF16, bool FP8, int RB, bool V, int NW>
__device__ __forceinline__ void dma_half(const PrefillParams& p, int h,
                                         int pid, int npages, int last,
                                         int tile, uint8_t* lds, int wave,
                                         int lane) {
  using C = PrefillCfg<D, BF16, FP8, RB>;
  constexpr int RPB = 1024 / C::ROWB;   // rows per 1 KiB block
  constexpr int CPR = C::ROWB / 16;     // chunks per row
  constexpr int NK = C::TILEB / 1024 / NW;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int blk = NW * k + wave;
    const int row0 = blk * RPB;
    const int j = uniform(row0 / kPage);  // page of the block within the tile
    const __amdgpu_buffer_rsrc_t r =
        page_rsrc<D, BF16, FP8, RB, V>(p, h, pid, npages, last, tile, j);
    const int row = row0 + lane / CPR;
    const int c = (lane % CPR) ^ swz<D>(row);
    const uint32_t off = (uint32_t)((row % kPage) * C::ROWB + c * 16);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)(lds + blk * 1024), 16, off,
        0, 0, 0);
  }
}

// e4m3 pools: register loads of one half of a K/V tile (16 elements per
// lane and load at D = 128, 8 at D = 64) plus the four page scales.
template <int D, bool BF16, bool FP8, int RB, bool V>
__device__ __forceinline__ void load_half(HalfRegs<D, BF16, FP8, RB>& hr,
                                          const PrefillParams& p, int h,
                                          int pid, int npages, int last,
                                          int tile, int wave, int lane) {
  using C = PrefillCfg<D, BF16, FP8, RB>;
  using H = HalfRegs<D, BF16, FP8, RB>;
  constexpr int E = H::WIDE ? 16 : 8;  // elements per lane and load
#pragma unroll
  for (int k = 0; k < H::NL; ++k) {
    const int c = lane + 64 * wave + C::THREADS * k;
    const int tok = c / (D / E);
    const int d0 = (c % (D / E)) * E;
    // the 64 pieces of a wave lie in one page of the tile
    const int j = uniform((64 * wave + C::THREADS * k) / (D / E) / kPage);
    const __amdgpu_buffer_rsrc_t r =
        page_rsrc<D, BF16, FP8, RB, V>(p, h, pid, npages, last, tile, j);
    if constexpr (H::WIDE) {
      hr.x[k] = buf_load16(r, (uint32_t)((tok % kPage) * D + d0));
    } else {
      hr.x[k] = buf_load8(r, (uint32_t)((tok % kPage) * D + d0));
    }
  }
  hr.sc = 0.f;
  if (lane < 4 && pid >= 0 && pid < p.num_pages)
    hr.sc = p.kv_scales[((int64_t)pid * 2 + (V ? 1 : 0)) * p.hkv + h];
}

// e4m3 -> 16-bit conversion and store of a staged half tile, swizzled.
template <int D, bool BF16, bool FP8, int RB>
__device__ __forceinline__ void store_half(const HalfRegs<D, BF16, FP8, RB>& hr,
                                           uint8_t* lds, int wave, int lane) {
  using C = PrefillCfg<D, BF16, FP8, RB>;
  using H = HalfRegs<D, BF16, FP8, RB>;
  constexpr int E = H::WIDE ? 16 : 8;
#pragma unroll
  for (int k = 0; k < H::NL; ++k) {
    const int c = lane + 64 * wave + C::THREADS * k;
    const int tok = c / (D / E);
    const int chunk = (c % (D / E)) * (E / 8);
#pragma unroll
    for (int q = 0; q < E / 8; ++q) {
      u32x4 x;
      x[0] = e4m3x2_to16<BF16, false>(hr.x[k][2 * q]);
      x[1] = e4m3x2_to16<BF16, true>(hr.x[k][2 * q]);
      x[2] = e4m3x2_to16<BF16, false>(hr.x[k][2 * q + 1]);
      x[3] = e4m3x2_to16<BF16, true>(hr.x[k][2 * q + 1]);
      *reinterpret_cast<u32x4*>(lds + lds_off<D>(tok, chunk + q)) = x;
    }
  }
}

__device__ __forceinline__ float lane_value(float v, int i) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), i));
}

// Rescale threshold (log2 units): the running max of a row is only moved
// when a tile raises it by more than this, so P = 2^(s - m) <= 2^8 and the
// rescale of O and l runs on few tiles.
constexpr float kRescaleSlack = 8.f;

template <int D, bool BF16, bool FP8, int RB>
__global__ void __launch_bounds__(64 * kPrefillWaves, 1) prefill_kernel(PrefillParams p) {
  using C = PrefillCfg<D, BF16, FP8, RB>;
  constexpr int BN = C::BN;
  // Two stages, each a K tile then a V tile.  Tile t lives in stage t & 1;
  // tile t + 1 is loaded into the other stage while tile t is computed.
  // Separate arrays (not one indexed array) let the compiler see that the
  // direct-to-LDS loads into one stage never alias reads of the other, so it
  // does not wait for them before those reads.
  __shared__ __attribute__((aligned(1024))) uint8_t stage0[2 * C::TILEB];
  __shared__ __attribute__((aligned(1024))) uint8_t stage1[2 * C::TILEB];
  // The second head's stages of a paired tile.  Pairing is built for
  // 16-bit pools at D = 128 only: at D = 64 its registers would cost the
  // second workgroup per CU.
  constexpr bool PAIRS = !FP8 && D == 128;
  __shared__ __attribute__((aligned(1024))) uint8_t stage2[PAIRS ? 2 * C::TILEB : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t stage3[PAIRS ? 2 * C::TILEB : 16];

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int col = lane & 31;   // row of the 32-row block this lane owns
  const int half = lane >> 5;  // k-half of the MFMA operands
  // Workgroup w runs KV head w % Hkv of item w / Hkv.  Workgroups are dealt
  // to the 8 XCDs round-robin by id, so one KV head's work stays on one XCD
  // (Hkv = 8) or a fixed pair of them, and the q-tiles that re-read the same
  // K/V pages (and prefix pages shared between sequences) hit that XCD's L2.
  const int h = (int)(blockIdx.x % (unsigned)p.hkv);
  const int item = (int)(blockIdx.x / (unsigned)p.hkv);
  const int g = p.g;
  // a work list that does not match this launch is skipped, never followed
  // (every condition is uniform over the workgroup)
  if (item >= p.n_items) return;
  const int32_t* itp = reinterpret_cast<const int32_t*>(p.items + item);
  const int b = uniform(load_invariant(itp + 0));
  if (b < 0 || b >= p.batch_size) return;
  const int qo_start = uniform(load_invariant(p.qo_indptr + b));
  const int qo_len = max(0, uniform(load_invariant(p.qo_indptr + b + 1)) - qo_start);
  const int q_lo = max(0, uniform(load_invariant(itp + 1)));
  const int q_hi = min(uniform(load_invariant(itp + 2)), qo_len);
  if (q_lo >= q_hi) return;
  const int ind_lo = uniform(load_invariant(p.kv_indptr + b));
  const int npages = max(0, uniform(load_invariant(p.kv_indptr + b + 1)) - ind_lo);
  const int last = min(max(uniform(load_invariant(p.last_page_len + b)), 1), kPage);
  const int kv_len = npages > 0 ? (npages - 1) * kPage + last : 0;
  const int diag = kv_len - qo_len;  // row i sees kv j <= diag + i
  const int kv_end =
      p.causal ? min(kv_len, max(0, diag + q_hi)) : kv_len;
  const int clean_end =
      p.causal ? min(kv_len, max(0, diag + q_lo + 1)) : kv_len;
  const int n_tiles = (kv_end + BN - 1) / BN;
  // A paired tile (flagged by the planner; at most half the workgroup's rows)
  // is run for KV heads h0 = h & ~1 and h0 + 1 by one workgroup of the pair,
  // the even head's (flag 1) or the odd head's (flag 2): waves
  // 0 .. WAVES/2 - 1 take head h0, the others head h0 + 1, each group with
  // its own K/V stages.  Both groups walk the same tiles, so they meet at
  // every barrier.  The pair's other workgroup has nothing left to do.
  const int pflag = uniform(load_invariant(itp + 3));
  const bool paired = PAIRS && (p.hkv & 1) == 0 && (pflag == 1 || pflag == 2) &&
                      (q_hi - q_lo) * g <= C::ROWS / 2;
  if (paired && (h & 1) != pflag - 1) return;

  // The tile loop of one head group: NW waves, wave index `wave` within the
  // group, KV head `h`, LDS stages st0 / st1.
  auto body = [&](auto pair_tag, uint8_t* st0, uint8_t* st1, const int wave,
                  const int h) __attribute__((always_inline)) {
    constexpr int NW = decltype(pair_tag)::value ? C::WAVES / 2 : C::WAVES;

    // ---- Q^T fragments (B operand): lane -> row, 8 consecutive d per k-step
    u32x4 qf[RB][C::KS];
    int lim[RB];       // last visible kv index of the lane's row
    bool rvalid[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = 32 * (RB * wave + rb) + col;
      const int qi = q_lo + row / g;
      rvalid[rb] = qi < q_hi;
      lim[rb] = p.causal ? min(diag + qi, kv_len - 1) : kv_len - 1;
      const uint16_t* qp =
          p.q + (int64_t)(qo_start + (rvalid[rb] ? qi : q_lo)) * p.q_sn +
          (int64_t)(h * g + row % g) * p.q_sh + 8 * half;
#pragma unroll
      for (int ks_ = 0; ks_ < C::KS; ++ks_) {
        u32x4 z = {0u, 0u, 0u, 0u};
        if (rvalid[rb]) z = *reinterpret_cast<const u32x4*>(qp + 16 * ks_);
        qf[rb][ks_] = z;
      }
    }

    // whether any row of this wave lies in the tile
    const bool wave_rows = 32 * RB * wave < (q_hi - q_lo) * g;

    f32x16 o[RB][C::DT];
    float m[RB], l[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) o[rb][dt] = f32x16{};
      m[rb] = -INFINITY;
      l[rb] = 0.f;
    }

    // Per-lane LDS byte offsets (swizzled) of the MFMA operand reads, fixed
    // for the whole loop: K rows 32 mt + col, chunk 2 ks + half (mt adds
    // 32 rows, which keeps the swizzle); V transpose reads at rows
    // 16 st + 4 half + L/4 (+8), chunk 4 dt + 2 (qg & 1) + (L & 3) / 2.
    int koff[C::KS];
#pragma unroll
    for (int ks_ = 0; ks_ < C::KS; ++ks_) koff[ks_] = lds_off<D>(col, 2 * ks_ + half);
    const int L = lane & 15;
    const int qg = lane >> 4;
    int voff[C::DT][2];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
        voff[dt][hi] = C::TILEB +
                       lds_off<D>(4 * half + (L >> 2) + 8 * hi,
                                  4 * dt + 2 * (qg & 1) + ((L & 3) >> 1)) +
                       8 * (L & 1);

    HalfRegs<D, BF16, FP8, RB> kr, vr;  // e4m3 staging only
    float ksc_l = 0.f, vsc_l = 0.f;     // e4m3 scales of the computed tile
    int pid = fetch_page_ids(p, ind_lo, npages, 0, lane);
    if (n_tiles > 0) {
      if constexpr (FP8) {
        load_half<D, BF16, FP8, RB, false>(kr, p, h, pid, npages, last, 0, wave, lane);
        load_half<D, BF16, FP8, RB, true>(vr, p, h, pid, npages, last, 0, wave, lane);
      } else {
        dma_half<D, BF16, FP8, RB, false, NW>(p, h, pid, npages, last, 0, st0, wave, lane);
        dma_half<D, BF16, FP8, RB, true, NW>(p, h, pid, npages, last, 0, st0 + C::TILEB,
                                             wave, lane);
      }
    }
    int pid_next = fetch_page_ids(p, ind_lo, npages, 1, lane);

    // Tile t's QK, softmax and PV from stage `cur` (e4m3: with the register
    // loads of tile t + 1, pages pid_ld, issued between its phases).
    auto compute = [&](auto mask_tag, int t, uint8_t* cur, int pid_ld) __attribute__((always_inline)) {
      constexpr bool MASK = decltype(mask_tag)::value;
      // ---- S^T = K . Q^T
      f32x16 s[RB][2];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) s[rb][0] = s[rb][1] = f32x16{};
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int ks_ = 0; ks_ < C::KS; ++ks_) {
          const u32x4 a =
              *reinterpret_cast<const u32x4*>(cur + 32 * mt * C::ROWB + koff[ks_]);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) s[rb][mt] = mfma32<BF16>(a, qf[rb][ks_], s[rb][mt]);
        }
        if (mt == 0) {
          if constexpr (FP8)
            load_half<D, BF16, FP8, RB, false>(kr, p, h, pid_ld, npages, last, t + 1, wave, lane);
        }
      }

      // ---- online softmax in log2 units; lane holds 32 of the tile's 64
      // tokens of its row (token 32 mt + 8 (i/4) + 4 half + i%4 in register i)
      const int tok0 = t * BN;
      float ksc[4], vsc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ksc[i] = FP8 ? fmaxf(lane_value(ksc_l, i) * p.scale_log2, FLT_MIN) : p.scale_log2;
        vsc[i] = FP8 ? lane_value(vsc_l, i) : 1.f;
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if constexpr (MASK) {
          const int rel = lim[rb] - tok0 - 4 * half;  // visible iff offset <= rel
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i)
              if (32 * mt + 8 * (i >> 2) + (i & 3) > rel) s[rb][mt][i] = -INFINITY;
        }
        // e4m3: the page scale (> 0; FLT_MIN stands in for an empty page,
        // whose K rows are zero) multiplies each page's max once and enters
        // the exponent's FMA, since max commutes with a positive factor
        float mxs = -INFINITY;
        if constexpr (FP8) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float pm = -INFINITY;
#pragma unroll
            for (int i = 0; i < 8; ++i) pm = fmaxf(pm, s[rb][q >> 1][8 * (q & 1) + i]);
            mxs = fmaxf(mxs, pm * ksc[q]);
          }
        } else {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) mxs = fmaxf(mxs, s[rb][mt][i]);
          mxs *= p.scale_log2;  // > 0: max commutes with it
        }
        {
          const float2 hv = swap_halves32(mxs);  // the row's two halves of the tile
          mxs = fmaxf(hv.x, hv.y);
        }
        if (__builtin_amdgcn_ballot_w64(mxs > m[rb] + kRescaleSlack)) {
          const float m_new = fmaxf(m[rb], mxs);
          const float alpha =
              m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m[rb] - m_new);
          l[rb] *= alpha;
#pragma unroll
          for (int dt = 0; dt < C::DT; ++dt) o[rb][dt] *= alpha;
          m[rb] = m_new;
        }
        const float mu = m[rb] == -INFINITY ? 0.f : m[rb];
        float rs = 0.f;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float c = FP8 ? ksc[2 * mt + (i >> 3)] : p.scale_log2;
            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rb][mt][i], c, -mu));
            s[rb][mt][i] = e;
            rs += e;
          }
        }
        l[rb] += rs;
      }

      // ---- O^T += V^T . P^T over 4 steps of 16 tokens
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        if (st == 1) {
          if constexpr (FP8)
            load_half<D, BF16, FP8, RB, true>(vr, p, h, pid_ld, npages, last, t + 1, wave, lane);
        }
        u32x4 pb[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r0 = 8 * (st & 1) + 2 * i;
            pb[rb][i] = pack2_16<BF16>(s[rb][st >> 1][r0] * vsc[st],
                                       s[rb][st >> 1][r0 + 1] * vsc[st]);
          }
        }
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_i16x4*)(cur + 16 * st * C::ROWB + voff[dt][0]));
          const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_i16x4*)(cur + 16 * st * C::ROWB + voff[dt][1]));
          const u32x2 lo2 = __builtin_bit_cast(u32x2, lo);
          const u32x2 hi2 = __builtin_bit_cast(u32x2, hi);
          const u32x4 a = {lo2[0], lo2[1], hi2[0], hi2[1]};
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) o[rb][dt] = mfma32<BF16>(a, pb[rb], o[rb][dt]);
        }
      }
    };
    // Iteration t: (e4m3: convert and store tile t) -- barrier -- issue tile
    // t + 1's loads into the other stage, interleaved with tile t's MFMAs.
    // The loads are issued on every tile (on the last one with no page, so
    // they read nothing) and tiles that need no mask run a copy of the step
    // without it: the step is then one branch-free block apart from the
    // rare rescale, and the compiler can overlap its LDS reads, exps and
    // MFMAs across the phases.
    auto step = [&](auto mask_tag, int t, uint8_t* cur, uint8_t* nxt) __attribute__((always_inline)) {
      if constexpr (FP8) {
        store_half<D, BF16, FP8, RB>(kr, cur, wave, lane);
        store_half<D, BF16, FP8, RB>(vr, cur + C::TILEB, wave, lane);
        ksc_l = kr.sc;
        vsc_l = vr.sc;
      }
      // Every wave's direct-to-LDS loads of tile t are complete before any wave
      // passes the barrier and reads them.  The barrier itself waits only for
      // LDS operations (workgroup-scope release), so this wait is explicit
      // rather than left to the compiler's alias tracking of the loads.
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      __syncthreads();
      pid = pid_next;
      pid_next = fetch_page_ids(p, ind_lo, npages, t + 2, lane);
      const int pid_ld = t + 1 < n_tiles ? pid : -1;  // past the last tile: no pages
      if constexpr (!FP8) {
        // tile t + 1 straight into the other stage, K and V, a whole tile
        // ahead of the barrier that waits for it
        dma_half<D, BF16, FP8, RB, false, NW>(p, h, pid_ld, npages, last, t + 1, nxt, wave, lane);
        dma_half<D, BF16, FP8, RB, true, NW>(p, h, pid_ld, npages, last, t + 1, nxt + C::TILEB,
                                             wave, lane);
      }
      // paired tiles: a wave with no row of the tile only loads
      if (!decltype(pair_tag)::value || wave_rows) compute(mask_tag, t, cur, pid_ld);
    };


    // tiles [0, n_clean) lie wholly at or below the first row's diagonal
    // (and inside the sequence): no mask; the rest are masked.  Tile t uses
    // stage t & 1 (the prologue loaded tile 0 into stage 0).
    const int n_clean = min(n_tiles, clean_end / BN);
    int t = 0;
    auto run_tiles = [&](auto mask_tag, const int t_end) __attribute__((always_inline)) {
      if (t < t_end && (t & 1)) {
        step(mask_tag, t, st1, st0);
        ++t;
      }
      for (; t + 1 < t_end; t += 2) {
        step(mask_tag, t, st0, st1);
        step(mask_tag, t + 1, st1, st0);
      }
      if (t < t_end) {
        step(mask_tag, t, st0, st1);
        ++t;
      }
    };
    run_tiles(std::false_type{}, n_clean);
    run_tiles(std::true_type{}, n_tiles);
    // the last tile's loads (of no page) are complete before the workgroup
    // can end and its LDS be handed on
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

    // ---- epilogue: O^T / l, lane's row, 4 consecutive d per register quad
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const float2 lh = swap_halves32(l[rb]);
      const float l_tot = lh.x + lh.y;
      if (!rvalid[rb]) continue;
      const int row = 32 * (RB * wave + rb) + col;
      const int qi = q_lo + row / g;
      const int head = h * g + row % g;
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
      uint16_t* orow = p.out + ((int64_t)(qo_start + qi) * p.hq + head) * D;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          u32x2 w;
          w[0] = pack2_16<BF16>(o[rb][dt][4 * i4] * inv, o[rb][dt][4 * i4 + 1] * inv);
          w[1] = pack2_16<BF16>(o[rb][dt][4 * i4 + 2] * inv, o[rb][dt][4 * i4 + 3] * inv);
          *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * i4 + 4 * half) = w;
        }
      }
      if (p.lse && half == 0)
        p.lse[(int64_t)(qo_start + qi) * p.hq + head] =
            l_tot > 0.f ? (m[rb] + log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
    }
  };

  if constexpr (PAIRS) {
    if (paired) {
      const int h0 = h & ~1;
      // The odd head's row blocks run in reverse wave order.  Waves w and
      // w + WAVES/2 share a SIMD, so a pair of tiles with few rows puts its
      // working waves on different SIMDs (waves without rows skip the
      // compute).
      if (wave < C::WAVES / 2)
        body(std::true_type{}, stage0, stage1, wave, h0);
      else
        body(std::true_type{}, stage2, stage3, C::WAVES - 1 - wave, h0 + 1);
      return;
    }
  }
  body(std::false_type{}, stage0, stage1, wave, h);
}

using PrefillFn = void (*)(PrefillParams);

template <int D, bool BF16, bool FP8>
PrefillFn prefill_fn() {
  return prefill_kernel<D, BF16, FP8, kPrefillRB>;
}

static PrefillFn pick_prefill(int d, bool bf16, bool fp8) {
  if (d == 64) {
    if (bf16) return fp8 ? prefill_fn<64, true, true>() : prefill_fn<64, true, false>();
    return fp8 ? prefill_fn<64, false, true>() : prefill_fn<64, false, false>();
  }
  if (bf16) return fp8 ? prefill_fn<128, true, true>() : prefill_fn<128, true, false>();
  return fp8 ? prefill_fn<128, false, true>() : prefill_fn<128, false, false>();
}

// ----------------------------------------------------------------------------
// Device plan (pagedattn_prefill_plan_device): one workgroup builds the
// q-tile list that pagedattn_prefill_plan builds on the host, from the
// qo_indptr / kv_indptr / kv_last_page_len of the run, so a prefill step
// needs no host copy of its metadata and can be captured in a HIP graph.
// Tiles are cut per sequence exactly as the host planner cuts them; up to
// kPrefillDevSortMax tiles are ordered by the kv tokens their last row sees,
// longest first (ties in sequence order, as the host's stable sort), more
// keep sequence order.  The order only schedules the workgroups: every
// tile's output is the same wherever it runs.  Entries past the tiles, up to
// the plan's capacity, get b = -1 (the attention workgroups return at once);
// tiles beyond the capacity are dropped and counted in `dropped`.
struct PrefillPlanArgs {
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* last_page_len;
  int32_t batch_size, q_tile, g, pair, cap;
  PrefillItem* items;
  int32_t* dropped;
};

constexpr int kPrefillPlanThreads = 1024;

__global__ void __launch_bounds__(kPrefillPlanThreads) prefill_plan_kernel(PrefillPlanArgs a) {
  static_assert(kPrefillDevMaxBatch <= 4 * kPrefillPlanThreads, "four sequences per thread");
  static_assert(kPrefillDevSortMax <= kPrefillPlanThreads, "one sorted tile per thread");
  __shared__ int start[kPrefillDevMaxBatch + 1];  // first tile of each sequence
  __shared__ int red[kPrefillPlanThreads / kWave];
  __shared__ long long key[kPrefillDevSortMax];
  const int t = threadIdx.x;
  const int B = min(max(a.batch_size, 0), kPrefillDevMaxBatch);
  auto qo_len = [&](int b) {
    return (int)min<int64_t>(max<int64_t>((int64_t)a.qo_indptr[b + 1] - a.qo_indptr[b], 0),
                             INT_MAX);
  };
  // tiles of sequences 4t .. 4t + 3, each clamped to cap + 1 so that the
  // sums stay in int32 and a too-large total is still seen as one
  int c[4];
  int mine = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int b = 4 * t + k;
    int n = 0;
    if (b < B) {
      const int qo = qo_len(b);
      n = (int)min<int64_t>(((int64_t)qo + a.q_tile - 1) / a.q_tile, (int64_t)a.cap + 1);
    }
    c[k] = n;
    mine += n;
  }
  int total = 0;
  int run = block_excl_scan<kPrefillPlanThreads>(mine, &total, red);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int b = 4 * t + k;
    if (b <= B) start[b] = run;
    run += c[k];
  }
  __syncthreads();
  const int n_tiles = min(total, a.cap);
  if (t == 0 && total > a.cap && a.dropped) atomicAdd(a.dropped, total - a.cap);
  // tile i: the last sequence whose first tile is <= i (sequences without
  // tiles share their successor's start and are passed over)
  auto tile = [&](int i, int64_t* cost) {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (start[mid] <= i) lo = mid;
      else hi = mid - 1;
    }
    const int b = lo;
    const int qo = qo_len(b);
    const int q_lo = (i - start[b]) * a.q_tile;  // < qo
    const int q_hi = qo - q_lo > a.q_tile ? q_lo + a.q_tile : qo;
    if (cost) {
      const int np = max(a.kv_indptr[b + 1] - a.kv_indptr[b], 0);
      const int last = min(max(a.last_page_len[b], 1), kPage);
      const int64_t kv_len = np > 0 ? (int64_t)(np - 1) * kPage + last : 0;
      *cost = max<int64_t>(0, min<int64_t>(kv_len, kv_len - qo + q_hi));
    }
    const int flag = a.pair && (int64_t)(q_hi - q_lo) * a.g <= kPrefillRows / 2 ? 1 : -1;
    return PrefillItem{b, q_lo, q_hi, flag};
  };
  if (n_tiles <= kPrefillDevSortMax) {
    // one tile per thread; its rank among unique keys (cost, then sequence
    // order) is its place in the list
    PrefillItem it{-1, 0, 0, -1};
    if (t < n_tiles) {
      int64_t cost = 0;
      it = tile(t, &cost);
      key[t] = (cost << 10) | (kPrefillDevSortMax - 1 - t);
    }
    __syncthreads();
    if (t < n_tiles) {
      const long long mk = key[t];
      int rank = 0;
      for (int j = 0; j < n_tiles; ++j) rank += key[j] > mk ? 1 : 0;
      // paired tiles alternate between the even and the odd head of a head
      // pair by list position, so both XCDs of the pair share them
      if (it.slot > 0) it.slot = 1 + (rank & 1);
      a.items[rank] = it;
    }
  } else {
    for (int i = t; i < n_tiles; i += kPrefillPlanThreads) {
      PrefillItem it = tile(i, nullptr);
      if (it.slot > 0) it.slot = 1 + (i & 1);
      a.items[i] = it;
    }
  }
  for (int i = n_tiles + t; i < a.cap; i += kPrefillPlanThreads)
    a.items[i] = PrefillItem{-1, 0, 0, -1};
}

}  // namespace pa

namespace pa {

// The q-tile list of a device prefill plan, cut from the metadata on the
// device by one workgroup (prefill_plan_kernel) on `stream`.
static int launch_prefill_plan(const pagedattn_plan* plan, const int32_t* qo_indptr,
                               const int32_t* kv_indptr, const int32_t* kv_last_page_len,
                               void* stream, const char* who) {
  PrefillPlanArgs a{qo_indptr, kv_indptr, kv_last_page_len, plan->batch_size,
                    plan->q_tile, plan->hq / plan->hkv, plan->prefill_pair ? 1 : 0,
                    plan->n_items, static_cast<PrefillItem*>(plan->items_dev),
                    reinterpret_cast<int32_t*>(static_cast<char*>(plan->workspace) + 12)};
  hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(kPrefillPlanThreads), 0,
                     (hipStream_t)stream, a);
  return check_launch(who);
}

}  // namespace pa

using namespace pa;

extern "C" {

int pagedattn_prefill_plan_device_update(pagedattn_plan* plan, const int32_t* qo_indptr,
                                         const int32_t* kv_indptr,
                                         const int32_t* kv_last_page_len, void* stream) {
  const char* who = "prefill_plan_device_update";
  if (!plan || plan->mode != kPlanPrefill || !plan->implicit)
    return set_error(PAGEDATTN_ERR_PLAN, "%s: no device prefill plan (call plan_device first)",
                     who);
  if (!qo_indptr || !kv_indptr || !kv_last_page_len)
    return set_error(PAGEDATTN_ERR_INVALID, "%s: null pointer", who);
  if (plan->batch_size > kPrefillDevMaxBatch)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: device plan of %d sequences", who,
                     plan->batch_size);
  if (plan->n_items == 0) {
    plan->dev_table = true;
    return PAGEDATTN_OK;
  }
  const int rc = launch_prefill_plan(plan, qo_indptr, kv_indptr, kv_last_page_len, stream, who);
  if (rc) return rc;
  plan->dev_table = true;
  return PAGEDATTN_OK;
}

int pagedattn_prefill_run(const pagedattn_plan* plan, const void* q,
                          int64_t q_stride_n, int64_t q_stride_h,
                          int32_t q_dtype, const int32_t* qo_indptr,
                          const void* paged_kv_cache, int32_t kv_dtype,
                          const float* kv_scales, int32_t num_pages,
                          const int32_t* kv_indices, int32_t num_indices,
                          const int32_t* kv_indptr,
                          const int32_t* kv_last_page_len, void* out,
                          float* lse, int32_t causal, float sm_scale,
                          void* stream) {
  const char* who = "prefill_run";
  if (!plan || plan->mode != kPlanPrefill)
    return set_error(PAGEDATTN_ERR_PLAN,
                     "%s: no prefill plan (call plan first)", who);
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
  if (!(sm_scale > 0.f) || !std::isfinite(sm_scale))
    return set_error(PAGEDATTN_ERR_UNSUPPORTED,
                     "%s: sm_scale must be a positive finite number", who);
  if (plan->n_items == 0) return PAGEDATTN_OK;
  if (plan->implicit && plan->batch_size > kPrefillDevMaxBatch)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: device plan of %d sequences", who,
                     plan->batch_size);
  if ((int64_t)plan->n_items * plan->hkv > INT32_MAX)
    return set_error(PAGEDATTN_ERR_UNSUPPORTED, "%s: too many work items", who);
  if (!q || !qo_indptr || !paged_kv_cache || !kv_indices || !kv_indptr ||
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
  PrefillParams p;
  p.items = static_cast<const PrefillItem*>(plan->items_dev);
  p.n_items = plan->n_items;
  p.batch_size = plan->batch_size;
  p.q = static_cast<const uint16_t*>(q);
  p.q_sn = q_stride_n;
  p.q_sh = q_stride_h;
  p.qo_indptr = qo_indptr;
  p.cache = static_cast<const uint8_t*>(paged_kv_cache);
  p.kv_scales = kv_scales;
  p.num_pages = num_pages;
  p.kv_indices = kv_indices;
  p.num_indices = num_indices;
  p.kv_indptr = kv_indptr;
  p.last_page_len = kv_last_page_len;
  p.out = static_cast<uint16_t*>(out);
  p.lse = lse;
  p.hq = plan->hq;
  p.hkv = plan->hkv;
  p.g = plan->hq / plan->hkv;
  p.causal = causal ? 1 : 0;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  PrefillFn fn = pick_prefill(plan->d, q_dtype == PAGEDATTN_BF16, fp8);
  if (plan->implicit && !plan->dev_table) {
    // the work list of this run, built on the device ahead of the attention
    // (unless pagedattn_prefill_plan_device_update built it for the step)
    int rc = launch_prefill_plan(plan, qo_indptr, kv_indptr, kv_last_page_len, stream, who);
    if (rc) return rc;
  }
  hipLaunchKernelGGL(fn, dim3(plan->n_items * plan->hkv), dim3(64 * kPrefillWaves), 0,
                     (hipStream_t)stream, p);
  return check_launch(who);
}

}  // extern "C"
