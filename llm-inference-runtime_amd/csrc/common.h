// Shared definitions for the gfx950 paged-attention kernels and their host
// launchers.  Everything here is CDNA4-specific: wave64, MFMA builtins,
// buffer resources with hardware range checking.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "pagedattn.h"

namespace pa {

// ----------------------------------------------------------------------------
// host-side error reporting (thread-local message, status code returned)
int set_error(int code, const char* fmt, ...)
    __attribute__((format(printf, 2, 3)));
// Checks hipGetLastError() after a launch; returns PAGEDATTN_OK or
// PAGEDATTN_ERR_HIP with the message set.
int check_launch(const char* what);
// CU count of the current device, cached per device.
int device_cu_count();

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// ----------------------------------------------------------------------------
// device types
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
constexpr int kPage = 16;  // page_size baked into the kernels (EngineConfig.block_size)

// Buffer resource word 3 for raw (stride 0) gfx9 buffers: 32-bit data format,
// no swizzle.  Loads at byte offsets >= num_records return 0 without touching
// memory, which is how partial and absent pages are read.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base,
                                                            uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)bytes, kRsrcWord3);
}

// Cache policy of buffer loads: kCachePolicyStream marks data read once as
// non-temporal (the 16-bit K/V pages of a decode pass; each kernel picks the
// policy it measured faster).
constexpr int kCachePolicyDefault = 0;
constexpr int kCachePolicyStream = 2;

template <int POLICY = kCachePolicyDefault>
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r,
                                            uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POLICY);
}
template <int POLICY = kCachePolicyDefault>
__device__ __forceinline__ u32x2 buf_load8(__amdgpu_buffer_rsrc_t r,
                                           uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POLICY);
}
template <int POLICY = kCachePolicyDefault>
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r,
                                              uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POLICY);
}

__device__ __forceinline__ int uniform(int x) {
  return __builtin_amdgcn_readfirstlane(x);
}

// Load of data that no thread writes during the kernel (metadata, work
// lists), through the constant address space: with a wave-uniform address
// the compiler emits a scalar load instead of a vector load plus a wait on
// every outstanding vector load.
template <typename T>
__device__ __forceinline__ T load_invariant(const T* ptr) {
  using CT = const __attribute__((address_space(4))) T;
  return *reinterpret_cast<CT*>(reinterpret_cast<uintptr_t>(ptr));
}

// 16-bit element helpers.  Storage is raw uint16 bits; IS_BF16 selects the
// interpretation.
template <bool IS_BF16>
__device__ __forceinline__ float h2f(uint16_t h) {
  if constexpr (IS_BF16) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, h);
  }
}

template <bool IS_BF16>
__device__ __forceinline__ uint16_t f2h(float f) {
  if constexpr (IS_BF16) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
}

// Two floats -> two 16-bit values in one dword (element a low), round to
// nearest even: one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <bool IS_BF16>
__device__ __forceinline__ uint32_t pack2_16(float a, float b) {
  const f32x2 v = {a, b};
  if constexpr (IS_BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
}

// fp32 -> fp8 e4m3fn (OCP, the gfx950 fp8 format) through the hardware
// converter, round to nearest even.  It saturates nothing by itself: callers
// clamp to +-448 first.
__device__ __forceinline__ uint32_t f32_to_e4m3x4(float a, float b, float c,
                                                  float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// Eight 16-bit values (u32x4) -> eight e4m3 bytes with a fixed scale:
// round_to_nearest_even(clamp(x / scale, -448, 448)).  *clamped is set when
// a value had |x / scale| > 448 (or x / scale was NaN) and the clamp changed
// it.  A scale that is not positive and finite writes zero codes and sets
// *clamped.  Every kernel that appends with a fixed scale uses this one, so
// the stand-alone, RoPE-fused and decode-fused appends store the same bytes.
template <bool IS_BF16>
__device__ __forceinline__ u32x2 quant8_e4m3(u32x4 x, float scale, bool* clamped) {
  float f[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = h2f<IS_BF16>((uint16_t)(x[e] & 0xffffu));
    f[2 * e + 1] = h2f<IS_BF16>((uint16_t)(x[e] >> 16));
  }
  bool over = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float y = f[e] / scale;
    over |= !(__builtin_fabsf(y) <= 448.f);
    f[e] = fminf(fmaxf(y, -448.f), 448.f);
  }
  u32x2 o;
  o[0] = f32_to_e4m3x4(f[0], f[1], f[2], f[3]);
  o[1] = f32_to_e4m3x4(f[4], f[5], f[6], f[7]);
  const bool scale_ok = scale > 0.f && scale < __builtin_huge_valf();
  if (!scale_ok) o = u32x2{0u, 0u};
  *clamped = over || !scale_ok;
  return o;
}

// Adds the number of active lanes with `hit` set to *counter (a device int32;
// may be null) with one atomic per wave, issued by the first such lane.
// Lanes that call it from different branches are counted by their own call.
__device__ __forceinline__ void count_lanes(int32_t* counter, bool hit) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(hit);
  if (m == 0 || counter == nullptr) return;
  const int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  if (lane == __builtin_ctzll(m)) atomicAdd(counter, (int32_t)__builtin_popcountll(m));
}

// RoPE (src/models/llama.py:175-182 via flashinfer.apply_rope_pos_ids_inplace):
// angle of frequency i at position pos, inv_freq = theta^(-2i/rotary_dim),
// pos / rope_scale, formed and reduced mod 2 pi in fp64 so that positions up
// to 2^17 keep fp32 accuracy in the sin / cos.  Every kernel that rotates
// uses these two functions, so fused and stand-alone rotations agree bit for
// bit.
__device__ __forceinline__ void rope_cos_sin(int pos, int i, int rotary_dim,
                                             double inv_scale, double log2_theta,
                                             float* c, float* s) {
  const double inv_freq = exp2(-(double)(2 * i) / (double)rotary_dim * log2_theta);
  double ang = (double)pos * inv_scale * inv_freq;
  constexpr double kTwoPi = 6.283185307179586476925286766559;
  ang -= kTwoPi * rint(ang * (1.0 / kTwoPi));
  sincosf((float)ang, s, c);
}

// (x0, x1) rotated by the angle with cosine c and sine s, with one fixed
// rounding order.
__device__ __forceinline__ void rope_rotate(float x0, float x1, float c, float s,
                                            float* y0, float* y1) {
  *y0 = __builtin_fmaf(x0, c, -(x1 * s));
  *y1 = __builtin_fmaf(x1, c, x0 * s);
}

// Eight consecutive 16-bit elements (u32x4) rotated against their partners
// half a head away: lo holds elements i .. i+7, hi elements i+D/2 .. i+D/2+7.
template <bool IS_BF16>
__device__ __forceinline__ void rope8(u32x4& lo, u32x4& hi, const float (&c)[8],
                                      const float (&s)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    float y[4];
    rope_rotate(h2f<IS_BF16>((uint16_t)(lo[w] & 0xffffu)),
                h2f<IS_BF16>((uint16_t)(hi[w] & 0xffffu)), c[2 * w], s[2 * w], &y[0],
                &y[1]);
    rope_rotate(h2f<IS_BF16>((uint16_t)(lo[w] >> 16)), h2f<IS_BF16>((uint16_t)(hi[w] >> 16)),
                c[2 * w + 1], s[2 * w + 1], &y[2], &y[3]);
    lo[w] = (uint32_t)f2h<IS_BF16>(y[0]) | ((uint32_t)f2h<IS_BF16>(y[2]) << 16);
    hi[w] = (uint32_t)f2h<IS_BF16>(y[1]) | ((uint32_t)f2h<IS_BF16>(y[3]) << 16);
  }
}

// wave-level reductions over lanes that differ in bits 4 and 5 (the four
// 16-lane groups of a 16x16 MFMA tile).  v_permlane16_swap / 32_swap
// exchange 16-lane rows (lanes l and l ^ 16) and the two 32-lane halves
// (l and l ^ 32) in the VALU, where a 64-lane shuffle would take a round
// trip through the LDS crossbar; each returns {this row's value, the
// partner's} in an order that is the same pair on both lanes, and max and
// fp32 addition are commutative, so the results equal the shuffles' bits.
__device__ __forceinline__ float2 swap_rows16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v),
                                                  __builtin_bit_cast(uint32_t, v), false, false);
  return float2{__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ float2 swap_halves32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                  __builtin_bit_cast(uint32_t, v), false, false);
  return float2{__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ float max_over_groups16(float v) {
  float2 p = swap_rows16(v);
  v = fmaxf(p.x, p.y);
  p = swap_halves32(v);
  return fmaxf(p.x, p.y);
}
__device__ __forceinline__ float sum_over_groups16(float v) {
  float2 p = swap_rows16(v);
  v = p.x + p.y;
  p = swap_halves32(v);
  return p.x + p.y;
}

// Exclusive prefix sum of v over the THREADS threads of the workgroup (every
// thread calls it); *total gets the sum.  `red` holds THREADS / 64 wave
// totals in LDS.
template <int THREADS>
__device__ __forceinline__ int block_excl_scan(int v, int* total, int* red) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) red[wave] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < THREADS / kWave; ++w) {
    const int t = red[w];
    before += w < wave ? t : 0;
    all += t;
  }
  __syncthreads();
  *total = all;
  return before + x - v;
}

}  // namespace pa
