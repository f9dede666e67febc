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

// Cache policy of buffer loads: kCachePolicyStream marks data read once
// (K/V pages of a decode pass) as non-temporal.
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

// wave-level reductions over lanes that differ in bits 4 and 5 (the four
// 16-lane groups of a 16x16 MFMA tile).
__device__ __forceinline__ float max_over_groups16(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
__device__ __forceinline__ float sum_over_groups16(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

}  // namespace pa
