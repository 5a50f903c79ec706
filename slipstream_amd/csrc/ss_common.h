// Shared device helpers for the gfx950 kernels: vector types, MFMA wrappers,
// 16-bit packing and wavefront exchanges. CDNA4 only (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>


#include "../../include/slipstream_hip.h"

namespace ss {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

constexpr int kWave = 64;
// A finite stand-in for -inf as the running max: exp2(x - kNegBig) stays well
// defined while every key seen so far is masked.
constexpr float kNegBig = -1.0e30f;
constexpr float kLog2e = 1.4426950408889634f;

// 16-bit element traits: MFMA 16x16x32 with fp32 accumulation, packing of two
// fp32 values into one dword of this type and unpacking them again.
template <typename T>
struct Elem;

template <>
struct Elem<bf16_t> {
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    bf16x2 v = {(bf16_t)lo, (bf16_t)hi};  // v_cvt_pk_bf16_f32, round to nearest even
    return __builtin_bit_cast(uint32_t, v);
  }
  // the low / high element of a packed pair, exactly
  static __device__ __forceinline__ float lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }
};

template <>
struct Elem<f16_t> {
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    f16x2 v = {(f16_t)lo, (f16_t)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[0]; }
  static __device__ __forceinline__ float hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[1]; }
};

// Byte-select of two dwords: result = (lo16 of `a` half ha, hi16 = `b` half hb),
// where half 0 is bits 0..15 and half 1 is bits 16..31 (v_perm_b32).
template <int HA, int HB>
__device__ __forceinline__ uint32_t pick_halves(uint32_t a, uint32_t b) {
  // v_perm_b32 dst, s0, s1, sel: byte k of dst = byte sel[k] of {s0:s1}, where
  // bytes 0..3 come from s1 and 4..7 from s0.
  constexpr uint32_t sel = (uint32_t)(2 * HA) | ((uint32_t)(2 * HA + 1) << 8) |
                           ((uint32_t)(4 + 2 * HB) << 16) | ((uint32_t)(5 + 2 * HB) << 24);
  return __builtin_amdgcn_perm(b, a, sel);
}

// All-reduce across the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48)
// with the gfx950 lane-swap instructions.
__device__ __forceinline__ float max_across_rows(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto s32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  float y = fmaxf(__builtin_bit_cast(float, (uint32_t)s32[0]),
                  __builtin_bit_cast(float, (uint32_t)s32[1]));
  uint32_t w = __builtin_bit_cast(uint32_t, y);
  auto s16 = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)s16[0]),
               __builtin_bit_cast(float, (uint32_t)s16[1]));
}

__device__ __forceinline__ float sum_across_rows(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto s32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  float y = __builtin_bit_cast(float, (uint32_t)s32[0]) + __builtin_bit_cast(float, (uint32_t)s32[1]);
  uint32_t w = __builtin_bit_cast(uint32_t, y);
  auto s16 = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return __builtin_bit_cast(float, (uint32_t)s16[0]) + __builtin_bit_cast(float, (uint32_t)s16[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// log2-domain log-sum-exp of a softmax row from its running (max, sum); -inf for no key.
__device__ __forceinline__ float row_lse(float m, float l) {
  return l > 0.f ? m + __builtin_amdgcn_logf(l) : -__builtin_inff();
}

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void store16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

}  // namespace ss

// Host-side helpers shared by the C-ABI wrappers.
namespace ss_host {
void set_error(const char* fmt, ...);
int launch_status(const char* what);
int device_cu_count();
}  // namespace ss_host
