// Shared device helpers for the gstar_evict HIP kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gstar_evict.h"

#define GSE_DEVICE __device__ __forceinline__

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

// Wavefront size on CDNA is 64.
constexpr int kWave = 64;

GSE_DEVICE float bf16_to_f32(uint16_t x) { return __uint_as_float(uint32_t(x) << 16); }

// Round-to-nearest-even float -> bf16 (NaN stays NaN).
GSE_DEVICE uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

GSE_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  return uint32_t(f32_to_bf16(lo)) | (uint32_t(f32_to_bf16(hi)) << 16);
}

GSE_DEVICE bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// 16x16x32 bf16 MFMA, fp32 accumulate. Lane l supplies A[l%16][8*(l/16)+e] and
// B[8*(l/16)+e][l%16] for e = 0..7, and holds D[4*(l/16)+r][l%16] for r = 0..3.
GSE_DEVICE f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

GSE_DEVICE float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T>
GSE_DEVICE int64_t load_index(const void* p, int64_t i) {
  return int64_t(static_cast<const T*>(p)[i]);
}

GSE_DEVICE int64_t load_index_dyn(const void* p, int dtype, int64_t i) {
  return dtype == GSE_I64 ? static_cast<const int64_t*>(p)[i] : int64_t(static_cast<const int32_t*>(p)[i]);
}

GSE_DEVICE float load_float_dyn(const void* p, int dtype, int64_t i) {
  return dtype == GSE_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

GSE_DEVICE float wave_max_xor(float v, int mask) { return fmaxf(v, __shfl_xor(v, mask, kWave)); }
GSE_DEVICE float wave_sum_xor(float v, int mask) { return v + __shfl_xor(v, mask, kWave); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
