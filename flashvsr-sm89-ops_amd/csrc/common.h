// Shared device helpers for the gfx950 operator pack.
//
// Every kernel in this library works on raw bit patterns: bf16 tensors are
// uint16_t, e4m3fn tensors are uint8_t.  Conversions use the gfx950
// instructions whose rounding was checked against torch's casts:
//   fp32 -> bf16   v_cvt_pk_bf16_f32 (round to nearest even)
//   fp32 -> e4m3fn v_cvt_pk_fp8_f32  (round to nearest even; inputs are
//                  always clamped to +-448 first, so overflow never occurs)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fvsr.h"

#define FVSR_DEV static __device__ __forceinline__

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

FVSR_DEV float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
FVSR_DEV float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
FVSR_DEV float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Two fp32 -> packed bf16x2 (lo = a), round to nearest even.
FVSR_DEV uint32_t pack_bf16x2(float a, float b) {
  bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
// fp32 -> bf16 -> fp32 (the "round-trip through bf16" of eager).
FVSR_DEV float round_bf16(float a) { return bf_lo(pack_bf16x2(a, 0.0f)); }

// Four fp32 (already within +-448) -> four e4m3fn codes in one dword.
FVSR_DEV uint32_t pack_e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

FVSR_DEV float clamp448(float v) { return fminf(fmaxf(v, -448.0f), 448.0f); }

// Wavefront (64-lane) reductions.
FVSR_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
FVSR_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Shared fp32 exp: Cody-Waite reduction by ln2 split in two parts, degree-7
// Taylor polynomial in Horner form, two exact power-of-two scalings.  Every
// step is a single IEEE binary32 multiply or add (the translation units that
// use it are compiled with contraction off), so the CPU oracle's C copy of the
// same sequence returns identical bits.
FVSR_DEV float fvsr_expf(float x) {
  const float LOG2E = 1.44269502162933349609375f;
  const float LN2_HI = 0.693145751953125f;
  const float LN2_LO = 1.428606765330187045e-06f;
  if (x != x) return x;
  if (x > 88.7228394f) return __builtin_huge_valf();
  if (x < -103.972084f) return 0.0f;
  float t = x * LOG2E;
  float n = __builtin_rintf(t);
  float r = x - n * LN2_HI;
  r = r - n * LN2_LO;
  float p = 1.984126984126984e-04f;
  p = p * r + 1.388888888888889e-03f;
  p = p * r + 8.333333333333333e-03f;
  p = p * r + 4.166666666666666e-02f;
  p = p * r + 1.666666666666667e-01f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  int ni = (int)n;
  int h = ni / 2;
  float s1 = __uint_as_float((uint32_t)(h + 127) << 23);
  float s2 = __uint_as_float((uint32_t)(ni - h + 127) << 23);
  return (p * s1) * s2;
}

// tanh-GELU via 1 - 2/(exp(2u)+1), rounded to bf16 (returned as fp32),
// operation order of flashvsr_sm89_ops/fp8_ffn.py:26-30.
FVSR_DEV float gelu_tanh_bf16(float x) {
  const float C0 = 0.7978845608028654f;
  float u = C0 * (x + ((0.044715f * x) * x) * x);
  float t = 1.0f - 2.0f / (fvsr_expf(2.0f * u) + 1.0f);
  float g = (0.5f * x) * (1.0f + t);
  return round_bf16(g);
}

static inline int fvsr_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FVSR_OK : FVSR_EHIP;
}
