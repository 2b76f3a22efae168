// Shared device helpers for the gfx950 operator pack.
//
// Every kernel in this library works on raw bit patterns: bf16 tensors are
// uint16_t, e4m3fn tensors are uint8_t.  Conversions use the gfx950
// instructions whose rounding was checked against torch's casts:
//   fp32 -> bf16   v_cvt_pk_bf16_f32 (round to nearest even)
//   fp32 -> e4m3fn v_cvt_pk_fp8_f32  (round to nearest even; magnitudes in
//                  (448, 464] give 448, the tie at 464 included, and larger
//                  ones NaN, so inputs are either clamped to +-448 first or
//                  known to stay below 464)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fvsr.h"

#define FVSR_DEV static __device__ __forceinline__

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));

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
// The same round trip in one instruction: bf16(a) converted into the high
// half with +0 in the low half is the fp32 bit pattern of bf16(a).  (Written
// out: the compiler would otherwise merge two of these into one conversion
// plus byte permutes.)
FVSR_DEV float rbf16(float a) {
  float r;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(a));
  return r;
}

// Four fp32 (of magnitude below 464) -> four e4m3fn codes in one dword.
FVSR_DEV uint32_t pack_e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

FVSR_DEV float clamp448(float v) { return fminf(fmaxf(v, -448.0f), 448.0f); }

// The scale an activation quantisation returns, amax / 448 as torch computes
// it on the GPU: the reference returns `amax / FP8_MAX` (a device tensor
// divided by a Python float, flashvsr_sm89_ops/fp8_quant.py:54 and
// fp8_ffn.py:72), which torch evaluates as amax * fl(1/448), its
// reciprocal-multiply path for a host-scalar divisor.  That differs from the
// IEEE quotient by one ulp for about half of all amax values.  (The scale the
// codes are divided by, max(amax, 1e-12) / 448, is a true division inside the
// reference's kernels and stays one here.)
FVSR_DEV float act_scale(float amax) { return amax * (1.0f / 448.0f); }

// Element access of the dtype-generic kernels (FVSR_DT_* codes, uniform per
// launch).  Loads widen to fp32 exactly, as the reference's kernels load every
// input with .to(tl.float32).  st_elem takes a result already rounded to bf16
// (every output of these ops is) and writes it in the tensor's type: exactly
// for bf16 and fp32, rounded to nearest even for fp16 (v_cvt_f16_f32).
FVSR_DEV float ld_elem(const void* p, int dt, int64_t i) {
  if (dt == FVSR_DT_F32) return ((const float*)p)[i];
  if (dt == FVSR_DT_F16) return (float)((const _Float16*)p)[i];
  return bf2f(((const uint16_t*)p)[i]);
}
FVSR_DEV void st_elem(void* p, int dt, int64_t i, float v) {
  if (dt == FVSR_DT_F32)
    ((float*)p)[i] = v;
  else if (dt == FVSR_DT_F16)
    ((_Float16*)p)[i] = (_Float16)v;
  else
    ((uint16_t*)p)[i] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffff);
}
// v rounded to the precision of type dt (nearest even), as fp32.
FVSR_DEV float round_to(int dt, float v) {
  if (dt == FVSR_DT_F32) return v;
  if (dt == FVSR_DT_F16) return (float)(_Float16)v;
  return round_bf16(v);
}

// torch's fp32 -> float8_e4m3fn cast: round to nearest even, magnitudes above
// 464 (and NaN) give the NaN code 0x7F with the value's sign (e4m3fn has no
// infinity); v_cvt_pk_fp8_f32 gives the same codes up to 464 but 0xFF for
// every NaN.
FVSR_DEV uint8_t e4m3_cast(float v) {
  const uint32_t u = __float_as_uint(v);
  if (!(fabsf(v) <= 464.0f)) return (uint8_t)(((u >> 24) & 0x80u) | 0x7Fu);
  return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false) & 0xff);
}

// Lane id, recomputed where it is used.  Address arithmetic derived from it
// cannot be hoisted out of a loop by the compiler, which otherwise keeps a
// loop-invariant offset per load alive (and spills them) for the whole loop.
FVSR_DEV int lane_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Chunk index for an unconditional row load: chunks past the end of the row
// read the row's last chunk (n >= 1) instead, so a wave issues all of its
// row loads back to back rather than one per divergent branch.
FVSR_DEV int64_t clamp_chunk(int64_t c, int64_t n) { return c < n ? c : n - 1; }

// Wavefront (64-lane) reductions on the VALU through DPP lane moves (no LDS
// round trips): quad swaps, half-row and row mirrors leave every lane of a
// 16-lane row with the row's result; two row broadcasts fold rows 0..3 into
// lane 63, which is read into a scalar register, so the result is uniform.
// Lanes of rows outside a broadcast's row mask receive 0 (the identity for
// sums, and for maxima of non-negative values).
template <int CTRL, int ROWS>
FVSR_DEV float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xf, false));
}
FVSR_DEV float lane63(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
FVSR_DEV float wave_sum(float v) {
  v += dpp_f32<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141, 0xf>(v);  // row_half_mirror
  v += dpp_f32<0x140, 0xf>(v);  // row_mirror
  v += dpp_f32<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
  v += dpp_f32<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
  return lane63(v);
}
// Maximum of non-negative values (|x| maxima): compared as unsigned bit
// patterns, which orders non-negative floats and lets a NaN win.
FVSR_DEV float umax_f32(float a, float b) {
  const uint32_t x = __builtin_bit_cast(uint32_t, a), y = __builtin_bit_cast(uint32_t, b);
  return __builtin_bit_cast(float, x > y ? x : y);
}
FVSR_DEV float wave_max_abs(float v) {
  v = umax_f32(v, dpp_f32<0xB1, 0xf>(v));
  v = umax_f32(v, dpp_f32<0x4E, 0xf>(v));
  v = umax_f32(v, dpp_f32<0x141, 0xf>(v));
  v = umax_f32(v, dpp_f32<0x140, 0xf>(v));
  v = umax_f32(v, dpp_f32<0x142, 0xa>(v));
  v = umax_f32(v, dpp_f32<0x143, 0xc>(v));
  return lane63(v);
}
// Maximum of any values: the row broadcasts fill masked-out rows with 0, so
// they are replaced by a final lane-63 read of each row's own maximum.
FVSR_DEV float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1, 0xf>(v));
  v = fmaxf(v, dpp_f32<0x4E, 0xf>(v));
  v = fmaxf(v, dpp_f32<0x141, 0xf>(v));
  v = fmaxf(v, dpp_f32<0x140, 0xf>(v));
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Shared fp32 exp for y clamped to [-40, 40] (the GELU below is saturated
// outside): Cody-Waite reduction by ln2 in two fused steps, degree-6 Taylor
// polynomial in fused Horner form, exact ldexp.  Every step is one IEEE
// operation, so the CPU oracle's C copy of this sequence (fmaf, nearbyintf,
// ldexpf) returns identical bits.
FVSR_DEV float fvsr_expf(float y) {
#pragma clang fp contract(off)
  const float LOG2E = 1.44269502162933349609375f;
  const float LN2_HI = 0.693145751953125f;
  const float LN2_LO = 1.428606765330187045e-06f;
  if (y != y) return y;
  y = y < -40.0f ? -40.0f : (y > 40.0f ? 40.0f : y);
  const float n = __builtin_rintf(y * LOG2E);
  float r = __builtin_fmaf(-n, LN2_HI, y);
  r = __builtin_fmaf(-n, LN2_LO, r);
  float p = 1.388888888888889e-03f;
  p = __builtin_fmaf(p, r, 8.333333333333333e-03f);
  p = __builtin_fmaf(p, r, 4.166666666666666e-02f);
  p = __builtin_fmaf(p, r, 1.666666666666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

// tanh-GELU in the form of flashvsr_sm89_ops/fp8_ffn.py:24-30, rounded to bf16
// (returned as fp32): u = sqrt(2/pi)(x + 0.044715 x^3), t = 1 - 2/(exp(2u)+1),
// g = bf16(0.5 x (1 + t)).  IEEE division.
FVSR_DEV float gelu_tanh_bf16(float x) {
#pragma clang fp contract(off)
  const float C2 = 1.5957691216057308f;  // 2*sqrt(2/pi)
  const float x2 = x * x;
  const float inner = __builtin_fmaf(0.044715f * x2, x, x);
  const float e = fvsr_expf(C2 * inner);
  const float t = 1.0f - 2.0f / (e + 1.0f);
  return round_bf16((0.5f * x) * (1.0f + t));
}

// Four fp32 -> four e4m3fn codes; both halves of the destination are written,
// so its prior contents (here a's bits, dead after this) do not matter.
FVSR_DEV uint32_t e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
}

// max(m, |a|, |b|) in one v_max3_f32.  A NaN operand is passed over as
// fmaxf does (the kernels' NaNs are quiet: bf16 data and conversions), and
// the operands need no canonicalising maximum first.
FVSR_DEV float max3_abs(float m, float a, float b) {
  float r;
  asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
  return r;
}

// Packed bf16 pair -> the two floats.
FVSR_DEV float lo_f(uint32_t p) { return __uint_as_float(p << 16); }
FVSR_DEV float hi_f(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// |v| / s without a division: q0 = |v| * r with r = fl(1/s), the residual
// e = |v| - q0 * s by one fma, and q0 + e * r by another (Markstein's
// correction).  Its e4m3 code equals that of the IEEE quotient fl(|v| / s)
// for every bf16 v and every bf16 amax >= |v|, with s = fl(max(amax, 1e-12) /
// 448), including amax = inf (sc = min(s, FLT_MAX) keeps the residual finite
// there): checked exhaustively over all 1.07e9 such pairs
// (tests/native/fma_quotient_check.c).  The quotient is formed on |v| and the
// sign put into the code afterwards, so -0 keeps its sign.  |v| <= amax bounds
// the result by 448 * (1 + 2^-23), which the conversion rounds to 448 without
// a clamp.
FVSR_DEV float quot_abs(float v, float r, float sc) {
  const float a = fabsf(v);
  const float q0 = a * r;
  const float e = fmaf(-q0, sc, a);
  return fmaf(e, r, q0);
}

// The same quotient on the signed value, for code paths that hold unpacked
// floats (no sign bits to gather): q0 = v * r, t = q0 * s - v (the negated
// residual) and q0 - t * r.  Every step is odd in v under round-to-nearest, so
// the result is -quot(|v|) for negative v, and equals quot_abs's value for
// v > 0 (t is exactly -e, or both are +0).  For v = -0 it is -0 (q0 = -0,
// t = +0, -0 - 0 = -0), so the conversion's own sign gives the code.  Checked
// over the same pairs, both signs, by tests/native/fma_quotient_check.c.  (A
// NaN's sign may come out either way; v_cvt_pk_fp8_f32 writes 0xFF for every
// NaN in any case.)
FVSR_DEV float quot_signed(float v, float r, float sc) {
  const float q0 = v * r;
  const float t = fmaf(q0, sc, -v);
  return fmaf(t, -r, q0);
}

// Codes of one chunk (8 packed bf16 values) divided by s (r = fl(1/s),
// sc = min(s, FLT_MAX)), every value bounded by the amax s was made from.
// The sign bits of the inputs (bit 7 of bytes 1 and 3 of each dword) are
// gathered by one byte permute per four values.
FVSR_DEV u32x2_t chunk_codes_fma(u32x4_t p, float r, float sc) {
  u32x2_t out;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t p0 = p[2 * h], p1 = p[2 * h + 1];
    const uint32_t c = e4m3x4(quot_abs(lo_f(p0), r, sc), quot_abs(hi_f(p0), r, sc),
                              quot_abs(lo_f(p1), r, sc), quot_abs(hi_f(p1), r, sc));
    out[h] = c | (__builtin_amdgcn_perm(p1, p0, 0x07050301u) & 0x80808080u);
  }
  return out;
}

// Largest |GELU| over negative inputs is 0.16992 (exhaustive over bf16), and
// the bf16 GELU above is non-decreasing for x >= -0.75; so for a row whose
// largest element is h_max, max|gelu(row)| == gelu(h_max) whenever that value
// exceeds this bound.
#define FVSR_GELU_NEG_BOUND 0.17f

static inline int fvsr_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FVSR_OK : FVSR_EHIP;
}
