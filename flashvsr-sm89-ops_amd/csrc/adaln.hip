// AdaLN elementwise chains (contracts LN and GA), bandwidth bound.
//
// ln_modulate: one wavefront per row, the row lives in registers between the
// mean pass, the variance pass and the output, so x is read from HBM once.
// The optional fused output is the per-row e4m3 quantisation of the modulated
// row (what the following FP8 linear would compute), produced from the same
// registers: the bf16 row never has to be written when only codes are needed.
//
// gate_add: 16-byte vector loads/stores, eager's bf16 rounding chain, bitwise
// equal to x + gate*res in bf16.
#pragma clang fp contract(off)
#include "common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
#ifndef FVSR_LN_ROWS
#define FVSR_LN_ROWS 2
#endif
constexpr int kLnRows = FVSR_LN_ROWS;  // rows per wavefront in ln_modulate_vec

FVSR_DEV void unpack8(u32x4_t c, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf_lo(c[i]);
    f[2 * i + 1] = bf_hi(c[i]);
  }
}

// Packed bf16 pair whose halves are then read back separately: the empty asm
// keeps the single two-value conversion (the compiler otherwise rewrites each
// half's read-back into its own conversion).
FVSR_DEV uint32_t pack_bf16x2_once(float a, float b) {
  uint32_t w = pack_bf16x2(a, b);
  asm("" : "+v"(w));
  return w;
}

FVSR_DEV u32x4_t pack8(const float* f) {
  u32x4_t c;
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return c;
}

// bf16(v_e / den) for the eight values of a chunk, as four packed bf16 pairs,
// from the reciprocal rd = 1/den (IEEE).  For normal y = fl(v * rd), y lies
// within 1.5 * 2^-23 (relative) of fl(v / den), so fl(v / den) lies between
// fl(y * (1 - 2^-21)) and fl(y * (1 + 2^-21)); bf16 rounding is monotone, so
// when both ends round to the same bf16 that is the result.  Lanes whose ends
// disagree set `bad`.  The caller guarantees that no y is subnormal, infinite
// or NaN (see ln_fast_ok).
FVSR_DEV u32x4_t bf16_quot8(const float* v, float rd, bool& bad) {
  const float kLo = 0.99999952316284180f, kHi = 1.00000047683715820f;  // 1 -+ 2^-21
  u32x4_t out;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float y0 = v[2 * p] * rd, y1 = v[2 * p + 1] * rd;
    const uint32_t lo = pack_bf16x2_once(y0 * kLo, y1 * kLo);
    const uint32_t hi = pack_bf16x2(y0 * kHi, y1 * kHi);
    bad |= lo != hi;
    out[p] = lo;
  }
  return out;
}

// Row-level precondition of bf16_quot8.  A nonzero v = fl(x - mean), x bf16
// and mean fp32 normal, has |v| >= |mean| * 2^-24: within a factor of two of
// mean (Sterbenz) both are multiples of mean's fp32 ulp, otherwise
// |v| >= |mean| / 2.  So |mean| * rd >= 2^-100 keeps every nonzero
// y = v * rd above 2^-125 (normal); y is bounded by sqrt(D) (a normalised
// value).  NaN or infinite rows fail the test and take the division.
FVSR_DEV bool ln_fast_ok(float mean, float rd) {
  const float am = fabsf(mean);
  return am >= 0x1p-125f && am * rd >= 0x1p-100f && rd <= 0x1p100f;
}

// R rows of one batch element per wavefront: the modulation vectors
// bf16(1 + scale) and shift are loaded and prepared once for the R rows, and
// all R rows are loaded before any arithmetic, so each wave keeps R row loads
// in flight.  Row groups never straddle a batch element; a group running
// past the batch's last row recomputes that row and stores nothing for it.
//
// GATE: the row is first formed as x1 = bf16(x + bf16(gate * res)) (the
// gated residual of the op before, fused_gate_add's arithmetic) and written
// to x1_out; the LayerNorm then runs on x1 from registers.
template <int VPL, int R, bool WRITE_OUT, bool QUANT, bool GATE = false>
__global__ __launch_bounds__(kThreads) void ln_modulate_vec(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ shift, uint16_t* __restrict__ out, int64_t B, int64_t L,
    int64_t D, float eps, uint8_t* __restrict__ codes, float* __restrict__ row_scale,
    const uint16_t* __restrict__ gate = nullptr, const uint16_t* __restrict__ res = nullptr,
    uint16_t* __restrict__ x1_out = nullptr) {
  const int lane = threadIdx.x & 63;
  const int64_t groups = (L + R - 1) / R;
  const int64_t g = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (g >= B * groups) return;
  const int64_t b = g / groups;
  const int64_t l0 = (g - b * groups) * R;
  const int64_t nchunk = D >> 3;
  const int64_t pb = b * D;
  int64_t row[R];
#pragma unroll
  for (int r = 0; r < R; ++r) row[r] = b * L + (l0 + r < L ? l0 + r : L - 1);
  // All loads unconditional (past-the-end chunks read the last chunk again)
  // so they are in flight together; repeated chunks are masked out of the
  // sums below and change no maximum.
  u32x4_t raw[R][VPL], sraw[VPL], shraw[VPL];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      raw[r][j] = *(const u32x4_t*)(x + row[r] * D + clamp_chunk(lane + 64 * j, nchunk) * 8);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t cc = clamp_chunk(lane + 64 * j, nchunk);
    sraw[j] = *(const u32x4_t*)(scale + pb + cc * 8);
    shraw[j] = *(const u32x4_t*)(shift + pb + cc * 8);
  }
  if (GATE) {
    u32x4_t rraw[R][VPL], graw[VPL];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < VPL; ++j)
        rraw[r][j] = *(const u32x4_t*)(res + row[r] * D + clamp_chunk(lane + 64 * j, nchunk) * 8);
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      graw[j] = *(const u32x4_t*)(gate + pb + clamp_chunk(lane + 64 * j, nchunk) * 8);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t t = pack_bf16x2_once(bf_lo(graw[j][p]) * bf_lo(rraw[r][j][p]),
                                              bf_hi(graw[j][p]) * bf_hi(rraw[r][j][p]));
          raw[r][j][p] = pack_bf16x2_once(bf_lo(raw[r][j][p]) + bf_lo(t),
                                          bf_hi(raw[r][j][p]) + bf_hi(t));
        }
        const int64_t c = lane + 64 * j;
        if (c < nchunk && l0 + r < L) *(u32x4_t*)(x1_out + row[r] * D + c * 8) = raw[r][j];
      }
  }
  float v[R][VPL][8], sum[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    sum[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      unpack8(raw[r][j], v[r][j]);
      float cs = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) cs += v[r][j][e];
      sum[r] += lane + 64 * j < nchunk ? cs : 0.0f;
    }
  }
  float sq[R], mean_r[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float mean = wave_sum(sum[r]) / (float)D;
    sq[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float cs = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[r][j][e] -= mean;
        cs = __builtin_fmaf(v[r][j][e], v[r][j][e], cs);
      }
      sq[r] += lane + 64 * j < nchunk ? cs : 0.0f;
    }
    mean_r[r] = mean;
  }
  float s1[VPL][8], sh[VPL][8];  // bf16(1 + scale) and shift
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    unpack8(shraw[j], sh[j]);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t w = pack_bf16x2_once(1.0f + bf_lo(sraw[j][p]), 1.0f + bf_hi(sraw[j][p]));
      s1[j][2 * p] = bf_lo(w);
      s1[j][2 * p + 1] = bf_hi(w);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float den = sqrtf(wave_sum(sq[r]) / (float)D + eps);
    const float rd = 1.0f / den;
    u32x4_t xn[VPL];
    bool bad = !ln_fast_ok(mean_r[r], rd);
    if (!bad) {
#pragma unroll
      for (int j = 0; j < VPL; ++j) xn[j] = bf16_quot8(v[r][j], rd, bad);
    }
    if (__builtin_amdgcn_ballot_w64(bad)) {
      if (bad) {
#pragma unroll
        for (int j = 0; j < VPL; ++j)
#pragma unroll
          for (int p = 0; p < 4; ++p)
            xn[j][p] = pack_bf16x2_once(v[r][j][2 * p] / den, v[r][j][2 * p + 1] / den);
      }
    }
    // y = bf16(xn * bf16(1 + s)); out = bf16(y + shift), two values per
    // conversion.  The row's largest |out| as the quantisation takes it
    // (NaNs passed over, as fmaxf does).
    u32x4_t o[VPL];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t y = pack_bf16x2_once(bf_lo(xn[j][p]) * s1[j][2 * p],
                                            bf_hi(xn[j][p]) * s1[j][2 * p + 1]);
        o[j][p] = pack_bf16x2_once(bf_lo(y) + sh[j][2 * p], bf_hi(y) + sh[j][2 * p + 1]);
        if (QUANT) m = max3_abs(m, bf_lo(o[j][p]), bf_hi(o[j][p]));
      }
      const int64_t c = lane + 64 * j;
      if (WRITE_OUT && c < nchunk && l0 + r < L) *(u32x4_t*)(out + row[r] * D + c * 8) = o[j];
    }
    if (QUANT) {
      const float amax = wave_max_abs(m);
      const float qs = fmaxf(amax, 1e-12f) / 448.0f, qr = 1.0f / qs;
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int64_t c = lane + 64 * j;
        if (c < nchunk && l0 + r < L) {
          *(u32x2_t*)(codes + row[r] * D + c * 8) = chunk_codes_fma(o[j], qr, fminf(qs, 3.40282347e38f));
        }
      }
      if (lane == 0 && l0 + r < L) row_scale[row[r]] = act_scale(amax);
    }
  }
}

// One row per wavefront, for workgroups whose four rows belong to one batch
// element (B == 1, or L a multiple of 4): the modulation vectors
// (bf16(1 + scale) and shift, and the gate for GATE) are formed once per
// workgroup, as fp32, in LDS, and each wave reads its chunks' values from
// there, so a row costs no per-column VALU work beyond its own chain.  Same
// arithmetic as ln_modulate_vec, bit for bit, with two changes of method:
// bf16(v / den) takes the division only for values whose y = v * (1/den)
// lies within 3 ulps of a bf16 rounding tie (y is within 3 ulps of fl(v /
// den): 1/den and the product are each rounded once), and the codes come
// from the signed quotient (quot_signed).  D % 8 == 0, D <= 1536.
constexpr int kRowChunks = 192;  // 1536 / 8
template <bool WRITE_OUT, bool QUANT, bool GATE>
__global__ __launch_bounds__(kThreads) void ln_modulate_row(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ shift, uint16_t* __restrict__ out, int64_t B, int64_t L,
    int64_t D, float eps, uint8_t* __restrict__ codes, float* __restrict__ row_scale,
    const uint16_t* __restrict__ gate, const uint16_t* __restrict__ res,
    uint16_t* __restrict__ x1_out) {
  constexpr int VPL = 3;
  constexpr int NP = GATE ? 6 : 4;  // s1 lo/hi halves, shift lo/hi, gate lo/hi
  __shared__ f32x4_t prm[NP][kRowChunks];
  const int lane = threadIdx.x & 63;
  const int64_t rows = B * L;
  const int64_t row0 = (int64_t)blockIdx.x * kWaves;
  const int64_t rw = row0 + (threadIdx.x >> 6);
  const bool live = rw < rows;
  const int64_t row = live ? rw : rows - 1;
  const int64_t pb = (row0 / L) * D;
  const int nchunk = (int)(D >> 3);
  // The row (and residual) loads go first; they are in flight while the
  // parameters are formed.
  u32x4_t raw[VPL], rraw[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int cc = min(lane + 64 * j, nchunk - 1);
    raw[j] = *(const u32x4_t*)(x + row * D + cc * 8);
    if (GATE) rraw[j] = *(const u32x4_t*)(res + row * D + cc * 8);
  }
  if ((int)threadIdx.x < nchunk) {
    const int c = threadIdx.x;
    const u32x4_t sc = *(const u32x4_t*)(scale + pb + c * 8);
    const u32x4_t sh = *(const u32x4_t*)(shift + pb + c * 8);
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = pack_bf16x2_once(1.0f + bf_lo(sc[i]), 1.0f + bf_hi(sc[i]));
      f[2 * i] = bf_lo(w);
      f[2 * i + 1] = bf_hi(w);
    }
    prm[0][c] = f32x4_t{f[0], f[1], f[2], f[3]};
    prm[1][c] = f32x4_t{f[4], f[5], f[6], f[7]};
    unpack8(sh, f);
    prm[2][c] = f32x4_t{f[0], f[1], f[2], f[3]};
    prm[3][c] = f32x4_t{f[4], f[5], f[6], f[7]};
    if (GATE) {
      unpack8(*(const u32x4_t*)(gate + pb + c * 8), f);
      prm[NP - 2][c] = f32x4_t{f[0], f[1], f[2], f[3]};
      prm[NP - 1][c] = f32x4_t{f[4], f[5], f[6], f[7]};
    }
  }
  __syncthreads();
  if (!live) return;
  // Every bf16 rounding of the chain is one rbf16 (the value stays fp32).
  float v[VPL][8];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    unpack8(raw[j], v[j]);
    if (GATE) {
      // x1 = bf16(x + bf16(gate * res)), written out, normalised below.
      const int cc = min(lane + 64 * j, nchunk - 1);
      const f32x4_t g0 = prm[NP - 2][cc], g1 = prm[NP - 1][cc];
      const float g[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
      float r[8];
      unpack8(rraw[j], r);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = rbf16(v[j][e] + rbf16(g[e] * r[e]));
      if (lane + 64 * j < nchunk) *(u32x4_t*)(x1_out + row * D + (lane + 64 * j) * 8) = pack8(v[j]);
    }
  }
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    float cs = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) cs += v[j][e];
    sum += lane + 64 * j < nchunk ? cs : 0.0f;
  }
  const float mean = wave_sum(sum) / (float)D;
  float sq = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    float cs = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[j][e] -= mean;
      cs = __builtin_fmaf(v[j][e], v[j][e], cs);
    }
    sq += lane + 64 * j < nchunk ? cs : 0.0f;
  }
  const float den = sqrtf(wave_sum(sq) / (float)D + eps);
  const float rd = 1.0f / den;
  // xn = bf16(v / den) from y = v * (1/den): y lies within 3 ulps of
  // fl(v / den) (1/den and the product are each rounded once), so their bf16
  // roundings agree unless y's low 16 bits are within 3 of the tie 0x8000,
  // i.e. (bits + 0x8003) mod 2^16 <= 6.  The lane keeps the smallest such
  // distance; values near a tie (rare) and rows failing ln_fast_ok divide.
  const bool fast = ln_fast_ok(mean, rd);
  float xn[VPL][8];
  uint16_t near = fast ? (uint16_t)0xffff : (uint16_t)0;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = v[j][e] * rd;
      xn[j][e] = rbf16(y);
      near = min(near, (uint16_t)(__float_as_uint(y) + 0x8003u));
    }
  if (__builtin_amdgcn_ballot_w64(near <= 6)) {
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = v[j][e] * rd;
        if (!fast || (uint16_t)(__float_as_uint(y) + 0x8003u) <= 6) xn[j][e] = rbf16(v[j][e] / den);
      }
  }
  // o = bf16(bf16(xn * bf16(1 + s)) + shift); the row's largest |o|.
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int cc = min(lane + 64 * j, nchunk - 1);
    const f32x4_t sa = prm[0][cc], sb = prm[1][cc], ha = prm[2][cc], hb = prm[3][cc];
    const float s1[8] = {sa[0], sa[1], sa[2], sa[3], sb[0], sb[1], sb[2], sb[3]};
    const float sh[8] = {ha[0], ha[1], ha[2], ha[3], hb[0], hb[1], hb[2], hb[3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) xn[j][e] = rbf16(rbf16(xn[j][e] * s1[e]) + sh[e]);
    // a repeated chunk (past the row's end) changes no maximum
#pragma unroll
    for (int e = 0; e < 8; e += 2) m = max3_abs(m, xn[j][e], xn[j][e + 1]);
    if (WRITE_OUT && lane + 64 * j < nchunk)
      *(u32x4_t*)(out + row * D + (lane + 64 * j) * 8) = pack8(xn[j]);
  }
  if (QUANT) {
    const float amax = wave_max_abs(m);
    const float qs = fmaxf(amax, 1e-12f) / 448.0f, qr = 1.0f / qs;
    const float qsf = fminf(qs, 3.40282347e38f);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const float* o = xn[j];
      u32x2_t q;
      q[0] = e4m3x4(quot_signed(o[0], qr, qsf), quot_signed(o[1], qr, qsf),
                    quot_signed(o[2], qr, qsf), quot_signed(o[3], qr, qsf));
      q[1] = e4m3x4(quot_signed(o[4], qr, qsf), quot_signed(o[5], qr, qsf),
                    quot_signed(o[6], qr, qsf), quot_signed(o[7], qr, qsf));
      if (lane + 64 * j < nchunk) *(u32x2_t*)(codes + row * D + (lane + 64 * j) * 8) = q;
    }
    if (lane == 0) row_scale[row] = act_scale(amax);
  }
}

// Any D and any input types (x, scale, shift of types xt, st, ht; out of
// type xt): three passes over the row from global memory (L2-resident after
// the first).
__global__ __launch_bounds__(kThreads) void ln_modulate_generic(
    const void* __restrict__ x, int xt, const void* __restrict__ scale, int st,
    const void* __restrict__ shift, int ht, void* __restrict__ out, int64_t rows, int64_t L,
    int64_t D, float eps, uint8_t* __restrict__ codes, float* __restrict__ row_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t xr = row * D;
  float sum = 0.0f;
  for (int64_t d = lane; d < D; d += 64) sum += ld_elem(x, xt, xr + d);
  const float mean = wave_sum(sum) / (float)D;
  float sq = 0.0f;
  for (int64_t d = lane; d < D; d += 64) {
    const float t = ld_elem(x, xt, xr + d) - mean;
    sq += t * t;
  }
  const float den = sqrtf(wave_sum(sq) / (float)D + eps);
  const int64_t pb = (row / L) * D;
  float amax = 0.0f;
  for (int64_t d = lane; d < D; d += 64) {
    const float xn = round_bf16((ld_elem(x, xt, xr + d) - mean) / den);
    const float y = round_bf16(xn * round_bf16(1.0f + ld_elem(scale, st, pb + d)));
    const float o = round_bf16(y + ld_elem(shift, ht, pb + d));
    amax = fmaxf(amax, fabsf(o));
    if (out) st_elem(out, xt, xr + d, o);
  }
  if (codes) {
    amax = wave_max(amax);
    const float qs = fmaxf(amax, 1e-12f) / 448.0f;
    for (int64_t d = lane; d < D; d += 64) {
      const float xn = round_bf16((ld_elem(x, xt, xr + d) - mean) / den);
      const float y = round_bf16(xn * round_bf16(1.0f + ld_elem(scale, st, pb + d)));
      const float o = round_bf16(y + ld_elem(shift, ht, pb + d));
      codes[row * D + d] =
          (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(o / qs), 0.0f, 0, false) & 0xff);
    }
    if (lane == 0) row_scale[row] = act_scale(amax);
  }
}

// LayerNorm with affine weight and bias (the DiT block's norm3 before the
// cross-attention), in torch's arithmetic for bf16 tensors: mean and variance
// in fp32, y = bf16(w * ((x - mean) * rstd) + b) in fp32 with
// rstd = rsqrt(var + eps), one rounding.  R rows per wavefront, rows in
// registers as in ln_modulate_vec; optional per-row e4m3 codes of y.
// GATE: the rows are first x1 = bf16(x + bf16(gate * res)) (fused_gate_add,
// gate [B, 1, D] per batch element of L rows), written to x1_out, then
// normalised from the registers.
template <int VPL, int R, bool WRITE_OUT, bool QUANT, bool GATE = false>
__global__ __launch_bounds__(kThreads) void layer_norm_vec(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int64_t rows, int64_t D,
    float eps, uint8_t* __restrict__ codes, float* __restrict__ row_scale,
    const uint16_t* __restrict__ gate = nullptr, const uint16_t* __restrict__ res = nullptr,
    uint16_t* __restrict__ x1_out = nullptr, int64_t L = 1) {
  const int lane = threadIdx.x & 63;
  const int64_t r0 = ((int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
  if (r0 >= rows) return;
  const int64_t nchunk = D >> 3;
  int64_t row[R];
#pragma unroll
  for (int r = 0; r < R; ++r) row[r] = r0 + r < rows ? r0 + r : rows - 1;
  u32x4_t raw[R][VPL], wraw[VPL], braw[VPL];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      raw[r][j] = *(const u32x4_t*)(x + row[r] * D + clamp_chunk(lane + 64 * j, nchunk) * 8);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t cc = clamp_chunk(lane + 64 * j, nchunk);
    wraw[j] = *(const u32x4_t*)(w + cc * 8);
    braw[j] = *(const u32x4_t*)(bias + cc * 8);
  }
  if (GATE) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t pg = (row[r] / L) * D;
      u32x4_t rraw[VPL], graw[VPL];
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int64_t cc = clamp_chunk(lane + 64 * j, nchunk);
        rraw[j] = *(const u32x4_t*)(res + row[r] * D + cc * 8);
        graw[j] = *(const u32x4_t*)(gate + pg + cc * 8);
      }
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t t = pack_bf16x2_once(bf_lo(graw[j][p]) * bf_lo(rraw[j][p]),
                                              bf_hi(graw[j][p]) * bf_hi(rraw[j][p]));
          raw[r][j][p] = pack_bf16x2_once(bf_lo(raw[r][j][p]) + bf_lo(t),
                                          bf_hi(raw[r][j][p]) + bf_hi(t));
        }
        const int64_t c = lane + 64 * j;
        if (c < nchunk && r0 + r < rows) *(u32x4_t*)(x1_out + row[r] * D + c * 8) = raw[r][j];
      }
    }
  }
  float v[R][VPL][8], sum[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    sum[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      unpack8(raw[r][j], v[r][j]);
      float cs = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) cs += v[r][j][e];
      sum[r] += lane + 64 * j < nchunk ? cs : 0.0f;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float mean = wave_sum(sum[r]) / (float)D;
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float cs = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[r][j][e] -= mean;
        cs = __builtin_fmaf(v[r][j][e], v[r][j][e], cs);
      }
      sq += lane + 64 * j < nchunk ? cs : 0.0f;
    }
    const float rstd = rsqrtf(wave_sum(sq) / (float)D + eps);
    u32x4_t o[VPL];
    float m = 0.0f;  // the row's largest |y|, NaNs passed over as fmaxf does
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float y0 = __builtin_fmaf(bf_lo(wraw[j][p]), v[r][j][2 * p] * rstd, bf_lo(braw[j][p]));
        const float y1 =
            __builtin_fmaf(bf_hi(wraw[j][p]), v[r][j][2 * p + 1] * rstd, bf_hi(braw[j][p]));
        o[j][p] = pack_bf16x2_once(y0, y1);
        if (QUANT) m = max3_abs(m, bf_lo(o[j][p]), bf_hi(o[j][p]));
      }
      const int64_t c = lane + 64 * j;
      if (WRITE_OUT && c < nchunk && r0 + r < rows) *(u32x4_t*)(out + row[r] * D + c * 8) = o[j];
    }
    if (QUANT) {
      const float amax = wave_max_abs(m);
      const float qs = fmaxf(amax, 1e-12f) / 448.0f, qr = 1.0f / qs;
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int64_t c = lane + 64 * j;
        if (c < nchunk && r0 + r < rows) {
          *(u32x2_t*)(codes + row[r] * D + c * 8) = chunk_codes_fma(o[j], qr, fminf(qs, 3.40282347e38f));
        }
      }
      if (lane == 0 && r0 + r < rows) row_scale[row[r]] = act_scale(amax);
    }
  }
}

// Any D: passes over the row from global memory.
__global__ __launch_bounds__(kThreads) void layer_norm_generic(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int64_t rows, int64_t D,
    float eps, uint8_t* __restrict__ codes, float* __restrict__ row_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + row * D;
  float sum = 0.0f;
  for (int64_t d = lane; d < D; d += 64) sum += bf2f(xr[d]);
  const float mean = wave_sum(sum) / (float)D;
  float sq = 0.0f;
  for (int64_t d = lane; d < D; d += 64) {
    const float t = bf2f(xr[d]) - mean;
    sq = __builtin_fmaf(t, t, sq);
  }
  const float rstd = rsqrtf(wave_sum(sq) / (float)D + eps);
  float amax = 0.0f;
  for (int64_t d = lane; d < D; d += 64) {
    const float o = round_bf16(__builtin_fmaf(bf2f(w[d]), (bf2f(xr[d]) - mean) * rstd, bf2f(bias[d])));
    amax = fmaxf(amax, fabsf(o));
    if (out) out[row * D + d] = (uint16_t)(pack_bf16x2(o, 0.0f) & 0xffff);
  }
  if (codes) {
    amax = wave_max(amax);
    const float qs = fmaxf(amax, 1e-12f) / 448.0f;
    for (int64_t d = lane; d < D; d += 64) {
      const float o = round_bf16(__builtin_fmaf(bf2f(w[d]), (bf2f(xr[d]) - mean) * rstd, bf2f(bias[d])));
      codes[row * D + d] =
          (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(o / qs), 0.0f, 0, false) & 0xff);
    }
    if (lane == 0) row_scale[row] = act_scale(amax);
  }
}

constexpr int kGateUnroll = 2;

__global__ __launch_bounds__(kThreads) void gate_add_vec(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gate,
    const uint16_t* __restrict__ res, uint16_t* __restrict__ out, int64_t nchunk, int64_t LD,
    int64_t D) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t c0 = (int64_t)blockIdx.x * kThreads + threadIdx.x; c0 < nchunk;
       c0 += stride * kGateUnroll) {
    u32x4_t xv[kGateUnroll], rv[kGateUnroll], gv[kGateUnroll];
#pragma unroll
    for (int u = 0; u < kGateUnroll; ++u) {
      const int64_t i = clamp_chunk(c0 + u * stride, nchunk) * 8;
      xv[u] = *(const u32x4_t*)(x + i);
      rv[u] = *(const u32x4_t*)(res + i);
      gv[u] = *(const u32x4_t*)(gate + (i / LD) * D + (i % D));
    }
#pragma unroll
    for (int u = 0; u < kGateUnroll; ++u) {
      const int64_t c = c0 + u * stride;
      if (c < nchunk) {
        u32x4_t o;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float y0 = round_bf16(bf_lo(gv[u][w]) * bf_lo(rv[u][w]));
          const float y1 = round_bf16(bf_hi(gv[u][w]) * bf_hi(rv[u][w]));
          o[w] = pack_bf16x2(bf_lo(xv[u][w]) + y0, bf_hi(xv[u][w]) + y1);
        }
        *(u32x4_t*)(out + c * 8) = o;
      }
    }
  }
}

// Any shape and input types (x, gate, res of types xt, gt, rt; out of type xt).
__global__ __launch_bounds__(kThreads) void gate_add_generic(
    const void* __restrict__ x, int xt, const void* __restrict__ gate, int gt,
    const void* __restrict__ res, int rt, void* __restrict__ out, int64_t n, int64_t LD,
    int64_t D) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const float y = round_bf16(ld_elem(gate, gt, (i / LD) * D + (i % D)) * ld_elem(res, rt, i));
    st_elem(out, xt, i, round_bf16(ld_elem(x, xt, i) + y));
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool dtype_ok(int dt) { return dt == FVSR_DT_BF16 || dt == FVSR_DT_F16 || dt == FVSR_DT_F32; }

}  // namespace

extern "C" int fvsr_ln_modulate(const void* x, const void* scale, const void* shift, void* out,
                                int64_t B, int64_t L, int64_t D, float eps, void* codes,
                                float* row_scale, void* stream) {
  if (B < 0 || L < 0 || D <= 0) return FVSR_EINVAL;
  const int64_t rows = B * L;
  if (rows == 0) return FVSR_OK;
  if (!x || !scale || !shift || (!out && !codes) || (codes && !row_scale)) return FVSR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves)), block(kThreads);
  const uint16_t *xp = (const uint16_t*)x, *sp = (const uint16_t*)scale,
                 *hp = (const uint16_t*)shift;
  uint16_t* op = (uint16_t*)out;
  uint8_t* qp = (uint8_t*)codes;
  const bool vec = D % 8 == 0 && D <= 512 * 3 && aligned16(x) && aligned16(scale) &&
                   aligned16(shift) && (!out || aligned16(out)) && (!codes || aligned16(codes));
  if (vec && (B == 1 || L % kWaves == 0)) {
    // one row per wave, the workgroup's modulation vectors in LDS
    const uint16_t* none = nullptr;
    uint16_t* none_out = nullptr;
    if (out && codes)
      hipLaunchKernelGGL((ln_modulate_row<true, true, false>), grid, block, 0, st, xp, sp, hp, op,
                         B, L, D, eps, qp, row_scale, none, none, none_out);
    else if (out)
      hipLaunchKernelGGL((ln_modulate_row<true, false, false>), grid, block, 0, st, xp, sp, hp, op,
                         B, L, D, eps, qp, row_scale, none, none, none_out);
    else
      hipLaunchKernelGGL((ln_modulate_row<false, true, false>), grid, block, 0, st, xp, sp, hp, op,
                         B, L, D, eps, qp, row_scale, none, none, none_out);
  } else if (vec) {
    const int64_t groups = B * ((L + kLnRows - 1) / kLnRows);
    const dim3 vgrid((unsigned)((groups + kWaves - 1) / kWaves));
    if (out && codes)
      hipLaunchKernelGGL((ln_modulate_vec<3, kLnRows, true, true>), vgrid, block, 0, st, xp, sp,
                         hp, op, B, L, D, eps, qp, row_scale);
    else if (out)
      hipLaunchKernelGGL((ln_modulate_vec<3, kLnRows, true, false>), vgrid, block, 0, st, xp, sp,
                         hp, op, B, L, D, eps, qp, row_scale);
    else
      hipLaunchKernelGGL((ln_modulate_vec<3, kLnRows, false, true>), vgrid, block, 0, st, xp, sp,
                         hp, op, B, L, D, eps, qp, row_scale);
  } else {
    hipLaunchKernelGGL(ln_modulate_generic, grid, block, 0, st, x, FVSR_DT_BF16, scale,
                       FVSR_DT_BF16, shift, FVSR_DT_BF16, out, rows, L, D, eps, qp, row_scale);
  }
  return fvsr_launch_status();
}

extern "C" int fvsr_layer_norm(const void* x, const void* weight, const void* bias, void* out,
                               int64_t rows, int64_t D, float eps, void* codes, float* row_scale,
                               void* stream) {
  if (rows < 0 || D <= 0) return FVSR_EINVAL;
  if (rows == 0) return FVSR_OK;
  if (!x || !weight || !bias || (!out && !codes) || (codes && !row_scale)) return FVSR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *xp = (const uint16_t*)x, *wp = (const uint16_t*)weight,
                 *bp = (const uint16_t*)bias;
  uint16_t* op = (uint16_t*)out;
  uint8_t* qp = (uint8_t*)codes;
  const bool vec = D % 8 == 0 && D <= 512 * 3 && aligned16(x) && aligned16(weight) &&
                   aligned16(bias) && (!out || aligned16(out)) && (!codes || aligned16(codes));
  if (vec) {
    const int64_t groups = (rows + kLnRows - 1) / kLnRows;
    const dim3 vgrid((unsigned)((groups + kWaves - 1) / kWaves)), block(kThreads);
    if (out && codes)
      hipLaunchKernelGGL((layer_norm_vec<3, kLnRows, true, true>), vgrid, block, 0, st, xp, wp,
                         bp, op, rows, D, eps, qp, row_scale);
    else if (out)
      hipLaunchKernelGGL((layer_norm_vec<3, kLnRows, true, false>), vgrid, block, 0, st, xp, wp,
                         bp, op, rows, D, eps, qp, row_scale);
    else
      hipLaunchKernelGGL((layer_norm_vec<3, kLnRows, false, true>), vgrid, block, 0, st, xp, wp,
                         bp, op, rows, D, eps, qp, row_scale);
  } else {
    hipLaunchKernelGGL(layer_norm_generic, dim3((unsigned)((rows + kWaves - 1) / kWaves)),
                       dim3(kThreads), 0, st, xp, wp, bp, op, rows, D, eps, qp, row_scale);
  }
  return fvsr_launch_status();
}

extern "C" int fvsr_gate_add_ln_modulate(const void* x, const void* gate, const void* res,
                                         void* x1, const void* scale, const void* shift,
                                         void* out, int64_t B, int64_t L, int64_t D, float eps,
                                         void* codes, float* row_scale, void* stream) {
  if (B < 0 || L < 0 || D <= 0) return FVSR_EINVAL;
  if (B * L == 0) return FVSR_OK;
  if (!x || !gate || !res || !x1 || !scale || !shift || (!out && !codes) ||
      (codes && !row_scale))
    return FVSR_EINVAL;
  const bool vec = D % 8 == 0 && D <= 512 * 3 && aligned16(x) && aligned16(gate) &&
                   aligned16(res) && aligned16(x1) && aligned16(scale) && aligned16(shift) &&
                   (!out || aligned16(out)) && (!codes || aligned16(codes));
  if (!vec) return FVSR_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *xp = (const uint16_t*)x, *sp = (const uint16_t*)scale,
                 *hp = (const uint16_t*)shift, *gp = (const uint16_t*)gate,
                 *rp = (const uint16_t*)res;
  uint16_t *op = (uint16_t*)out, *x1p = (uint16_t*)x1;
  uint8_t* qp = (uint8_t*)codes;
  const dim3 block(kThreads);
  if (B == 1 || L % kWaves == 0) {
    // one row per wave, the workgroup's modulation vectors and gate in LDS
    const dim3 grid((unsigned)((B * L + kWaves - 1) / kWaves));
    if (out && codes)
      hipLaunchKernelGGL((ln_modulate_row<true, true, true>), grid, block, 0, st, xp, sp, hp, op,
                         B, L, D, eps, qp, row_scale, gp, rp, x1p);
    else if (out)
      hipLaunchKernelGGL((ln_modulate_row<true, false, true>), grid, block, 0, st, xp, sp, hp, op,
                         B, L, D, eps, qp, row_scale, gp, rp, x1p);
    else
      hipLaunchKernelGGL((ln_modulate_row<false, true, true>), grid, block, 0, st, xp, sp, hp, op,
                         B, L, D, eps, qp, row_scale, gp, rp, x1p);
    return fvsr_launch_status();
  }
  const int64_t groups = B * ((L + kLnRows - 1) / kLnRows);
  const dim3 vgrid((unsigned)((groups + kWaves - 1) / kWaves));
  if (out && codes)
    hipLaunchKernelGGL((ln_modulate_vec<3, kLnRows, true, true, true>), vgrid, block, 0, st, xp, sp,
                       hp, op, B, L, D, eps, qp, row_scale, gp, rp, x1p);
  else if (out)
    hipLaunchKernelGGL((ln_modulate_vec<3, kLnRows, true, false, true>), vgrid, block, 0, st, xp,
                       sp, hp, op, B, L, D, eps, qp, row_scale, gp, rp, x1p);
  else
    hipLaunchKernelGGL((ln_modulate_vec<3, kLnRows, false, true, true>), vgrid, block, 0, st, xp,
                       sp, hp, op, B, L, D, eps, qp, row_scale, gp, rp, x1p);
  return fvsr_launch_status();
}

extern "C" int fvsr_gate_add_dt(const void* x, int x_dtype, const void* gate, int gate_dtype,
                                const void* res, int res_dtype, void* out, int64_t B, int64_t L,
                                int64_t D, void* stream) {
  if (B < 0 || L < 0 || D <= 0 || !dtype_ok(x_dtype) || !dtype_ok(gate_dtype) ||
      !dtype_ok(res_dtype))
    return FVSR_EINVAL;
  const int64_t n = B * L * D;
  if (n == 0) return FVSR_OK;
  if (!x || !gate || !res || !out) return FVSR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *xp = (const uint16_t*)x, *gp = (const uint16_t*)gate,
                 *rp = (const uint16_t*)res;
  uint16_t* op = (uint16_t*)out;
  const bool bf16 = x_dtype == FVSR_DT_BF16 && gate_dtype == FVSR_DT_BF16 &&
                    res_dtype == FVSR_DT_BF16;
  const bool vec = bf16 && D % 8 == 0 && aligned16(x) && aligned16(gate) && aligned16(res) &&
                   aligned16(out);
  if (vec) {
    const int64_t nchunk = n / 8;
    int64_t blocks = (nchunk + kThreads * kGateUnroll - 1) / (kThreads * kGateUnroll);
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(gate_add_vec, dim3((unsigned)blocks), dim3(kThreads), 0, st, xp, gp, rp,
                       op, nchunk, L * D, D);
  } else {
    int64_t blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(gate_add_generic, dim3((unsigned)blocks), dim3(kThreads), 0, st, x,
                       x_dtype, gate, gate_dtype, res, res_dtype, out, n, L * D, D);
  }
  return fvsr_launch_status();
}

extern "C" int fvsr_gate_add(const void* x, const void* gate, const void* res, void* out,
                             int64_t B, int64_t L, int64_t D, void* stream) {
  return fvsr_gate_add_dt(x, FVSR_DT_BF16, gate, FVSR_DT_BF16, res, FVSR_DT_BF16, out, B, L, D,
                          stream);
}

extern "C" int fvsr_ln_modulate_dt(const void* x, int x_dtype, const void* scale, int scale_dtype,
                                   const void* shift, int shift_dtype, void* out, int64_t B,
                                   int64_t L, int64_t D, float eps, void* stream) {
  if (B < 0 || L < 0 || D <= 0 || !dtype_ok(x_dtype) || !dtype_ok(scale_dtype) ||
      !dtype_ok(shift_dtype))
    return FVSR_EINVAL;
  if (x_dtype == FVSR_DT_BF16 && scale_dtype == FVSR_DT_BF16 && shift_dtype == FVSR_DT_BF16)
    return fvsr_ln_modulate(x, scale, shift, out, B, L, D, eps, nullptr, nullptr, stream);
  const int64_t rows = B * L;
  if (rows == 0) return FVSR_OK;
  if (!x || !scale || !shift || !out) return FVSR_EINVAL;
  hipLaunchKernelGGL(ln_modulate_generic, dim3((unsigned)((rows + kWaves - 1) / kWaves)),
                     dim3(kThreads), 0, (hipStream_t)stream, x, x_dtype, scale, scale_dtype,
                     shift, shift_dtype, out, rows, L, D, eps, (uint8_t*)nullptr,
                     (float*)nullptr);
  return fvsr_launch_status();
}

extern "C" int fvsr_gate_add_layer_norm(const void* x, const void* gate, const void* res,
                                        void* x1, const void* weight, const void* bias,
                                        void* out, int64_t B, int64_t L, int64_t D, float eps,
                                        void* codes, float* row_scale, void* stream) {
  if (B < 0 || L < 0 || D <= 0) return FVSR_EINVAL;
  const int64_t rows = B * L;
  if (rows == 0) return FVSR_OK;
  if (!x || !gate || !res || !x1 || !weight || !bias || (!out && !codes) ||
      (codes && !row_scale))
    return FVSR_EINVAL;
  const bool vec = D % 8 == 0 && D <= 512 * 3 && aligned16(x) && aligned16(gate) &&
                   aligned16(res) && aligned16(x1) && aligned16(weight) && aligned16(bias) &&
                   (!out || aligned16(out)) && (!codes || aligned16(codes));
  if (!vec) return FVSR_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *xp = (const uint16_t*)x, *gp = (const uint16_t*)gate, *rp = (const uint16_t*)res,
                 *wp = (const uint16_t*)weight, *bp = (const uint16_t*)bias;
  uint16_t *x1p = (uint16_t*)x1, *op = (uint16_t*)out;
  uint8_t* qp = (uint8_t*)codes;
  const int64_t groups = (rows + kLnRows - 1) / kLnRows;
  const dim3 vgrid((unsigned)((groups + kWaves - 1) / kWaves)), block(kThreads);
  if (out && codes)
    hipLaunchKernelGGL((layer_norm_vec<3, kLnRows, true, true, true>), vgrid, block, 0, st, xp, wp,
                       bp, op, rows, D, eps, qp, row_scale, gp, rp, x1p, L);
  else if (out)
    hipLaunchKernelGGL((layer_norm_vec<3, kLnRows, true, false, true>), vgrid, block, 0, st, xp,
                       wp, bp, op, rows, D, eps, qp, row_scale, gp, rp, x1p, L);
  else
    hipLaunchKernelGGL((layer_norm_vec<3, kLnRows, false, true, true>), vgrid, block, 0, st, xp,
                       wp, bp, op, rows, D, eps, qp, row_scale, gp, rp, x1p, L);
  return fvsr_launch_status();
}
