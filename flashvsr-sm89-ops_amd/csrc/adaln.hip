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

FVSR_DEV void unpack8(u32x4_t c, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf_lo(c[i]);
    f[2 * i + 1] = bf_hi(c[i]);
  }
}

FVSR_DEV u32x4_t pack8(const float* f) {
  u32x4_t c;
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return c;
}

template <int VPL, bool WRITE_OUT, bool QUANT>
__global__ __launch_bounds__(kThreads) void ln_modulate_vec(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ shift, uint16_t* __restrict__ out, int64_t rows, int64_t L,
    int64_t D, float eps, uint8_t* __restrict__ codes, float* __restrict__ row_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t nchunk = D >> 3;
  const uint16_t* xr = x + row * D;
  float v[VPL][8];
  u32x4_t raw[VPL], sraw[VPL], shraw[VPL];
  const int64_t pb = (row / L) * D;
  // All loads unconditional (past-the-end chunks read the last chunk again)
  // so they are in flight together; repeated chunks are masked out of the
  // sums below and change no maximum.
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t cc = clamp_chunk(lane + 64 * j, nchunk);
    raw[j] = *(const u32x4_t*)(xr + cc * 8);
    sraw[j] = *(const u32x4_t*)(scale + pb + cc * 8);
    shraw[j] = *(const u32x4_t*)(shift + pb + cc * 8);
  }
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const bool in = lane + 64 * j < nchunk;
    unpack8(raw[j], v[j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += in ? v[j][e] : 0.0f;
  }
  const float mean = wave_sum(sum) / (float)D;
  float sq = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const bool in = lane + 64 * j < nchunk;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[j][e] -= mean;
      sq += in ? v[j][e] * v[j][e] : 0.0f;
    }
  }
  const float var = wave_sum(sq) / (float)D;
  const float den = sqrtf(var + eps);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t c = lane + 64 * j;
    float s[8], sh[8];
    unpack8(sraw[j], s);
    unpack8(shraw[j], sh);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float xn = round_bf16(v[j][e] / den);
      const float y = round_bf16(xn * round_bf16(1.0f + s[e]));
      v[j][e] = round_bf16(y + sh[e]);
      amax = fmaxf(amax, fabsf(v[j][e]));
    }
    if (WRITE_OUT && c < nchunk) *(u32x4_t*)(out + row * D + c * 8) = pack8(v[j]);
  }
  if (QUANT) {
    amax = wave_max(amax);
    const float qs = fmaxf(amax, 1e-12f) / 448.0f, qr = 1.0f / qs;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int64_t c = lane + 64 * j;
      if (c < nchunk) {
        u32x2_t q;
        q[0] = e4m3x4_div(v[j][0], v[j][1], v[j][2], v[j][3], qs, qr);
        q[1] = e4m3x4_div(v[j][4], v[j][5], v[j][6], v[j][7], qs, qr);
        *(u32x2_t*)(codes + row * D + c * 8) = q;
      }
    }
    if (lane == 0) row_scale[row] = amax / 448.0f;
  }
}

// Any D: three passes over the row from global memory (L2-resident after the first).
__global__ __launch_bounds__(kThreads) void ln_modulate_generic(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ scale,
    const uint16_t* __restrict__ shift, uint16_t* __restrict__ out, int64_t rows, int64_t L,
    int64_t D, float eps, uint8_t* __restrict__ codes, float* __restrict__ row_scale) {
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
    sq += t * t;
  }
  const float den = sqrtf(wave_sum(sq) / (float)D + eps);
  const int64_t pb = (row / L) * D;
  float amax = 0.0f;
  for (int64_t d = lane; d < D; d += 64) {
    const float xn = round_bf16((bf2f(xr[d]) - mean) / den);
    const float y = round_bf16(xn * round_bf16(1.0f + bf2f(scale[pb + d])));
    const float o = round_bf16(y + bf2f(shift[pb + d]));
    amax = fmaxf(amax, fabsf(o));
    if (out) out[row * D + d] = (uint16_t)(pack_bf16x2(o, 0.0f) & 0xffff);
  }
  if (codes) {
    amax = wave_max(amax);
    const float qs = fmaxf(amax, 1e-12f) / 448.0f;
    for (int64_t d = lane; d < D; d += 64) {
      const float xn = round_bf16((bf2f(xr[d]) - mean) / den);
      const float y = round_bf16(xn * round_bf16(1.0f + bf2f(scale[pb + d])));
      const float o = round_bf16(y + bf2f(shift[pb + d]));
      codes[row * D + d] =
          (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(clamp448(o / qs), 0.0f, 0, false) & 0xff);
    }
    if (lane == 0) row_scale[row] = amax / 448.0f;
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

__global__ __launch_bounds__(kThreads) void gate_add_generic(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gate,
    const uint16_t* __restrict__ res, uint16_t* __restrict__ out, int64_t n, int64_t LD,
    int64_t D) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const float y = round_bf16(bf2f(gate[(i / LD) * D + (i % D)]) * bf2f(res[i]));
    out[i] = (uint16_t)(pack_bf16x2(bf2f(x[i]) + y, 0.0f) & 0xffff);
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

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
  if (vec) {
    if (out && codes)
      hipLaunchKernelGGL((ln_modulate_vec<3, true, true>), grid, block, 0, st, xp, sp, hp, op,
                         rows, L, D, eps, qp, row_scale);
    else if (out)
      hipLaunchKernelGGL((ln_modulate_vec<3, true, false>), grid, block, 0, st, xp, sp, hp, op,
                         rows, L, D, eps, qp, row_scale);
    else
      hipLaunchKernelGGL((ln_modulate_vec<3, false, true>), grid, block, 0, st, xp, sp, hp, op,
                         rows, L, D, eps, qp, row_scale);
  } else {
    hipLaunchKernelGGL(ln_modulate_generic, grid, block, 0, st, xp, sp, hp, op, rows, L, D, eps,
                       qp, row_scale);
  }
  return fvsr_launch_status();
}

extern "C" int fvsr_gate_add(const void* x, const void* gate, const void* res, void* out,
                             int64_t B, int64_t L, int64_t D, void* stream) {
  if (B < 0 || L < 0 || D <= 0) return FVSR_EINVAL;
  const int64_t n = B * L * D;
  if (n == 0) return FVSR_OK;
  if (!x || !gate || !res || !out) return FVSR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *xp = (const uint16_t*)x, *gp = (const uint16_t*)gate,
                 *rp = (const uint16_t*)res;
  uint16_t* op = (uint16_t*)out;
  const bool vec = D % 8 == 0 && aligned16(x) && aligned16(gate) && aligned16(res) &&
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
    hipLaunchKernelGGL(gate_add_generic, dim3((unsigned)blocks), dim3(kThreads), 0, st, xp, gp,
                       rp, op, n, L * D, D);
  }
  return fvsr_launch_status();
}
