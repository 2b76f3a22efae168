// Dynamic and static e4m3fn quantisation (contracts Q-A, Q-W, G).
//
// Row mode keeps one row per wavefront in registers: one HBM read of the bf16
// row, a 64-lane max reduction, then the codes are produced from registers
// (3 bytes of HBM traffic per element).  Tensor mode writes per-workgroup
// partial maxima in a first launch and every workgroup of the second launch
// re-reduces those partials (at most 1024 floats) before quantising, so no
// atomics and no memset are needed.
//
// Bit-exactness: the codes are those of the IEEE division x/s, formed
// without dividing (quot_abs / quot_signed in common.h: one product and two
// fmas, checked exhaustively over bf16 values and scales); the fp32 -> e4m3fn
// conversion is v_cvt_pk_fp8_f32.
//
// GELU of bf16 data (the FFN requantisation) is a lookup: the 65536 bf16
// results, generated at build time from the operation sequence of
// gelu_tanh_bf16 (csrc/gelu_table_gen.c), sit in every workgroup's LDS.
#pragma clang fp contract(off)
#include <atomic>
#include <mutex>

#include "common.h"

namespace {

constexpr int kWaves = 4;            // wavefronts per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kMaxPartials = 1024;   // tensor-mode partial maxima

// Element i of x (type dt, FVSR_DT_*) as fp32, or its tanh-GELU rounded to
// bf16: the scalar paths, which also take fp16 and fp32 inputs.
template <bool GELU>
FVSR_DEV float load_val(const void* x, int dt, int64_t i) {
  const float v = ld_elem(x, dt, i);
  return GELU ? gelu_tanh_bf16(v) : v;
}

// Apply GELU to a packed chunk of 8 bf16 (the result is bf16-valued, so it is
// stored back packed).
FVSR_DEV u32x4_t gelu_chunk(u32x4_t c) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = pack_bf16x2(gelu_tanh_bf16(bf_lo(c[i])), gelu_tanh_bf16(bf_hi(c[i])));
  return r;
}

FVSR_DEV float chunk_absmax(u32x4_t c) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf_lo(c[i])), fabsf(bf_hi(c[i]))));
  return m;
}

FVSR_DEV float qscale(float amax) { return fmaxf(amax, 1e-12f) / 448.0f; }
// The residual's copy of s, kept finite (s = inf when amax = inf).
FVSR_DEV float qscale_fin(float s) { return fminf(s, 3.40282347e38f); }

// ---------------------------------------------------------------------------
// Row mode, register resident: cols % 8 == 0, cols <= 512*VPL, 16-byte rows.
// The row is held as fp32 (one shift or mask per value), the maximum taken by
// v_max3_f32 on magnitudes and the codes by quot_signed: 2% less time at
// 16896 x 1536 than packed bf16 with the sign bits gathered separately.
// ---------------------------------------------------------------------------
template <int VPL, bool GELU>
__global__ __launch_bounds__(kThreads) void quant_rows_vec(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, int64_t ld,
    uint8_t* __restrict__ codes, float* __restrict__ scale_out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + row * ld;
  const int64_t nchunk = cols >> 3;
  u32x4_t v[VPL];
  // Every lane loads VPL chunks, past-the-end ones clamped to the row's last
  // chunk: the loads stay unconditional (so they are all in flight at once)
  // and a repeated chunk cannot change the row's max.
#pragma unroll
  for (int j = 0; j < VPL; ++j) v[j] = *(const u32x4_t*)(xr + clamp_chunk(lane + 64 * j, nchunk) * 8);
  float m = 0.0f;
  float f[VPL][8];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    if (GELU) v[j] = gelu_chunk(v[j]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[j][2 * i] = lo_f(v[j][i]);
      f[j][2 * i + 1] = hi_f(v[j][i]);
      m = max3_abs(m, f[j][2 * i], f[j][2 * i + 1]);
    }
  }
  const float amax = wave_max_abs(m);
  const float s = qscale(amax), r = 1.0f / s, sc = qscale_fin(s);
  uint8_t* qr = codes + row * cols;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t c = lane + 64 * j;
    u32x2_t q;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      q[h] = e4m3x4(quot_signed(f[j][4 * h], r, sc), quot_signed(f[j][4 * h + 1], r, sc),
                    quot_signed(f[j][4 * h + 2], r, sc), quot_signed(f[j][4 * h + 3], r, sc));
    if (c < nchunk) *(u32x2_t*)(qr + c * 8) = q;
  }
  if (lane == 0) scale_out[row] = act_scale(amax);
}

// ---------------------------------------------------------------------------
// GELU by table: persistent workgroups (one per CU: the 128 KB table fills
// most of its LDS), one row per wave at a time, the row in registers
// (cols % 8 == 0, cols <= 512*VPL, 16-byte rows).
// ---------------------------------------------------------------------------
__device__ const uint16_t kGeluTable[65536] __attribute__((aligned(16))) = {
#include "gelu_table.inc"
};

// Waves per workgroup.  Per-token requantisation keeps a row's GELU values as
// fp32 (162 registers per lane: 2 waves per SIMD); the tensor-mode kernels
// keep packed bf16 (<= 128 registers) and run 11.  Measured at the C5 shape
// (16896 rows of 8960), per token: 8 waves 80.4 us, 10: 82.6, 11: 81.6, 12:
// 81.4; packed bf16 at 11 waves 82.8.
constexpr int kTabWaves = 11;
constexpr int kRowTabWaves = 8;

// First row of this wave: the waves of a workgroup take rows one grid apart
// (row = block + wave * grid, then steps of grid * waves), so one CU never
// streams a run of neighbouring rows.  Same work, same per-row code; a CU
// taking 8 adjacent rows at a time ran the per-token requantisation at 87.8
// us against 80.4, and a pure row-streaming kernel at 80.3 us against 76.1.
FVSR_DEV int64_t first_table_row() {
  return (int64_t)blockIdx.x + (int64_t)(threadIdx.x >> 6) * gridDim.x;
}

// Load row `row` (chunks past the end of the row repeat its last chunk).
// Streamed once: non-temporal loads (and stores of the codes) keep the
// caches for the table and the other waves' rows (104 -> 97.5 us at 16 waves).
template <int VPL>
FVSR_DEV void load_row(u32x4_t (&v)[VPL], const uint16_t* x, int64_t row, int64_t ld, int nchunk) {
  const int lane = lane_here();
  const uint8_t* xr = (const uint8_t*)(x + row * ld);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int c = lane + 64 * j < nchunk ? lane + 64 * j : nchunk - 1;
    v[j] = __builtin_nontemporal_load((const u32x4_t*)(xr + (uint32_t)c * 16u));
  }
}


// Row `row` is in v (bf16).  Its GELU values are looked up straight into fp32
// registers (the bf16 result shifted into the high half: one operation per
// value, 8 registers per chunk), their maximum magnitude taken by v_max3_f32,
// and the codes formed from the signed values (quot_signed: no sign bits to
// gather).  Against packed bf16 (4 registers per chunk, unpacked once for the
// maximum and again for the codes) this is 21% fewer VALU instructions per
// row.
template <int VPL>
FVSR_DEV void gelu_quant_row(const u32x4_t (&v)[VPL], const uint16_t* tab, int64_t row,
                             int64_t cols, int nchunk, uint8_t* codes, float* scale_out) {
  float f[VPL][8];
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[j][2 * i] = __uint_as_float((uint32_t)tab[v[j][i] & 0xffffu] << 16);
      f[j][2 * i + 1] = __uint_as_float((uint32_t)tab[v[j][i] >> 16] << 16);
      m = max3_abs(m, f[j][2 * i], f[j][2 * i + 1]);
    }
  }
  const float amax = wave_max_abs(m);  // a repeated chunk changes no maximum
  const float s = qscale(amax), r = 1.0f / s, sc = qscale_fin(s);
  const int lane = lane_here();
  uint8_t* qr = codes + row * cols;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    u32x2_t q;
    q[0] = e4m3x4(quot_signed(f[j][0], r, sc), quot_signed(f[j][1], r, sc),
                  quot_signed(f[j][2], r, sc), quot_signed(f[j][3], r, sc));
    q[1] = e4m3x4(quot_signed(f[j][4], r, sc), quot_signed(f[j][5], r, sc),
                  quot_signed(f[j][6], r, sc), quot_signed(f[j][7], r, sc));
    // Past the row's end the chunk is a copy of its last one (load_row), so
    // its codes go to that chunk's place: same bytes, and no branch.
    const int c = min(lane + 64 * j, nchunk - 1);
    __builtin_nontemporal_store(q, (u32x2_t*)(qr + (uint32_t)c * 8u));
  }
  if (lane == 0) scale_out[row] = act_scale(amax);
}

// Codes of one row's GELU values against a given scale (the per-tensor
// requantisation): lookup in place, then the same conversion and stores as
// gelu_quant_row.
template <int VPL>
FVSR_DEV void gelu_codes_row(u32x4_t (&v)[VPL], const uint16_t* tab, int64_t row, int64_t cols,
                             int nchunk, float r, float sc, uint8_t* codes) {
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v[j][i] = (uint32_t)tab[v[j][i] & 0xffffu] | ((uint32_t)tab[v[j][i] >> 16] << 16);
  const int lane = lane_here();
  uint8_t* qr = codes + row * cols;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    // Packed values only: the unpacked lookups are not kept for this loop.
    asm volatile("" : "+v"(v[j]));
    const u32x2_t q = chunk_codes_fma(v[j], r, sc);
    const int c = min(lane + 64 * j, nchunk - 1);
    __builtin_nontemporal_store(q, (u32x2_t*)(qr + (uint32_t)c * 8u));
  }
}

// Per-tensor GELU requantisation by table: the tensor's amax comes from
// per-block partial maxima of |GELU| (every wave reduces them all: at most
// 1024 floats), then rows as in quant_rows_gelu_table.  Same codes and scale
// as quant_tensor<true, true>, whose GELU is evaluated per element.
template <int VPL>
__global__ __launch_bounds__(kTabWaves * 64) void quant_tensor_gelu_table(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, int64_t ld,
    const float* __restrict__ part, int nparts, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out) {
  __shared__ __attribute__((aligned(16))) uint16_t tab[65536];
  for (int i = threadIdx.x; i < 65536 / 8; i += kTabWaves * 64)
    ((u32x4_t*)tab)[i] = ((const u32x4_t*)kGeluTable)[i];
  const int lane = threadIdx.x & 63;
  float m = 0.0f;
  for (int i = lane; i < nparts; i += 64) m = fmaxf(m, part[i]);
  const float amax = wave_max_abs(m);
  __syncthreads();
  const float s = qscale(amax), r = 1.0f / s, sc = qscale_fin(s);
  if (blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = act_scale(amax);
  const int nchunk = (int)(cols >> 3);
  const int64_t stride = (int64_t)gridDim.x * kTabWaves;
  u32x4_t v[VPL];
  for (int64_t row = first_table_row(); row < rows; row += stride) {
    load_row(v, x, row, ld, nchunk);
    gelu_codes_row<VPL>(v, tab, row, cols, nchunk, r, sc, codes);
  }
}

// Per-workgroup maxima of |GELU(x)| by table (the amax pass of the two-pass
// per-tensor requantisation): part[blockIdx.x] for a persistent grid.
template <int VPL>
__global__ __launch_bounds__(kTabWaves * 64) void amax_gelu_table(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, int64_t ld,
    float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint16_t tab[65536];
  __shared__ float red[kTabWaves];
  for (int i = threadIdx.x; i < 65536 / 8; i += kTabWaves * 64)
    ((u32x4_t*)tab)[i] = ((const u32x4_t*)kGeluTable)[i];
  __syncthreads();
  const int nchunk = (int)(cols >> 3);
  const int64_t stride = (int64_t)gridDim.x * kTabWaves;
  float m = 0.0f;
  u32x4_t v[VPL];
  for (int64_t row = first_table_row(); row < rows; row += stride) {
    load_row(v, x, row, ld, nchunk);  // a repeated chunk changes no maximum
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        m = max3_abs(m, bf2f(tab[v[j][i] & 0xffffu]), bf2f(tab[v[j][i] >> 16]));
  }
  m = wave_max_abs(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = 0.0f;
    for (int w = 0; w < kTabWaves; ++w) b = fmaxf(b, red[w]);
    part[blockIdx.x] = b;
  }
}

template <int VPL>
__global__ __launch_bounds__(kRowTabWaves * 64) void quant_rows_gelu_table(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, int64_t ld,
    uint8_t* __restrict__ codes, float* __restrict__ scale_out) {
  __shared__ __attribute__((aligned(16))) uint16_t tab[65536];
  for (int i = threadIdx.x; i < 65536 / 8; i += kRowTabWaves * 64)
    ((u32x4_t*)tab)[i] = ((const u32x4_t*)kGeluTable)[i];
  __syncthreads();
  const int nchunk = (int)(cols >> 3);
  const int64_t stride = (int64_t)gridDim.x * kRowTabWaves;
  u32x4_t v[VPL];
  for (int64_t row = first_table_row(); row < rows; row += stride) {
    load_row(v, x, row, ld, nchunk);
    gelu_quant_row<VPL>(v, tab, row, cols, nchunk, codes, scale_out);
  }
}

// Row mode, any shape and input type: two passes over the row (the second
// hits L2).  The codes are those of the IEEE quotient v / s.
template <bool GELU>
__global__ __launch_bounds__(kThreads) void quant_rows_generic(
    const void* __restrict__ x, int dt, int64_t rows, int64_t cols, int64_t ld,
    uint8_t* __restrict__ codes, float* __restrict__ scale_out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t xr = row * ld;
  float m = 0.0f;
  for (int64_t c = lane; c < cols; c += 64) m = fmaxf(m, fabsf(load_val<GELU>(x, dt, xr + c)));
  const float amax = wave_max_abs(m);
  const float s = qscale(amax);
  uint8_t* qr = codes + row * cols;
  for (int64_t c = lane; c < cols; c += 64) {
    float q = clamp448(load_val<GELU>(x, dt, xr + c) / s);
    qr[c] = (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(q, 0.0f, 0, false) & 0xff);
  }
  if (lane == 0) scale_out[row] = act_scale(amax);
}

// ---------------------------------------------------------------------------
// Tensor mode.
// ---------------------------------------------------------------------------
FVSR_DEV float block_max(float m, float* red) {
  m = wave_max_abs(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = fmaxf(r, red[w]);
  return r;
}

// Partial |x| maxima: workgroup b covers rows b, b+G, ... (one wave per row).
// VEC: bf16 rows in 16-byte chunks; otherwise element loads of type dt.
template <bool GELU, bool VEC>
__global__ __launch_bounds__(kThreads) void amax_partial(
    const void* __restrict__ x, int dt, int64_t rows, int64_t cols, int64_t ld,
    float* __restrict__ part) {
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63;
  float m = 0.0f;
  for (int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); row < rows;
       row += (int64_t)gridDim.x * kWaves) {
    if (VEC) {
      const uint16_t* xr = (const uint16_t*)x + row * ld;
      for (int64_t c = lane; c < (cols >> 3); c += 64) {
        u32x4_t v = *(const u32x4_t*)(xr + c * 8);
        if (GELU) v = gelu_chunk(v);
        m = fmaxf(m, chunk_absmax(v));
      }
    } else {
      for (int64_t c = lane; c < cols; c += 64)
        m = fmaxf(m, fabsf(load_val<GELU>(x, dt, row * ld + c)));
    }
  }
  m = block_max(m, red);
  if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// Signed max of n floats -> part[blockIdx.x] (maxima of h, which may be negative).
__global__ __launch_bounds__(kThreads) void max_reduce_signed(const float* __restrict__ in,
                                                              int64_t n, float* __restrict__ part) {
  __shared__ float red[kWaves];
  float m = -__builtin_huge_valf();
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    m = fmaxf(m, in[i]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0)
    part[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

FVSR_DEV float reduce_partials(const float* __restrict__ part, int nparts, float* red) {
  float m = 0.0f;
  for (int i = threadIdx.x; i < nparts; i += kThreads) m = fmaxf(m, part[i]);
  return block_max(m, red);
}

// Codes against the tensor's scale (the partial maxima reduced again by every
// workgroup).  VEC: bf16 rows in 16-byte chunks; otherwise element loads of
// type dt and the IEEE quotient.
template <bool GELU, bool VEC>
__global__ __launch_bounds__(kThreads) void quant_tensor(
    const void* __restrict__ x, int dt, int64_t rows, int64_t cols, int64_t ld,
    const float* __restrict__ part, int nparts, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out) {
  __shared__ float red[kWaves];
  const float amax = reduce_partials(part, nparts, red);
  const float s = qscale(amax), r = 1.0f / s;
  if (blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = act_scale(amax);
  const int lane = threadIdx.x & 63;
  for (int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); row < rows;
       row += (int64_t)gridDim.x * kWaves) {
    uint8_t* qr = codes + row * cols;
    if (VEC) {
      const uint16_t* xr = (const uint16_t*)x + row * ld;
      for (int64_t c = lane; c < (cols >> 3); c += 64) {
        u32x4_t v = *(const u32x4_t*)(xr + c * 8);
        if (GELU) v = gelu_chunk(v);
        *(u32x2_t*)(qr + c * 8) = chunk_codes_fma(v, r, qscale_fin(s));
      }
    } else {
      for (int64_t c = lane; c < cols; c += 64) {
        float q = clamp448(load_val<GELU>(x, dt, row * ld + c) / s);
        qr[c] = (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(q, 0.0f, 0, false) & 0xff);
      }
    }
  }
}

// Per-tensor GELU quantisation after a row-max GEMM epilogue.  Step 2: every
// workgroup reduces the partial maxima of h to h_max; if gelu(h_max) exceeds
// the largest |GELU| of a negative input it is the tensor's max|gelu| and the
// workgroup just records it, otherwise it scans its rows (GELU evaluated).
__global__ __launch_bounds__(kThreads) void gelu_amax_from_hmax(
    const uint16_t* __restrict__ h, int64_t rows, int64_t cols, const float* __restrict__ hpart,
    int nh, float* __restrict__ gpart) {
  __shared__ float red[kWaves];
  float hm = -__builtin_huge_valf();
  for (int i = threadIdx.x; i < nh; i += kThreads) hm = fmaxf(hm, hpart[i]);
  hm = wave_max(hm);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = hm;
  __syncthreads();
  hm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float a = gelu_tanh_bf16(hm);
  if (a > FVSR_GELU_NEG_BOUND) {
    if (threadIdx.x == 0) gpart[blockIdx.x] = a;
    return;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  float m = 0.0f;
  for (int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); row < rows;
       row += (int64_t)gridDim.x * kWaves)
    for (int64_t c = lane; c < cols; c += 64) m = fmaxf(m, fabsf(gelu_tanh_bf16(bf2f(h[row * cols + c]))));
  m = block_max(m, red);
  if (threadIdx.x == 0) gpart[blockIdx.x] = m;
}

// ---------------------------------------------------------------------------
// Static weight quantisation (fp8_linear.py:17-22 and its per-channel form).
// ---------------------------------------------------------------------------
// `(w.abs().amax() / FP8_MAX).clamp(min=1e-12).float()` evaluated in the
// weight's type dt: the division by a Python float is amax * fl(1/448) on the
// GPU, rounded to dt; the clamp compares in fp32 against 1e-12 rounded to dt
// (0 in fp16) and keeps a NaN.  For bf16 weights t(amax * fl(1/448)) equals
// t(amax / 448) for every amax (checked exhaustively on the host).
FVSR_DEV float weight_scale(float amax, int dt) {
  const float s = round_to(dt, amax * (1.0f / 448.0f));
  const float lo = round_to(dt, 1e-12f);
  return s < lo ? lo : s;
}

// Code of one weight element: per tensor, w / s is evaluated in the weight's
// type (a 0-dim fp32 scale does not promote it) and rounded to dt before the
// cast; per channel the [N, 1] fp32 scales promote the quotient to fp32.
FVSR_DEV uint8_t weight_code(float w, float s, bool per_channel, int dt) {
  const float v = w / s;
  return e4m3_cast(per_channel ? v : round_to(dt, v));
}

__global__ __launch_bounds__(kThreads) void quant_weight_rows(
    const void* __restrict__ w, int dt, int64_t n, int64_t k, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= n) return;
  float m = 0.0f;
  for (int64_t c = lane; c < k; c += 64) m = fmaxf(m, fabsf(ld_elem(w, dt, row * k + c)));
  const float s = weight_scale(wave_max_abs(m), dt);
  for (int64_t c = lane; c < k; c += 64)
    codes[row * k + c] = weight_code(ld_elem(w, dt, row * k + c), s, true, dt);
  if (lane == 0) scale_out[row] = s;
}

__global__ __launch_bounds__(kThreads) void quant_weight_tensor(
    const void* __restrict__ w, int dt, int64_t n, int64_t k, const float* __restrict__ part,
    int nparts, uint8_t* __restrict__ codes, float* __restrict__ scale_out) {
  __shared__ float red[kWaves];
  const float s = weight_scale(reduce_partials(part, nparts, red), dt);
  if (blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = s;
  const int64_t total = n * k;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kThreads)
    codes[i] = weight_code(ld_elem(w, dt, i), s, false, dt);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
int partial_blocks(int64_t rows) {
  int64_t b = (rows + kWaves - 1) / kWaves;
  return (int)(b < kMaxPartials ? (b > 0 ? b : 1) : kMaxPartials);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool dtype_ok(int dt) { return dt == FVSR_DT_BF16 || dt == FVSR_DT_F16 || dt == FVSR_DT_F32; }

// Compute units of the current device (persistent grids).
int64_t cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    cus = 256;
  return cus;
}

template <bool GELU>
int launch_rows(const uint16_t* x, int64_t rows, int64_t cols, int64_t ld, uint8_t* q,
                float* s, hipStream_t st) {
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves)), block(kThreads);
  const bool vec = (cols % 8 == 0) && (ld % 8 == 0) && aligned16(x) && aligned16(q);
  const int64_t vpl = (cols / 8 + 63) / 64;
  if (GELU && vec && vpl <= 18) {
    const int64_t want = (rows + kRowTabWaves - 1) / kRowTabWaves;
    const int64_t g = want < cu_count() ? want : cu_count();
    hipLaunchKernelGGL((quant_rows_gelu_table<18>), dim3((unsigned)g), dim3(kRowTabWaves * 64), 0,
                       st, x, rows, cols, ld, q, s);
  } else if (vec && vpl <= 3) {
    hipLaunchKernelGGL((quant_rows_vec<3, GELU>), grid, block, 0, st, x, rows, cols, ld, q, s);
  } else if (vec && vpl <= 6) {
    hipLaunchKernelGGL((quant_rows_vec<6, GELU>), grid, block, 0, st, x, rows, cols, ld, q, s);
  } else if (vec && vpl <= 18) {
    hipLaunchKernelGGL((quant_rows_vec<18, GELU>), grid, block, 0, st, x, rows, cols, ld, q, s);
  } else {
    hipLaunchKernelGGL((quant_rows_generic<GELU>), grid, block, 0, st, x, FVSR_DT_BF16, rows,
                       cols, ld, q, s);
  }
  return fvsr_launch_status();
}

// The per-tensor GELU quant pass: by table when rows fit 18 chunks per lane.
void launch_gelu_tensor_codes(const uint16_t* x, int64_t rows, int64_t cols, int64_t ld,
                              const float* part, int P, uint8_t* q, float* s, hipStream_t st) {
  if ((cols / 8 + 63) / 64 <= 18) {
    const int64_t want = (rows + kTabWaves - 1) / kTabWaves;
    const int64_t g = want < cu_count() ? want : cu_count();
    hipLaunchKernelGGL((quant_tensor_gelu_table<18>), dim3((unsigned)g), dim3(kTabWaves * 64), 0,
                       st, x, rows, cols, ld, part, P, q, s);
  } else {
    hipLaunchKernelGGL((quant_tensor<true, true>), dim3(P), dim3(kThreads), 0, st, x,
                       FVSR_DT_BF16, rows, cols, ld, part, P, q, s);
  }
}

// Per-tensor quantisation by element loads of type dt (two launches).
template <bool GELU>
int launch_tensor_scalar(const void* x, int dt, int64_t rows, int64_t cols, int64_t ld,
                         uint8_t* q, float* s, float* ws, hipStream_t st) {
  const int P = partial_blocks(rows);
  hipLaunchKernelGGL((amax_partial<GELU, false>), dim3(P), dim3(kThreads), 0, st, x, dt, rows,
                     cols, ld, ws);
  hipLaunchKernelGGL((quant_tensor<GELU, false>), dim3(P), dim3(kThreads), 0, st, x, dt, rows,
                     cols, ld, ws, P, q, s);
  return fvsr_launch_status();
}

template <bool GELU>
int launch_tensor(const uint16_t* x, int64_t rows, int64_t cols, int64_t ld, uint8_t* q,
                  float* s, float* ws, hipStream_t st) {
  const int P = partial_blocks(rows);
  const bool vec = (cols % 8 == 0) && (ld % 8 == 0) && aligned16(x) && aligned16(q);
  if (vec && GELU && (cols / 8 + 63) / 64 <= 18) {
    // both passes by table; the grid is persistent, one partial per workgroup
    const int64_t want = (rows + kTabWaves - 1) / kTabWaves;
    int64_t g = want < cu_count() ? want : cu_count();
    g = g < P ? g : P;
    hipLaunchKernelGGL((amax_gelu_table<18>), dim3((unsigned)g), dim3(kTabWaves * 64), 0, st, x,
                       rows, cols, ld, ws);
    hipLaunchKernelGGL((quant_tensor_gelu_table<18>), dim3((unsigned)g), dim3(kTabWaves * 64), 0,
                       st, x, rows, cols, ld, ws, (int)g, q, s);
  } else if (vec && GELU) {
    hipLaunchKernelGGL((amax_partial<GELU, true>), dim3(P), dim3(kThreads), 0, st, x,
                       FVSR_DT_BF16, rows, cols, ld, ws);
    launch_gelu_tensor_codes(x, rows, cols, ld, ws, P, q, s, st);
  } else if (vec) {
    hipLaunchKernelGGL((amax_partial<GELU, true>), dim3(P), dim3(kThreads), 0, st, x,
                       FVSR_DT_BF16, rows, cols, ld, ws);
    hipLaunchKernelGGL((quant_tensor<GELU, true>), dim3(P), dim3(kThreads), 0, st, x,
                       FVSR_DT_BF16, rows, cols, ld, ws, P, q, s);
  } else {
    return launch_tensor_scalar<GELU>(x, FVSR_DT_BF16, rows, cols, ld, q, s, ws, st);
  }
  return fvsr_launch_status();
}

}  // namespace

extern "C" int64_t fvsr_quant_workspace_floats(int64_t rows, int64_t cols, int mode) {
  (void)cols;
  return mode == FVSR_SCALE_ROW ? 0 : partial_blocks(rows);
}

extern "C" int fvsr_quant_fp8(const void* x, int64_t rows, int64_t cols, int64_t ld, int mode,
                              int gelu, void* codes, float* scale_out, float* workspace,
                              int64_t workspace_floats, void* stream) {
  if (rows < 0 || cols < 0 || ld < cols || (mode != FVSR_SCALE_TENSOR && mode != FVSR_SCALE_ROW))
    return FVSR_EINVAL;
  if (rows == 0 || cols == 0) return FVSR_OK;
  if (!x || !codes || !scale_out) return FVSR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  uint8_t* qp = (uint8_t*)codes;
  if (mode == FVSR_SCALE_ROW)
    return gelu ? launch_rows<true>(xp, rows, cols, ld, qp, scale_out, st)
                : launch_rows<false>(xp, rows, cols, ld, qp, scale_out, st);
  if (!workspace || workspace_floats < partial_blocks(rows)) return FVSR_EWORKSPACE;
  return gelu ? launch_tensor<true>(xp, rows, cols, ld, qp, scale_out, workspace, st)
              : launch_tensor<false>(xp, rows, cols, ld, qp, scale_out, workspace, st);
}

extern "C" int fvsr_gelu_quant_fp8_tensor(const void* h, int64_t rows, int64_t cols,
                                          const float* hmax_part, int64_t nparts, void* codes,
                                          float* scale_out, float* workspace,
                                          int64_t workspace_floats, void* stream) {
  if (rows < 0 || cols < 0 || nparts <= 0) return FVSR_EINVAL;
  if (rows == 0 || cols == 0) return FVSR_OK;
  if (!h || !codes || !scale_out || !hmax_part) return FVSR_EINVAL;
  const int P = partial_blocks(rows);
  if (!workspace || workspace_floats < 2 * P) return FVSR_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* hp = (const uint16_t*)h;
  uint8_t* qp = (uint8_t*)codes;
  float* hpart = workspace;
  float* gpart = workspace + P;
  hipLaunchKernelGGL(max_reduce_signed, dim3(P), dim3(kThreads), 0, st, hmax_part, rows * nparts,
                     hpart);
  hipLaunchKernelGGL(gelu_amax_from_hmax, dim3(P), dim3(kThreads), 0, st, hp, rows, cols, hpart,
                     P, gpart);
  const bool vec = (cols % 8 == 0) && aligned16(h) && aligned16(codes);
  if (vec)
    launch_gelu_tensor_codes(hp, rows, cols, cols, gpart, P, qp, scale_out, st);
  else
    hipLaunchKernelGGL((quant_tensor<true, false>), dim3(P), dim3(kThreads), 0, st, hp,
                       FVSR_DT_BF16, rows, cols, cols, gpart, P, qp, scale_out);
  return fvsr_launch_status();
}

extern "C" int fvsr_quant_weight_fp8_dt(const void* w, int w_dtype, int64_t n, int64_t k,
                                        int mode, void* codes, float* scale_out,
                                        float* workspace, int64_t workspace_floats,
                                        void* stream) {
  if (n < 0 || k < 0 || (mode != FVSR_SCALE_TENSOR && mode != FVSR_SCALE_ROW) ||
      !dtype_ok(w_dtype))
    return FVSR_EINVAL;
  if (n == 0 || k == 0) return FVSR_OK;
  if (!w || !codes || !scale_out) return FVSR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  uint8_t* qp = (uint8_t*)codes;
  if (mode == FVSR_SCALE_ROW) {
    hipLaunchKernelGGL(quant_weight_rows, dim3((unsigned)((n + kWaves - 1) / kWaves)),
                       dim3(kThreads), 0, st, w, w_dtype, n, k, qp, scale_out);
    return fvsr_launch_status();
  }
  const int P = partial_blocks(n);
  if (!workspace || workspace_floats < P) return FVSR_EWORKSPACE;
  hipLaunchKernelGGL((amax_partial<false, false>), dim3(P), dim3(kThreads), 0, st, w, w_dtype, n,
                     k, k, workspace);
  hipLaunchKernelGGL(quant_weight_tensor, dim3(P), dim3(kThreads), 0, st, w, w_dtype, n, k,
                     workspace, P, qp, scale_out);
  return fvsr_launch_status();
}

extern "C" int fvsr_quant_weight_fp8(const void* w, int64_t n, int64_t k, int mode, void* codes,
                                     float* scale_out, float* workspace, int64_t workspace_floats,
                                     void* stream) {
  return fvsr_quant_weight_fp8_dt(w, FVSR_DT_BF16, n, k, mode, codes, scale_out, workspace,
                                  workspace_floats, stream);
}

extern "C" int fvsr_quant_fp8_dt(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                 int64_t ld, int mode, int gelu, void* codes, float* scale_out,
                                 float* workspace, int64_t workspace_floats, void* stream) {
  if (!dtype_ok(x_dtype)) return FVSR_EINVAL;
  if (x_dtype == FVSR_DT_BF16)
    return fvsr_quant_fp8(x, rows, cols, ld, mode, gelu, codes, scale_out, workspace,
                          workspace_floats, stream);
  if (rows < 0 || cols < 0 || ld < cols || (mode != FVSR_SCALE_TENSOR && mode != FVSR_SCALE_ROW))
    return FVSR_EINVAL;
  if (rows == 0 || cols == 0) return FVSR_OK;
  if (!x || !codes || !scale_out) return FVSR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  uint8_t* qp = (uint8_t*)codes;
  if (mode == FVSR_SCALE_ROW) {
    const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves)), block(kThreads);
    if (gelu)
      hipLaunchKernelGGL((quant_rows_generic<true>), grid, block, 0, st, x, x_dtype, rows, cols,
                         ld, qp, scale_out);
    else
      hipLaunchKernelGGL((quant_rows_generic<false>), grid, block, 0, st, x, x_dtype, rows, cols,
                         ld, qp, scale_out);
    return fvsr_launch_status();
  }
  if (!workspace || workspace_floats < partial_blocks(rows)) return FVSR_EWORKSPACE;
  return gelu ? launch_tensor_scalar<true>(x, x_dtype, rows, cols, ld, qp, scale_out, workspace, st)
              : launch_tensor_scalar<false>(x, x_dtype, rows, cols, ld, qp, scale_out, workspace,
                                            st);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of fvsr_quant_fp8, for callers that cannot allocate
// (code under stream capture, serving loops).  The per-tensor partial maxima
// live in a file-scope device array instead of a caller workspace.  Each GPU
// holds its own copy of the array at its own address, resolved once per device
// by hipGetSymbolAddress with that device current; host code passes only that
// resolved address to kernels, never the array's name (a host-side stand-in).
// Calls that overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
constexpr int kScratchFloats = kMaxPartials;  // 4 KiB per GPU
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on device `dev`.
int scratch_on(int dev, float** out) {
  if (dev < 0 || dev >= kMaxDevices) return FVSR_EUNSUPPORTED;
  float* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      int cur = 0;
      if (hipGetDevice(&cur) != hipSuccess) return FVSR_EHIP;
      if (cur != dev && hipSetDevice(dev) != hipSuccess) return FVSR_EHIP;
      void* addr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (cur != dev && hipSetDevice(cur) != hipSuccess) return FVSR_EHIP;
      if (e != hipSuccess || addr == nullptr) return FVSR_EHIP;
      p = (float*)addr;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FVSR_OK;
}
}  // namespace

extern "C" int fvsr_quant_fp8_noalloc(const void* x, int64_t rows, int64_t cols, int64_t ld,
                                      int mode, int gelu, void* codes, float* scale_out,
                                      void* stream) {
  if (rows < 0 || cols < 0 || ld < cols || (mode != FVSR_SCALE_TENSOR && mode != FVSR_SCALE_ROW))
    return FVSR_EINVAL;
  if (rows == 0 || cols == 0) return FVSR_OK;
  if (!x || !codes || !scale_out) return FVSR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  uint8_t* qp = (uint8_t*)codes;
  if (mode == FVSR_SCALE_ROW)
    return gelu ? launch_rows<true>(xp, rows, cols, ld, qp, scale_out, st)
                : launch_rows<false>(xp, rows, cols, ld, qp, scale_out, st);
  if (partial_blocks(rows) > kScratchFloats) return FVSR_EWORKSPACE;
  int dev = 0;
  if ((st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev)) != hipSuccess) return FVSR_EHIP;
  float* ws = nullptr;
  const int rc = scratch_on(dev, &ws);
  if (rc != FVSR_OK) return rc;
  // every partial the second pass reads is written by the first: nothing to clear
  return gelu ? launch_tensor<true>(xp, rows, cols, ld, qp, scale_out, ws, st)
              : launch_tensor<false>(xp, rows, cols, ld, qp, scale_out, ws, st);
}

extern "C" const char* fvsr_version(void) { return "fvsr 0.1.0 gfx950"; }
