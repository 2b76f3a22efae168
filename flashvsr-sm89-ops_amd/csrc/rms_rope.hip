// RMSNorm over the full hidden dim + interleaved RoPE per head (contract R),
// bandwidth bound.
//
// One wavefront per row.  Each lane holds 8 contiguous elements per chunk, so
// a RoPE pair (2i, 2i+1) is always inside one lane's registers and the partner
// swap costs nothing.  The (cos, sin) table is read in its interleaved
// [L, head_dim/2, 2] fp32 layout — the view_as_real of the complex freqs_cis —
// as two 16-byte loads per chunk.
//
// Products and sums are contracted into fmas only where written out (the
// sum of squares and the rotation), so the results do not depend on the
// compiler's choices.
#pragma clang fp contract(off)
#include "common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

template <int VPL, bool ROPE>
FVSR_DEV void rms_rope_row(const uint16_t* xr, const uint16_t* __restrict__ w,
                           const float* __restrict__ cs_row, uint16_t* outr,
                           int64_t D, int64_t head_dim, float eps, int lane) {
  const int64_t nchunk = D >> 3;
  u32x4_t v[VPL];
  // Unconditional loads (past-the-end chunks read the last chunk again, and
  // are masked out of the sum) so that the row's loads are in flight together.
#pragma unroll
  for (int j = 0; j < VPL; ++j) v[j] = *(const u32x4_t*)(xr + clamp_chunk(lane + 64 * j, nchunk) * 8);
  float sq = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const bool in = lane + 64 * j < nchunk;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = bf_lo(v[j][i]), b = bf_hi(v[j][i]);
      sq = in ? __builtin_fmaf(b, b, __builtin_fmaf(a, a, sq)) : sq;
    }
  }
  // Weights and (cos, sin) for every chunk, loaded before the reduction
  // completes (same clamping).
  u32x4_t wv[VPL];
  f32x4_t cs0[VPL], cs1[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t cc = clamp_chunk(lane + 64 * j, nchunk);
    wv[j] = *(const u32x4_t*)(w + cc * 8);
    if (ROPE) {
      const int64_t i0 = ((cc * 8) % head_dim) >> 1;  // first pair index of this chunk
      cs0[j] = *(const f32x4_t*)(cs_row + 2 * i0);     // c0 s0 c1 s1
      cs1[j] = *(const f32x4_t*)(cs_row + 2 * i0 + 4); // c2 s2 c3 s3
    }
  }
  const float r = rsqrtf(wave_sum(sq) / (float)D + eps);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t c = lane + 64 * j;
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ye = rbf16(bf_lo(v[j][i]) * r) * bf_lo(wv[j][i]);
      const float yo = rbf16(bf_hi(v[j][i]) * r) * bf_hi(wv[j][i]);
      if (ROPE) {
        const float cc = i < 2 ? cs0[j][2 * i] : cs1[j][2 * (i - 2)];
        const float ss = i < 2 ? cs0[j][2 * i + 1] : cs1[j][2 * (i - 2) + 1];
        o[i] = pack_bf16x2(__builtin_fmaf(ye, cc, -(yo * ss)), __builtin_fmaf(ye, ss, yo * cc));
      } else {
        o[i] = pack_bf16x2(ye, yo);
      }
    }
    if (c < nchunk) *(u32x4_t*)(outr + c * 8) = o;
  }
}

template <int VPL, bool ROPE>
__global__ __launch_bounds__(kThreads) void rms_rope_vec(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const float* __restrict__ cs,
    uint16_t* __restrict__ out, int64_t rows, int64_t L, int64_t D, int64_t head_dim, float eps) {
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  rms_rope_row<VPL, ROPE>(x + row * D, w, ROPE ? cs + (row % L) * head_dim : nullptr,
                          out + row * D, D, head_dim, eps, threadIdx.x & 63);
}

// q and k rows in one grid: blockIdx.y selects the tensor.
// Row strides ld_in / ld_out let q and k be column slices of a fused QKV
// projection output and be normalised in place (each wave reads its whole row
// into registers before it writes).
template <int VPL>
__global__ __launch_bounds__(kThreads) void rms_rope_qk_vec(
    const uint16_t* q, const uint16_t* k, const uint16_t* __restrict__ wq,
    const uint16_t* __restrict__ wk, const float* __restrict__ cs, uint16_t* oq, uint16_t* ok,
    int64_t rows, int64_t L, int64_t D, int64_t head_dim, float eps, int64_t ld_in,
    int64_t ld_out) {
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bool isk = blockIdx.y != 0;
  rms_rope_row<VPL, true>((isk ? k : q) + row * ld_in, isk ? wk : wq, cs + (row % L) * head_dim,
                          (isk ? ok : oq) + row * ld_out, D, head_dim, eps, threadIdx.x & 63);
}

// q (in place or to out_q, same rows), k and v to rows kv_rows[r] of out_k and
// out_v (the window-ordered K/V buffer of the attention): blockIdx.y picks the
// tensor; v is a plain row copy.  Rows whose target is outside [0, kv_cap)
// are not written.
template <int VPL>
__global__ __launch_bounds__(kThreads) void rms_rope_qkv_rows_vec(
    const uint16_t* q, const uint16_t* k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ wq, const uint16_t* __restrict__ wk,
    const float* __restrict__ cs, uint16_t* oq, uint16_t* __restrict__ ok,
    uint16_t* __restrict__ ov, const int32_t* __restrict__ kv_rows, int64_t kv_cap,
    int64_t rows, int64_t L, int64_t D, int64_t head_dim, float eps, int64_t ld_in,
    int64_t ld_out, int64_t ld_kv) {
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  if (blockIdx.y == 0) {
    rms_rope_row<VPL, true>(q + row * ld_in, wq, cs + (row % L) * head_dim, oq + row * ld_out, D,
                            head_dim, eps, lane);
    return;
  }
  const int64_t dst = kv_rows[row];
  if (dst < 0 || dst >= kv_cap) return;
  if (blockIdx.y == 1) {
    rms_rope_row<VPL, true>(k + row * ld_in, wk, cs + (row % L) * head_dim, ok + dst * ld_kv, D,
                            head_dim, eps, lane);
    return;
  }
  const int64_t nchunk = D >> 3;
  const uint16_t* src = v + row * ld_in;
  uint16_t* out = ov + dst * ld_kv;
  u32x4_t t[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) t[j] = *(const u32x4_t*)(src + clamp_chunk(lane + 64 * j, nchunk) * 8);
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (lane + 64 * j < nchunk) *(u32x4_t*)(out + (lane + 64 * j) * 8) = t[j];
}

// Any shape and input types (x and w of types xt, wt; out of type xt): scalar
// loads, partner element read directly.  Each lane sums the squares of its
// 8-element chunks in order (then the last D % 8 elements), as rms_rope_row
// does, so rows of bf16 values give that kernel's results bit for bit.
__global__ __launch_bounds__(kThreads) void rms_rope_generic(
    const void* __restrict__ x, int xt, const void* __restrict__ w, int wt,
    const float* __restrict__ cs, void* __restrict__ out, int64_t rows, int64_t L, int64_t D,
    int64_t head_dim, float eps, int rope) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t xr = row * D;
  float sq = 0.0f;
  for (int64_t c = lane; c < (D >> 3); c += 64) {
    for (int e = 0; e < 8; ++e) {
      const float a = ld_elem(x, xt, xr + c * 8 + e);
      sq = __builtin_fmaf(a, a, sq);
    }
  }
  for (int64_t d = (D & ~(int64_t)7) + lane; d < D; d += 64) {
    const float a = ld_elem(x, xt, xr + d);
    sq = __builtin_fmaf(a, a, sq);
  }
  const float r = rsqrtf(wave_sum(sq) / (float)D + eps);
  const int64_t s = row % L;
  for (int64_t d = lane; d < D; d += 64) {
    const float y = rbf16(ld_elem(x, xt, xr + d) * r) * ld_elem(w, wt, d);
    float o = y;
    if (rope) {
      const int64_t dp = d ^ 1;
      const float yp = rbf16(ld_elem(x, xt, xr + dp) * r) * ld_elem(w, wt, dp);
      const int64_t i = (d % head_dim) >> 1;
      const float cc = cs[(s * (head_dim >> 1) + i) * 2], ss = cs[(s * (head_dim >> 1) + i) * 2 + 1];
      // the same expressions as the vector kernel (ye, yo = even, odd)
      o = (d & 1) ? __builtin_fmaf(yp, ss, y * cc) : __builtin_fmaf(y, cc, -(yp * ss));
    }
    st_elem(out, xt, xr + d, round_bf16(o));
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool dtype_ok(int dt) { return dt == FVSR_DT_BF16 || dt == FVSR_DT_F16 || dt == FVSR_DT_F32; }

}  // namespace

extern "C" int fvsr_rms_rope(const void* x, const void* weight, const float* cs, void* out,
                             int64_t B, int64_t L, int64_t D, int64_t head_dim, float eps,
                             int rope, void* stream) {
  if (B < 0 || L < 0 || D <= 0) return FVSR_EINVAL;
  if (rope && (head_dim <= 0 || head_dim % 2 || D % head_dim || !cs)) return FVSR_EINVAL;
  const int64_t rows = B * L;
  if (rows == 0) return FVSR_OK;
  if (!x || !weight || !out) return FVSR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves)), block(kThreads);
  const uint16_t *xp = (const uint16_t*)x, *wp = (const uint16_t*)weight;
  uint16_t* op = (uint16_t*)out;
  const bool vec = D % 8 == 0 && D <= 512 * 3 && aligned16(x) && aligned16(weight) &&
                   aligned16(out) && (!rope || (head_dim % 8 == 0 && aligned16(cs)));
  if (vec && rope)
    hipLaunchKernelGGL((rms_rope_vec<3, true>), grid, block, 0, st, xp, wp, cs, op, rows, L, D,
                       head_dim, eps);
  else if (vec)
    hipLaunchKernelGGL((rms_rope_vec<3, false>), grid, block, 0, st, xp, wp, cs, op, rows, L, D,
                       head_dim > 0 ? head_dim : D, eps);
  else
    hipLaunchKernelGGL(rms_rope_generic, grid, block, 0, st, x, FVSR_DT_BF16, weight,
                       FVSR_DT_BF16, cs, out, rows, L, D, head_dim > 0 ? head_dim : D, eps, rope);
  return fvsr_launch_status();
}

extern "C" int fvsr_rms_rope_dt(const void* x, int x_dtype, const void* weight, int weight_dtype,
                                const float* cs, void* out, int64_t B, int64_t L, int64_t D,
                                int64_t head_dim, float eps, int rope, void* stream) {
  if (!dtype_ok(x_dtype) || !dtype_ok(weight_dtype)) return FVSR_EINVAL;
  if (x_dtype == FVSR_DT_BF16 && weight_dtype == FVSR_DT_BF16)
    return fvsr_rms_rope(x, weight, cs, out, B, L, D, head_dim, eps, rope, stream);
  if (B < 0 || L < 0 || D <= 0) return FVSR_EINVAL;
  if (rope && (head_dim <= 0 || head_dim % 2 || D % head_dim || !cs)) return FVSR_EINVAL;
  const int64_t rows = B * L;
  if (rows == 0) return FVSR_OK;
  if (!x || !weight || !out) return FVSR_EINVAL;
  hipLaunchKernelGGL(rms_rope_generic, dim3((unsigned)((rows + kWaves - 1) / kWaves)),
                     dim3(kThreads), 0, (hipStream_t)stream, x, x_dtype, weight, weight_dtype, cs,
                     out, rows, L, D, head_dim > 0 ? head_dim : D, eps, rope);
  return fvsr_launch_status();
}

extern "C" int fvsr_rms_rope_qk(const void* q, const void* k, const void* wq, const void* wk,
                                const float* cs, void* out_q, void* out_k, int64_t B, int64_t L,
                                int64_t D, int64_t head_dim, float eps, int64_t ld_in,
                                int64_t ld_out, void* stream) {
  if (B < 0 || L < 0 || D <= 0 || head_dim <= 0 || head_dim % 8 || D % head_dim) return FVSR_EINVAL;
  if (ld_in < D || ld_out < D) return FVSR_EINVAL;
  const int64_t rows = B * L;
  if (rows == 0) return FVSR_OK;
  if (!q || !k || !wq || !wk || !cs || !out_q || !out_k) return FVSR_EINVAL;
  const bool vec = D % 8 == 0 && D <= 512 * 3 && ld_in % 8 == 0 && ld_out % 8 == 0 &&
                   aligned16(q) && aligned16(k) && aligned16(wq) && aligned16(wk) &&
                   aligned16(cs) && aligned16(out_q) && aligned16(out_k);
  if (!vec) return FVSR_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL((rms_rope_qk_vec<3>), dim3((unsigned)((rows + kWaves - 1) / kWaves), 2),
                     dim3(kThreads), 0, st, (const uint16_t*)q, (const uint16_t*)k,
                     (const uint16_t*)wq, (const uint16_t*)wk, cs, (uint16_t*)out_q,
                     (uint16_t*)out_k, rows, L, D, head_dim, eps, ld_in, ld_out);
  return fvsr_launch_status();
}

extern "C" int fvsr_rms_rope_qkv_rows(const void* q, const void* k, const void* v, const void* wq,
                                      const void* wk, const float* cs, void* out_q, void* out_k,
                                      void* out_v, const int32_t* kv_rows, int64_t kv_cap,
                                      int64_t B, int64_t L, int64_t D, int64_t head_dim,
                                      float eps, int64_t ld_in, int64_t ld_out, int64_t ld_kv,
                                      void* stream) {
  if (B < 0 || L < 0 || D <= 0 || head_dim <= 0 || head_dim % 8 || D % head_dim) return FVSR_EINVAL;
  if (ld_in < D || ld_out < D || ld_kv < D || kv_cap < 0) return FVSR_EINVAL;
  const int64_t rows = B * L;
  if (rows == 0) return FVSR_OK;
  if (!q || !k || !v || !wq || !wk || !cs || !out_q || !out_k || !out_v || !kv_rows)
    return FVSR_EINVAL;
  const bool vec = D % 8 == 0 && D <= 512 * 3 && ld_in % 8 == 0 && ld_out % 8 == 0 &&
                   ld_kv % 8 == 0 && aligned16(q) && aligned16(k) && aligned16(v) &&
                   aligned16(wq) && aligned16(wk) && aligned16(cs) && aligned16(out_q) &&
                   aligned16(out_k) && aligned16(out_v);
  if (!vec) return FVSR_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL((rms_rope_qkv_rows_vec<3>), dim3((unsigned)((rows + kWaves - 1) / kWaves), 3),
                     dim3(kThreads), 0, st, (const uint16_t*)q, (const uint16_t*)k,
                     (const uint16_t*)v, (const uint16_t*)wq, (const uint16_t*)wk, cs,
                     (uint16_t*)out_q, (uint16_t*)out_k, (uint16_t*)out_v, kv_rows, kv_cap, rows,
                     L, D, head_dim, eps, ld_in, ld_out, ld_kv);
  return fvsr_launch_status();
}
