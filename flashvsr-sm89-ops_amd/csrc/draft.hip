// Draft block mask of the sparse self-attention on the device, reference
// draft_block_mask (flashvsr_sm89_ops/lcsa/reference.py:37-64) on bf16 q/k with
// the rounding torch applies to bf16 tensors at every stage:
//   avg[n]  = bf16(fp32(sum of the 128 tokens of block n) * 2^-7)   (torch.mean)
//   raw     = bf16(fp32(avg_q[l][h] . avg_k[m][h]))                 (einsum)
//   score   = bf16(raw * fp32(1 / fp32(sqrt(D))))                   (/ math.sqrt(D))
//             or -inf outside local[l % sq][m % sk]                 (+ bias)
//   attn    = bf16(fp32(exp(score - max)) / fp32(sum of those))     (softmax)
//   per (head, query time row t): thr = the (topk+1)-th largest attn over the
//   time row's query blocks x all key blocks (torch.topk order: NaN largest);
//   keep = attn > thr.
// Sums are taken in fp64, where they are exact for bf16 data of any realistic
// range, then rounded once: the results do not depend on summation order.
// Four launches (pool, scores+softmax, threshold, index), no host synchronisation.
#include "common.h"

namespace {

constexpr int kBlk = 128;
constexpr int kThreads = 256;
constexpr uint32_t kNaN16 = 0x7fc0u;

// fp32 -> bf16 bits, round to nearest even, NaN -> 0x7fc0 (torch's convention).
FVSR_DEV uint32_t bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return kNaN16;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
FVSR_DEV float bf16_val(float f) { return __uint_as_float(bf16_bits(f) << 16); }

FVSR_DEV double wave_sum_f64(double v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// avg[n][c] for the NQ query blocks (blockIdx.x < NQ) and the NK key blocks
// (the rest): token j of block n is row map[n*128 + j] (n*128 + j without a
// map), rows ts elements apart.  A workgroup covers 512 channels of one block:
// lane g owns 8 channels, wave w adds tokens 16w..16w+15 in four batches of 4
// (each batch's loads issued before its first add), and the eight partial
// fp64 sums meet in LDS.  The (NQ + NK) * ceil(C/512) workgroups fit the GPU
// in one round at the C5 shape.  Measured at the C5 geometry (whole draft):
// 4 waves x 2 batches of 16: 52.2 us; 8 x 4 of 4: 47.2; 8 x 2 of 8: 48.1;
// 8 x 1 of 16: 54.3; 16 waves: 54.5-55.9.
constexpr int kPoolWaves = 8;
constexpr int kPoolBatch = 4;

__global__ __launch_bounds__(kPoolWaves * 64) void pool_kernel(
    const uint16_t* __restrict__ q, int64_t qts, const int32_t* __restrict__ qmap,
    const uint16_t* __restrict__ k, int64_t kts, const int32_t* __restrict__ kmap, int64_t NQ,
    int64_t C, uint16_t* __restrict__ avg) {
  __shared__ double part[kPoolWaves - 1][8][64];
  // The channel slices of one block are neighbours in dispatch order.
  const int64_t ny = (C + 511) / 512;
  const int64_t blk = blockIdx.x / ny, y = blockIdx.x % ny;
  const bool is_q = blk < NQ;
  const int64_t n = is_q ? blk : blk - NQ;
  const uint16_t* x = is_q ? q : k;
  const int64_t ts = is_q ? qts : kts;
  const int32_t* map = is_q ? qmap : kmap;
  const int g = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c0 = (y * 64 + g) * 8;
  const bool active = c0 < C;
  double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (active) {
#pragma unroll 1
    for (int b = 0; b < kBlk / kPoolWaves / kPoolBatch; ++b) {
      u32x4_t v[kPoolBatch];
      const int64_t p0 = n * kBlk + (w * (kBlk / kPoolWaves) + b * kPoolBatch);
#pragma unroll
      for (int j = 0; j < kPoolBatch; ++j) {
        const int64_t tok = map ? (int64_t)map[p0 + j] : p0 + j;
        v[j] = *(const u32x4_t*)(x + tok * ts + c0);
      }
#pragma unroll
      for (int j = 0; j < kPoolBatch; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] += (double)bf_lo(v[j][i]);
          acc[2 * i + 1] += (double)bf_hi(v[j][i]);
        }
      }
    }
  }
  if (w > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) part[w - 1][e][g] = acc[e];
  }
  __syncthreads();
  if (w == 0 && active) {
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t h2[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int e = 2 * i + b;
        double s = acc[e];
#pragma unroll
        for (int u = 0; u < kPoolWaves - 1; ++u) s += part[u][e][g];
        h2[b] = bf16_bits((float)s * 0.0078125f);
      }
      o[i] = h2[0] | (h2[1] << 16);
    }
    const int64_t row = is_q ? n : NQ + n;
    *(u32x4_t*)(avg + row * C + c0) = u32x4_t{o[0], o[1], o[2], o[3]};
  }
}

// Four query blocks l0..l0+3 of one head h per workgroup.  Pass 1: thread m
// (m = tid, tid+256, ...) forms the four masked scores of key block m, reading
// each avg_k value once for the four dot products (query values as fp64 in
// LDS, four 16-byte key loads kept in flight); pass 2: wave w takes row l0+w,
// its maximum, exponentials and sum by wave reductions, and writes the
// softmax as bf16 bits to attn[h][l0+w][:] and, for the threshold search, the
// row's histogram of nonzero patterns by high byte to hist[h][l0+w][0..127]
// (attn <= 1 or the NaN 0x7fc0, so the high byte is below 128).
constexpr int kRowsPerScoreWg = 4;

__global__ __launch_bounds__(kThreads) void score_softmax_kernel(
    const uint16_t* __restrict__ avg_q, const uint16_t* __restrict__ avg_k, int64_t H, int64_t D,
    int64_t NQ, int64_t NK, const uint8_t* __restrict__ local, int64_t sq, int64_t sk,
    float inv_sqrt_d, uint16_t* __restrict__ attn, uint16_t* __restrict__ hist) {
  extern __shared__ double smem_d[];  // query values [4][D] (fp64), scores [4][NK] (fp32)
  __shared__ int rh[kRowsPerScoreWg][128];
  constexpr int R = kRowsPerScoreWg;
  const int64_t groups = (NQ + R - 1) / R;
  const int64_t h = blockIdx.x / groups, l0 = (blockIdx.x % groups) * R;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t C = H * D;
  double* aq = smem_d;
  float* srow = (float*)(smem_d + R * D);
  for (int64_t i = tid; i < R * D; i += kThreads) {
    const int64_t l = l0 + i / D;
    aq[i] = l < NQ ? (double)bf2f(avg_q[l * C + h * D + i % D]) : 0.0;
  }
  for (int i = tid; i < R * 128; i += kThreads) rh[i / 128][i % 128] = 0;
  __syncthreads();
  const int64_t nch = D / 8;
  for (int64_t m = tid; m < NK; m += kThreads) {
    const u32x4_t* ak = (const u32x4_t*)(avg_k + m * C + h * D);
    double p[R] = {};
    auto chunk = [&](const u32x4_t& v, int64_t c) {
      const double* a = aq + 8 * c;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const double k0 = (double)bf_lo(v[i]), k1 = (double)bf_hi(v[i]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          p[r] = __builtin_fma(a[r * D + 2 * i], k0, p[r]);
          p[r] = __builtin_fma(a[r * D + 2 * i + 1], k1, p[r]);
        }
      }
    };
    const u32x4_t zero = {0u, 0u, 0u, 0u};
    u32x4_t v0 = ak[0], v1 = nch > 1 ? ak[1] : zero, v2 = nch > 2 ? ak[2] : zero,
            v3 = nch > 3 ? ak[3] : zero;
#pragma unroll 1
    for (int64_t c = 0; c < nch; c += 4) {
      chunk(v0, c);
      if (c + 4 < nch) v0 = ak[c + 4];
      if (c + 1 < nch) chunk(v1, c + 1);
      if (c + 5 < nch) v1 = ak[c + 5];
      if (c + 2 < nch) chunk(v2, c + 2);
      if (c + 6 < nch) v2 = ak[c + 6];
      if (c + 3 < nch) chunk(v3, c + 3);
      if (c + 7 < nch) v3 = ak[c + 7];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bool allowed = local[((l0 + r) % sq) * sk + m % sk] != 0;
      srow[r * NK + m] =
          allowed ? bf16_val(bf16_val((float)p[r]) * inv_sqrt_d) : -__builtin_huge_valf();
    }
  }
  __syncthreads();
  const int64_t l = l0 + wave;
  if (l < NQ) {
    float* row = srow + wave * NK;
    float mx = -__builtin_huge_valf();
    for (int64_t m = lane; m < NK; m += 64) mx = fmaxf(mx, row[m]);
    mx = wave_max(mx);
    double sum = 0.0;
    for (int64_t m = lane; m < NK; m += 64) {
      const float e = (float)exp((double)(row[m] - mx));
      row[m] = e;
      sum += (double)e;
    }
    const float tot = (float)wave_sum_f64(sum);
    uint16_t* arow = attn + (h * NQ + l) * NK;
    for (int64_t m = lane; m < NK; m += 64) {
      const uint32_t b = bf16_bits(row[m] / tot);
      arow[m] = (uint16_t)b;
      if (b != 0u) atomicAdd(&rh[wave][b >> 8], 1);
    }
  }
  __syncthreads();
  if (l < NQ) {
    uint16_t* hrow = hist + (h * NQ + l) * 128;
    hrow[lane] = (uint16_t)rh[wave][lane];
    hrow[lane + 64] = (uint16_t)rh[wave][lane + 64];
  }
}

// Of the 256 bins hist[0..255] (in LDS), the largest b with sum(hist[b..255])
// >= r, and r minus sum(hist[b+1..255]); b = -1 if the total is below r.  Run
// by one whole wave; every lane returns the answer.
FVSR_DEV int2 find_bin(const int* hist, int r) {
  const int lane = threadIdx.x & 63;
  int c[4], lsum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = hist[lane * 4 + i];
    lsum += c[i];
  }
  int suf = lsum;  // becomes the sum over lanes >= lane
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_down(suf, o, 64);
    if (lane + o < 64) suf += t;
  }
  const uint64_t ok = __ballot(suf >= r);
  if (!ok) return make_int2(-1, r);
  const int top = 63 - __clzll(ok);
  int bin = 0, rest = 0;
  if (lane == top) {
    int above = suf - lsum;  // bins of higher lanes
    int b = 3;
    while (above + c[b] < r) above += c[b--];
    bin = lane * 4 + b;
    rest = r - above;
  }
  return make_int2(__shfl(bin, top, 64), __shfl(rest, top, 64));
}

// One (head, query time row) per workgroup: the threshold pattern of the
// joint top-k over the slab attn[h][t*S .. t*S+S)[:] (S = NQ / q_temporal,
// n = S*NK values), the (k+1)-th largest pattern with k = min(topk, n - 1).
// attn is non-negative or the NaN 0x7fc0, so patterns order like values with
// NaN largest, as torch.topk orders them.  Zeros (the masked blocks) are left
// out of the histograms: if fewer than k+1 values are nonzero the threshold is
// 0.  Otherwise the rows' high-byte histograms give the threshold's high byte
// and its rank r2 among the values sharing it; one pass over the slab then
// builds the low-byte histogram of those values in LDS.
constexpr int kSelPer = 16;

__global__ __launch_bounds__(kThreads) void threshold_kernel(const uint16_t* __restrict__ attn,
                                                             const uint16_t* __restrict__ hist,
                                                             int64_t NQ, int64_t NK,
                                                             int64_t q_temporal, int64_t topk,
                                                             uint32_t* __restrict__ thr) {
  __shared__ int bins[256];
  __shared__ int upper[128];
  __shared__ int2 pick;
  const int64_t h = blockIdx.x / q_temporal, t = blockIdx.x % q_temporal;
  const int64_t S = NQ / q_temporal, n = S * NK;
  const int tid = threadIdx.x;
  const int r = (int)((topk < n - 1 ? topk : n - 1) + 1);

  // High-byte totals: thread tid sums bin tid % 128 over rows of parity tid / 128.
  const uint16_t* hs = hist + (h * NQ + t * S) * 128;
  int c = 0;
  for (int64_t r0 = tid >> 7; r0 < S; r0 += 16) {
    uint32_t x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = r0 + 2 * u < S ? hs[(r0 + 2 * u) * 128 + (tid & 127)] : 0u;
#pragma unroll
    for (int u = 0; u < 8; ++u) c += (int)x[u];
  }
  if (tid >= 128) upper[tid - 128] = c;
  __syncthreads();
  if (tid < 128) bins[tid] = c + upper[tid];
  else bins[tid] = 0;
  __syncthreads();
  if (tid < 64) {
    const int2 f = find_bin(bins, r);
    if (tid == 0) pick = f;
  }
  __syncthreads();
  const int hb = pick.x, r2 = pick.y;
  if (hb < 0) {  // fewer than k+1 nonzero values: the threshold is 0
    if (tid == 0) thr[blockIdx.x] = 0u;
    return;
  }
  bins[tid] = 0;
  __syncthreads();
  const uint16_t* vals = attn + (h * NQ + t * S) * NK;
  for (int64_t base = 0; base < n; base += kSelPer * kThreads) {
    uint32_t v[kSelPer];
#pragma unroll
    for (int i = 0; i < kSelPer; ++i) {
      const int64_t idx = base + i * kThreads + tid;
      v[i] = idx < n ? (uint32_t)vals[idx] : 0u;
    }
#pragma unroll
    for (int i = 0; i < kSelPer; ++i)
      if (v[i] != 0u && (int)(v[i] >> 8) == hb) atomicAdd(&bins[v[i] & 0xff], 1);
  }
  __syncthreads();
  if (tid < 64) {
    const int2 f = find_bin(bins, r2);
    if (tid == 0) thr[blockIdx.x] = ((uint32_t)hb << 8) | (uint32_t)f.x;
  }
}

// One row (h, l) per wave: keep = attn > thr (as floats, so the NaN threshold
// keeps nothing) and/or the row's kept key blocks ascending in sel, count in cnt.
__global__ __launch_bounds__(kThreads) void index_kernel(const uint16_t* __restrict__ attn,
                                                         const uint32_t* __restrict__ thr,
                                                         int64_t rows, int64_t NQ, int64_t NK,
                                                         int64_t q_temporal,
                                                         uint8_t* __restrict__ keep,
                                                         int32_t* __restrict__ sel,
                                                         int32_t* __restrict__ cnt) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t h = row / NQ, l = row % NQ, S = NQ / q_temporal;
  const float th = bf2f((uint16_t)thr[h * q_temporal + l / S]);
  const uint16_t* ar = attn + row * NK;
  int base = 0;
  for (int64_t c0 = 0; c0 < NK; c0 += 8 * 64) {
    uint32_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t m = c0 + u * 64 + lane;
      v[u] = m < NK ? (uint32_t)ar[m] : 0u;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t m = c0 + u * 64 + lane;
      const bool f = m < NK && bf2f((uint16_t)v[u]) > th;
      if (keep && m < NK) keep[row * NK + m] = f ? 1 : 0;
      if (sel) {
        const uint64_t bal = __ballot(f);
        if (f) sel[row * NK + base + __popcll(bal & ((1ull << lane) - 1ull))] = (int32_t)m;
        base += __popcll(bal);
      }
    }
  }
  if (sel && lane == 0) cnt[row] = base;
}

constexpr int64_t align64(int64_t n) { return (n + 63) & ~(int64_t)63; }

}  // namespace

extern "C" int64_t fvsr_draft_workspace_floats(int64_t H, int64_t D, int64_t NQ, int64_t NK) {
  if (H <= 0 || D <= 0 || NQ < 0 || NK < 0) return 0;
  // In 16-bit units, each region 128-byte aligned: bf16 avg_q [NQ, H*D] and
  // avg_k [NK, H*D], bf16 attn [H, NQ, NK], uint16 hist [H, NQ, 128] and the
  // uint32 thresholds [H * q_temporal] (at most H * NQ); + 256 bytes of slack.
  const int64_t units = align64((NQ + NK) * H * D) + align64(H * NQ * NK) +
                        align64(H * NQ * 128) + align64(2 * H * NQ);
  return units / 2 + 64;
}

extern "C" int fvsr_draft_block_mask(const void* q, int64_t q_tok_stride, const int32_t* q_map,
                                     const void* k, int64_t k_tok_stride, const int32_t* k_map,
                                     int64_t H, int64_t D, int64_t NQ, int64_t NK,
                                     int64_t q_temporal, const uint8_t* local, int64_t sq,
                                     int64_t sk, int64_t topk, uint8_t* keep, int32_t* sel,
                                     int32_t* cnt, float* workspace, int64_t workspace_floats,
                                     void* stream) {
  if (H <= 0 || D <= 0 || NQ < 0 || NK < 0 || q_temporal <= 0 || sq <= 0 || sk <= 0 || topk < 0)
    return FVSR_EINVAL;
  if (NQ == 0) return FVSR_OK;
  if (NK == 0 || !q || !k || !local || !workspace || (!keep && !sel) || (!sel != !cnt))
    return FVSR_EINVAL;
  if (NQ % q_temporal || NQ % sq || NK % sk) return FVSR_EINVAL;
  if (D % 8 || q_tok_stride % 8 || k_tok_stride % 8 || ((uintptr_t)q & 15) || ((uintptr_t)k & 15) ||
      ((uintptr_t)workspace & 15))
    return FVSR_EUNSUPPORTED;
  if (workspace_floats < fvsr_draft_workspace_floats(H, D, NQ, NK)) return FVSR_EWORKSPACE;
  // LDS holds 4 * D doubles and 4 * NK floats (at most 62 KB).
  if (2 * D + NK > 3968 || (NQ / q_temporal) * NK > 0x7fffffff || H * NQ > 0x7fffffff ||
      (NQ + NK) * ((H * D + 511) / 512) > 0x7fffffff)
    return FVSR_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int64_t C = H * D;
  uint16_t* avg = (uint16_t*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  uint16_t* attn = avg + align64((NQ + NK) * C);
  hipLaunchKernelGGL(pool_kernel, dim3((unsigned)((NQ + NK) * ((C + 511) / 512))),
                     dim3(kPoolWaves * 64), 0, st, (const uint16_t*)q, q_tok_stride, q_map,
                     (const uint16_t*)k, k_tok_stride, k_map, NQ, C, avg);
  const float inv_sqrt_d = 1.0f / (float)sqrt((double)D);
  uint16_t* hist = attn + align64(H * NQ * NK);
  uint32_t* thr = (uint32_t*)(hist + align64(H * NQ * 128));
  const int64_t groups = (NQ + kRowsPerScoreWg - 1) / kRowsPerScoreWg;
  hipLaunchKernelGGL(score_softmax_kernel, dim3((unsigned)(H * groups)), dim3(kThreads),
                     kRowsPerScoreWg * (D * sizeof(double) + NK * sizeof(float)), st, avg,
                     avg + NQ * C, H, D, NQ, NK, local, sq, sk, inv_sqrt_d, attn, hist);
  hipLaunchKernelGGL(threshold_kernel, dim3((unsigned)(H * q_temporal)), dim3(kThreads), 0, st,
                     attn, hist, NQ, NK, q_temporal, topk, thr);
  const int64_t rows = H * NQ;
  hipLaunchKernelGGL(index_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(kThreads), 0, st, attn,
                     thr, rows, NQ, NK, q_temporal, keep, sel, cnt);
  return fvsr_launch_status();
}
