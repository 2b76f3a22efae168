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
// Three launches (pool, scores+softmax, select), no host synchronisation.
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
// lane g owns 8 channels, wave w adds tokens 32w..32w+31, and the four partial
// fp64 sums meet in LDS.
__global__ __launch_bounds__(kThreads) void pool_kernel(const uint16_t* __restrict__ q, int64_t qts,
                                                        const int32_t* __restrict__ qmap,
                                                        const uint16_t* __restrict__ k, int64_t kts,
                                                        const int32_t* __restrict__ kmap, int64_t NQ,
                                                        int64_t C, uint16_t* __restrict__ avg) {
  __shared__ double part[3][8][64];
  const bool is_q = blockIdx.x < NQ;
  const int64_t n = is_q ? (int64_t)blockIdx.x : (int64_t)blockIdx.x - NQ;
  const uint16_t* x = is_q ? q : k;
  const int64_t ts = is_q ? qts : kts;
  const int32_t* map = is_q ? qmap : kmap;
  const int g = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c0 = ((int64_t)blockIdx.y * 64 + g) * 8;
  const bool active = c0 < C;
  double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (active) {
#pragma unroll 8
    for (int j = w * 32; j < w * 32 + 32; ++j) {
      const int64_t tok = map ? (int64_t)map[n * kBlk + j] : n * kBlk + j;
      const u32x4_t v = *(const u32x4_t*)(x + tok * ts + c0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += (double)bf_lo(v[i]);
        acc[2 * i + 1] += (double)bf_hi(v[i]);
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
        const double s = acc[e] + part[0][e][g] + part[1][e][g] + part[2][e][g];
        h2[b] = bf16_bits((float)s * 0.0078125f);
      }
      o[i] = h2[0] | (h2[1] << 16);
    }
    const int64_t row = is_q ? n : NQ + n;
    *(u32x4_t*)(avg + row * C + c0) = u32x4_t{o[0], o[1], o[2], o[3]};
  }
}

// One (head h, query block l) per workgroup: the NK masked scores, then their
// softmax, written as bf16 bits to attn[h][l][:].  A thread owns key blocks
// m = tid, tid+256, ... and keeps its scores in LDS between the passes.
__global__ __launch_bounds__(kThreads) void score_softmax_kernel(
    const uint16_t* __restrict__ avg_q, const uint16_t* __restrict__ avg_k, int64_t H, int64_t D,
    int64_t NQ, int64_t NK, const uint8_t* __restrict__ local, int64_t sq, int64_t sk,
    float inv_sqrt_d, uint16_t* __restrict__ attn) {
  extern __shared__ float smem[];  // D query values, NK scores
  __shared__ float redf[4];
  __shared__ double redd[4];
  float* aq = smem;
  float* srow = smem + D;
  const int64_t h = blockIdx.x / NQ, l = blockIdx.x % NQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t C = H * D;
  for (int64_t d = tid; d < D; d += kThreads) aq[d] = bf2f(avg_q[l * C + h * D + d]);
  __syncthreads();
  const uint8_t* lrow = local + (l % sq) * sk;
  float mx = -__builtin_huge_valf();
  for (int64_t m = tid; m < NK; m += kThreads) {
    const uint16_t* ak = avg_k + m * C + h * D;
    double p = 0.0;
    for (int64_t d0 = 0; d0 < D; d0 += 8) {
      const u32x4_t v = *(const u32x4_t*)(ak + d0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p = __builtin_fma((double)aq[d0 + 2 * i], (double)bf_lo(v[i]), p);
        p = __builtin_fma((double)aq[d0 + 2 * i + 1], (double)bf_hi(v[i]), p);
      }
    }
    float s = bf16_val(bf16_val((float)p) * inv_sqrt_d);
    if (!lrow[m % sk]) s = -__builtin_huge_valf();
    srow[m] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  if (lane == 0) redf[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
  double sum = 0.0;
  for (int64_t m = tid; m < NK; m += kThreads) {
    const float e = (float)exp((double)(srow[m] - mx));
    srow[m] = e;
    sum += (double)e;
  }
  sum = wave_sum_f64(sum);
  if (lane == 0) redd[wave] = sum;
  __syncthreads();
  const float tot = (float)(redd[0] + redd[1] + redd[2] + redd[3]);
  uint16_t* arow = attn + (h * NQ + l) * NK;
  for (int64_t m = tid; m < NK; m += kThreads) arow[m] = (uint16_t)bf16_bits(srow[m] / tot);
}

// Of the 256 bins hist[0..255], the largest b with sum(hist[b..255]) >= r,
// and r minus sum(hist[b+1..255]).  Run by wave 0; the answer goes to out[0..1].
FVSR_DEV void find_bin(const int* hist, int r, int* out) {
  const int lane = threadIdx.x & 63;
  int c[4], lsum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = hist[lane * 4 + i];
    lsum += c[i];
  }
  int suf = lsum;  // becomes sum over lanes >= lane
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_down(suf, o, 64);
    if (lane + o < 64) suf += t;
  }
  const uint64_t ok = __ballot(suf >= r);
  const int top = 63 - __clzll(ok);
  if (lane == top) {
    int above = suf - lsum;  // bins of higher lanes
    int b = 3;
    while (above + c[b] < r) above += c[b--];
    out[0] = lane * 4 + b;
    out[1] = r - above;
  }
}

// One (head, query time row) per workgroup.  The slab attn[h][t*S .. t*S+S)[:]
// (S = NQ / q_temporal) is contiguous.  The threshold is the (k+1)-th largest
// bf16 pattern (k = min(topk, S*NK - 1); attn is non-negative or the NaN
// 0x7fc0, so patterns order like values with NaN largest), found by two
// 256-bin histogram passes over the high and low bytes.  keep = attn > thr as
// floats; sel/cnt (if given) list each row's kept key blocks ascending.
__global__ __launch_bounds__(kThreads) void select_kernel(const uint16_t* __restrict__ attn,
                                                          int64_t NQ, int64_t NK, int64_t q_temporal,
                                                          int64_t topk, uint8_t* __restrict__ keep,
                                                          int32_t* __restrict__ sel,
                                                          int32_t* __restrict__ cnt) {
  __shared__ int hist[256];
  __shared__ int pick[2];
  const int64_t h = blockIdx.x / q_temporal, t = blockIdx.x % q_temporal;
  const int64_t S = NQ / q_temporal, n = S * NK;
  const int64_t off = (h * NQ + t * S) * NK;
  const uint16_t* vals = attn + off;
  const int tid = threadIdx.x;
  const int r = (int)((topk < n - 1 ? topk : n - 1) + 1);

  hist[tid] = 0;
  __syncthreads();
  for (int64_t i = tid; i < n; i += kThreads) atomicAdd(&hist[vals[i] >> 8], 1);
  __syncthreads();
  if (tid < 64) find_bin(hist, r, pick);
  __syncthreads();
  const uint32_t hi = (uint32_t)pick[0];
  const int r2 = pick[1];
  __syncthreads();
  hist[tid] = 0;
  __syncthreads();
  for (int64_t i = tid; i < n; i += kThreads) {
    const uint32_t v = vals[i];
    if ((v >> 8) == hi) atomicAdd(&hist[v & 0xff], 1);
  }
  __syncthreads();
  if (tid < 64) find_bin(hist, r2, pick);
  __syncthreads();
  const float thr = __uint_as_float(((hi << 8) | (uint32_t)pick[0]) << 16);

  if (keep)
    for (int64_t i = tid; i < n; i += kThreads) keep[off + i] = bf2f(vals[i]) > thr ? 1 : 0;
  if (sel) {
    const int lane = tid & 63;
    for (int64_t row = tid >> 6; row < S; row += kThreads / 64) {
      const uint16_t* ar = vals + row * NK;
      int32_t* sr = sel + off + row * NK;
      int base = 0;
      for (int64_t c0 = 0; c0 < NK; c0 += 64) {
        const bool f = c0 + lane < NK && bf2f(ar[c0 + lane]) > thr;
        const uint64_t bal = __ballot(f);
        if (f) sr[base + __popcll(bal & ((1ull << lane) - 1ull))] = (int32_t)(c0 + lane);
        base += __popcll(bal);
      }
      if (lane == 0) cnt[h * NQ + t * S + row] = base;
    }
  }
}

constexpr int64_t align64(int64_t n) { return (n + 63) & ~(int64_t)63; }

}  // namespace

extern "C" int64_t fvsr_draft_workspace_floats(int64_t H, int64_t D, int64_t NQ, int64_t NK) {
  if (H <= 0 || D <= 0 || NQ < 0 || NK < 0) return 0;
  // bf16 avg_q [NQ, H*D], avg_k [NK, H*D] and attn [H, NQ, NK], 256-byte aligned.
  return (align64((NQ + NK) * H * D) + align64(H * NQ * NK)) / 2 + 64;
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
  // LDS holds D + NK floats; the select pass counts a slab in int.
  if (D + NK > 12288 || (NQ / q_temporal) * NK > 0x7fffffff || H * NQ > 0x7fffffff ||
      NQ + NK > 0x7fffffff)
    return FVSR_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int64_t C = H * D;
  uint16_t* avg = (uint16_t*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  uint16_t* attn = avg + align64((NQ + NK) * C);
  hipLaunchKernelGGL(pool_kernel, dim3((unsigned)(NQ + NK), (unsigned)((C + 511) / 512)),
                     dim3(kThreads), 0, st, (const uint16_t*)q, q_tok_stride, q_map,
                     (const uint16_t*)k, k_tok_stride, k_map, NQ, C, avg);
  const float inv_sqrt_d = 1.0f / (float)sqrt((double)D);
  hipLaunchKernelGGL(score_softmax_kernel, dim3((unsigned)(H * NQ)), dim3(kThreads),
                     (D + NK) * sizeof(float), st, avg, avg + NQ * C, H, D, NQ, NK, local, sq, sk,
                     inv_sqrt_d, attn);
  hipLaunchKernelGGL(select_kernel, dim3((unsigned)(H * q_temporal)), dim3(kThreads), 0, st, attn,
                     NQ, NK, q_temporal, topk, keep, sel, cnt);
  return fvsr_launch_status();
}
