// Block-sparse attention over 128-token blocks (contract BSA) and the device
// block-index builder.
//
// Work unit: one workgroup per (head, query block) = 128 queries, 4 wavefronts
// of 32 queries.  For every kept key block (ids from the block index, never
// touching skipped blocks):
//   S^T = K Q^T     v_mfma_f32_32x32x16_bf16, K from LDS, Q^T from registers.
//                   Each lane owns one query column, so the softmax row
//                   statistics are lane-local (plus one lane^32 exchange).
//   online softmax  exp2 with sm_scale*log2(e) folded in, fp32.
//   O^T += V^T P^T  P^T stays in the S^T registers (converted to bf16): with
//                   the 32x32 accumulator layout, accumulator registers
//                   8*gp..8*gp+7 of key subtile jk are exactly one MFMA
//                   K-operand once the key order inside the reduction is
//                   permuted consistently on both operands.
//   V^T is written transposed into LDS (dword = two keys of one dim), K is
//   stored row-major; both are XOR-swizzled and double-buffered (128 KB).
// Rows whose block list is empty produce zeros (lcsa/triton_lcsa.py:59-60).
#include "common.h"

namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kBlk = 128;       // tokens per block
constexpr int kD = 128;         // head dim
constexpr int kThreads = 256;
constexpr int kTileBytes = kBlk * kD * 2;  // 32 KB
constexpr int kStage = 2 * kTileBytes;     // K + V^T

FVSR_DEV v8bf as_bf(u32x4_t v) { return __builtin_bit_cast(v8bf, v); }

// K tile: row = key (256 B = 16 chunks of 16 B), chunk ^ (key & 15).
FVSR_DEV int k_off(int key, int chunk) { return key * 256 + ((chunk ^ (key & 15)) << 4); }
// V^T tile: row = dim (256 B = 32 units of 8 B = 4 keys), unit ^ (dim & 31).
FVSR_DEV int vt_off(int dim, int unit) { return dim * 256 + ((unit ^ (dim & 31)) << 3); }

struct Regs {
  u32x4_t k[8];  // 8 K chunks
  u32x4_t v[8];  // 4 d-chunks x 2 keys
};

FVSR_DEV int64_t tok_of(const int32_t* map, int64_t pos) { return map ? (int64_t)map[pos] : pos; }

FVSR_DEV void load_kv(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                      int64_t tok_stride, const int32_t* __restrict__ kv_map, int blk, Regs& r) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int id = t + kThreads * i;
    const int key = id >> 4, c = id & 15;
    r.k[i] = *(const u32x4_t*)(k + tok_of(kv_map, (int64_t)blk * kBlk + key) * tok_stride + c * 8);
  }
  const int kp = t & 63, dg = t >> 6;
  const int64_t t0 = tok_of(kv_map, (int64_t)blk * kBlk + 2 * kp);
  const int64_t t1 = tok_of(kv_map, (int64_t)blk * kBlk + 2 * kp + 1);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    r.v[2 * c] = *(const u32x4_t*)(v + t0 * tok_stride + dg * 32 + c * 8);
    r.v[2 * c + 1] = *(const u32x4_t*)(v + t1 * tok_stride + dg * 32 + c * 8);
  }
}

FVSR_DEV void store_kv(uint8_t* stage, const Regs& r) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int id = t + kThreads * i;
    *(u32x4_t*)(stage + k_off(id >> 4, id & 15)) = r.k[i];
  }
  uint8_t* vt = stage + kTileBytes;
  const int kp = t & 63, dg = t >> 6;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t a = r.v[2 * c][w], b = r.v[2 * c + 1][w];
      const int d = dg * 32 + c * 8 + 2 * w;
      // dims d (low halves) and d+1 (high halves) of keys 2kp, 2kp+1
      *(uint32_t*)(vt + vt_off(d, kp >> 1) + (kp & 1) * 4) = (a & 0xffffu) | (b << 16);
      *(uint32_t*)(vt + vt_off(d + 1, kp >> 1) + (kp & 1) * 4) = (a >> 16) | (b & 0xffff0000u);
    }
  }
}

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void bsa_fwd_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, int64_t q_ts,
                    int64_t q_hs, int64_t kv_ts, int64_t kv_hs, int64_t o_ts, int64_t o_hs,
                    const int32_t* __restrict__ sel, const int32_t* __restrict__ cnt,
                    int64_t maxk, int NQ, float scale_log2, const int32_t* __restrict__ q_map,
                    const int32_t* __restrict__ kv_map) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStage];
  const int h = blockIdx.x / NQ, qb = blockIdx.x % NQ;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5;
  const int n = cnt[(int64_t)h * NQ + qb];
  const int32_t* blocks = sel + ((int64_t)h * NQ + qb) * maxk;
  const uint16_t* kh = k + (int64_t)h * kv_hs;
  const uint16_t* vh = v + (int64_t)h * kv_hs;

  // This lane's query (MFMA column) and its Q^T operand: step kk covers dims
  // kk*16 + half*8 .. +8.
  const int qpos = wave * 32 + (lane & 31);
  const int64_t qtok = tok_of(q_map, (int64_t)qb * kBlk + qpos);
  u32x4_t qf[8];
  {
    const uint16_t* qr = q + qtok * q_ts + (int64_t)h * q_hs;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = *(const u32x4_t*)(qr + kk * 16 + half * 8);
  }

  v16f acc[4];  // O^T, dim subtile jd
#pragma unroll
  for (int jd = 0; jd < 4; ++jd)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[jd][e] = 0.0f;
  float m_run = -__builtin_huge_valf(), l_run = 0.0f;

  Regs pre;
  if (n > 0) {
    load_kv(kh, vh, kv_ts, kv_map, blocks[0], pre);
    store_kv(smem, pre);
  }
  __syncthreads();

  for (int it = 0; it < n; ++it) {
    const uint8_t* st = smem + (it & 1) * kStage;
    const bool more = it + 1 < n;
    if (more) load_kv(kh, vh, kv_ts, kv_map, blocks[it + 1], pre);

    // S^T[key][q] for the 4 key subtiles.
    v16f s[4];
#pragma unroll
    for (int jk = 0; jk < 4; ++jk) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[jk][e] = 0.0f;
      const int key = jk * 32 + (lane & 31);
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const u32x4_t kf = *(const u32x4_t*)(st + k_off(key, kk * 2 + half));
        s[jk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(kf), as_bf(qf[kk]), s[jk], 0, 0, 0);
      }
    }

    // Online softmax for this lane's query (its 64 keys + the partner lane's 64).
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int jk = 0; jk < 4; ++jk)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[jk][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx * scale_log2);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.0f;
    u32x4_t pf[8];  // P^T operands, step (jk, gp) -> pf[jk*2+gp]
#pragma unroll
    for (int jk = 0; jk < 4; ++jk) {
      float p[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        p[e] = __builtin_amdgcn_exp2f(s[jk][e] * scale_log2 - m_new);
        psum += p[e];
      }
#pragma unroll
      for (int gp = 0; gp < 2; ++gp)
        pf[jk * 2 + gp] = u32x4_t{pack_bf16x2(p[gp * 8 + 0], p[gp * 8 + 1]),
                                  pack_bf16x2(p[gp * 8 + 2], p[gp * 8 + 3]),
                                  pack_bf16x2(p[gp * 8 + 4], p[gp * 8 + 5]),
                                  pack_bf16x2(p[gp * 8 + 6], p[gp * 8 + 7])};
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[jd][e] *= alpha;

    // O^T[d][q] += V^T[d][key] P^T[key][q].  Step (jk, gp): lane half h
    // supplies keys jk*32 + gp*16 + h*4 + {0..3} and the same + 8.
    const uint8_t* vt = st + kTileBytes;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd) {
      const int d = jd * 32 + (lane & 31);
#pragma unroll
      for (int jk = 0; jk < 4; ++jk) {
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) {
          const int u = jk * 8 + gp * 4 + half;
          const u32x2_t lo = *(const u32x2_t*)(vt + vt_off(d, u));
          const u32x2_t hi = *(const u32x2_t*)(vt + vt_off(d, u + 2));
          const u32x4_t vf = {lo[0], lo[1], hi[0], hi[1]};
          acc[jd] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(vf), as_bf(pf[jk * 2 + gp]),
                                                            acc[jd], 0, 0, 0);
        }
      }
    }
    if (more) store_kv(smem + ((it + 1) & 1) * kStage, pre);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  uint16_t* orow = o + tok_of(q_map, (int64_t)qb * kBlk + qpos) * o_ts + (int64_t)h * o_hs;
#pragma unroll
  for (int jd = 0; jd < 4; ++jd)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = jd * 32 + g * 8 + half * 4;
      *(u32x2_t*)(orow + d) = u32x2_t{pack_bf16x2(acc[jd][g * 4 + 0] * inv, acc[jd][g * 4 + 1] * inv),
                                      pack_bf16x2(acc[jd][g * 4 + 2] * inv, acc[jd][g * 4 + 3] * inv)};
    }
}

// One wavefront per (head, query block) row: ballot compaction of the kept ids.
__global__ __launch_bounds__(256) void block_index_kernel(const uint8_t* __restrict__ keep,
                                                          int64_t rows, int64_t NK,
                                                          int32_t* __restrict__ sel,
                                                          int32_t* __restrict__ cnt) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint8_t* kr = keep + row * NK;
  int32_t* sr = sel + row * NK;
  int base = 0;
  for (int64_t c0 = 0; c0 < NK; c0 += 64) {
    const bool f = c0 + lane < NK && kr[c0 + lane] != 0;
    const uint64_t bal = __ballot(f);
    if (f) sr[base + __popcll(bal & ((1ull << lane) - 1ull))] = (int32_t)(c0 + lane);
    base += __popcll(bal);
  }
  if (lane == 0) cnt[row] = base;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int fvsr_block_index(const uint8_t* keep, int64_t H, int64_t NQ, int64_t NK,
                                int32_t* sel, int32_t* cnt, void* stream) {
  if (H < 0 || NQ < 0 || NK < 0) return FVSR_EINVAL;
  const int64_t rows = H * NQ;
  if (rows == 0) return FVSR_OK;
  if (!keep || !sel || !cnt) return FVSR_EINVAL;
  hipLaunchKernelGGL(block_index_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, keep, rows, NK, sel, cnt);
  return fvsr_launch_status();
}

extern "C" int fvsr_bsa_fwd(const void* q, const void* k, const void* v, void* o,
                            int64_t q_tok_stride, int64_t q_head_stride, int64_t kv_tok_stride,
                            int64_t kv_head_stride, int64_t o_tok_stride, int64_t o_head_stride,
                            const int32_t* sel, const int32_t* cnt, int64_t maxk, int64_t H,
                            int64_t NQ, int64_t NK, int64_t head_dim, float sm_scale,
                            const int32_t* q_map, const int32_t* kv_map, void* stream) {
  if (H < 0 || NQ < 0 || NK < 0 || maxk < 0) return FVSR_EINVAL;
  if (H * NQ == 0) return FVSR_OK;
  if (!q || !k || !v || !o || !sel || !cnt) return FVSR_EINVAL;
  if (head_dim != kD) return FVSR_EUNSUPPORTED;
  // 16-byte rows: token strides and head offsets must keep every row aligned.
  if ((q_tok_stride | q_head_stride | kv_tok_stride | kv_head_stride) % 8) return FVSR_EUNSUPPORTED;
  if ((o_tok_stride | o_head_stride) % 4) return FVSR_EUNSUPPORTED;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || ((uintptr_t)o & 7)) return FVSR_EUNSUPPORTED;
  if (H * NQ > 0x7fffffff || NQ > 0x7fffffff) return FVSR_EUNSUPPORTED;
  const float scale_log2 = sm_scale * 1.4426950408889634f;
  hipLaunchKernelGGL(bsa_fwd_kernel, dim3((unsigned)(H * NQ)), dim3(kThreads), 0,
                     (hipStream_t)stream, (const uint16_t*)q, (const uint16_t*)k,
                     (const uint16_t*)v, (uint16_t*)o, q_tok_stride, q_head_stride, kv_tok_stride,
                     kv_head_stride, o_tok_stride, o_head_stride, sel, cnt, maxk, (int)NQ,
                     scale_log2, q_map, kv_map);
  return fvsr_launch_status();
}
