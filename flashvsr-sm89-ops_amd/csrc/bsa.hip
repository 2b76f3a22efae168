// Block-sparse attention over 128-token blocks (contract BSA) and the device
// block-index builder.
//
// Work unit: one workgroup per (head, query block) = 128 queries, 4 wavefronts
// of 32 queries; two workgroups share a CU (64 KB of LDS each, <= 256
// registers per lane), so one workgroup's softmax overlaps the other's MFMAs.
// Kept key blocks (ids from the block index; skipped blocks are never read)
// are streamed in halves of 64 keys through a double-buffered LDS stage:
//   K, V half tiles [64 keys][128 dims] bf16, row-major, loaded straight from
//   global memory into LDS (global_load_lds_dwordx4: no staging registers);
//   S^T = K Q^T       v_mfma_f32_32x32x16_bf16, Q^T held in registers, so each
//                     lane owns one query and the softmax statistics are
//                     lane-local (plus one lane^32 exchange);
//   online softmax    exp2 with sm_scale*log2(e) folded in; the running max is
//                     only moved (and O rescaled) when it grows by more than
//                     2^8, decided per wavefront;
//   O^T += V^T P^T    P^T stays in the S^T registers: accumulator registers
//                     8*gp..8*gp+7 of key subtile jk are one MFMA K-operand
//                     once the key order inside the reduction is permuted the
//                     same way on both operands; V^T comes from the row-major
//                     V tile through ds_read_b64_tr_b16 (lane i of each
//                     16-lane group receives element i%4 of the 8 bytes
//                     addressed by lane 4j + i/4, for j = 0..3).
// Rows whose block list is empty produce zeros (lcsa/triton_lcsa.py:59-60).
#include "common.h"

namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
#define LDS_AS __attribute__((address_space(3)))

constexpr int kBlk = 128;              // tokens per block
constexpr int kHalf = 64;              // keys per pipeline stage
constexpr int kD = 128;                // head dim
constexpr int kThreads = 256;
constexpr int kTile = kHalf * kD * 2;  // 16 KB: one K or V half tile
constexpr int kStage = 2 * kTile;      // K + V

FVSR_DEV v8bf as_bf(u32x4_t v) { return __builtin_bit_cast(v8bf, v); }

// K tile: 16-byte chunk c of key row r sits at chunk c ^ (r & 15): the 16
// lanes of a ds_read_b128 phase read 16 consecutive rows at one chunk.
FVSR_DEV int k_swz(int r, int c) { return c ^ (r & 15); }
// V tile: chunk c of row r sits at c ^ (4*(r & 3)): a transposed read touches
// 4 consecutive rows x 32 bytes per 16-lane group, and the two groups of a
// half-wave read adjacent 32-byte column blocks; this spreads them over 64 banks.
FVSR_DEV int v_swz(int r, int c) { return c ^ ((r & 3) << 2); }

// Stream one 64-key half of key block `blk` into `stage`.  Each wave issues
// 8 direct loads of 1 KB (4 rows); lane i of a load lands at row 4*seg + i/16,
// physical chunk i%16, and fetches the logical chunk that belongs there.
// The token indices are gathered first (one wait), then the eight loads go
// out back to back.  Waves 0-1 stream K, waves 2-3 stream V.
template <bool MAP>
FVSR_DEV void issue_half(uint8_t LDS_AS* stage, const uint16_t* __restrict__ kh,
                         const uint16_t* __restrict__ vh, int64_t ts,
                         const int32_t* __restrict__ kv_map, int blk, int half, int wave,
                         int lane) {
  const bool isv = wave >= 2;  // wave-uniform
  const uint16_t* base = isv ? vh : kh;
  uint8_t LDS_AS* tile = stage + (isv ? kTile : 0);
  int64_t tok[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int r = ((wave & 1) * 8 + t) * 4 + (lane >> 4);
    const int64_t pos = (int64_t)blk * kBlk + half * kHalf + r;
    tok[t] = MAP ? (int64_t)kv_map[pos] : pos;
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int seg = (wave & 1) * 8 + t;  // 1 KB segment = rows 4*seg .. 4*seg+3
    const int r = seg * 4 + (lane >> 4);
    const int p = lane & 15;
    const int c = isv ? v_swz(r, p) : k_swz(r, p);  // the swizzles are involutions
    __builtin_amdgcn_global_load_lds(base + tok[t] * ts + c * 8,
                                     (void LDS_AS*)(tile + seg * 1024), 16, 0, 0);
  }
}

struct StepCtx {
  const uint16_t* kh;
  const uint16_t* vh;
  int64_t ts;
  const int32_t* kv_map;
  const int32_t* blocks;
  int steps, wave, lane, half, g16, s16;
  float scale_log2;
};

// One 64-key half step: wait for `cur`, start streaming step it+1 into
// `nxt`, then S^T, softmax and O^T on `cur`.  `cur` and `nxt` are distinct
// LDS objects, so the compiler can tell the direct loads into `nxt` apart from
// the reads of `cur` and does not serialise them.
template <bool MAP>
FVSR_DEV void bsa_step(uint8_t LDS_AS* cur, uint8_t LDS_AS* nxt, int it, const StepCtx& c,
                       const u32x4_t (&qf)[8], v16f (&acc)[4], float& m_run, float& l_run) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of step `it` have landed
  __syncthreads();                // ... and everyone's; `nxt` is no longer being read
  if (it + 1 < c.steps)
    issue_half<MAP>(nxt, c.kh, c.vh, c.ts, c.kv_map, c.blocks[(it + 1) >> 1], (it + 1) & 1,
                    c.wave, c.lane);
  const uint8_t LDS_AS* kt = cur;
  const uint8_t LDS_AS* vt = cur + kTile;
  const int lane = c.lane, half = c.half;

  // S^T[key][q] for the two 32-key subtiles of this half.
  v16f s[2];
#pragma unroll
  for (int jk = 0; jk < 2; ++jk) {
#pragma unroll
    for (int e = 0; e < 16; ++e) s[jk][e] = 0.0f;
    const int r = jk * 32 + (lane & 31);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const u32x4_t kf = *(const u32x4_t LDS_AS*)(kt + r * 256 + (k_swz(r, kk * 2 + half) << 4));
      s[jk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(kf), as_bf(qf[kk]), s[jk], 0, 0, 0);
    }
  }

  // Online softmax for this lane's query over the 64 keys of the half.
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int jk = 0; jk < 2; ++jk)
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[jk][e]);
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c.scale_log2;
  if (__ballot(mx > m_run + 8.0f) != 0) {  // move the max (wave-uniform)
    asm volatile("" :::);  // keep this a branch: the rescale is rare after the first steps
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[jd][e] *= alpha;
  }
  float psum = 0.0f;
  u32x4_t pf[4];  // P^T operands, step (jk, gp) -> pf[jk*2+gp]
#pragma unroll
  for (int jk = 0; jk < 2; ++jk) {
    float p[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = __builtin_amdgcn_exp2f(s[jk][e] * c.scale_log2 - m_run);
      psum += p[e];
    }
#pragma unroll
    for (int gp = 0; gp < 2; ++gp)
      pf[jk * 2 + gp] = u32x4_t{pack_bf16x2(p[gp * 8 + 0], p[gp * 8 + 1]),
                                pack_bf16x2(p[gp * 8 + 2], p[gp * 8 + 3]),
                                pack_bf16x2(p[gp * 8 + 4], p[gp * 8 + 5]),
                                pack_bf16x2(p[gp * 8 + 6], p[gp * 8 + 7])};
  }
  l_run += psum;

  // O^T[d][q] += V^T[d][key] P^T[key][q].  Step (jk, gp): lane half h
  // supplies keys kb0 + 0..3 and kb0 + 8 + 0..3, kb0 = jk*32 + gp*16 + h*4;
  // a transposed read gives lane (g16, s16) dims dbase + s16 of keys kb..kb+3
  // from the 8 bytes at row kb + s16/4, dims dbase + 4*(s16%4).
#pragma unroll
  for (int jd = 0; jd < 4; ++jd) {
    const int dcol = jd * 32 + (c.g16 & 1) * 16 + 4 * (c.s16 & 3);
    const int cch = dcol >> 3, cof = (dcol & 7) * 2;
#pragma unroll
    for (int jk = 0; jk < 2; ++jk) {
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        const int r0 = jk * 32 + gp * 16 + half * 4 + (c.s16 >> 2);
        const int r1 = r0 + 8;
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (v4s LDS_AS*)(vt + r0 * 256 + (v_swz(r0, cch) << 4) + cof));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (v4s LDS_AS*)(vt + r1 * 256 + (v_swz(r1, cch) << 4) + cof));
        const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
        const u32x4_t vf = {l2[0], l2[1], h2[0], h2[1]};
        acc[jd] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(vf), as_bf(pf[jk * 2 + gp]),
                                                          acc[jd], 0, 0, 0);
      }
    }
  }
}

template <bool MAP>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2, 2)))
void bsa_fwd_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, int64_t q_ts,
                    int64_t q_hs, int64_t kv_ts, int64_t kv_hs, int64_t o_ts, int64_t o_hs,
                    const int32_t* __restrict__ sel, const int32_t* __restrict__ cnt,
                    int64_t maxk, int NQ, float scale_log2, const int32_t* __restrict__ q_map,
                    const int32_t* __restrict__ kv_map) {
  __shared__ __attribute__((aligned(1024))) uint8_t stage0[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t stage1[kStage];
  uint8_t LDS_AS* st0 = (uint8_t LDS_AS*)stage0;
  uint8_t LDS_AS* st1 = (uint8_t LDS_AS*)stage1;
  // Workgroup ids are dispatched round robin over the 8 XCDs; give each XCD a
  // contiguous range of (head, query block) units so that neighbouring query
  // blocks, whose local windows share most key blocks, share one L2.
  const int total = (int)gridDim.x, per = total / 8, rem = total % 8;
  const int xcd = blockIdx.x % 8, loc = blockIdx.x / 8;
  const int unit = xcd < rem ? xcd * (per + 1) + loc : rem * (per + 1) + (xcd - rem) * per + loc;
  const int h = unit / NQ, qb = unit % NQ;
  const int lane = threadIdx.x & 63, half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = cnt[(int64_t)h * NQ + qb];
  StepCtx c{k + (int64_t)h * kv_hs, v + (int64_t)h * kv_hs, kv_ts, kv_map,
            sel + ((int64_t)h * NQ + qb) * maxk, 2 * n, wave, lane, half, lane >> 4, lane & 15,
            scale_log2};

  if (c.steps > 0) issue_half<MAP>(st0, c.kh, c.vh, c.ts, c.kv_map, c.blocks[0], 0, wave, lane);

  // This lane's query (MFMA column) and its Q^T operand: d-step kk covers
  // dims kk*16 + half*8 .. +8.
  const int qpos = wave * 32 + (lane & 31);
  const int64_t qtok = MAP ? (int64_t)q_map[(int64_t)qb * kBlk + qpos] : (int64_t)qb * kBlk + qpos;
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

  for (int it = 0; it < c.steps; it += 2) {  // steps is even: two halves per block
    bsa_step<MAP>(st0, st1, it, c, qf, acc, m_run, l_run);
    bsa_step<MAP>(st1, st0, it + 1, c, qf, acc, m_run, l_run);
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  uint16_t* orow = o + qtok * o_ts + (int64_t)h * o_hs;
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
  if ((q_map == nullptr) != (kv_map == nullptr)) return FVSR_EUNSUPPORTED;
  const float scale_log2 = sm_scale * 1.4426950408889634f;
  if (q_map)
    hipLaunchKernelGGL(bsa_fwd_kernel<true>, dim3((unsigned)(H * NQ)), dim3(kThreads), 0,
                       (hipStream_t)stream, (const uint16_t*)q, (const uint16_t*)k,
                       (const uint16_t*)v, (uint16_t*)o, q_tok_stride, q_head_stride,
                       kv_tok_stride, kv_head_stride, o_tok_stride, o_head_stride, sel, cnt, maxk,
                       (int)NQ, scale_log2, q_map, kv_map);
  else
    hipLaunchKernelGGL(bsa_fwd_kernel<false>, dim3((unsigned)(H * NQ)), dim3(kThreads), 0,
                       (hipStream_t)stream, (const uint16_t*)q, (const uint16_t*)k,
                       (const uint16_t*)v, (uint16_t*)o, q_tok_stride, q_head_stride,
                       kv_tok_stride, kv_head_stride, o_tok_stride, o_head_stride, sel, cnt, maxk,
                       (int)NQ, scale_log2, q_map, kv_map);
  return fvsr_launch_status();
}
