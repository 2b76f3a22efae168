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

// Per-lane state of the K/V stream.  Each wave issues 8 direct loads of 1 KB
// (4 rows of 256 bytes) per 64-key half: load t covers rows 4*seg .. 4*seg+3
// of the tile, seg = (wave & 1) * 8 + t, lane i landing at row 4*seg + i/16,
// physical chunk i%16 and fetching the logical chunk that belongs there.
// Waves 0-1 stream K, waves 2-3 stream V.  The chunk a lane fetches depends
// only on t % 4 (K) or not at all (V), so `lbase[t % 4]` (the tile base
// pointer plus the chunk offset) is fixed for the whole kernel, and a load's
// address is lbase + token row * row stride: one multiply-add per load.
// With a token map the 8 rows' tokens of the next-but-one half are gathered
// one step ahead, so no load ever waits on the map.
struct Stream {
  const uint8_t* lbase[4];
  uint32_t ts2;             // token row stride in bytes
  const int32_t* kv_map;
  int blk[2];               // key blocks of the current and the next block step
  int tok[8];               // MAP: tokens of the rows of the next half to issue
};

FVSR_DEV int stream_row(int wave, int t, int lane) { return ((wave & 1) * 8 + t) * 4 + (lane >> 4); }

// First position of half `hf` of key block `blk`.
FVSR_DEV int64_t half_pos(int blk, int hf) { return (int64_t)blk * kBlk + hf * kHalf; }

template <bool MAP>
FVSR_DEV void gather_tokens(Stream& s, int blk, int hf, int wave, int lane) {
  if (MAP) {
    const int64_t p0 = half_pos(blk, hf);
#pragma unroll
    for (int t = 0; t < 8; ++t) s.tok[t] = s.kv_map[p0 + stream_row(wave, t, lane)];
  }
}

// Token rows are non-negative and below 2^31, so a load's address is one
// 32 x 32 -> 64-bit multiply-add onto the lane's base pointer.
template <bool MAP>
FVSR_DEV void issue_half(uint8_t LDS_AS* stage, const Stream& s, int blk, int hf, int wave,
                         int lane) {
  uint8_t LDS_AS* tile = stage + (wave >= 2 ? kTile : 0);
  const uint32_t p0 = MAP ? 0u : (uint32_t)half_pos(blk, hf);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int seg = (wave & 1) * 8 + t;
    const uint32_t row = MAP ? (uint32_t)s.tok[t] : p0 + (uint32_t)stream_row(wave, t, lane);
    __builtin_amdgcn_global_load_lds(s.lbase[t & 3] + (uint64_t)row * s.ts2,
                                     (void LDS_AS*)(tile + seg * 1024), 16, 0, 0);
  }
}

struct StepCtx {
  int steps, wave, lane, half, g16, s16;
  float scale_log2;
};

// The four V^T operands of dim subtile jd (steps (jk, gp) -> j = jk*2 + gp),
// read with inline-asm ds_read_b64_tr_b16: the compiler cannot tell the
// builtin's reads from the direct loads streaming into the other stage and
// would wait for those loads (vmcnt(0)) first.  The caller waits (lgkmcnt)
// before using the operands.
FVSR_DEV void read_vt(const uint8_t LDS_AS* vt, const StepCtx& c, int jd, u32x4_t (&vf)[4]) {
  const int dcol = jd * 32 + (c.g16 & 1) * 16 + 4 * (c.s16 & 3);
  const int cch = dcol >> 3, cof = (dcol & 7) * 2;
  const int rl = c.half * 4 + (c.s16 >> 2);  // row within each 16-key group; rl & 3 = (s16 >> 2) & 3
  const uint32_t a = (uint32_t)(uintptr_t)vt + rl * 256 + (v_swz(rl, cch) << 4) + cof;
#define FVSR_TR(J, OFF, DST)                                                            \
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(DST) : "v"(a), "i"(OFF))
  u32x2_t lo0, hi0, lo1, hi1, lo2, hi2, lo3, hi3;
  FVSR_TR(0, 0 * 256, lo0);
  FVSR_TR(0, 8 * 256, hi0);
  FVSR_TR(1, 16 * 256, lo1);
  FVSR_TR(1, 24 * 256, hi1);
  FVSR_TR(2, 32 * 256, lo2);
  FVSR_TR(2, 40 * 256, hi2);
  FVSR_TR(3, 48 * 256, lo3);
  FVSR_TR(3, 56 * 256, hi3);
#undef FVSR_TR
  vf[0] = u32x4_t{lo0[0], lo0[1], hi0[0], hi0[1]};
  vf[1] = u32x4_t{lo1[0], lo1[1], hi1[0], hi1[1]};
  vf[2] = u32x4_t{lo2[0], lo2[1], hi2[0], hi2[1]};
  vf[3] = u32x4_t{lo3[0], lo3[1], hi3[0], hi3[1]};
}

// s_waitcnt immediate (gfx9 encoding): vmcnt in bits 3:0 and 15:14 (63 =
// left open), expcnt 6:4 (left open), lgkmcnt 11:8.
constexpr int kWaitLgkm0 = 15 | (3 << 14) | (7 << 4) | (0 << 8);

FVSR_DEV void wait_lds() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_sched_barrier(0);
}

// One 64-key half step: wait for `cur`, start streaming step it+1 into
// `nxt` (and gather the tokens of step it+2), then S^T, softmax and O^T on
// `cur`.  All sixteen K fragments are read before the S^T MFMAs and all
// sixteen V^T fragments before the softmax, so the MFMAs never wait on a
// read issued just before them and the V reads complete under the softmax.
// `cur` and `nxt` are distinct LDS objects, so the compiler can tell the
// direct loads into `nxt` apart from the reads of `cur` and does not
// serialise them.
template <bool MAP>
FVSR_DEV void bsa_step(uint8_t LDS_AS* cur, uint8_t LDS_AS* nxt, int it, const StepCtx& c,
                       Stream& st, const u32x4_t (&qf)[8], v16f (&acc)[4], float& m_run,
                       float& l_run) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of step `it` have landed
  __syncthreads();                // ... and everyone's; `nxt` is no longer being read
  // Step it+1 is the second half of this block (it even) or the first half of
  // the next; step it+2 the first or second half of the next block.
  const int hf = it & 1;
  if (it + 1 < c.steps) issue_half<MAP>(nxt, st, st.blk[hf], hf ^ 1, c.wave, c.lane);
  if (MAP && it + 2 < c.steps) gather_tokens<MAP>(st, st.blk[1], hf, c.wave, c.lane);
  const uint8_t LDS_AS* kt = cur;
  const uint8_t LDS_AS* vt = cur + kTile;
  const int lane = c.lane, half = c.half;

  // S^T[key][q] for the two 32-key subtiles of this half.
  u32x4_t kf[2][8];
#pragma unroll
  for (int jk = 0; jk < 2; ++jk) {
    const int r = jk * 32 + (lane & 31);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      kf[jk][kk] = *(const u32x4_t LDS_AS*)(kt + r * 256 + (k_swz(r, kk * 2 + half) << 4));
  }
  v16f s[2];
#pragma unroll
  for (int jk = 0; jk < 2; ++jk) {
    const v16f z = {};
    s[jk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(kf[jk][0]), as_bf(qf[0]), z, 0, 0, 0);
#pragma unroll
    for (int kk = 1; kk < 8; ++kk)
      s[jk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(kf[jk][kk]), as_bf(qf[kk]), s[jk], 0,
                                                      0, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // the 16 K reads
  __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);  // then the 16 S^T MFMAs

  // V^T operands of step (jd, jk, gp): lane half h supplies keys kb0 + 0..3
  // and kb0 + 8 + 0..3, kb0 = jk*32 + gp*16 + h*4; a transposed read gives
  // lane (g16, s16) dims dbase + s16 of keys kb..kb+3 from the 8 bytes at row
  // kb + s16/4, dims dbase + 4*(s16%4).  Dim subtiles 0-1 are read before the
  // softmax, 2-3 under the MFMAs of 0-1.
  u32x4_t vf[4][4];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int jd = 0; jd < 2; ++jd) read_vt(vt, c, jd, vf[jd]);
  // Online softmax for this lane's query over the 64 keys of the half.
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int jk = 0; jk < 2; ++jk)
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[jk][e]);
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false,
                                                     false);  // lane l and l ^ 32
    mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * c.scale_log2;
  }
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

  // O^T[d][q] += V^T[d][key] P^T[key][q].
  wait_lds();  // V operands of dim subtiles 0-1
  read_vt(vt, c, 2, vf[2]);
  read_vt(vt, c, 3, vf[3]);
#pragma unroll
  for (int jd = 0; jd < 4; ++jd) {
    if (jd == 2) wait_lds();  // ... and 2-3
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[jd] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(vf[jd][j]), as_bf(pf[j]), acc[jd], 0,
                                                        0, 0);
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
  const StepCtx c{2 * n, wave, lane, half, lane >> 4, lane & 15, scale_log2};
  const int32_t* blocks = sel + ((int64_t)h * NQ + qb) * maxk;
  Stream st;
  {
    const uint16_t* base = (wave >= 2 ? v : k) + (int64_t)h * kv_hs;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = stream_row(wave, t, lane), p = lane & 15;
      st.lbase[t] = (const uint8_t*)(base + (wave >= 2 ? v_swz(r, p) : k_swz(r, p)) * 8);  // involutions
    }
    st.ts2 = (uint32_t)(kv_ts * 2);
    st.kv_map = kv_map;
  }
  if (n > 0) {
    st.blk[0] = blocks[0];
    st.blk[1] = blocks[n > 1 ? 1 : 0];
    gather_tokens<MAP>(st, st.blk[0], 0, wave, lane);
    issue_half<MAP>(st0, st, st.blk[0], 0, wave, lane);
    gather_tokens<MAP>(st, st.blk[0], 1, wave, lane);
  }

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

  for (int b = 0; b < n; ++b) {  // two 64-key halves per kept block
    // The block after next loads under this block's steps (a full wait opens
    // every step) and becomes st.blk[1] when the block moves on.
    const int ahead = blocks[b + 2 < n ? b + 2 : n - 1];
    bsa_step<MAP>(st0, st1, 2 * b, c, st, qf, acc, m_run, l_run);
    bsa_step<MAP>(st1, st0, 2 * b + 1, c, st, qf, acc, m_run, l_run);
    st.blk[0] = st.blk[1];
    st.blk[1] = ahead;
  }

  const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run),
                                                    false, false);
  const float l_tot = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
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
