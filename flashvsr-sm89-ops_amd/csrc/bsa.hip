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
// How a block position (block id, row within the block) becomes a stored
// token row: kDirect the position itself; kMap an int32 map gathered from
// memory; kWin the (2, 8, 8) window partition of a raster-order latent grid
// (WindowPartition3D, reference integrate.py:70-94), in closed form.
enum { kDirect = 0, kMap = 1, kWin = 2 };

// Latent grid of the kWin mode: row width W and frame size HW in tokens;
// windows per row nww = W / 8 and per frame pair nwhw = (H / 8) * nww.
struct WinGeo {
  int W, HW, nww, nwhw;
};

// First raster token of window `wi` (its frame-pair, window row and column).
FVSR_DEV int64_t win_base(int wi, const WinGeo& g) {
  const int wf = wi / g.nwhw, rem = wi - wf * g.nwhw;
  const int whi = rem / g.nww, wwi = rem - whi * g.nww;
  return (int64_t)wf * 2 * g.HW + (int64_t)whi * 8 * g.W + wwi * 8;
}

// Token offset of slot s (0..127) of a window from the window's first token:
// slot = (frame in pair) * 64 + (row in window) * 8 + (column in window).
FVSR_DEV int win_slot(int s, const WinGeo& g) {
  return (s >> 6) * g.HW + ((s >> 3) & 7) * g.W + (s & 7);
}

struct Stream {
  const uint8_t* lbase[4];
  uint32_t ts2;             // token row stride in bytes
  const int32_t* kv_map;
  int blk[2];               // key blocks of the current and the next block step
  int tok[8];               // kMap: tokens of the rows of the next half to issue
  uint32_t woff[8];         // kWin: byte offsets of this lane's rows in half 0
  uint32_t hw2;             // kWin: bytes from half 0 to half 1 (the next frame)
  WinGeo geo;
};

// With NW waves, the first NW/2 stream K and the others V, 32/NW loads of
// 4 rows each per wave and half tile (NW = 8: the dense pair mode below).
template <int NW>
FVSR_DEV int stream_row(int wave, int t, int lane) {
  return ((wave % (NW / 2)) * (32 / NW) + t) * 4 + (lane >> 4);
}

// First position of half `hf` of key block `blk`.
FVSR_DEV int64_t half_pos(int blk, int hf) { return (int64_t)blk * kBlk + hf * kHalf; }

template <int KM, int NW>
FVSR_DEV void gather_tokens(Stream& s, int blk, int hf, int wave, int lane) {
  if (KM == kMap) {
    const int64_t p0 = half_pos(blk, hf);
#pragma unroll
    for (int t = 0; t < 32 / NW; ++t) s.tok[t] = s.kv_map[p0 + stream_row<NW>(wave, t, lane)];
  }
}

// Token rows are non-negative and below 2^31, so a load's address is one
// 32 x 32 -> 64-bit multiply-add onto the lane's base pointer (kWin: the
// window's first row, uniform, plus the lane's 32-bit offset).
template <int KM, int NW>
FVSR_DEV void issue_half(uint8_t LDS_AS* stage, const Stream& s, int blk, int hf, int wave,
                         int lane) {
  uint8_t LDS_AS* tile = stage + (wave >= NW / 2 ? kTile : 0);
  const uint32_t p0 = KM == kDirect ? (uint32_t)half_pos(blk, hf) : 0u;
  const uint64_t wb = KM == kWin ? (uint64_t)win_base(blk, s.geo) * s.ts2 + hf * s.hw2 : 0u;
#pragma unroll
  for (int t = 0; t < 32 / NW; ++t) {
    const int seg = (wave % (NW / 2)) * (32 / NW) + t;
    const uint8_t* src;
    if (KM == kWin) {
      src = s.lbase[t & 3] + wb + s.woff[t];
    } else {
      const uint32_t row =
          KM == kMap ? (uint32_t)s.tok[t] : p0 + (uint32_t)stream_row<NW>(wave, t, lane);
      src = s.lbase[t & 3] + (uint64_t)row * s.ts2;
    }
    __builtin_amdgcn_global_load_lds(src, (void LDS_AS*)(tile + seg * 1024), 16, 0, 0);
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
template <int KM, int NW>
FVSR_DEV void bsa_step(uint8_t LDS_AS* cur, uint8_t LDS_AS* nxt, int it, const StepCtx& c,
                       Stream& st, const u32x4_t (&qf)[8], v16f (&acc)[4], float& m_run,
                       float& l_run) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of step `it` have landed
  __syncthreads();                // ... and everyone's; `nxt` is no longer being read
  // Step it+1 is the second half of this block (it even) or the first half of
  // the next; step it+2 the first or second half of the next block.
  const int hf = it & 1;
  if (it + 1 < c.steps) issue_half<KM, NW>(nxt, st, st.blk[hf], hf ^ 1, c.wave, c.lane);
  if (KM == kMap && it + 2 < c.steps) gather_tokens<KM, NW>(st, st.blk[1], hf, c.wave, c.lane);
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

// QM / KM: how query and key/value block positions become stored token rows
// (kDirect, kMap or kWin, see above); the output rows are the query rows.
// DENSE: every key block 0..maxk-1 is kept for every query block (the
// cross-attention over the cached prompt, integrate.py:132-143): no block
// index is read and a workgroup of 8 waves takes two query blocks (waves 0-3
// and 4-7) over one K/V stream, so the per-unit start-up and the K/V stream
// are paid once per two query blocks (2 waves per SIMD, as two 4-wave
// workgroups would give).
template <int QM, int KM, bool DENSE>
__global__ __attribute__((amdgpu_flat_work_group_size(DENSE ? 512 : 256, DENSE ? 512 : 256),
                          amdgpu_waves_per_eu(2, 2)))
void bsa_fwd_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, int64_t q_ts,
                    int64_t q_hs, int64_t kv_ts, int64_t kv_hs, int64_t o_ts, int64_t o_hs,
                    const int32_t* __restrict__ sel, const int32_t* __restrict__ cnt,
                    int64_t maxk, int NQ, float scale_log2, const int32_t* __restrict__ q_map,
                    const int32_t* __restrict__ kv_map, WinGeo geo, int o_rows16) {
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
  constexpr int NW = DENSE ? 8 : 4;
  const int units_per_head = DENSE ? (NQ + 1) / 2 : NQ;
  const int h = unit / units_per_head, up = unit % units_per_head;
  const int lane = threadIdx.x & 63, half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // A dense pair's second query block may lie past NQ (odd NQ): its waves
  // follow the stream on the last block and store nothing.
  const int qb_raw = DENSE ? 2 * up + (wave >> 2) : up;
  const bool q_live = qb_raw < NQ;
  const int qb = q_live ? qb_raw : NQ - 1;
  const int n = DENSE ? (int)maxk : cnt[(int64_t)h * NQ + qb];
  const StepCtx c{2 * n, wave, lane, half, lane >> 4, lane & 15, scale_log2};
  const int32_t* blocks = DENSE ? nullptr : sel + ((int64_t)h * NQ + qb) * maxk;
  // The first two block ids load together with the count (the row holds maxk
  // entries; those past the count are unspecified and then unused), so the
  // first K/V addresses wait for one memory round trip, not two.
  int b0 = 0, b1 = maxk > 1 ? 1 : 0;
  if (!DENSE && maxk > 0) {
    b0 = blocks[0];
    b1 = blocks[maxk > 1 ? 1 : 0];
  }
  Stream st;
  {
    const uint16_t* base = (wave >= NW / 2 ? v : k) + (int64_t)h * kv_hs;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = stream_row<NW>(wave, t, lane), p = lane & 15;
      st.lbase[t] = (const uint8_t*)(base + (wave >= NW / 2 ? v_swz(r, p) : k_swz(r, p)) * 8);  // involutions
    }
    st.ts2 = (uint32_t)(kv_ts * 2);
    st.kv_map = kv_map;
    st.geo = geo;
    if (KM == kWin) {
      st.hw2 = (uint32_t)geo.HW * st.ts2;
#pragma unroll
      for (int t = 0; t < 32 / NW; ++t)
        st.woff[t] = (uint32_t)win_slot(stream_row<NW>(wave, t, lane), geo) * st.ts2;
    }
  }
  if (n > 0) {
    st.blk[0] = b0;
    st.blk[1] = n > 1 ? b1 : b0;
    gather_tokens<KM, NW>(st, st.blk[0], 0, wave, lane);
    issue_half<KM, NW>(st0, st, st.blk[0], 0, wave, lane);
    gather_tokens<KM, NW>(st, st.blk[0], 1, wave, lane);
  }

  // This lane's query (MFMA column) and its Q^T operand: d-step kk covers
  // dims kk*16 + half*8 .. +8.
  const int qpos = (wave & 3) * 32 + (lane & 31);
  const int64_t qtok = QM == kMap   ? (int64_t)q_map[(int64_t)qb * kBlk + qpos]
                       : QM == kWin ? win_base(qb, geo) + win_slot(qpos, geo)
                                    : (int64_t)qb * kBlk + qpos;
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
    const int ahead = DENSE ? (b + 2 < n ? b + 2 : n - 1) : blocks[b + 2 < n ? b + 2 : n - 1];
    bsa_step<KM, NW>(st0, st1, 2 * b, c, st, qf, acc, m_run, l_run);
    bsa_step<KM, NW>(st1, st0, 2 * b + 1, c, st, qf, acc, m_run, l_run);
    st.blk[0] = st.blk[1];
    st.blk[1] = ahead;
  }

  const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run),
                                                    false, false);
  const float l_tot = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (DENSE) {
    __syncthreads();  // waves 4-7 stage through stage1, which the last step reads
    if (!q_live) return;
  }
  if (!o_rows16) {
    uint16_t* orow = o + qtok * o_ts + (int64_t)h * o_hs;
#pragma unroll
    for (int jd = 0; jd < 4; ++jd)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = jd * 32 + g * 8 + half * 4;
        *(u32x2_t*)(orow + d) =
            u32x2_t{pack_bf16x2(acc[jd][g * 4 + 0] * inv, acc[jd][g * 4 + 1] * inv),
                    pack_bf16x2(acc[jd][g * 4 + 2] * inv, acc[jd][g * 4 + 3] * inv)};
      }
    return;
  }
  // 16-byte aligned output rows leave through stage0, free once the last
  // step's barrier has passed (that step reads stage1; no load targets
  // stage0 after it): each wave writes its 32 x 128 bf16 tile there and then
  // stores whole 256-byte rows, 4 rows per instruction, where the lanes'
  // own accumulators would give 16-byte pieces of 32 rows (F3's 4-block
  // units 83 -> 74 us, C5 566 -> 559 us; the same bytes).
  uint8_t LDS_AS* ot = (wave < 4 ? st0 : st1) + (wave & 3) * 8192;
  const int ql = lane & 31;
#pragma unroll
  for (int jd = 0; jd < 4; ++jd)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int ch = jd * 4 + g;
      *(u32x2_t LDS_AS*)(ot + ql * 256 + ((ch ^ (ql & 15)) << 4) + half * 8) =
          u32x2_t{pack_bf16x2(acc[jd][g * 4 + 0] * inv, acc[jd][g * 4 + 1] * inv),
                  pack_bf16x2(acc[jd][g * 4 + 2] * inv, acc[jd][g * 4 + 3] * inv)};
    }
  const int c16 = lane & 15;
  const int tq = (int)qtok;  // token rows are below 2^31
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = (lane >> 4) + 4 * i;
    const u32x4_t val = *(const u32x4_t LDS_AS*)(ot + r * 256 + ((c16 ^ (r & 15)) << 4));
    const int64_t tr = __shfl(tq, r, 64);
    *(u32x4_t*)(o + tr * o_ts + (int64_t)h * o_hs + c16 * 8) = val;
  }
}

// One row of the block index per wave: the kept block ids ascending, then the
// other ids ascending -- the order of the reference's stable descending
// argsort of keep (lcsa/triton_lcsa.py:67-68) -- and the kept count.  The
// first pass counts the kept ids, so the second can place both groups.
__global__ __launch_bounds__(256) void block_index_kernel(const uint8_t* __restrict__ keep,
                                                          int64_t rows, int64_t NK,
                                                          int32_t* __restrict__ sel,
                                                          int32_t* __restrict__ cnt) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint8_t* kr = keep + row * NK;
  int32_t* sr = sel + row * NK;
  int kept = 0;
  for (int64_t c0 = 0; c0 < NK; c0 += 64)
    kept += __popcll(__ballot(c0 + lane < NK && kr[c0 + lane] != 0));
  int base = 0, rest = kept;
  for (int64_t c0 = 0; c0 < NK; c0 += 64) {
    const bool in = c0 + lane < NK;
    const bool f = in && kr[c0 + lane] != 0;
    const uint64_t below = (1ull << lane) - 1ull;
    const uint64_t bk = __ballot(f), bn = __ballot(in && !f);
    if (f) sr[base + __popcll(bk & below)] = (int32_t)(c0 + lane);
    if (in && !f) sr[rest + __popcll(bn & below)] = (int32_t)(c0 + lane);
    base += __popcll(bk);
    rest += __popcll(bn);
  }
  if (lane == 0) cnt[row] = kept;
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

namespace {

template <int QM, int KM, bool DENSE = false>
void launch_bsa(const void* q, const void* k, const void* v, void* o, int64_t q_ts, int64_t q_hs,
                int64_t kv_ts, int64_t kv_hs, int64_t o_ts, int64_t o_hs, const int32_t* sel,
                const int32_t* cnt, int64_t maxk, int64_t H, int64_t NQ, float scale_log2,
                const int32_t* q_map, const int32_t* kv_map, WinGeo geo, hipStream_t st) {
  const int64_t units = H * (DENSE ? (NQ + 1) / 2 : NQ);
  hipLaunchKernelGGL((bsa_fwd_kernel<QM, KM, DENSE>), dim3((unsigned)units),
                     dim3(DENSE ? 2 * kThreads : kThreads), 0, st,
                     (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o,
                     q_ts, q_hs, kv_ts, kv_hs, o_ts, o_hs, sel, cnt, maxk, (int)NQ, scale_log2,
                     q_map, kv_map, geo, (int)(aligned16(o) && (o_ts | o_hs) % 8 == 0));
}

// Checks shared by both entry points.
int bsa_args_ok(const void* q, const void* k, const void* v, const void* o, int64_t q_ts,
                int64_t q_hs, int64_t kv_ts, int64_t kv_hs, int64_t o_ts, int64_t o_hs,
                const int32_t* sel, const int32_t* cnt, int64_t head_dim, int64_t H,
                int64_t NQ) {
  if (!q || !k || !v || !o || !sel || !cnt) return FVSR_EINVAL;
  if (head_dim != kD) return FVSR_EUNSUPPORTED;
  // 16-byte rows: token strides and head offsets must keep every row aligned.
  if ((q_ts | q_hs | kv_ts | kv_hs) % 8) return FVSR_EUNSUPPORTED;
  if ((o_ts | o_hs) % 4) return FVSR_EUNSUPPORTED;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || ((uintptr_t)o & 7)) return FVSR_EUNSUPPORTED;
  if (H * NQ > 0x7fffffff || NQ > 0x7fffffff) return FVSR_EUNSUPPORTED;
  return FVSR_OK;
}

}  // namespace

extern "C" int fvsr_bsa_fwd(const void* q, const void* k, const void* v, void* o,
                            int64_t q_tok_stride, int64_t q_head_stride, int64_t kv_tok_stride,
                            int64_t kv_head_stride, int64_t o_tok_stride, int64_t o_head_stride,
                            const int32_t* sel, const int32_t* cnt, int64_t maxk, int64_t H,
                            int64_t NQ, int64_t NK, int64_t head_dim, float sm_scale,
                            const int32_t* q_map, const int32_t* kv_map, void* stream) {
  if (H < 0 || NQ < 0 || NK < 0 || maxk < 0) return FVSR_EINVAL;
  if (H * NQ == 0) return FVSR_OK;
  const int rc = bsa_args_ok(q, k, v, o, q_tok_stride, q_head_stride, kv_tok_stride,
                             kv_head_stride, o_tok_stride, o_head_stride, sel, cnt, head_dim, H,
                             NQ);
  if (rc != FVSR_OK) return rc;
  if ((q_map == nullptr) != (kv_map == nullptr)) return FVSR_EUNSUPPORTED;
  const float scale_log2 = sm_scale * 1.4426950408889634f;
  const WinGeo geo{0, 0, 1, 1};
  if (q_map)
    launch_bsa<kMap, kMap>(q, k, v, o, q_tok_stride, q_head_stride, kv_tok_stride,
                           kv_head_stride, o_tok_stride, o_head_stride, sel, cnt, maxk, H, NQ,
                           scale_log2, q_map, kv_map, geo, (hipStream_t)stream);
  else
    launch_bsa<kDirect, kDirect>(q, k, v, o, q_tok_stride, q_head_stride, kv_tok_stride,
                                 kv_head_stride, o_tok_stride, o_head_stride, sel, cnt, maxk, H,
                                 NQ, scale_log2, nullptr, nullptr, geo, (hipStream_t)stream);
  return fvsr_launch_status();
}

extern "C" int fvsr_bsa_fwd_window(const void* q, const void* k, const void* v, void* o,
                                   int64_t q_tok_stride, int64_t q_head_stride,
                                   int64_t kv_tok_stride, int64_t kv_head_stride,
                                   int64_t o_tok_stride, int64_t o_head_stride,
                                   const int32_t* sel, const int32_t* cnt, int64_t maxk,
                                   int64_t H, int64_t NQ, int64_t NK, int64_t head_dim,
                                   float sm_scale, int64_t frames, int64_t height, int64_t width,
                                   int kv_raster, void* stream) {
  if (H < 0 || NQ < 0 || NK < 0 || maxk < 0 || frames < 0 || height < 0 || width < 0)
    return FVSR_EINVAL;
  if (frames % 2 || height % 8 || width % 8) return FVSR_EINVAL;
  if (frames * height * width != NQ * kBlk) return FVSR_EINVAL;
  if (kv_raster && NK != NQ) return FVSR_EINVAL;
  if (H * NQ == 0) return FVSR_OK;
  const int rc = bsa_args_ok(q, k, v, o, q_tok_stride, q_head_stride, kv_tok_stride,
                             kv_head_stride, o_tok_stride, o_head_stride, sel, cnt, head_dim, H,
                             NQ);
  if (rc != FVSR_OK) return rc;
  // In-window byte offsets of the K/V stream are 32-bit: two frames of rows.
  const int64_t hw = height * width;
  if (kv_raster && 2 * hw * kv_tok_stride * 2 > 0xffffffffLL) return FVSR_EUNSUPPORTED;
  if (hw > 0x3fffffff) return FVSR_EUNSUPPORTED;
  const float scale_log2 = sm_scale * 1.4426950408889634f;
  const WinGeo geo{(int)width, (int)hw, (int)(width / 8), (int)((height / 8) * (width / 8))};
  if (kv_raster)
    launch_bsa<kWin, kWin>(q, k, v, o, q_tok_stride, q_head_stride, kv_tok_stride, kv_head_stride,
                           o_tok_stride, o_head_stride, sel, cnt, maxk, H, NQ, scale_log2,
                           nullptr, nullptr, geo, (hipStream_t)stream);
  else
    launch_bsa<kWin, kDirect>(q, k, v, o, q_tok_stride, q_head_stride, kv_tok_stride,
                              kv_head_stride, o_tok_stride, o_head_stride, sel, cnt, maxk, H, NQ,
                              scale_log2, nullptr, nullptr, geo, (hipStream_t)stream);
  return fvsr_launch_status();
}

extern "C" int fvsr_attn_dense(const void* q, const void* k, const void* v, void* o,
                               int64_t q_tok_stride, int64_t q_head_stride, int64_t kv_tok_stride,
                               int64_t kv_head_stride, int64_t o_tok_stride, int64_t o_head_stride,
                               int64_t H, int64_t NQ, int64_t NK, int64_t head_dim, float sm_scale,
                               void* stream) {
  if (H < 0 || NQ < 0 || NK < 0) return FVSR_EINVAL;
  if (H * NQ == 0) return FVSR_OK;
  static const int32_t kNone = 0;  // no block index is read in the dense mode
  const int rc = bsa_args_ok(q, k, v, o, q_tok_stride, q_head_stride, kv_tok_stride,
                             kv_head_stride, o_tok_stride, o_head_stride, &kNone, &kNone,
                             head_dim, H, NQ);
  if (rc != FVSR_OK) return rc;
  if (NK > 0x3fffffff) return FVSR_EUNSUPPORTED;
  const WinGeo geo{0, 0, 1, 1};
  launch_bsa<kDirect, kDirect, true>(q, k, v, o, q_tok_stride, q_head_stride, kv_tok_stride,
                                     kv_head_stride, o_tok_stride, o_head_stride, nullptr,
                                     nullptr, NK, H, NQ, sm_scale * 1.4426950408889634f,
                                     nullptr, nullptr, geo, (hipStream_t)stream);
  return fvsr_launch_status();
}
