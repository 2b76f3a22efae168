// FP8 (OCP e4m3fn) GEMM on CDNA4 matrix cores, contract M:
//   C[m,n] = epilogue( sum_k A[m,k] * B[n,k] )      A [M,K], B [N,K], K-contiguous
// which is torch._scaled_mm(x8, W8.t(), ...) of FP8Linear._mm
// (flashvsr_sm89_ops/fp8_linear.py:28-30).
//
// One workgroup = 4 wavefronts (one per SIMD) computes a 256 x 256 tile; each
// wave owns a 128 x 128 quadrant = 4 x 4 v_mfma_f32_32x32x64_f8f6f4 tiles with
// fp32 accumulators (256 per lane).  The weight operand is fed as the MFMA "A"
// side and the activation as the "B" side, so each lane's accumulators hold 4
// consecutive output columns of one output row.
//
// Main loop (K a multiple of 256, at least 512): a persistent kernel, one
// workgroup per CU, streaming K through two 64 KB LDS pair slots (128 bytes
// of K for the 256 A rows and 256 B rows) filled by buffer_load ... lds
// straight from memory, one load per MFMA; the last K steps of a tile already
// load the next tile's first pairs (details at gemm_fp8_ring).  Other K (a
// multiple of 16) use a register-staged loop with K step 128.
//
// Epilogue: y = acc * (sa[m] * sb[n]) + bias[n], rounded to bf16, leaves
// through a per-wave LDS staging area as 16-byte row chunks:
//   FVSR_EPI_BIAS      C = y
//   FVSR_EPI_ROWMAX    C = y, plus max(C) over each row's 128-column slab
//   FVSR_EPI_GATE_ADD  C = bf16(res + bf16(gate[n] * y))
// Workgroups are renumbered so each XCD (workgroup ids are dispatched round
// robin over the 8 XCDs) walks a contiguous, M-grouped range of tiles.
#include <utility>

#include "common.h"

// Buffer loads straight into LDS (buffer_load_dwordx4 ... lds): the 16 bytes
// at base + voffset + soffset of every lane land at M0 + 16 * lane.
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__device__ void fvsr_buffer_load_lds(i32x4_t rsrc, __attribute__((address_space(3))) void* lds,
                                     int size, int voffset, int soffset, int offset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.lds");
// Raw buffer store of 16 bytes at base + voffset + soffset; a store whose
// voffset lies past the descriptor's byte count is dropped by the hardware.
__device__ void fvsr_buffer_store_b128(u32x4_t data, i32x4_t rsrc, int voffset, int soffset,
                                       int aux) __asm("llvm.amdgcn.raw.buffer.store.v4i32");

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
#define LDS_AS __attribute__((address_space(3)))

constexpr int BM = 256, BN = 256;
constexpr int kThreads = 256;
constexpr int kGroupM = 8;

struct EpiArgs {
  const float* sa;
  const float* sb;
  const uint16_t* bias;
  uint16_t* c;
  int64_t ldc;
  float* amax_part;
  int64_t nparts;
  const uint16_t* res;
  const uint16_t* gate;
  int sa_row, sb_col;
  int vec_params;  // sb (per column) 16-byte aligned and bias 8-byte aligned
  int res_vec;     // gate-add: N, ldc multiples of 8 and res / c / gate 16-byte aligned
  int direct;      // c 16-byte aligned, ldc % 8 == 0, (M + 256) * ldc * 2 below 2^32
};

FVSR_DEV void map_tile(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int q = total / 8, r = total % 8;
  const int xcd = bid % 8, loc = bid / 8;
  const int logical = xcd < r ? xcd * (q + 1) + loc : r * (q + 1) + (xcd - r) * q + loc;
  const int per_group = kGroupM * tiles_n;
  const int group = logical / per_group;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = logical % per_group;
  if (tiles_n <= 8) {
    // Narrow N (the 1536-wide projections: 6 column tiles): the column tiles
    // of one row panel run side by side, so the panel (K = 8960 for ffn2) is
    // fetched once per round (ffn2 232 -> 228 us, o 56.5 -> 55.6 us).
    tm = first_m + in_group / tiles_n;
    tn = in_group % tiles_n;
  } else {
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
  }
}

FVSR_DEV void zero_acc(v16f (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
}

template <int MJ>
FVSR_DEV void mfma_block(v16f (&acc)[4][MJ], const v8i (&fa)[MJ], const v8i (&fb)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[i], fa[j], acc[i][j], 0, 0,
                                                                   0, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Epilogue through a bf16 [256][256] LDS tile held in four 64-row pieces.
// ---------------------------------------------------------------------------
struct CTile {
  uint16_t LDS_AS* part[4];  // rows 64*i .. 64*i+63
  __device__ __forceinline__ uint16_t LDS_AS* row(int r) const { return part[r >> 6] + (r & 63) * BN; }
};

template <int EPI>
FVSR_DEV void epilogue(const v16f (&acc)[4][4], const CTile& ct, int64_t m0, int64_t n0,
                       int64_t M, int64_t N, const EpiArgs& ep, int wm, int wn, int lane) {
  // Phase 1: acc[i][j][g*4+r] is row ml = wm*128 + j*32 + (lane&31), column
  // nl = wn*128 + i*32 + g*8 + (lane>>5)*4 + r.  8-byte units are XOR-swizzled
  // with the row so 32 lanes writing 32 rows do not share banks.
  float sam[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t mg = m0 + wm * 128 + j * 32 + (lane & 31);
    sam[j] = ep.sa[ep.sa_row ? (mg < M ? mg : M - 1) : 0];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = wn * 128 + i * 32 + g * 8 + (lane >> 5) * 4;
      float sbv[4], bv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t ng = n0 + nl + r < N ? n0 + nl + r : N - 1;
        sbv[r] = ep.sb[ep.sb_col ? ng : 0];
        bv[r] = ep.bias ? bf2f(ep.bias[ng]) : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ml = wm * 128 + j * 32 + (lane & 31);
        float y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = acc[i][j][g * 4 + r] * (sam[j] * sbv[r]) + bv[r];
        const int unit = (nl >> 2) ^ (ml & 63);
        *(u32x2_t LDS_AS*)(ct.row(ml) + unit * 4) =
            u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
      }
    }
  }
  __syncthreads();

  // Phase 2: 32 threads per 512-byte row, 16 bytes (8 columns) each.
  const int cpos = threadIdx.x & 31;
  const int64_t slab0 = n0 / 128;
  for (int rr = threadIdx.x >> 5; rr < BM; rr += kThreads / 32) {
    const int64_t m = m0 + rr;
    const int nl = cpos * 8;
    const int64_t n = n0 + nl;
    const uint16_t LDS_AS* crow = ct.row(rr);
    const u32x2_t lo = *(const u32x2_t LDS_AS*)(crow + (((nl >> 2) ^ (rr & 63)) * 4));
    const u32x2_t hi = *(const u32x2_t LDS_AS*)(crow + ((((nl >> 2) + 1) ^ (rr & 63)) * 4));
    u32x4_t v = {lo[0], lo[1], hi[0], hi[1]};
    float vmax = -__builtin_huge_valf();
    if (EPI == FVSR_EPI_ROWMAX) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if (n + 2 * w < N) vmax = fmaxf(vmax, bf_lo(v[w]));
        if (n + 2 * w + 1 < N) vmax = fmaxf(vmax, bf_hi(v[w]));
      }
    }
    if (m < M && n < N) {
      uint16_t* cp = ep.c + m * ep.ldc + n;
      if (EPI == FVSR_EPI_GATE_ADD) {
        const uint16_t* rp = ep.res + m * ep.ldc + n;
        if (n + 7 < N && ((((uintptr_t)cp) | (uintptr_t)rp | (uintptr_t)(ep.gate + n)) & 15) == 0) {
          const u32x4_t rv = *(const u32x4_t*)rp;
          const u32x4_t gv = *(const u32x4_t*)(ep.gate + n);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float t0 = round_bf16(bf_lo(gv[w]) * bf_lo(v[w]));
            const float t1 = round_bf16(bf_hi(gv[w]) * bf_hi(v[w]));
            v[w] = pack_bf16x2(bf_lo(rv[w]) + t0, bf_hi(rv[w]) + t1);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (n + e >= N) break;
            const float y = (e & 1) ? bf_hi(v[e >> 1]) : bf_lo(v[e >> 1]);
            const float t = round_bf16(bf2f(ep.gate[n + e]) * y);
            const float o = round_bf16(bf2f(rp[e]) + t);
            const uint32_t ob = pack_bf16x2(o, 0.0f) & 0xffffu;
            v[e >> 1] = (e & 1) ? ((v[e >> 1] & 0xffffu) | (ob << 16))
                                : ((v[e >> 1] & 0xffff0000u) | ob);
          }
        }
      }
      if (n + 7 < N && (((uintptr_t)cp) & 15) == 0) {
        *(u32x4_t*)cp = v;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n + e < N) cp[e] = (uint16_t)((e & 1) ? (v[e >> 1] >> 16) : (v[e >> 1] & 0xffffu));
      }
    }
    if (EPI == FVSR_EPI_ROWMAX) {
      // 16 threads cover one 128-column slab of this row.
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, o, 64));
      const int64_t slab = slab0 + (cpos >> 4);
      if ((cpos & 15) == 0 && m < M && n < N && slab < ep.nparts)
        ep.amax_part[m * ep.nparts + slab] = vmax;
    }
  }
}

// ---------------------------------------------------------------------------
// Main loop, K % 64 == 0 and K >= 256: persistent direct-to-LDS ring.
// ---------------------------------------------------------------------------
// Tile shapes of the ring kernel: 256 output columns (B rows) by TM = 64 * MJ
// output rows (A rows); each of the 4 waves owns TM / 2 rows (MJ blocks of
// 32) by 128 columns (4 blocks).  MJ = 4 (256 x 256) everywhere except where
// a single round of 128-row tiles covers the output that 256-row tiles would
// leave mostly idle (C1: 4224 x 1536 is 102 tiles of 256 rows, 198 of 128).
template <int MJ>
struct Tile {
  static constexpr int TM = 64 * MJ;
  static constexpr int kPairBytes = (TM + BN) * 128;  // 64 KB (MJ 4) or 48 KB (MJ 2)
  static constexpr int kLoadsA = TM / 32;              // A loads per wave per pair
};

// The ring holds K in pairs of 64-byte steps: a pair slot keeps 128 bytes of
// every A row and B row, so each load covers whole 128-byte lines.
// 16-byte chunk c of row r sits at chunk position c ^ (r & 7) ^ ((r >> 3) & 1):
// any 8 consecutive rows read at one logical chunk hit 8 distinct 16-byte
// bank groups, and any 16 consecutive rows 16 distinct (row parity, chunk)
// pairs, so ds_read_b128 is conflict-free whether the LDS serves 8 or 16
// lanes per cycle.
FVSR_DEV int swz128(int r, int c) { return c ^ (r & 7) ^ ((r >> 3) & 1); }

// Per-lane byte offsets of the 16-byte pieces this lane streams for one pair:
// load t of an operand covers 8 of the wave's rows (A: TM / 4 rows per wave,
// B: 64), lane l taking row 8*t + l/8 (clamped to the matrix) and the chunk
// that lands at position l % 8.  Offsets fit 32 bits (checked on the host),
// so each load is a uniform base plus a per-lane 32-bit offset.
template <int MJ>
struct DmaOffs {
  uint32_t a[Tile<MJ>::kLoadsA], b[8];
  uint32_t ta, tb;  // L2 prefetch (long K): row starts of this lane's A row and B row
};

template <int MJ>
FVSR_DEV void dma_offsets(DmaOffs<MJ>& o, int64_t m0, int64_t n0, int64_t M, int64_t N,
                          int64_t lda, int64_t ldb, int wave, int lane) {
  const int rl = lane >> 3;
  const int c = lane & 7;
#pragma unroll
  for (int t = 0; t < Tile<MJ>::kLoadsA; ++t) {
    const int r = wave * (Tile<MJ>::TM / 4) + t * 8 + rl;
    const int64_t ga = m0 + r < M ? m0 + r : M - 1;
    o.a[t] = (uint32_t)(ga * lda + swz128(r, c) * 16);  // the swizzle is an involution in c
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int r = wave * 64 + t * 8 + rl;
    const int64_t gb = n0 + r < N ? n0 + r : N - 1;
    o.b[t] = (uint32_t)(gb * ldb + swz128(r, c) * 16);
  }
  {
    const int64_t ra = m0 + wave * (Tile<MJ>::TM / 4) + lane % (Tile<MJ>::TM / 4);
    const int64_t rb = n0 + wave * 64 + lane;
    o.ta = (uint32_t)((ra < M ? ra : M - 1) * lda);
    o.tb = (uint32_t)((rb < N ? rb : N - 1) * ldb);
  }
}

// Raw buffer descriptor over `base` (stride 0, range `bytes`; no range limit
// below 4 GB by default).
FVSR_DEV i32x4_t make_rsrc(const void* base, uint32_t bytes = 0xffffffffu) {
  const uint64_t p = (uint64_t)base;
  return i32x4_t{(int)(uint32_t)p, (int)(uint32_t)(p >> 32), (int)bytes, 0x00020000};
}

// Stream one pair (A and B bytes [k0, k0+128) of the tile's rows) into a pair
// slot.  The per-lane offsets stay in VGPRs and k0 rides in the scalar offset.
template <int MJ>
FVSR_DEV void issue_pair(uint8_t LDS_AS* slot, i32x4_t ra, i32x4_t rb, int k0,
                         const DmaOffs<MJ>& o, int wave) {
  constexpr int LA = Tile<MJ>::kLoadsA;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (t < LA)
      fvsr_buffer_load_lds(ra, (void LDS_AS*)(slot + (wave * LA + t) * 1024), 16,
                           __builtin_bit_cast(int, o.a[t]), k0, 0, 0);
    fvsr_buffer_load_lds(rb, (void LDS_AS*)(slot + Tile<MJ>::TM * 128 + (wave * 8 + t) * 1024),
                         16, __builtin_bit_cast(int, o.b[t]), k0, 0, 0);
  }
}

// MFMA fragment of one 64-byte step (half `hs` of a pair) of row r: lane
// half h takes logical chunks 4hs + 2h and 4hs + 2h + 1.
FVSR_DEV v8i read_frag(const uint8_t LDS_AS* base, int r, int c0) {
  const u32x4_t lo = *(const u32x4_t LDS_AS*)(base + r * 128 + (swz128(r, c0) << 4));
  const u32x4_t hi = *(const u32x4_t LDS_AS*)(base + r * 128 + (swz128(r, c0 + 1) << 4));
  return v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
             (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// All fragments of one step (the wave's A rows, then its B rows).
template <int MJ>
FVSR_DEV void read_step(const uint8_t LDS_AS* slot, int hs, int wm, int wn, int lane,
                        v8i (&fa)[MJ], v8i (&fb)[4]) {
  const int c0 = 4 * hs + 2 * (lane >> 5);
  const int ra = wm * (32 * MJ) + (lane & 31), rb = wn * 128 + (lane & 31);
#pragma unroll
  for (int j = 0; j < MJ; ++j) fa[j] = read_frag(slot, ra + 32 * j, c0);
#pragma unroll
  for (int i = 0; i < 4; ++i) fb[i] = read_frag(slot + Tile<MJ>::TM * 128, rb + 32 * i, c0);
}

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSgMfma = 0x008, kSgVmemRead = 0x020, kSgDsRead = 0x100;

// s_waitcnt immediate (gfx9 encoding): vmcnt in bits 3:0 and 15:14, expcnt
// 6:4 (left open), lgkmcnt 11:8 (15 = left open).
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8);
}
constexpr int kWaitVm0 = waitcnt_imm(0, 15);

struct RingCtx {
  i32x4_t ra, rb;
  int wave, wm, wn, lane;
  int kmax;               // K offset of the last pair
  uint8_t LDS_AS* touch;  // 512 bytes of LDS that nothing reads
};

// Long K (ffn2, K = 8960): the operand panels are used by few tiles, so most
// pair loads miss L2, and the two LDS pair slots put them only one pair ahead
// of the MFMAs.  Each pair step also fetches, into a dummy LDS word, the
// first 4 bytes of this lane's A row and B row two pairs further on: the
// 128-byte lines land in L2 ahead of the pair's own loads.  Exactly two such
// loads follow every pair's loads, so a pair is waited for with vmcnt(2).
// (ffn2 218 -> 208 us; at K = 1536 the panels stay in L2 and the extra loads
// cost 5-8%, so they are only issued for K >= 4096.)
constexpr int kTouchAhead = 2;
template <int MJ>
FVSR_DEV void touch_pairs(const RingCtx& c, const DmaOffs<MJ>& o, int k0) {
  const int kt = min(k0 + kTouchAhead * 128, c.kmax);
  fvsr_buffer_load_lds(c.ra, (void LDS_AS*)c.touch, 4, __builtin_bit_cast(int, o.ta), kt, 0, 0);
  fvsr_buffer_load_lds(c.rb, (void LDS_AS*)(c.touch + 256), 4, __builtin_bit_cast(int, o.tb), kt,
                       0, 0);
}

// One 64-byte K step s of a tile (fragments of s in fa/fb):
//   PAIR (s odd): wait until this wave's loads of the next pair (steps s+1,
//     s+2) have landed and its reads of step s are done, then barrier: the
//     pair is in LDS for every wave and the pair slot holding steps s-1, s
//     is free; stream the pair of steps s+3, s+4 into it (`ds`, K offset k0,
//     per-lane offsets `o`: the next tile's when past the end) -- two steps
//     ahead of the reads that need it;
//   read step s+1's fragments (pair slot `rd`, half RH) into na/nb;
//   run the 4 * MJ MFMAs of step s (ZERO: start the accumulators from 0).
// The loads are spread evenly over the MFMAs (a burst of them stalls the
// wave's instruction stream) and the reads go with the first half of the
// MFMAs, leaving the second half of the step for them to land.
// Scheduling of one step: MFMA q is preceded by its share of the NL loads
// (PAIR steps) and, in the first half of the step, followed by its share of
// the ND fragment reads.
template <bool PAIR, int NM, int NL, int ND, int Q>
FVSR_DEV void sched_slot() {
  if (PAIR) __builtin_amdgcn_sched_group_barrier(kSgVmemRead, NL * (Q + 1) / NM - NL * Q / NM, 0);
  __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
  if (2 * Q < NM)
    __builtin_amdgcn_sched_group_barrier(kSgDsRead, ND * (Q + 1) / (NM / 2) - ND * Q / (NM / 2),
                                         0);
}

template <bool PAIR, int NM, int NL, int ND, int... Q>
FVSR_DEV void sched_step(std::integer_sequence<int, Q...>) {
  (sched_slot<PAIR, NM, NL, ND, Q>(), ...);
}

template <int MJ, bool PAIR, int RH, bool ZERO, bool TOUCH>
FVSR_DEV void ring_step(const RingCtx& c, const DmaOffs<MJ>& o, int k0, const uint8_t LDS_AS* rd,
                        uint8_t LDS_AS* ds, v16f (&acc)[4][MJ], const v8i (&fa)[MJ],
                        const v8i (&fb)[4], v8i (&na)[MJ], v8i (&nb)[4]) {
  __builtin_amdgcn_sched_barrier(0);  // nothing (MFMAs included) moves across a step boundary
  if (PAIR) {
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(TOUCH ? 2 : 0, 0));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS access may move across the barrier
    __builtin_amdgcn_sched_barrier(0);
    issue_pair(ds, c.ra, c.rb, k0, o, c.wave);
    if (TOUCH) touch_pairs<MJ>(c, o, k0);
  }
  read_step<MJ>(rd, RH, c.wm, c.wn, c.lane, na, nb);
  if (ZERO) {
    const v16f z = {};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < MJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[i], fa[j], z, 0, 0, 0, 0,
                                                                     0, 0);
  } else {
    mfma_block<MJ>(acc, fa, fb);
  }
  sched_step<PAIR, 4 * MJ, Tile<MJ>::kLoadsA + 8, 2 * (MJ + 4)>(
      std::make_integer_sequence<int, 4 * MJ>{});
}

// Per-wave epilogue area: 32 rows x 64 columns of bf16 staging (4 KB, one
// eighth of the wave's 128 x 128 quadrant per pass; 8-byte units XOR-swizzled
// with the row so that 16 lanes writing 16 rows cover all banks), then the
// quadrant's epilogue parameters as fp32: sa of its 128 rows, sb and bias of
// its 128 columns (1.5 KB).
constexpr int kEpiStageBytes = 32 * 128;
constexpr int kEpiWaveBytes = kEpiStageBytes + 3 * 128 * 4;
FVSR_DEV int epi_off(int row, int unit) { return row * 128 + ((unit ^ (row & 15)) << 3); }

// This lane's share of the wave's parameters (rows / columns q*64 + lane of
// the wave's `wrows` rows and 128 columns; rows past them are loaded but not
// used), loaded into registers ahead of time and parked in LDS by
// put_epi_params.
struct EpiParamRegs {
  float sa[2], sb[2];
  uint32_t bias[2];
};

FVSR_DEV void fetch_epi_params(EpiParamRegs& r, const EpiArgs& e, int64_t m0, int64_t n0,
                               int64_t M, int64_t N, int wm, int wn, int wrows, int lane) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int64_t m = m0 + wm * wrows + q * 64 + lane, n = n0 + wn * 128 + q * 64 + lane;
    const int64_t mc = m < M ? m : M - 1, nc = n < N ? n : N - 1;
    r.sa[q] = e.sa[e.sa_row ? mc : 0];
    r.sb[q] = e.sb[e.sb_col ? nc : 0];
    r.bias[q] = e.bias ? (uint32_t)e.bias[nc] << 16 : 0u;
  }
}

FVSR_DEV void put_epi_params(const EpiParamRegs& r, uint8_t LDS_AS* prm, int lane) {
  float LDS_AS* sa_l = (float LDS_AS*)prm;
  float LDS_AS* sb_l = sa_l + 128;
  uint32_t LDS_AS* bi_l = (uint32_t LDS_AS*)(sb_l + 128);
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    sa_l[q * 64 + lane] = r.sa[q];
    sb_l[q * 64 + lane] = r.sb[q];
    bi_l[q * 64 + lane] = r.bias[q];
  }
}

// Phase 1 of pass (ip, j): y = acc * (sa * sb) + bias for column blocks
// 2ip, 2ip+1 and row block j, as bf16 into the staging area.
FVSR_DEV void epi_stage(const v16f (&acc)[4][4], uint16_t LDS_AS* stg,
                        const uint8_t LDS_AS* prm, int lane, int ip, int j) {
  const float LDS_AS* sa_l = (const float LDS_AS*)prm;
  const float LDS_AS* sb_l = sa_l + 128;
  const float LDS_AS* bi_l = sb_l + 128;
  const int h = lane >> 5;
  const int row = lane & 31;
  const float sam = sa_l[j * 32 + row];
#pragma unroll
  for (int ii = 0; ii < 2; ++ii)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int cl = (2 * ip + ii) * 32 + g * 8 + h * 4;
      const f32x4_t sb = *(const f32x4_t LDS_AS*)(sb_l + cl);
      const f32x4_t bw = *(const f32x4_t LDS_AS*)(bi_l + cl);
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = acc[2 * ip + ii][j][g * 4 + r] * (sam * sb[r]) + bw[r];
      *(u32x2_t LDS_AS*)((uint8_t LDS_AS*)stg + epi_off(row, ii * 8 + g * 2 + h)) =
          u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
    }
}

// Phase 2 of pass (ip, j): 32 rows of 64 columns leave as 16-byte chunks (8
// lanes per row), with the gate-add / row-max epilogues applied on the way.
template <int EPI>
FVSR_DEV void epi_store(const uint16_t LDS_AS* stg, int64_t mw, int64_t nw, int64_t M, int64_t N,
                        const EpiArgs& e, int lane, int ip, int j, float (&vmax)[4]) {
  const int c8 = lane & 7;
  const int64_t n = nw + ip * 64 + c8 * 8;
  // Gate-add with vector rows: the pass's four residual rows and its gate
  // columns are loaded before any store (the stores may alias them when c ==
  // res, which would otherwise order each load after the previous store).
  u32x4_t rv[4], gv = {0u, 0u, 0u, 0u};
  if (EPI == FVSR_EPI_GATE_ADD && e.res_vec) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int64_t m = mw + j * 32 + s * 8 + (lane >> 3);
      const bool ok = m < M && n < N;
      rv[s] = *(const u32x4_t*)(e.res + (ok ? m : 0) * e.ldc + (ok ? n : 0));
    }
    gv = *(const u32x4_t*)(e.gate + (n < N ? n : 0));
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int row = s * 8 + (lane >> 3);
    const int64_t m = mw + j * 32 + row;
    const u32x2_t lo = *(const u32x2_t LDS_AS*)((const uint8_t LDS_AS*)stg + epi_off(row, 2 * c8));
    const u32x2_t hi =
        *(const u32x2_t LDS_AS*)((const uint8_t LDS_AS*)stg + epi_off(row, 2 * c8 + 1));
    u32x4_t v = {lo[0], lo[1], hi[0], hi[1]};
    if (EPI == FVSR_EPI_ROWMAX) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if (n + 2 * w < N) vmax[s] = fmaxf(vmax[s], bf_lo(v[w]));
        if (n + 2 * w + 1 < N) vmax[s] = fmaxf(vmax[s], bf_hi(v[w]));
      }
    }
    if (m < M && n < N) {
      uint16_t* cp = e.c + m * e.ldc + n;
      if (EPI == FVSR_EPI_GATE_ADD) {
        const uint16_t* rp = e.res + m * e.ldc + n;
        if (e.res_vec) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float t0 = round_bf16(bf_lo(gv[w]) * bf_lo(v[w]));
            const float t1 = round_bf16(bf_hi(gv[w]) * bf_hi(v[w]));
            v[w] = pack_bf16x2(bf_lo(rv[s][w]) + t0, bf_hi(rv[s][w]) + t1);
          }
        } else {
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            if (n + q >= N) break;
            const float y = (q & 1) ? bf_hi(v[q >> 1]) : bf_lo(v[q >> 1]);
            const float t = round_bf16(bf2f(e.gate[n + q]) * y);
            const float o = round_bf16(bf2f(rp[q]) + t);
            const uint32_t ob = pack_bf16x2(o, 0.0f) & 0xffffu;
            v[q >> 1] = (q & 1) ? ((v[q >> 1] & 0xffffu) | (ob << 16))
                                : ((v[q >> 1] & 0xffff0000u) | ob);
          }
        }
      }
      if (n + 7 < N && (((uintptr_t)cp) & 15) == 0) {
        *(u32x4_t*)cp = v;
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (n + q < N) cp[q] = (uint16_t)((q & 1) ? (v[q >> 1] >> 16) : (v[q >> 1] & 0xffffu));
      }
    }
  }
}

// Epilogue of tiles whose 256 columns all lie inside the output (bias and
// row-max epilogues).  The same eight 32 x 64 passes (column half ip, row
// block j) through the wave's staging area as epi_stage / epi_store, arranged
// so that nothing waits on LDS per value: the column scales and biases of one
// 64-column half are read into registers once (64 VGPRs), and the passes are
// software-pipelined -- pass p's staged rows are read back as 16-byte row
// chunks, pass p + 1 is converted and written over them, then pass p's chunks
// are stored (8 lanes = one 128-byte row segment).  A wave's LDS accesses
// execute in order, so the rewrite cannot overtake the reads.  Stores go
// through a buffer descriptor spanning the M output rows: stores of rows past
// M are dropped by its range check.
struct FastParams {
  f32x4_t sb[2][4], bias[2][4];
};

FVSR_DEV void fast_params(FastParams& fp, const uint8_t LDS_AS* prm, int ip, int h) {
  const float LDS_AS* sb_l = (const float LDS_AS*)prm + 128;
  const float LDS_AS* bi_l = sb_l + 128;
#pragma unroll
  for (int ii = 0; ii < 2; ++ii)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int cl = (2 * ip + ii) * 32 + g * 8 + h * 4;
      fp.sb[ii][g] = *(const f32x4_t LDS_AS*)(sb_l + cl);
      fp.bias[ii][g] = *(const f32x4_t LDS_AS*)(bi_l + cl);
    }
}

// Convert pass (ip, j) and write it to the staging area.
template <int MJ>
FVSR_DEV void fast_stage(const v16f (&acc)[4][MJ], const FastParams& fp, float sam,
                         uint16_t LDS_AS* stg, int ip, int j, int row, int h) {
#pragma unroll
  for (int ii = 0; ii < 2; ++ii)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        y[r] = acc[2 * ip + ii][j][g * 4 + r] * (sam * fp.sb[ii][g][r]) + fp.bias[ii][g][r];
      *(u32x2_t LDS_AS*)((uint8_t LDS_AS*)stg + epi_off(row, ii * 8 + g * 2 + h)) =
          u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
    }
}

// Read the staged pass back: row s * 8 + lane / 8, 16-byte chunk lane % 8.
FVSR_DEV void fast_read(const uint16_t LDS_AS* stg, u32x4_t (&v)[4], int lane) {
  const int c8 = lane & 7;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int r8 = s * 8 + (lane >> 3);
    const u32x2_t lo = *(const u32x2_t LDS_AS*)((const uint8_t LDS_AS*)stg + epi_off(r8, 2 * c8));
    const u32x2_t hi =
        *(const u32x2_t LDS_AS*)((const uint8_t LDS_AS*)stg + epi_off(r8, 2 * c8 + 1));
    v[s] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
  }
}

// Byte offsets into the output are unsigned 32-bit (the host admits outputs
// below 4 GiB); the sum is formed in uint32_t and handed to the intrinsic's
// int operand bit for bit.  The stores are non-temporal (cache policy `nt`):
// every workgroup writes its 128 KB output tile at about the same moment, and
// allocating those lines in L2 evicted the operand panels the next tiles read
// (qkv 111 -> 107 us, ffn0 217 -> 207 us, C1 15.5 -> 14.1 us; bit-identical).
constexpr int kStoreNT = 2;  // aux bits of the raw buffer store: nt
template <int EPI>
FVSR_DEV void fast_store(const u32x4_t (&v)[4], float (&vmax)[4], i32x4_t rc, uint32_t voff,
                         int64_t ldc, int ip, int j) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (EPI == FVSR_EPI_ROWMAX) {
#pragma unroll
      for (int w = 0; w < 4; ++w) vmax[s] = fmaxf(vmax[s], fmaxf(bf_lo(v[s][w]), bf_hi(v[s][w])));
    }
    const uint32_t off = voff + (uint32_t)((j * 32 + s * 8) * ldc * 2 + ip * 128);
    fvsr_buffer_store_b128(v[s], rc, __builtin_bit_cast(int, off), 0, kStoreNT);
  }
}

template <int EPI, int MJ>
FVSR_DEV void epi_fast(const v16f (&acc)[4][MJ], uint16_t LDS_AS* stg, const uint8_t LDS_AS* prm,
                       int64_t mw, int64_t nw, int64_t M, const EpiArgs& e, i32x4_t rc,
                       int lane) {
  const float LDS_AS* sa_l = (const float LDS_AS*)prm;
  const int h = lane >> 5, row = lane & 31;
  float sam[MJ];
#pragma unroll
  for (int j = 0; j < MJ; ++j) sam[j] = sa_l[j * 32 + row];
  // Store offset of row lane / 8, chunk lane % 8; each pass adds its row
  // block, row group and column half (all in the offset the range check
  // covers).
  const uint32_t voff = (uint32_t)(((mw + (lane >> 3)) * e.ldc + nw + (lane & 7) * 8) * 2);
  float vmax[MJ][4];
#pragma unroll
  for (int j = 0; j < MJ; ++j)
#pragma unroll
    for (int s = 0; s < 4; ++s) vmax[j][s] = -__builtin_huge_valf();
  FastParams fp;
  fast_params(fp, prm, 0, h);
  fast_stage<MJ>(acc, fp, sam[0], stg, 0, 0, row, h);
  // Passes p = ip * MJ + j.
#pragma unroll
  for (int p = 0; p < 2 * MJ; ++p) {
    const int ip = p / MJ, j = p % MJ;
    u32x4_t v[4];
    fast_read(stg, v, lane);
    if (p == MJ - 1) fast_params(fp, prm, 1, h);
    if (p + 1 < 2 * MJ)
      fast_stage<MJ>(acc, fp, sam[(p + 1) % MJ], stg, (p + 1) / MJ, (p + 1) % MJ, row, h);
    fast_store<EPI>(v, vmax[j], rc, voff, e.ldc, ip, j);
  }
  if (EPI == FVSR_EPI_ROWMAX) {
    // 8 lanes per row cover 64 columns per pass; both halves = the slab.
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float v = vmax[j][s];
#pragma unroll
        for (int o = 4; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
        const int64_t m = mw + j * 32 + s * 8 + (lane >> 3);
        if ((lane & 7) == 0 && m < M) e.amax_part[m * e.nparts + nw / 128] = v;
      }
  }
}

FVSR_DEV void tile_origin(int t, int tiles_m, int tiles_n, int tile_rows, int64_t& m0,
                          int64_t& n0) {
  int tm, tn;
  map_tile(t, tiles_m, tiles_n, tm, tn);
  m0 = (int64_t)tm * tile_rows;
  n0 = (int64_t)tn * BN;
}

// Persistent kernel (K a multiple of 256, at least 512).  Workgroup b takes
// tiles b, b + G, b + 2G, ... (G = grid size, a multiple of 8, so its tiles
// stay within its XCD's M-grouped range).  The K steps of consecutive tiles
// form one stream through the two pair slots: the last two pair loads of a
// tile already fetch the next tile's pairs 0 and 1 (pair q lives in slot
// q % 2, and K/128 is even) and its last step reads the next tile's step-0
// fragments, so the epilogue overlaps the next tile's first loads.  The
// epilogue stages through a spare 32 KB that no load targets (8 KB per
// wave).  After a workgroup's last tile the same stream re-fetches that
// tile's first pairs (harmless) and the workgroup drains its loads before it
// exits.
template <int EPI, bool DIRECT, int MJ, bool TOUCH = false>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_fp8_ring(const uint8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B,
                   int64_t ldb, int64_t M, int64_t N, int64_t K, EpiArgs ep) {
  static_assert(MJ == 4 || (MJ == 2 && DIRECT), "128-row tiles take the fast epilogue only");
  constexpr int TM = Tile<MJ>::TM;
  __shared__ __attribute__((aligned(1024))) uint8_t pair0[Tile<MJ>::kPairBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t pair1[Tile<MJ>::kPairBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t spare[4 * kEpiWaveBytes];
  __shared__ __attribute__((aligned(256))) uint8_t touch_lds[TOUCH ? 512 : 4];
  uint8_t LDS_AS* p0 = (uint8_t LDS_AS*)pair0;
  uint8_t LDS_AS* p1 = (uint8_t LDS_AS*)pair1;

  const int tiles_m = (int)((M + TM - 1) / TM), tiles_n = (int)((N + BN - 1) / BN);
  const int tiles = tiles_m * tiles_n;
  int t = blockIdx.x;
  if (t >= tiles) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  uint8_t LDS_AS* epa = (uint8_t LDS_AS*)spare + wave * kEpiWaveBytes;
  uint16_t LDS_AS* stg = (uint16_t LDS_AS*)epa;
  uint8_t LDS_AS* prm = epa + kEpiStageBytes;
  const int KT = (int)(K / 64);

  RingCtx c{make_rsrc(A), make_rsrc(B), wave, wm, wn, lane, (int)K - 128,
            (uint8_t LDS_AS*)touch_lds};
  int64_t m0, n0;
  tile_origin(t, tiles_m, tiles_n, TM, m0, n0);
  DmaOffs<MJ> cur;
  dma_offsets<MJ>(cur, m0, n0, M, N, lda, ldb, wave, lane);
  issue_pair<MJ>(p0, c.ra, c.rb, 0, cur, wave);
  issue_pair<MJ>(p1, c.ra, c.rb, 128, cur, wave);
  if (TOUCH) touch_pairs<MJ>(c, cur, 128);
  // The first pair (the older half of the loads in flight) has landed.
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(Tile<MJ>::kLoadsA + 8 + (TOUCH ? 2 : 0), 15));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  v16f acc[4][MJ];
  v8i fa[MJ], fb[4], na[MJ], nb[4];
  read_step<MJ>(p0, 0, wm, wn, lane, fa, fb);

  for (;;) {
    // First trip: steps 0-3 (accumulators start from 0 at step 0).
    ring_step<MJ, false, 1, true, TOUCH>(c, cur, 0, p0, p0, acc, fa, fb, na, nb);
    ring_step<MJ, true, 0, false, TOUCH>(c, cur, 2 * 128, p1, p0, acc, na, nb, fa, fb);
    ring_step<MJ, false, 1, false, TOUCH>(c, cur, 0, p1, p1, acc, fa, fb, na, nb);
    ring_step<MJ, true, 0, false, TOUCH>(c, cur, 3 * 128, p0, p1, acc, na, nb, fa, fb);
    // Steady state: steps kt .. kt+3 load pairs kt/2 + 2 and kt/2 + 3.
    for (int kt = 4; kt < KT - 4; kt += 4) {
      ring_step<MJ, false, 1, false, TOUCH>(c, cur, 0, p0, p0, acc, fa, fb, na, nb);
      ring_step<MJ, true, 0, false, TOUCH>(c, cur, (kt + 4) * 64, p1, p0, acc, na, nb, fa, fb);
      ring_step<MJ, false, 1, false, TOUCH>(c, cur, 0, p1, p1, acc, fa, fb, na, nb);
      ring_step<MJ, true, 0, false, TOUCH>(c, cur, (kt + 6) * 64, p0, p1, acc, na, nb, fa, fb);
    }
    // Last trip: steps KT-4 .. KT-1; their loads are the next tile's pairs 0
    // and 1 and the last reads are the next tile's step 0.
    const int tn = t + (int)gridDim.x;
    int64_t m1 = m0, n1 = n0;
    if (tn < tiles) tile_origin(tn, tiles_m, tiles_n, TM, m1, n1);
    DmaOffs<MJ> nxt;
    dma_offsets<MJ>(nxt, m1, n1, M, N, lda, ldb, wave, lane);
    // This tile's epilogue parameters load under the last trip's MFMAs.
    EpiParamRegs epr;
    fetch_epi_params(epr, ep, m0, n0, M, N, wm, wn, TM / 2, lane);
    ring_step<MJ, false, 1, false, TOUCH>(c, nxt, 0, p0, p0, acc, fa, fb, na, nb);
    ring_step<MJ, true, 0, false, TOUCH>(c, nxt, 0, p1, p0, acc, na, nb, fa, fb);
    ring_step<MJ, false, 1, false, TOUCH>(c, nxt, 0, p1, p1, acc, fa, fb, na, nb);
    ring_step<MJ, true, 0, false, TOUCH>(c, nxt, 128, p0, p1, acc, na, nb, fa, fb);

    // Epilogue (fa/fb now hold the next tile's step-0 fragments): passes of
    // 32 rows x 64 columns through the wave's own staging area.
    const int el = lane_here();
    const int64_t mw = m0 + wm * (TM / 2), nw = n0 + wn * 128;
    put_epi_params(epr, prm, el);
    if constexpr (DIRECT) {
      epi_fast<EPI, MJ>(acc, stg, prm, mw, nw, M, ep,
                        make_rsrc(ep.c, (uint32_t)(M * ep.ldc * 2)), el);
    } else {
      float vmax[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s) vmax[j][s] = -__builtin_huge_valf();
#pragma unroll
      for (int ip = 0; ip < 2; ++ip)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          epi_stage(acc, stg, prm, el, ip, j);
          epi_store<EPI>(stg, mw, nw, M, N, ep, el, ip, j, vmax[j]);
        }
      if (EPI == FVSR_EPI_ROWMAX) {
        // 8 lanes per row cover 64 columns per pass; both ip passes = the slab.
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            float v = vmax[j][s];
#pragma unroll
            for (int o = 4; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
            const int64_t m = mw + j * 32 + s * 8 + (el >> 3);
            if ((el & 7) == 0 && m < M && nw < N) ep.amax_part[m * ep.nparts + nw / 128] = v;
          }
      }
    }
    // Stores and the next tile's loads drain before the ring moves on.
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    t = tn;
    if (t >= tiles) break;
    m0 = m1;
    n0 = n1;
    cur = nxt;
  }
}

// ---------------------------------------------------------------------------
// Main loop, any K % 16 == 0: register-staged, K step 128, LDS double buffer.
// ---------------------------------------------------------------------------
constexpr int BKG = 128;
constexpr int kStageG = (BM + BN) * BKG;  // 64 KB
constexpr int kChunksG = (BM * BKG / 16) / kThreads;  // 8

FVSR_DEV int swz_g(int row, int chunk) { return row * BKG + ((chunk ^ (row & 7)) << 4); }

FVSR_DEV void load_stage_g(const uint8_t* __restrict__ g, int64_t ld, int64_t row0, int64_t rows,
                           int64_t k0, int64_t K, u32x4_t (&r)[kChunksG]) {
#pragma unroll
  for (int i = 0; i < kChunksG; ++i) {
    const int id = threadIdx.x + kThreads * i;
    const int row = id >> 3, chunk = id & 7;
    int64_t gr = row0 + row;
    gr = gr < rows ? gr : rows - 1;
    const int64_t k = k0 + chunk * 16;
    r[i] = k < K ? *(const u32x4_t*)(g + gr * ld + k) : u32x4_t{0u, 0u, 0u, 0u};
  }
}

FVSR_DEV void store_stage_g(uint8_t LDS_AS* lds, const u32x4_t (&r)[kChunksG]) {
#pragma unroll
  for (int i = 0; i < kChunksG; ++i) {
    const int id = threadIdx.x + kThreads * i;
    *(u32x4_t LDS_AS*)(lds + swz_g(id >> 3, id & 7)) = r[i];
  }
}

FVSR_DEV v8i read_frag_g(const uint8_t LDS_AS* lds, int rb, int s, int lane) {
  const int row = rb + (lane & 31);
  const int c0 = s * 4 + (lane >> 5) * 2;
  const u32x4_t lo = *(const u32x4_t LDS_AS*)(lds + swz_g(row, c0));
  const u32x4_t hi = *(const u32x4_t LDS_AS*)(lds + swz_g(row, c0 + 1));
  return v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
             (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

template <int EPI>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_fp8_generic(const uint8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B,
                      int64_t ldb, int64_t M, int64_t N, int64_t K, EpiArgs ep) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kStageG];
  uint8_t LDS_AS* lds = (uint8_t LDS_AS*)smem;
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  int tm, tn;
  map_tile(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  v16f acc[4][4];
  zero_acc(acc);
  u32x4_t ra[kChunksG], rb[kChunksG];
  const int KT = (int)((K + BKG - 1) / BKG);
  load_stage_g(A, lda, m0, M, 0, K, ra);
  load_stage_g(B, ldb, n0, N, 0, K, rb);
  store_stage_g(lds, ra);
  store_stage_g(lds + BM * BKG, rb);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    uint8_t LDS_AS* cur = lds + (kt & 1) * kStageG;
    uint8_t LDS_AS* nxt = lds + ((kt + 1) & 1) * kStageG;
    const bool more = kt + 1 < KT;
    if (more) {
      load_stage_g(A, lda, m0, M, (int64_t)(kt + 1) * BKG, K, ra);
      load_stage_g(B, ldb, n0, N, (int64_t)(kt + 1) * BKG, K, rb);
    }
#pragma unroll
    for (int s = 0; s < BKG / 64; ++s) {
      v8i fa[4], fb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) fa[j] = read_frag_g(cur, wm * 128 + j * 32, s, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) fb[i] = read_frag_g(cur + BM * BKG, wn * 128 + i * 32, s, lane);
      mfma_block(acc, fa, fb);
    }
    if (more) {
      store_stage_g(nxt, ra);
      store_stage_g(nxt + BM * BKG, rb);
    }
    __syncthreads();
  }
  const CTile ct{{(uint16_t LDS_AS*)lds, (uint16_t LDS_AS*)(lds + 32768),
                  (uint16_t LDS_AS*)(lds + 65536), (uint16_t LDS_AS*)(lds + 98304)}};
  epilogue<EPI>(acc, ct, m0, n0, M, N, ep, wm, wn, lane);
}

enum class Path { kGeneric, kRing, kRingFast, kRingFast128 };
constexpr int64_t kTouchMinK = 4096;  // L2 prefetch of the pair loads from this K on

template <int EPI>
void launch(Path path, unsigned grid, hipStream_t st, const uint8_t* a, int64_t lda,
            const uint8_t* b, int64_t ldb, int64_t M, int64_t N, int64_t K, const EpiArgs& ep) {
  if constexpr (EPI != FVSR_EPI_GATE_ADD) {  // gate-add keeps the general epilogue
    if (path == Path::kRingFast) {
      if (K >= kTouchMinK)
        hipLaunchKernelGGL((gemm_fp8_ring<EPI, true, 4, true>), dim3(grid), dim3(kThreads), 0, st,
                           a, lda, b, ldb, M, N, K, ep);
      else
        hipLaunchKernelGGL((gemm_fp8_ring<EPI, true, 4>), dim3(grid), dim3(kThreads), 0, st, a,
                           lda, b, ldb, M, N, K, ep);
      return;
    }
    if (path == Path::kRingFast128) {
      hipLaunchKernelGGL((gemm_fp8_ring<EPI, true, 2>), dim3(grid), dim3(kThreads), 0, st, a, lda,
                         b, ldb, M, N, K, ep);
      return;
    }
  }
  if (path != Path::kGeneric)
    hipLaunchKernelGGL((gemm_fp8_ring<EPI, false, 4>), dim3(grid), dim3(kThreads), 0, st, a, lda,
                       b, ldb, M, N, K, ep);
  else
    hipLaunchKernelGGL(gemm_fp8_generic<EPI>, dim3(grid), dim3(kThreads), 0, st, a, lda, b, ldb,
                       M, N, K, ep);
}

// Workgroups of the persistent kernel: one per CU, rounded down to a multiple
// of the 8 XCDs.
int64_t persistent_slots() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 8)
    cus = 256;
  return (cus / 8) * 8;
}

}  // namespace

extern "C" int64_t fvsr_gemm_amax_parts(int64_t N) { return (N + 127) / 128; }

extern "C" int fvsr_fp8_gemm(const void* a, int64_t lda, const float* sa, int sa_mode,
                             const void* b, int64_t ldb, const float* sb, int sb_mode,
                             const void* bias, void* c, int64_t ldc, int64_t M, int64_t N,
                             int64_t K, int epilogue, float* amax_part, const void* res,
                             const void* gate, void* stream) {
  if (M < 0 || N < 0 || K < 0) return FVSR_EINVAL;
  if (epilogue != FVSR_EPI_BIAS && epilogue != FVSR_EPI_ROWMAX && epilogue != FVSR_EPI_GATE_ADD)
    return FVSR_EINVAL;
  if (M == 0 || N == 0) return FVSR_OK;
  if (!a || !b || !sa || !sb || !c) return FVSR_EINVAL;
  if (K % 16 || lda < K || ldb < K || lda % 16 || ldb % 16 || ldc < N) return FVSR_EUNSUPPORTED;
  if (((uintptr_t)a & 15) || ((uintptr_t)b & 15)) return FVSR_EUNSUPPORTED;
  if (epilogue == FVSR_EPI_ROWMAX && !amax_part) return FVSR_EINVAL;
  if (epilogue == FVSR_EPI_GATE_ADD && (!res || !gate)) return FVSR_EINVAL;
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > 0x7fffffff) return FVSR_EUNSUPPORTED;
  const int sb_col = sb_mode == FVSR_SCALE_ROW;
  const int vec_params = (!sb_col || ((uintptr_t)sb & 15) == 0) && ((uintptr_t)bias & 7) == 0;
  const int res_vec = epilogue == FVSR_EPI_GATE_ADD && N % 8 == 0 && ldc % 8 == 0 &&
                      ((((uintptr_t)res) | (uintptr_t)c | (uintptr_t)gate) & 15) == 0;
  const int direct = ((uintptr_t)c & 15) == 0 && ldc % 8 == 0 && (M + BM) * ldc * 2 <= 0xffffffffLL;
  EpiArgs ep{sa, sb, (const uint16_t*)bias, (uint16_t*)c, ldc, amax_part,
             fvsr_gemm_amax_parts(N), (const uint16_t*)res, (const uint16_t*)gate,
             sa_mode == FVSR_SCALE_ROW, sb_col, vec_params, res_vec, direct};
  hipStream_t st = (hipStream_t)stream;
  // Persistent ring: K a multiple of 256, at least 8 K steps, and every row
  // offset of either operand within 32 bits.
  const bool ring = K % 256 == 0 && K >= 512 && K < 0x7fffffffLL && (M - 1) * lda + K <= 0xffffffffLL &&
                    (N - 1) * ldb + K <= 0xffffffffLL;
  // The fast epilogue needs whole column tiles.  128-row tiles when one
  // round of them covers the output (a 128-row tile takes about half as long
  // as a 256-row one, and 256-row tiles would then be a partial round too).
  const bool fast = ring && epilogue != FVSR_EPI_GATE_ADD && direct && N % BN == 0;
  const int64_t slots = persistent_slots();
  const int64_t tiles128 = ((M + 127) / 128) * ((N + BN - 1) / BN);
  const Path path = !ring ? Path::kGeneric
                    : !fast ? Path::kRing
                    : tiles128 <= slots ? Path::kRingFast128 : Path::kRingFast;
  const int64_t units = path == Path::kRingFast128 ? tiles128 : tiles;
  // Persistent grid: the fewest workgroups (a multiple of the 8 XCDs) that
  // still finish in the same number of rounds as one per CU, so no CU holds
  // a round more than another (ffn0 2310 tiles: 232 workgroups of 10 tiles
  // and fewer instead of 256 of 9 or 10; qkv 240, o and ffn2 200): the
  // critical path is unchanged and the idle CUs' power goes to the others'
  // clock (ffn0 216 -> 210 us, o 40.8 -> 39.7 us on one box).
  int64_t grid64 = units;
  if (ring && units > slots) {
    const int64_t rounds = (units + slots - 1) / slots;
    grid64 = 8 * ((units + 8 * rounds - 1) / (8 * rounds));
  }
  const unsigned grid = (unsigned)grid64;
  const uint8_t *ap = (const uint8_t*)a, *bp = (const uint8_t*)b;
  switch (epilogue) {
    case FVSR_EPI_BIAS:
      launch<FVSR_EPI_BIAS>(path, grid, st, ap, lda, bp, ldb, M, N, K, ep);
      break;
    case FVSR_EPI_ROWMAX:
      launch<FVSR_EPI_ROWMAX>(path, grid, st, ap, lda, bp, ldb, M, N, K, ep);
      break;
    default:
      launch<FVSR_EPI_GATE_ADD>(path, grid, st, ap, lda, bp, ldb, M, N, K, ep);
      break;
  }
  return fvsr_launch_status();
}
