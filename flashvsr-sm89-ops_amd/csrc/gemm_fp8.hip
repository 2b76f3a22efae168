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
// Main loop (K a multiple of 64): a 4-slot LDS ring of 64-wide K steps
// (32 KB per slot: 256 A rows + 256 B rows of 64 bytes).  Operand tiles go
// from global memory straight into LDS (global_load_lds_dwordx4, no staging
// registers) three steps ahead of the MFMAs; each wave reads the MFMA
// fragments of step k+1 from LDS while the MFMAs of step k run.  The four slots
// are four distinct LDS objects and the loop is unrolled by four, so the
// compiler can see that the reads of one slot never alias the loads into
// another and does not serialise them.  Rows are 64 bytes = 4 chunks of 16;
// chunk c of row r sits at c ^ ((r >> 2) & 3), which makes the 16 rows one
// ds_read_b128 phase touches land on 16 distinct 16-byte bank groups.
// Other K (a multiple of 16) use a register-staged loop with K step 128.
//
// Epilogue: y = acc * sa[m] * sb[n] + bias[n] is written as bf16 into the (now
// free) LDS as a 256 x 256 tile, then every thread stores 16-byte row chunks:
//   FVSR_EPI_BIAS      C = y
//   FVSR_EPI_ROWMAX    C = y, plus max(C) over each row's 128-column slab
//   FVSR_EPI_GATE_ADD  C = bf16(res + bf16(gate[n] * y))
// Workgroups are renumbered so each XCD (workgroup ids are dispatched round
// robin over the 8 XCDs) walks a contiguous, M-grouped range of tiles.
#include "common.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
#define LDS_AS __attribute__((address_space(3)))

constexpr int BM = 256, BN = 256;
constexpr int kThreads = 256;
constexpr int kGroupM = 8;
constexpr int kSlotBytes = (BM + BN) * 64;  // 32 KB

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
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

FVSR_DEV void zero_acc(v16f (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
}

FVSR_DEV void mfma_block(v16f (&acc)[4][4], const v8i (&fa)[4], const v8i (&fb)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
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
// Main loop, K % 64 == 0: direct-to-LDS ring.
// ---------------------------------------------------------------------------
FVSR_DEV int swz64(int r, int c) { return c ^ ((r >> 2) & 3); }

// Stream K step kt (64 bytes of every row) into `slot`: wave w covers A rows
// and B rows 64w .. 64w+63, four 1 KB (16-row) loads each; lane i of a load
// lands at row 16*seg + i/4, physical chunk i%4.
FVSR_DEV void issue_step(uint8_t LDS_AS* slot, const uint8_t* __restrict__ A, int64_t lda,
                         const uint8_t* __restrict__ B, int64_t ldb, int64_t m0, int64_t n0,
                         int64_t M, int64_t N, int64_t k0, int wave, int lane) {
  const int p = lane & 3;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int seg = wave * 4 + t;
    const int r = seg * 16 + (lane >> 2);
    const int c = swz64(r, p);
    int64_t ga = m0 + r, gb = n0 + r;
    ga = ga < M ? ga : M - 1;
    gb = gb < N ? gb : N - 1;
    __builtin_amdgcn_global_load_lds(A + ga * lda + k0 + c * 16, (void LDS_AS*)(slot + seg * 1024),
                                     16, 0, 0);
    __builtin_amdgcn_global_load_lds(B + gb * ldb + k0 + c * 16,
                                     (void LDS_AS*)(slot + BM * 64 + seg * 1024), 16, 0, 0);
  }
}

// MFMA fragments of one K step: lane half h takes chunks 2h, 2h+1 of its row.
FVSR_DEV void read_step(const uint8_t LDS_AS* slot, int wm, int wn, int lane, v8i (&fa)[4],
                        v8i (&fb)[4]) {
  const int h = lane >> 5;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = wm * 128 + j * 32 + (lane & 31);
    const u32x4_t lo = *(const u32x4_t LDS_AS*)(slot + r * 64 + (swz64(r, 2 * h) << 4));
    const u32x4_t hi = *(const u32x4_t LDS_AS*)(slot + r * 64 + (swz64(r, 2 * h + 1) << 4));
    fa[j] = v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = wn * 128 + i * 32 + (lane & 31);
    const uint8_t LDS_AS* b = slot + BM * 64;
    const u32x4_t lo = *(const u32x4_t LDS_AS*)(b + r * 64 + (swz64(r, 2 * h) << 4));
    const u32x4_t hi = *(const u32x4_t LDS_AS*)(b + r * 64 + (swz64(r, 2 * h + 1) << 4));
    fb[i] = v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  }
}

struct LoopCtx {
  const uint8_t* A;
  const uint8_t* B;
  int64_t lda, ldb, m0, n0, M, N;
  int KT, wave, wm, wn, lane;
};

// s_waitcnt immediates (gfx9 encoding): vmcnt(n) with lgkmcnt/expcnt left open.
constexpr int kWaitVm16 = 0x4F70;  // vmcnt(16): two K steps of this wave's loads in flight
constexpr int kWaitVm8 = 0x0F78;   // vmcnt(8): one K step in flight
constexpr int kWaitVm0 = 0x0F70;   // vmcnt(0)

// Iteration kt: fragments of step kt are in (fa, fb).  Wait until step kt+1
// has landed (every wave), start the loads of step kt+3 into `dma_slot` (the
// slot of step kt-1, whose fragments every wave read before this barrier),
// read step kt+1's fragments from `rd_slot` into (na, nb), then run step kt's
// MFMAs.
FVSR_DEV void k_iter(int kt, const LoopCtx& c, uint8_t LDS_AS* rd_slot, uint8_t LDS_AS* dma_slot,
                     v16f (&acc)[4][4], v8i (&fa)[4], v8i (&fb)[4], v8i (&na)[4], v8i (&nb)[4]) {
  if (kt >= c.KT) return;
  if (kt + 1 < c.KT) {
    if (kt + 2 < c.KT)
      __builtin_amdgcn_s_waitcnt(kWaitVm8);
    else
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS access may move across the barrier
  }
  if (kt + 3 < c.KT)
    issue_step(dma_slot, c.A, c.lda, c.B, c.ldb, c.m0, c.n0, c.M, c.N, (int64_t)(kt + 3) * 64,
               c.wave, c.lane);
  if (kt + 1 < c.KT) read_step(rd_slot, c.wm, c.wn, c.lane, na, nb);
  mfma_block(acc, fa, fb);
}

template <int EPI>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_fp8_ring(const uint8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B,
                   int64_t ldb, int64_t M, int64_t N, int64_t K, EpiArgs ep) {
  __shared__ __attribute__((aligned(1024))) uint8_t slot0[kSlotBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t slot1[kSlotBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t slot2[kSlotBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t slot3[kSlotBytes];
  uint8_t LDS_AS* s0 = (uint8_t LDS_AS*)slot0;
  uint8_t LDS_AS* s1 = (uint8_t LDS_AS*)slot1;
  uint8_t LDS_AS* s2 = (uint8_t LDS_AS*)slot2;
  uint8_t LDS_AS* s3 = (uint8_t LDS_AS*)slot3;

  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  int tm, tn;
  map_tile(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  LoopCtx c{A, B, lda, ldb, (int64_t)tm * BM, (int64_t)tn * BN, M, N, (int)(K / 64), wave,
            wave & 1, wave >> 1, lane};

  v16f acc[4][4];
  zero_acc(acc);
  v8i fa[4], fb[4], na[4], nb[4];
  // Prologue: steps 0..2 in flight, wait for step 0, read its fragments.
  issue_step(s0, A, lda, B, ldb, c.m0, c.n0, M, N, 0, wave, lane);
  if (c.KT > 1) issue_step(s1, A, lda, B, ldb, c.m0, c.n0, M, N, 64, wave, lane);
  if (c.KT > 2) issue_step(s2, A, lda, B, ldb, c.m0, c.n0, M, N, 128, wave, lane);
  if (c.KT > 2)
    __builtin_amdgcn_s_waitcnt(kWaitVm16);
  else if (c.KT > 1)
    __builtin_amdgcn_s_waitcnt(kWaitVm8);
  else
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  read_step(s0, c.wm, c.wn, lane, fa, fb);
  for (int kt = 0; kt < c.KT; kt += 4) {
    k_iter(kt + 0, c, s1, s3, acc, fa, fb, na, nb);
    k_iter(kt + 1, c, s2, s0, acc, na, nb, fa, fb);
    k_iter(kt + 2, c, s3, s1, acc, fa, fb, na, nb);
    k_iter(kt + 3, c, s0, s2, acc, na, nb, fa, fb);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const CTile ct{{(uint16_t LDS_AS*)s0, (uint16_t LDS_AS*)s1, (uint16_t LDS_AS*)s2,
                  (uint16_t LDS_AS*)s3}};
  epilogue<EPI>(acc, ct, c.m0, c.n0, M, N, ep, c.wm, c.wn, lane);
}

// ---------------------------------------------------------------------------
// Main loop, any K % 16 == 0: register-staged, K step 128, LDS double buffer.
// ---------------------------------------------------------------------------
constexpr int BKG = 128;
constexpr int kStageG = (BM + BN) * BKG;  // 64 KB
constexpr int kChunksG = (BM * BKG / 16) / kThreads;  // 8

FVSR_DEV int swz128(int row, int chunk) { return row * BKG + ((chunk ^ (row & 7)) << 4); }

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
    *(u32x4_t LDS_AS*)(lds + swz128(id >> 3, id & 7)) = r[i];
  }
}

FVSR_DEV v8i read_frag_g(const uint8_t LDS_AS* lds, int rb, int s, int lane) {
  const int row = rb + (lane & 31);
  const int c0 = s * 4 + (lane >> 5) * 2;
  const u32x4_t lo = *(const u32x4_t LDS_AS*)(lds + swz128(row, c0));
  const u32x4_t hi = *(const u32x4_t LDS_AS*)(lds + swz128(row, c0 + 1));
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

template <int EPI>
void launch(bool ring, unsigned tiles, hipStream_t st, const uint8_t* a, int64_t lda,
            const uint8_t* b, int64_t ldb, int64_t M, int64_t N, int64_t K, const EpiArgs& ep) {
  if (ring)
    hipLaunchKernelGGL(gemm_fp8_ring<EPI>, dim3(tiles), dim3(kThreads), 0, st, a, lda, b, ldb, M,
                       N, K, ep);
  else
    hipLaunchKernelGGL(gemm_fp8_generic<EPI>, dim3(tiles), dim3(kThreads), 0, st, a, lda, b, ldb,
                       M, N, K, ep);
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
  EpiArgs ep{sa, sb, (const uint16_t*)bias, (uint16_t*)c, ldc, amax_part,
             fvsr_gemm_amax_parts(N), (const uint16_t*)res, (const uint16_t*)gate,
             sa_mode == FVSR_SCALE_ROW, sb_mode == FVSR_SCALE_ROW};
  hipStream_t st = (hipStream_t)stream;
  const bool ring = K % 64 == 0 && K > 0;
  const uint8_t *ap = (const uint8_t*)a, *bp = (const uint8_t*)b;
  switch (epilogue) {
    case FVSR_EPI_BIAS:
      launch<FVSR_EPI_BIAS>(ring, (unsigned)tiles, st, ap, lda, bp, ldb, M, N, K, ep);
      break;
    case FVSR_EPI_ROWMAX:
      launch<FVSR_EPI_ROWMAX>(ring, (unsigned)tiles, st, ap, lda, bp, ldb, M, N, K, ep);
      break;
    default:
      launch<FVSR_EPI_GATE_ADD>(ring, (unsigned)tiles, st, ap, lda, bp, ldb, M, N, K, ep);
      break;
  }
  return fvsr_launch_status();
}
