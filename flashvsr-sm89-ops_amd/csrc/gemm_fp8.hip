// FP8 (OCP e4m3fn) GEMM on CDNA4 matrix cores, contract M:
//   C[m,n] = epilogue( sum_k A[m,k] * B[n,k] )      A [M,K], B [N,K], K-contiguous
// which is torch._scaled_mm(x8, W8.t(), ...) of FP8Linear._mm
// (flashvsr_sm89_ops/fp8_linear.py:28-30).
//
// Tiling (one workgroup = 4 wavefronts = 256 threads, one per SIMD):
//   workgroup tile 256(M) x 256(N), K step 128 bytes, double-buffered in LDS
//   (2 stages x (32 KB A + 32 KB B) = 128 KB of the 160 KB LDS);
//   wave tile 128 x 128 = 4 x 4 v_mfma_f32_32x32x64_f8f6f4 tiles, fp32
//   accumulators (256 per lane).
// The weight operand is fed as the MFMA "A" side and the activation as the
// "B" side, so each lane's accumulators hold 4 consecutive output columns of
// one output row: the epilogue stores 8-byte bf16 quads.
// LDS rows are 128 bytes = 8 chunks of 16 bytes, chunk index XOR (row & 7),
// so the 32 lanes reading 32 rows at one K offset hit distinct banks.
// Workgroups are renumbered so each XCD (hardware dispatches workgroup ids
// round-robin over the 8 XCDs) walks a contiguous, M-grouped range of tiles
// and shares A/B panels in its own L2.
#include "common.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int kThreads = 256;
constexpr int kGroupM = 8;
constexpr int kStageBytes = (BM + BN) * BK;  // 64 KB
constexpr int kChunksPerThread = (BM * BK / 16) / kThreads;  // 8 for A and 8 for B

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

FVSR_DEV int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 4); }

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

// Global -> registers for one K step of one operand tile (rows clamped into
// range, chunks past K zero-filled).
FVSR_DEV void load_stage(const uint8_t* __restrict__ g, int64_t ld, int64_t row0, int64_t rows,
                         int64_t k0, int64_t K, u32x4_t (&r)[kChunksPerThread]) {
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int id = threadIdx.x + kThreads * i;
    const int row = id >> 3, chunk = id & 7;
    int64_t gr = row0 + row;
    gr = gr < rows ? gr : rows - 1;
    const int64_t k = k0 + chunk * 16;
    if (k < K)
      r[i] = *(const u32x4_t*)(g + gr * ld + k);
    else
      r[i] = u32x4_t{0u, 0u, 0u, 0u};
  }
}

FVSR_DEV void store_stage(uint8_t* lds, const u32x4_t (&r)[kChunksPerThread]) {
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int id = threadIdx.x + kThreads * i;
    *(u32x4_t*)(lds + swz(id >> 3, id & 7)) = r[i];
  }
}

// 32 bytes of K for MFMA step s (64 K) of subtile row base rb: lane half h
// takes bytes [s*64 + h*32, +32) of the row.
FVSR_DEV v8i read_frag(const uint8_t* lds, int rb, int s, int lane) {
  const int row = rb + (lane & 31);
  const int c0 = s * 4 + (lane >> 5) * 2;
  const u32x4_t lo = *(const u32x4_t*)(lds + swz(row, c0));
  const u32x4_t hi = *(const u32x4_t*)(lds + swz(row, c0 + 1));
  return v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
             (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

template <int EPI>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_fp8_kernel(const uint8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B,
                     int64_t ldb, int64_t M, int64_t N, int64_t K, EpiArgs ep) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStageBytes];
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  int tm, tn;
  map_tile(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;  // wave's 128x128 quadrant

  v16f acc[4][4];  // [n_sub][m_sub]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  u32x4_t ra[kChunksPerThread], rb[kChunksPerThread];
  const int KT = (int)((K + BK - 1) / BK);
  load_stage(A, lda, m0, M, 0, K, ra);
  load_stage(B, ldb, n0, N, 0, K, rb);
  store_stage(smem, ra);
  store_stage(smem + BM * BK, rb);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    uint8_t* cur = smem + (kt & 1) * kStageBytes;
    uint8_t* nxt = smem + ((kt + 1) & 1) * kStageBytes;
    const bool more = kt + 1 < KT;
    if (more) {
      load_stage(A, lda, m0, M, (int64_t)(kt + 1) * BK, K, ra);
      load_stage(B, ldb, n0, N, (int64_t)(kt + 1) * BK, K, rb);
    }
    const uint8_t* la = cur;
    const uint8_t* lb = cur + BM * BK;
#pragma unroll
    for (int s = 0; s < BK / 64; ++s) {
      v8i fa[4], fb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) fa[j] = read_frag(la, wm * 128 + j * 32, s, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) fb[i] = read_frag(lb, wn * 128 + i * 32, s, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[i], fa[j], acc[i][j], 0,
                                                                       0, 0, 0, 0, 0);
    }
    if (more) {
      store_stage(nxt, ra);
      store_stage(nxt + BM * BK, rb);
    }
    __syncthreads();
  }

  // Epilogue, phase 1: y = bf16(acc*sa*sb + bias) into a bf16 [256][256]
  // LDS tile (the operand buffers are free after the loop's final barrier).
  // acc[i][j][g*4+r] is row m = wm*128 + j*32 + (lane&31), column
  // n = wn*128 + i*32 + g*8 + (lane>>5)*4 + r.  8-byte units are XOR-swizzled
  // with the row so 32 lanes writing 32 rows do not share banks.
  uint16_t* ct = (uint16_t*)smem;
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
        *(u32x2_t*)(ct + ml * BN + unit * 4) =
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
    const u32x2_t lo = *(const u32x2_t*)(ct + rr * BN + ((((nl >> 2)) ^ (rr & 63)) * 4));
    const u32x2_t hi = *(const u32x2_t*)(ct + rr * BN + ((((nl >> 2) + 1) ^ (rr & 63)) * 4));
    u32x4_t v = {lo[0], lo[1], hi[0], hi[1]};
    float amax = 0.0f;
    if (EPI == FVSR_EPI_GELU) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float a = gelu_tanh_bf16(bf_lo(v[w])), b = gelu_tanh_bf16(bf_hi(v[w]));
        if (n + 2 * w < N) amax = fmaxf(amax, fabsf(a));
        if (n + 2 * w + 1 < N) amax = fmaxf(amax, fabsf(b));
        v[w] = pack_bf16x2(a, b);
      }
    }
    if (m < M && n < N) {
      uint16_t* cp = ep.c + m * ep.ldc + n;
      if (EPI == FVSR_EPI_GATE_ADD) {
        if (n + 7 < N && ((((uintptr_t)cp) | (uintptr_t)(ep.res + m * ep.ldc + n)) & 15) == 0) {
          const u32x4_t rv = *(const u32x4_t*)(ep.res + m * ep.ldc + n);
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
            const float o = round_bf16(bf2f(ep.res[m * ep.ldc + n + e]) + t);
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
    if (EPI == FVSR_EPI_GELU) {
      // 16 threads cover one 128-column slab of this row.
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
      const int64_t slab = slab0 + (cpos >> 4);
      if ((cpos & 15) == 0 && m < M && n < N && slab < ep.nparts)
        ep.amax_part[m * ep.nparts + slab] = amax;
    }
  }
}

}  // namespace

extern "C" int64_t fvsr_gemm_amax_parts(int64_t N) { return (N + 127) / 128; }

extern "C" int fvsr_fp8_gemm(const void* a, int64_t lda, const float* sa, int sa_mode,
                             const void* b, int64_t ldb, const float* sb, int sb_mode,
                             const void* bias, void* c, int64_t ldc, int64_t M, int64_t N,
                             int64_t K, int epilogue, float* amax_part, const void* res,
                             const void* gate, void* stream) {
  if (M < 0 || N < 0 || K < 0) return FVSR_EINVAL;
  if (M == 0 || N == 0) return FVSR_OK;
  if (!a || !b || !sa || !sb || !c) return FVSR_EINVAL;
  if (K % 16 || lda < K || ldb < K || lda % 16 || ldb % 16 || ldc < N) return FVSR_EUNSUPPORTED;
  if (((uintptr_t)a & 15) || ((uintptr_t)b & 15)) return FVSR_EUNSUPPORTED;
  if (epilogue == FVSR_EPI_GELU && !amax_part) return FVSR_EINVAL;
  if (epilogue == FVSR_EPI_GATE_ADD && (!res || !gate)) return FVSR_EINVAL;
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > 0x7fffffff) return FVSR_EUNSUPPORTED;
  EpiArgs ep{sa, sb, (const uint16_t*)bias, (uint16_t*)c, ldc, amax_part,
             fvsr_gemm_amax_parts(N), (const uint16_t*)res, (const uint16_t*)gate,
             sa_mode == FVSR_SCALE_ROW, sb_mode == FVSR_SCALE_ROW};
  hipStream_t st = (hipStream_t)stream;
  const size_t lds = 0;
  if (K == 0) {
    // An empty reduction: acc = 0, the epilogue still runs (bias, GELU, gate).
  }
  switch (epilogue) {
    case FVSR_EPI_BIAS:
      hipLaunchKernelGGL(gemm_fp8_kernel<FVSR_EPI_BIAS>, dim3((unsigned)tiles), dim3(kThreads),
                         lds, st, (const uint8_t*)a, lda, (const uint8_t*)b, ldb, M, N, K, ep);
      break;
    case FVSR_EPI_GELU:
      hipLaunchKernelGGL(gemm_fp8_kernel<FVSR_EPI_GELU>, dim3((unsigned)tiles), dim3(kThreads),
                         lds, st, (const uint8_t*)a, lda, (const uint8_t*)b, ldb, M, N, K, ep);
      break;
    case FVSR_EPI_GATE_ADD:
      hipLaunchKernelGGL(gemm_fp8_kernel<FVSR_EPI_GATE_ADD>, dim3((unsigned)tiles),
                         dim3(kThreads), lds, st, (const uint8_t*)a, lda, (const uint8_t*)b, ldb,
                         M, N, K, ep);
      break;
    default:
      return FVSR_EINVAL;
  }
  return fvsr_launch_status();
}
