/*
 * fvsr.h — C ABI of the MI355X (gfx950) FlashVSR DiT-block operator pack.
 *
 * One shared library, libfvsr.so, built from the HIP sources in
 * flashvsr-sm89-ops_amd/csrc.
 * The Python package flashvsr_sm89_ops binds these entry points with ctypes;
 * any other host language can bind them the same way.
 *
 * Conventions shared by every entry point:
 *  - Tensors are raw device pointers.  bf16 tensors hold uint16 bit patterns,
 *    e4m3fn tensors hold uint8 codes (OCP e4m3fn, max 448, 0x7F = NaN),
 *    scales are fp32.  Row-major, leading dimension = row length unless an
 *    explicit stride is given.
 *  - The library never allocates and never synchronises the host.  Outputs
 *    and scratch ("workspace") are caller-owned; every kernel is enqueued on
 *    the hipStream_t passed as `stream` (NULL = the default stream).
 *  - Return value: FVSR_OK (0) or a negative fvsr_status.  Argument checks
 *    run on the host before anything is enqueued.
 *  - Reentrant: no mutable global state, with one exception:
 *    fvsr_quant_fp8_noalloc (below) keeps its scratch in one device array per
 *    GPU plus a host table of those arrays' addresses, so calls of it that
 *    overlap on one GPU race; every other entry point is reentrant.
 *
 * Each declaration names the reference interface (aireet/flashvsr-sm89-ops,
 * file:line) whose work it carries.
 */
#ifndef FVSR_H
#define FVSR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  FVSR_OK = 0,
  FVSR_EINVAL = -1,       /* bad shape, stride, pointer or mode */
  FVSR_EHIP = -2,         /* a HIP launch failed (hipGetLastError) */
  FVSR_EUNSUPPORTED = -3, /* valid arguments outside what the kernels cover */
  FVSR_EWORKSPACE = -4    /* workspace too small */
} fvsr_status;

/* Granularity of an activation or weight scale. */
enum { FVSR_SCALE_TENSOR = 0, FVSR_SCALE_ROW = 1 };

/* Element types of the *_dt entry points' floating-point tensors. */
enum { FVSR_DT_BF16 = 0, FVSR_DT_F16 = 1, FVSR_DT_F32 = 2 };

/* GEMM epilogues. */
enum {
  FVSR_EPI_BIAS = 0,     /* C = bf16(acc*sa*sb + bias)                                  */
  FVSR_EPI_ROWMAX = 1,   /* C = bf16(acc*sa*sb + bias), plus max(C) (signed) per
                            (row, 128-column slab) into `amax_part`                      */
  FVSR_EPI_GATE_ADD = 2  /* C = bf16(res + bf16(gate[n] * bf16(acc*sa*sb + bias)))      */
};

/* Library version string ("fvsr <semver> gfx950"). */
const char* fvsr_version(void);

/* Number of 32-bit floats of workspace the quant entry points need: the
 * per-tensor partial maxima; 0 for FVSR_SCALE_ROW (no workspace, may be NULL). */
int64_t fvsr_quant_workspace_floats(int64_t rows, int64_t cols, int mode);

/*
 * Dynamic e4m3 quantisation of a bf16 [rows, cols] matrix (row stride ld
 * elements), optionally of tanh-GELU(x) (gelu = 1).
 *   mode FVSR_SCALE_TENSOR: one scale, reference quantize_fp8
 *     (flashvsr_sm89_ops/fp8_quant.py:42-55) and fused_gelu_quant_fp8
 *     (fp8_ffn.py:57-72); scale_out[0] = amax/448 as torch evaluates the
 *     reference's `amax / FP8_MAX` on the GPU, amax * fl(1/448).  The codes
 *     are those of x / (max(amax, 1e-12) / 448), true divisions.
 *   mode FVSR_SCALE_ROW: one scale per row, scale_out[rows], the same way.
 * codes: uint8 [rows, cols] contiguous.  workspace: fvsr_quant_workspace_floats.
 */
int fvsr_quant_fp8(const void* x, int64_t rows, int64_t cols, int64_t ld, int mode, int gelu,
                   void* codes, float* scale_out, float* workspace, int64_t workspace_floats,
                   void* stream);

/*
 * fvsr_quant_fp8 without a workspace argument: no counterpart in the
 * reference; for callers that cannot allocate (code under stream capture,
 * tight serving loops, harnesses that forbid allocation).  Same arguments,
 * codes and scales as fvsr_quant_fp8.  The per-tensor partial maxima live in a
 * library-owned device array of 1024 floats per GPU (every size fits: the
 * per-tensor pass uses at most 1024 partials; FVSR_EWORKSPACE otherwise),
 * resolved on the first call on each device.  Nothing is allocated.  Calls
 * that overlap on one GPU (two streams at once) share that array and race;
 * serialise them.
 */
int fvsr_quant_fp8_noalloc(const void* x, int64_t rows, int64_t cols, int64_t ld, int mode,
                           int gelu, void* codes, float* scale_out, void* stream);

/*
 * Per-tensor e4m3 quantisation of tanh-GELU(h), the FFN mid-section of FP8FFN
 * (fp8_ffn.py:43-72,84-96) in the reference's per-tensor mode, after an
 * FVSR_EPI_ROWMAX GEMM: h bf16 [rows, cols] contiguous, hmax_part float
 * [rows*nparts] the GEMM's per-slab maxima of h.  GELU is non-decreasing above
 * -0.75 and |GELU| < 0.17 below 0, so max|gelu(h)| is gelu(max h) whenever that
 * exceeds 0.17 and GELU runs once per element (otherwise one extra scan finds
 * the maximum).  Same codes and scale as fvsr_quant_fp8(h, gelu = 1, mode =
 * FVSR_SCALE_TENSOR).  workspace: 2 * fvsr_quant_workspace_floats(rows, cols, 0).
 * (Per-row mode needs no helper: fvsr_quant_fp8(gelu = 1, FVSR_SCALE_ROW) keeps
 * each row in registers and evaluates GELU once per element.)
 */
int fvsr_gelu_quant_fp8_tensor(const void* h, int64_t rows, int64_t cols, const float* hmax_part,
                               int64_t nparts, void* codes, float* scale_out, float* workspace,
                               int64_t workspace_floats, void* stream);

/*
 * Static weight quantisation, reference FP8Linear.__init__
 * (flashvsr_sm89_ops/fp8_linear.py:17-22).  mode FVSR_SCALE_TENSOR keeps the
 * eager bf16 roundings: s = fp32(bf16(amax/448) clamped at bf16(1e-12)),
 * q = e4m3(bf16(w/s)); FVSR_SCALE_ROW is the per-output-channel form,
 * q = e4m3(w/s_n) in fp32.  w: bf16 [n, k]; codes uint8 [n, k]; scale_out
 * [1] or [n]; workspace: fvsr_quant_workspace_floats(n, k, mode).
 */
int fvsr_quant_weight_fp8(const void* w, int64_t n, int64_t k, int mode, void* codes,
                          float* scale_out, float* workspace, int64_t workspace_floats,
                          void* stream);

/*
 * FP8 GEMM, C[M,N] = epilogue(sum_k A[m,k]*B[n,k]) with A e4m3 [M,K] (row
 * stride lda bytes) and B e4m3 [N,K] (row stride ldb bytes) — the
 * torch._scaled_mm(x8, W8.t(), scale_a, scale_b, bias, bf16) call of
 * FP8Linear._mm (fp8_linear.py:28-30).  sa: [1] or [M] (sa_mode), sb: [1] or
 * [N] (sb_mode).  bias: bf16 [N] or NULL.  C: bf16 [M,N] row stride ldc.
 * K must be a multiple of 16 and lda/ldb multiples of 16.
 * epilogue FVSR_EPI_ROWMAX also needs amax_part (float [M, ceil(N/128)]);
 * FVSR_EPI_GATE_ADD needs res (bf16 [M,N], row stride ldc) and gate (bf16 [N]).
 */
int fvsr_fp8_gemm(const void* a, int64_t lda, const float* sa, int sa_mode,
                  const void* b, int64_t ldb, const float* sb, int sb_mode,
                  const void* bias, void* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                  int epilogue, float* amax_part, const void* res, const void* gate,
                  void* stream);

/* Number of 128-column slabs FVSR_EPI_ROWMAX writes per row: ceil(N/128). */
int64_t fvsr_gemm_amax_parts(int64_t N);

/*
 * LayerNorm (no affine) + modulate, reference fused_ln_modulate
 * (flashvsr_sm89_ops/fused_adaln.py:22-42,60-71): x bf16 [B,L,D];
 * scale/shift bf16 [B,1,D].  out (bf16 [B,L,D]) may be NULL when codes is
 * given: then only the per-row e4m3 quantisation of the modulated rows is
 * written (codes uint8 [B*L, D], row_scale float [B*L]) — the activation
 * quantisation of the FP8 linear that consumes it, fused into the same pass.
 */
int fvsr_ln_modulate(const void* x, const void* scale, const void* shift, void* out,
                     int64_t B, int64_t L, int64_t D, float eps, void* codes, float* row_scale,
                     void* stream);

/*
 * The gated residual of the op before followed by the next AdaLN, in one
 * pass: x1 = bf16(x + bf16(gate*res)) (fused_gate_add, fused_adaln.py:74-85,
 * written to x1) then fvsr_ln_modulate of x1 with (scale, shift) into out
 * and/or the per-row e4m3 codes — the gate_add at the end of the
 * self-attention (or FFN) and the AdaLN at the start of the FFN (or the next
 * block's self-attention) of integrate.py:151-182.  x, res, x1 bf16 [B,L,D];
 * gate, scale, shift bf16 [B,1,D].  Requires D % 8 == 0, D <= 1536 and
 * 16-byte aligned tensors.
 */
int fvsr_gate_add_ln_modulate(const void* x, const void* gate, const void* res, void* x1,
                              const void* scale, const void* shift, void* out, int64_t B,
                              int64_t L, int64_t D, float eps, void* codes, float* row_scale,
                              void* stream);

/*
 * LayerNorm with affine weight and bias, the DiT block's norm3 before the
 * cross-attention (x + cross_attn(norm3(x)), integrate.py:171; upstream
 * nn.LayerNorm, elementwise_affine=True): x, out bf16 [rows, D]; weight, bias
 * bf16 [D]; y = bf16(w * ((x - mean) * rsqrt(var + eps)) + b) in fp32.  As
 * in fvsr_ln_modulate, out may be NULL when codes (uint8 [rows, D]) and
 * row_scale (float [rows]) take the per-row e4m3 quantisation of y for the
 * FP8 q projection that follows.
 */
int fvsr_layer_norm(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
                    int64_t D, float eps, void* codes, float* row_scale, void* stream);

/*
 * The self-attention's gated residual followed by norm3, one pass over the
 * rows (integrate.py:151-171: x = fused_gate_add(x, gate_msa, attn_out);
 * norm3(x)): x1 = bf16(x + bf16(gate * res)) written to x1 [B, L, D], then
 * the affine LayerNorm of x1 as fvsr_layer_norm into out (and/or codes +
 * row_scale).  gate bf16 [B, 1, D]; x, res, x1, out bf16 [B, L, D].  Same
 * results as fvsr_gate_add followed by fvsr_layer_norm; vector path only
 * (D % 8 == 0, D <= 1536, 16-byte aligned), else FVSR_EUNSUPPORTED.
 */
int fvsr_gate_add_layer_norm(const void* x, const void* gate, const void* res, void* x1,
                             const void* weight, const void* bias, void* out, int64_t B,
                             int64_t L, int64_t D, float eps, void* codes, float* row_scale,
                             void* stream);

/* out = bf16(x + bf16(gate*res)), reference fused_gate_add
 * (fused_adaln.py:45-57,74-85): x, res, out bf16 [B,L,D]; gate bf16 [B,1,D]. */
int fvsr_gate_add(const void* x, const void* gate, const void* res, void* out, int64_t B,
                  int64_t L, int64_t D, void* stream);

/*
 * RMSNorm over D + interleaved RoPE per head, reference fused_rms_rope
 * (flashvsr_sm89_ops/fused_rms_rope.py:21-83).  x, out: bf16 [B,L,D];
 * weight bf16 [D]; cs: fp32 [L, head_dim/2, 2] (cos, sin) pairs — the
 * view_as_real of the complex freqs_cis — or NULL with rope = 0.
 * Position of row r is r % L.
 */
int fvsr_rms_rope(const void* x, const void* weight, const float* cs, void* out, int64_t B,
                  int64_t L, int64_t D, int64_t head_dim, float eps, int rope, void* stream);

/*
 * fp16 and fp32 inputs.  The reference's kernels load every floating input
 * with .to(tl.float32) and store into torch.empty_like(x), so its ops take
 * bf16, fp16 or fp32 tensors, each in its own type (fp8_quant.py:20,33;
 * fused_adaln.py:29,37-38,53-55; fused_rms_rope.py:33,36,44).  These entry
 * points take one FVSR_DT_* code per floating tensor; the arithmetic,
 * including the bf16 roundings the reference makes, is that of the bf16
 * entry points above, and outputs (except codes and scales) are written in
 * x's type: a bf16-rounded result stored exactly in bf16 or fp32 and rounded
 * to nearest even in fp16.  With every tensor bf16 they run the bf16 entry
 * point's kernels.
 */

/* fvsr_quant_fp8 (fp8_quant.py:16-55, fp8_ffn.py:34-72) on x of type x_dtype;
 * fp16/fp32 codes are those of the IEEE quotient x / s.  Same workspace. */
int fvsr_quant_fp8_dt(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ld,
                      int mode, int gelu, void* codes, float* scale_out, float* workspace,
                      int64_t workspace_floats, void* stream);

/* fvsr_quant_weight_fp8 (fp8_linear.py:17-22) on a weight of type w_dtype,
 * with eager's arithmetic in that type: w_scale = fp32(t((amax * fl(1/448)))
 * clamped below at t(1e-12)) and codes e4m3(t(w / w_scale)), t() rounding to
 * w_dtype (the GPU evaluates amax / 448 as a product with the reciprocal;
 * t(1e-12) is 0 in fp16).  FVSR_SCALE_ROW: codes e4m3(w / s_n) in fp32.
 * Codes follow torch's e4m3fn cast (NaN and |v| > 464 give 0x7F | sign). */
int fvsr_quant_weight_fp8_dt(const void* w, int w_dtype, int64_t n, int64_t k, int mode,
                             void* codes, float* scale_out, float* workspace,
                             int64_t workspace_floats, void* stream);

/* fvsr_ln_modulate's out-only form (fused_adaln.py:22-42,60-71) on x, scale
 * and shift of any of the three types; out [B, L, D] has x's type. */
int fvsr_ln_modulate_dt(const void* x, int x_dtype, const void* scale, int scale_dtype,
                        const void* shift, int shift_dtype, void* out, int64_t B, int64_t L,
                        int64_t D, float eps, void* stream);

/* fvsr_gate_add (fused_adaln.py:45-57,74-85) on x, gate and res of any of the
 * three types; out [B, L, D] has x's type. */
int fvsr_gate_add_dt(const void* x, int x_dtype, const void* gate, int gate_dtype,
                     const void* res, int res_dtype, void* out, int64_t B, int64_t L, int64_t D,
                     void* stream);

/* fvsr_rms_rope (fused_rms_rope.py:21-83) on x and weight of any of the three
 * types; out [B, L, D] has x's type.  D and head_dim even. */
int fvsr_rms_rope_dt(const void* x, int x_dtype, const void* weight, int weight_dtype,
                     const float* cs, void* out, int64_t B, int64_t L, int64_t D,
                     int64_t head_dim, float eps, int rope, void* stream);

/* Both self-attention projections in one launch (q and k share the cos/sin
 * reads): the two fused_rms_rope calls of integrate.py:59-62.  Rows of q/k
 * are ld_in elements apart and rows of out_q/out_k ld_out apart (column
 * slices of a fused QKV projection; in place is allowed).  Requires
 * D % 8 == 0, D <= 1536, head_dim % 8 == 0 and 16-byte aligned rows. */
int fvsr_rms_rope_qk(const void* q, const void* k, const void* wq, const void* wk,
                     const float* cs, void* out_q, void* out_k, int64_t B, int64_t L, int64_t D,
                     int64_t head_dim, float eps, int64_t ld_in, int64_t ld_out, void* stream);

/*
 * The self-attention's q/k RMSNorm + RoPE together with the window-order
 * layout of K and V (F2), replacing integrate.py:59-62 (rope_fn on q and k)
 * and the WindowPartition3D.partition + KV-cache torch.cat copies of k and v
 * (integrate.py:70-83): q is normalised and rotated in place (or to out_q,
 * rows at ld_out); row r of k (normalised and rotated) and of v (copied) go
 * to row kv_rows[r] of out_k / out_v (ld_kv), the window-ordered K/V buffer
 * whose first rows the caller filled with the cached windows.  kv_rows int32
 * [B*L]; rows mapped outside [0, kv_cap) are skipped.  Same shape rules as
 * fvsr_rms_rope_qk.
 */
int fvsr_rms_rope_qkv_rows(const void* q, const void* k, const void* v, const void* wq,
                           const void* wk, const float* cs, void* out_q, void* out_k,
                           void* out_v, const int32_t* kv_rows, int64_t kv_cap, int64_t B,
                           int64_t L, int64_t D, int64_t head_dim, float eps, int64_t ld_in,
                           int64_t ld_out, int64_t ld_kv, void* stream);

/*
 * Block index from a bool block mask, reference build_csr
 * (flashvsr_sm89_ops/lcsa/triton_lcsa.py:64-71) without its host sync:
 * keep uint8 [H, NQ, NK] -> sel int32 [H, NQ, NK] and cnt int32 [H, NQ].
 * Each row of sel holds the kept block ids ascending, then the other ids
 * ascending: the reference's stable descending argsort of keep, before it
 * trims the rows to maxk = max(cnt) (a host read this entry point leaves to
 * the caller).
 */
int fvsr_block_index(const uint8_t* keep, int64_t H, int64_t NQ, int64_t NK, int32_t* sel,
                     int32_t* cnt, void* stream);

/* Number of 32-bit floats of workspace fvsr_draft_block_mask needs. */
int64_t fvsr_draft_workspace_floats(int64_t H, int64_t D, int64_t NQ, int64_t NK);

/*
 * Draft block mask, reference draft_block_mask (flashvsr_sm89_ops/lcsa/
 * reference.py:37-64), the work of the dit.generate_draft_block_mask call at
 * integrate.py:103-104: window-mean pooling of q and k over each 128-token
 * block, scores avg_q.avg_k / sqrt(D) per head, -inf outside the local rule
 * local[l % sq][m % sk] (uint8 [sq, sk]), softmax over key blocks, and a joint
 * top-k per (head, query time row) over the time row's NQ/q_temporal query
 * blocks x NK key blocks: keep = attn > the (topk+1)-th largest attn.  Every
 * stage is rounded to bf16 as torch does for bf16 q/k.
 * q, k: bf16, token j of block n at row map[n*128 + j] (row n*128 + j when the
 * map is NULL), rows q_tok_stride / k_tok_stride elements apart; H*D channels.
 * Outputs (either or both): keep uint8 [H, NQ, NK]; sel int32 [H, NQ, NK] and
 * cnt int32 [H, NQ]: the first cnt entries of each sel row are the kept block
 * ids ascending, as in fvsr_block_index; the rest of the row is unspecified.
 * workspace: fvsr_draft_workspace_floats(H, D, NQ, NK).
 * Requires D % 8 == 0, token strides % 8 == 0, 16-byte aligned q and k, and
 * 2*D + NK <= 3968.
 */
int fvsr_draft_block_mask(const void* q, int64_t q_tok_stride, const int32_t* q_map,
                          const void* k, int64_t k_tok_stride, const int32_t* k_map, int64_t H,
                          int64_t D, int64_t NQ, int64_t NK, int64_t q_temporal,
                          const uint8_t* local, int64_t sq, int64_t sk, int64_t topk,
                          uint8_t* keep, int32_t* sel, int32_t* cnt, float* workspace,
                          int64_t workspace_floats, void* stream);

/*
 * Block-sparse attention over 128-token blocks, reference _bsa_fwd_kernel /
 * block_sparse_attention (lcsa/triton_lcsa.py:19-61,74-94): for each head h
 * and query block i, softmax(Q_i K_J^T * sm_scale) V_J over the kept key
 * blocks J = sel[h,i,0..cnt[h,i]-1]; rows with cnt 0 are written as zeros.
 * q/k/v/o bf16, element (token t, head h, dim d) at ptr[t*tok_stride +
 * h*head_stride + d]; head_dim must be 128; sel row stride is maxk.
 * tok_map: NULL, or int32 [NQ*128] (queries/outputs) and [NK*128] (keys) maps
 * from block-order position to stored token index (kmap), letting raster-order
 * tensors be read in window order without a copy.
 */
int fvsr_bsa_fwd(const void* q, const void* k, const void* v, void* o, int64_t q_tok_stride,
                 int64_t q_head_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
                 int64_t o_tok_stride, int64_t o_head_stride, const int32_t* sel,
                 const int32_t* cnt, int64_t maxk, int64_t H, int64_t NQ, int64_t NK,
                 int64_t head_dim, float sm_scale, const int32_t* q_map, const int32_t* kv_map,
                 void* stream);

/*
 * fvsr_bsa_fwd with the window partition in closed form instead of token maps:
 * the same attention (lcsa/triton_lcsa.py:19-61,74-94) on q/k/v that the
 * reference's self-attention first permutes with WindowPartition3D
 * (integrate.py:70-94, lcsa/reference.py:15-21; windows of 2 x 8 x 8 tokens).
 * q and o rows are the raster tokens of a (frames, height, width) latent grid;
 * query block i is window i: its slot s = (f*8 + y)*8 + x is token
 * ((2*wf + f)*height + 8*wy + y)*width + 8*wx + x of window (wf, wy, wx).
 * kv_raster = 1: k and v rows are raster tokens of the same grid, key block j =
 * window j (NK == NQ); kv_raster = 0: k and v rows are already in window order
 * (row = block position, e.g. a window-ordered K/V cache), NK blocks.
 * No map is read: token rows are computed, so the first K/V loads of a block
 * wait on no other load.  Requires frames % 2 == 0, height % 8 == 0,
 * width % 8 == 0, frames*height*width == NQ*128, plus fvsr_bsa_fwd's
 * requirements.
 */
int fvsr_bsa_fwd_window(const void* q, const void* k, const void* v, void* o,
                        int64_t q_tok_stride, int64_t q_head_stride, int64_t kv_tok_stride,
                        int64_t kv_head_stride, int64_t o_tok_stride, int64_t o_head_stride,
                        const int32_t* sel, const int32_t* cnt, int64_t maxk, int64_t H,
                        int64_t NQ, int64_t NK, int64_t head_dim, float sm_scale, int64_t frames,
                        int64_t height, int64_t width, int kv_raster, void* stream);

/*
 * Dense attention: fvsr_bsa_fwd with every key block kept for every query
 * block, for the cross-attention's softmax(Q K^T * sm_scale) V over the
 * prompt K/V cached by init_cross_kv (integrate.py:132-143; upstream
 * self.attn(q, cache_k, cache_v)).  NQ*128 query tokens, NK*128 key tokens,
 * strides as in fvsr_bsa_fwd, no block index and no token map.  One
 * workgroup of 8 waves takes two query blocks over one K/V stream.
 */
int fvsr_attn_dense(const void* q, const void* k, const void* v, void* o, int64_t q_tok_stride,
                    int64_t q_head_stride, int64_t kv_tok_stride, int64_t kv_head_stride,
                    int64_t o_tok_stride, int64_t o_head_stride, int64_t H, int64_t NQ,
                    int64_t NK, int64_t head_dim, float sm_scale, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* FVSR_H */
