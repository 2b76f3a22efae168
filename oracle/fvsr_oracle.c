/*
 * CPU oracle for the FlashVSR DiT-block operator pack: the byte-exact parts.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels
 * are compared against; it is loaded by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg, never by the product path.
 *
 * Build: oracle/build_oracle.sh (gcc -O2 -ffp-contract=off, SSE float math,
 * so every float operation below is one IEEE-754 binary32 operation).
 *
 * What each function restates (reference = aireet/flashvsr-sm89-ops):
 *   orc_e4m3_encode   fp32 -> OCP e4m3fn, round-to-nearest-even, |x|>=480 or
 *                     (464,480) -> NaN code 0x7F|sign.  Same semantics as the
 *                     `.to(tl.float8e4nv)` store in flashvsr_sm89_ops/fp8_quant.py:35
 *                     and torch's float8_e4m3fn cast.
 *   orc_quant_rows    contract Q-A: amax -> s = max(amax,1e-12)/448 ->
 *                     e4m3(clamp(x/s, +-448)), returned scale amax/448
 *                     (fp8_quant.py:16-35,42-55), per tensor or per row.
 *                     The returned scale is `amax / FP8_MAX` of a device
 *                     tensor, which torch evaluates on the GPU as
 *                     amax * fl(1/448) (reciprocal multiply for a host-scalar
 *                     divisor), so that is the product formed here.
 *   orc_gelu_bf16     tanh-GELU through 1-2/(exp(2u)+1), rounded to bf16
 *                     (fp8_ffn.py:24-30), with orc_expf as the exp.
 *   orc_expf          fp32 exp by Cody-Waite reduction + degree-6 Taylor
 *                     polynomial (W. J. Cody, W. Waite, "Software Manual for
 *                     the Elementary Functions", 1980), fused multiply-adds and
 *                     an exact ldexp.  The HIP kernels run the same operation
 *                     sequence, so the GELU values (and therefore the FP8
 *                     codes) are bit-identical.
 *   orc_quant_weight  contract Q-W: per-tensor (fp8_linear.py:17-22, with the
 *                     bf16 intermediate roundings of eager type promotion) and
 *                     per-output-channel (fp32 division, single rounding).
 *   orc_quant_rows_f32, orc_quant_weight_f32
 *                     the same contracts on fp16 or fp32 inputs (given as
 *                     their exact fp32 values): the reference's kernels load
 *                     any floating input as fp32 (fp8_quant.py:20,33), and
 *                     FP8Linear's eager weight expressions run in the weight's
 *                     own type (fp8_linear.py:19-22).
 *   orc_f16_round     fp32 -> IEEE binary16, round to nearest even (subnormals,
 *                     overflow to inf), returned as fp32.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* bf16 round-to-nearest-even of an fp32 value, returned as fp32. NaN stays NaN. */
static inline float bf16r(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return u2f((u | 0x00400000u) & 0xffff0000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u2f(u & 0xffff0000u);
}
static inline float bf2f(uint16_t h) { return u2f((uint32_t)h << 16); }
static inline uint16_t f2bf(float f) { return (uint16_t)(f2u(bf16r(f)) >> 16); }

/* binary16 round-to-nearest-even of an fp32 value, returned as fp32.  Normal
 * range: 10 mantissa bits kept by the add-and-mask rounding; below 2^-14 the
 * grid is 2^-24 (subnormals); 65520 and above round to infinity. */
static float f16r(float f) {
    uint32_t u = f2u(f), sign = u & 0x80000000u, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return f;                       /* NaN */
    if (a >= 0x477ff000u) return u2f(sign | 0x7f800000u);
    if (a < 0x38800000u) {
        float m = nearbyintf(u2f(a) * 16777216.0f);      /* exact scale by 2^24, RNE */
        return u2f(sign | f2u(m / 16777216.0f));          /* exact */
    }
    a += 0xfffu + ((a >> 13) & 1u);
    return u2f(sign | (a & 0xffffe000u));
}

void orc_f16_round(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = f16r(x[i]);
}

/* Element type of the float-input entry points: 0 bf16, 1 fp16, 2 fp32. */
static float round_dt(float v, int dt) { return dt == 2 ? v : (dt == 1 ? f16r(v) : bf16r(v)); }

uint8_t orc_e4m3_one(float f) {
    uint32_t u = f2u(f);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7f;          /* NaN */
    if (a >= 0x43f00000u) return sign | 0x7f;         /* >= 480: no inf in e4m3fn */
    if (a < 0x3c800000u) {                            /* < 2^-6: subnormal grid 2^-9 */
        float scaled = u2f(a) * 512.0f;               /* exact: power-of-two scale */
        int m = (int)nearbyintf(scaled);              /* ties-to-even (default mode) */
        return sign | (uint8_t)m;                     /* m == 8 is the min normal */
    }
    a += 0x7ffffu + ((a >> 20) & 1u);                 /* RNE to 3 mantissa bits */
    return sign | (uint8_t)((a >> 20) - (120u << 3)); /* rebias 127 -> 7 */
}

float orc_e4m3_value(uint8_t c) {
    int s = c & 0x80, e = (c >> 3) & 15, m = c & 7;
    float v;
    if (e == 15 && m == 7) return NAN;
    v = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return s ? -v : v;
}

void orc_e4m3_encode(const float* x, uint8_t* q, int64_t n) {
    for (int64_t i = 0; i < n; ++i) q[i] = orc_e4m3_one(x[i]);
}

void orc_e4m3_decode(const uint8_t* q, float* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = orc_e4m3_value(q[i]);
}

void orc_bf16_round(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = bf16r(x[i]);
}

/* exp(y) for y clamped to [-40, 40]; the GELU below is already saturated
 * there (1 + exp(-40) == 1 and 2/(exp(40)+1) < 2^-25, so 1 - 2/(e+1) is
 * exactly -1 or 1 either way):  n = rint(y*log2e);  r = y - n*ln2 in two
 * fused steps (Cody & Waite 1980);  p = degree-6 Taylor polynomial of e^r in
 * fused Horner form;  result = ldexp(p, n), exact because the result is a
 * normal number.  Every step is one IEEE operation (fmaf is a single rounding),
 * so the device copy of this sequence returns identical bits. */
float orc_expf(float y) {
    const float LOG2E = 1.44269502162933349609375f;
    const float LN2_HI = 0.693145751953125f;
    const float LN2_LO = 1.428606765330187045e-06f;
    if (y != y) return y;
    y = y < -40.0f ? -40.0f : (y > 40.0f ? 40.0f : y);
    float n = nearbyintf(y * LOG2E);
    float r = fmaf(-n, LN2_HI, y);
    r = fmaf(-n, LN2_LO, r);
    float p = 1.388888888888889e-03f;                 /* 1/6! */
    p = fmaf(p, r, 8.333333333333333e-03f);          /* 1/5! */
    p = fmaf(p, r, 4.166666666666666e-02f);          /* 1/4! */
    p = fmaf(p, r, 1.666666666666667e-01f);          /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* tanh-GELU of one bf16-valued input, rounded to bf16 (as fp32), in the form
 * of fp8_ffn.py:24-30:  u = sqrt(2/pi) (x + 0.044715 x^3),
 * t = 1 - 2/(exp(2u) + 1) (= tanh u),  g = bf16(0.5 x (1 + t)). */
float orc_gelu_one(float x) {
    const float C2 = 1.5957691216057308f;             /* 2*sqrt(2/pi) */
    float x2 = x * x;
    float inner = fmaf(0.044715f * x2, x, x);         /* x + 0.044715 x^3 */
    float e = orc_expf(C2 * inner);                   /* exp(2u) */
    float t = 1.0f - 2.0f / (e + 1.0f);
    return bf16r((0.5f * x) * (1.0f + t));
}

void orc_gelu_bf16(const uint16_t* h, uint16_t* g, int64_t n) {
    for (int64_t i = 0; i < n; ++i) g[i] = f2bf(orc_gelu_one(bf2f(h[i])));
}

/* The same GELU on fp32 inputs (bf16-rounded results as fp32). */
void orc_gelu_f32(const float* x, float* g, int64_t n) {
    for (int64_t i = 0; i < n; ++i) g[i] = orc_gelu_one(x[i]);
}

/* Element i of x: bf16 bits (f32 = 0) or fp32 values (f32 = 1). */
static float ld_x(const void* x, int f32, int64_t i) {
    return f32 ? ((const float*)x)[i] : bf2f(((const uint16_t*)x)[i]);
}

/* Q-A over a [rows, cols] matrix (leading dimension ld elements).
 * per_row = 0: one scale for the whole matrix (scale[0]); per_row = 1: one per row.
 * gelu = 1 quantises gelu(x) instead of x (fp8_ffn.py:43-54). */
static void quant_rows(const void* x, int f32, int64_t rows, int64_t cols, int64_t ld,
                       int per_row, int gelu, uint8_t* q, float* scale_out) {
    const float FP8_MAX = 448.0f;
    int64_t groups = per_row ? rows : 1;
    int64_t rpg = per_row ? 1 : rows;
    for (int64_t g = 0; g < groups; ++g) {
        float amax = 0.0f;
        for (int64_t r = g * rpg; r < (g + 1) * rpg; ++r)
            for (int64_t c = 0; c < cols; ++c) {
                float v = ld_x(x, f32, r * ld + c);
                if (gelu) v = orc_gelu_one(v);
                v = fabsf(v);
                if (v > amax) amax = v;
            }
        float s = (amax > 1e-12f ? amax : 1e-12f) / FP8_MAX;
        for (int64_t r = g * rpg; r < (g + 1) * rpg; ++r)
            for (int64_t c = 0; c < cols; ++c) {
                float v = ld_x(x, f32, r * ld + c);
                if (gelu) v = orc_gelu_one(v);
                v = v / s;
                v = v < -FP8_MAX ? -FP8_MAX : v;
                v = v > FP8_MAX ? FP8_MAX : v;
                q[r * cols + c] = orc_e4m3_one(v);
            }
        scale_out[g] = amax * (1.0f / FP8_MAX);
    }
}

void orc_quant_rows(const uint16_t* x, int64_t rows, int64_t cols, int64_t ld,
                    int per_row, int gelu, uint8_t* q, float* scale_out) {
    quant_rows(x, 0, rows, cols, ld, per_row, gelu, q, scale_out);
}

/* Q-A on fp16 or fp32 inputs given as fp32 values. */
void orc_quant_rows_f32(const float* x, int64_t rows, int64_t cols, int64_t ld,
                        int per_row, int gelu, uint8_t* q, float* scale_out) {
    quant_rows(x, 1, rows, cols, ld, per_row, gelu, q, scale_out);
}

/* Q-W.  per_channel = 0 (fp8_linear.py:20-22):
 *   w_scale = fp32(bf16(bf16(amax) / 448).clamp_min(bf16(1e-12)))
 *   q = e4m3(bf16(fp32(w) / w_scale))
 * per_channel = 1 (row-wise generalisation, bf16[N,K] / fp32[N,1] promotes to fp32):
 *   s_n = fp32(bf16(amax_n / 448).clamp_min(bf16(1e-12)));  q = e4m3(fp32(w) / s_n) */
void orc_quant_weight(const uint16_t* w, int64_t n, int64_t k, int per_channel,
                      uint8_t* q, float* scale_out) {
    const float lo = bf16r(1e-12f);
    int64_t groups = per_channel ? n : 1;
    int64_t rpg = per_channel ? 1 : n;
    for (int64_t g = 0; g < groups; ++g) {
        float amax = 0.0f;
        for (int64_t r = g * rpg; r < (g + 1) * rpg; ++r)
            for (int64_t c = 0; c < k; ++c) {
                float v = fabsf(bf2f(w[r * k + c]));
                if (v > amax) amax = v;
            }
        float s = bf16r(amax / 448.0f);
        if (s < lo) s = lo;
        for (int64_t r = g * rpg; r < (g + 1) * rpg; ++r)
            for (int64_t c = 0; c < k; ++c) {
                float v = bf2f(w[r * k + c]) / s;
                if (!per_channel) v = bf16r(v);
                q[r * k + c] = orc_e4m3_one(v);
            }
        scale_out[g] = s;
    }
}

/* Q-W on a weight of type dt (0 bf16, 1 fp16, 2 fp32) given as fp32 values,
 * with eager torch's arithmetic in that type on the GPU:
 *   w_scale = fp32(t(amax * fl(1/448)) clamped below at t(1e-12))
 *     (a tensor divided by a Python float is multiplied by the float
 *     reciprocal there; the clamp compares in fp32 and its bound, rounded to
 *     t, is 0 in fp16; t() rounds to dt)
 *   per tensor:  q = e4m3(t(w / w_scale))   (a 0-dim fp32 scale does not
 *                promote w, so the quotient is rounded to dt)
 *   per channel: q = e4m3(w / s_n)          ([N, 1] fp32 scales promote it) */
void orc_quant_weight_f32(const float* w, int64_t n, int64_t k, int per_channel, int dt,
                          uint8_t* q, float* scale_out) {
    const float lo = round_dt(1e-12f, dt);
    int64_t groups = per_channel ? n : 1;
    int64_t rpg = per_channel ? 1 : n;
    for (int64_t g = 0; g < groups; ++g) {
        float amax = 0.0f;
        for (int64_t r = g * rpg; r < (g + 1) * rpg; ++r)
            for (int64_t c = 0; c < k; ++c) {
                float v = fabsf(w[r * k + c]);
                if (v > amax) amax = v;
            }
        float s = round_dt(amax * (1.0f / 448.0f), dt);
        if (s < lo) s = lo;
        for (int64_t r = g * rpg; r < (g + 1) * rpg; ++r)
            for (int64_t c = 0; c < k; ++c) {
                float v = w[r * k + c] / s;
                if (!per_channel) v = round_dt(v, dt);
                q[r * k + c] = orc_e4m3_one(v);
            }
        scale_out[g] = s;
    }
}
