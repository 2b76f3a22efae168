/*
 * Build-time generator of gelu_table.inc: the bf16 tanh-GELU of every bf16
 * bit pattern (65536 entries), computed with exactly the fp32 operation
 * sequence of gelu_tanh_bf16 in common.h (clamped Cody-Waite exp with fused
 * steps, IEEE division, bf16 round-to-nearest-even).  The kernels that need
 * GELU of bf16 data look it up instead of evaluating it per element.
 *
 * Build: gcc -O2 -std=c11 -ffp-contract=off -fno-fast-math gelu_table_gen.c -lm
 * Usage: gelu_table_gen > gelu_table.inc
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float round_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return u2f((u | 0x00400000u) & 0xffff0000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u2f(u & 0xffff0000u);
}

static float exp_clamped(float y) {
    const float LOG2E = 1.44269502162933349609375f;
    const float LN2_HI = 0.693145751953125f;
    const float LN2_LO = 1.428606765330187045e-06f;
    if (y != y) return y;
    y = y < -40.0f ? -40.0f : (y > 40.0f ? 40.0f : y);
    const float n = rintf(y * LOG2E);
    float r = fmaf(-n, LN2_HI, y);
    r = fmaf(-n, LN2_LO, r);
    float p = 1.388888888888889e-03f;
    p = fmaf(p, r, 8.333333333333333e-03f);
    p = fmaf(p, r, 4.166666666666666e-02f);
    p = fmaf(p, r, 1.666666666666667e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

static uint16_t gelu_bf16(uint16_t h) {
    const float C2 = 1.5957691216057308f;
    const float x = u2f((uint32_t)h << 16);
    const float x2 = x * x;
    const float inner = fmaf(0.044715f * x2, x, x);
    const float e = exp_clamped(C2 * inner);
    const float t = 1.0f - 2.0f / (e + 1.0f);
    return (uint16_t)(f2u(round_bf16((0.5f * x) * (1.0f + t))) >> 16);
}

int main(void) {
    for (uint32_t i = 0; i < 65536; ++i)
        printf("0x%04x,%s", gelu_bf16((uint16_t)i), (i % 8 == 7) ? "\n" : " ");
    return 0;
}
