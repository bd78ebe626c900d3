/* Exhaustive check of the division-free INT4 code computation used by the
 * quant_int4 kernel for bf16 / fp16 inputs (wush_int4_kernel_amd/csrc/quant.hip,
 * code_plus8) against the reference's division form
 * clamp(rint(RN(v / sf)), -7, 7) (my_int4/rtn_int4.py:50-51,
 * csrc/quant_int4.cu:90-93).
 *
 * For every bf16 scale sf >= 1e-8 (the smallest scale the sigma-clip formula
 * yields) and every finite bf16 and fp16 value v with |v| < 1.8e19 (a group
 * whose sum of squares is finite), with r = RN(1/sf):
 *     y = RN(v*r), e = fma(-y, sf, v), y1 = fma(e, r, y),
 *     code = clamp(rint(y1 + 8), 1, 15) - 8
 * must equal the division form.  Binary32 arithmetic, round to nearest even,
 * contraction off; fmaf is the IEEE fused multiply-add. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf16_value(uint32_t b) {
    uint32_t u = b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float f16_value(uint32_t h) {
    uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
    float f;
    if (e == 0) f = ldexpf((float)m, -24);
    else if (e == 31) f = m ? NAN : INFINITY;
    else f = ldexpf((float)(m | 1024), (int)e - 25);
    return s ? -f : f;
}

static int code_division(float v, float sf) {
    float q = v / sf;
    float c = rintf(q);
    if (c < -7.0f) c = -7.0f;
    if (c > 7.0f) c = 7.0f;
    return (int)c;
}

static int code_fma(float v, float sf, float r) {
    float y = v * r;
    float e = fmaf(-y, sf, v);
    float y1 = fmaf(e, r, y);
    float c = rintf(y1 + 8.0f);
    if (c < 1.0f) c = 1.0f;
    if (c > 15.0f) c = 15.0f;
    return (int)c - 8;
}

int main(void) {
    static float vals[65536];
    long bad = 0, checked = 0;
    for (int dt = 0; dt < 2; ++dt) {
        int nv = 0;
        for (uint32_t b = 0; b < 65536; ++b) {
            float v = dt ? f16_value(b) : bf16_value(b);
            if (isfinite(v) && fabsf(v) < 1.8e19f) vals[nv++] = v;
        }
#pragma omp parallel for reduction(+ : bad, checked) schedule(dynamic, 64)
        for (uint32_t sb = 0; sb < 0x7f80; ++sb) {
            float sf = bf16_value(sb);
            if (!(sf >= 1e-8f)) continue;
            float r = 1.0f / sf;
            for (int i = 0; i < nv; ++i) {
                int a = code_division(vals[i], sf), c = code_fma(vals[i], sf, r);
                checked++;
                if (a != c) {
                    if (bad < 10) printf("mismatch dtype=%s v=%a sf=%a division=%d fma=%d\n", dt ? "f16" : "bf16", vals[i], sf, a, c);
                    bad++;
                }
            }
        }
    }
    printf("checked %ld (v, sf) pairs, mismatches %ld\n", checked, bad);
    return bad != 0;
}
