/* Check of the division-free INT4 code computation used for fp32 values
 * (the quant_int4 kernel's fp32 inputs and the fused transform's fp32 x';
 * wush_int4_kernel_amd/csrc/wush_device.h, code_fp32) against the
 * reference's division form clamp(rint(RN(v / sf)), -7, 7)
 * (my_int4/rtn_int4.py:50-51, csrc/quant_int4.cu:90-93).
 *
 * With r = RN(1/sf) (sf a bf16 scale >= 1e-8) and |v| < 1.8e19 (a group whose
 * sum of squares is finite):
 *     q0 = RN(v*r), e0 = fma(-q0, sf, v), q1 = fma(e0, r, q0),
 *     e1 = fma(-q1, sf, v), q2 = fma(e1, r, q1),
 *     code = clamp(rint(q2) + 8, 1, 15) - 8
 * q2 must be RN(v/sf) itself (Markstein's correction: r = RN(1/sf), q1
 * within an ulp of v/sf, remainders exact), so the codes agree.  fp32 v has
 * too many values for an exhaustive sweep; the cases are
 *   - every bf16 scale >= 1e-8 against v = h*sf +- k ulps for every
 *     half-integer h in [-8, 8] and k = 0..64 (quotients at and next to the
 *     rounding ties, where a wrong last bit flips a code), and against v = h*sf
 *     scaled by 2^j (quotients near integers, half-integers at every binade);
 *   - 2^31 pseudo-random (v, sf) pairs over the whole exponent range.
 * q2 is compared with the division bit for bit, not only the code.
 *
 * The one-fma form (wush_device.h, code8_fast) is checked on the same cases:
 *     t = fma(v, r, 8), k = rint(t),
 *     code = clamp(k, 1, 15) - 8 when |t - k| < 0.5 - 2^-17,
 * otherwise the lane falls back to q2 above; its code must equal the
 * division's wherever the band test passes. */
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

static float f_from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t bits_of(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float quotient_fma(float v, float sf, float r) {
    float q0 = v * r;
    float e0 = fmaf(-q0, sf, v);
    float q1 = fmaf(e0, r, q0);
    float e1 = fmaf(-q1, sf, v);
    return fmaf(e1, r, q1);
}

static int code_of_q(float q) {
    float c = rintf(q) + 8.0f;
    if (c < 1.0f) c = 1.0f;
    if (c > 15.0f) c = 15.0f;
    return (int)c - 8;
}

/* code8_fast: the code, or 99 when the lane would take the exact fallback */
static int code_fast(float v, float r) {
    float t = fmaf(v, r, 8.0f);
    float k = rintf(t);
    if (fabsf(t - k) >= 0.5f - 0x1p-17f) return 99;
    if (k < 1.0f) k = 1.0f;
    if (k > 15.0f) k = 15.0f;
    return (int)k - 8;
}

static long bad = 0, checked = 0;
static long bad_fast = 0, fallback = 0;

static long bad_bits = 0;

/* Codes must agree everywhere; the quotient itself must equal the division
 * bit for bit wherever quotient and remainders are normal numbers (|v| and
 * |v/sf| >= 2^-100; below that a remainder or the quotient can underflow, but
 * then |v/sf| < 2^-73 and both codes are 0). */
static int check(float v, float sf, float r, long* nbad, long* nbits, long* nfast, long* nfall) {
    if (!isfinite(v) || fabsf(v) >= 1.8e19f) return 0;
    float qd = v / sf, qf = quotient_fma(v, sf, r);
    int cf = code_fast(v, r);
    if (cf == 99) {
        (*nfall)++;
    } else if (cf != code_of_q(qd)) {
        if (*nfast < 5) printf("one-fma code mismatch v=%a sf=%a division=%a\n", v, sf, qd);
        (*nfast)++;
    }
    if (code_of_q(qd) != code_of_q(qf)) {
        if (*nbad < 5) printf("code mismatch v=%a sf=%a division=%a fma=%a\n", v, sf, qd, qf);
        (*nbad)++;
    } else if (fabsf(v) >= 0x1p-100f && fabsf(qd) >= 0x1p-100f && bits_of(qd) != bits_of(qf)) {
        if (*nbits < 5) printf("quotient mismatch v=%a sf=%a division=%a fma=%a\n", v, sf, qd, qf);
        (*nbits)++;
    }
    return 1;
}

static uint32_t next_u32(uint64_t* st) {
    *st ^= *st << 13;
    *st ^= *st >> 7;
    *st ^= *st << 17;
    return (uint32_t)(*st >> 16);
}

int main(void) {
    /* ties and their neighbours, every bf16 scale */
#pragma omp parallel for reduction(+ : bad, bad_bits, checked, bad_fast, fallback) schedule(dynamic, 64)
    for (uint32_t sb = 0; sb < 0x7f80; ++sb) {
        float sf = bf16_value(sb);
        if (!(sf >= 1e-8f)) continue;
        float r = 1.0f / sf;
        for (int h2 = -16; h2 <= 16; ++h2) {
            float base = (float)h2 * 0.5f * sf;      /* exact: <= 5 + 8 significant bits */
            for (int j = -3; j <= 3; ++j) {
                float b = ldexpf(base, j);
                float up = b, dn = b;
                checked += check(b, sf, r, &bad, &bad_bits, &bad_fast, &fallback);
                for (int k = 0; k < 64; ++k) {
                    up = nextafterf(up, INFINITY);
                    dn = nextafterf(dn, -INFINITY);
                    checked += check(up, sf, r, &bad, &bad_bits, &bad_fast, &fallback);
                    checked += check(dn, sf, r, &bad, &bad_bits, &bad_fast, &fallback);
                }
            }
        }
    }
    /* pseudo-random pairs over the exponent range, 2^29 per run */
#pragma omp parallel for reduction(+ : bad, bad_bits, checked, bad_fast, fallback) schedule(static)
    for (int chunk = 0; chunk < 512; ++chunk) {
        uint64_t st = 0x9E3779B97F4A7C15ull ^ ((uint64_t)chunk * 0xD1B54A32D192ED03ull);
        for (long i = 0; i < (1L << 20); ++i) {
            uint32_t sb = 0x3280 + next_u32(&st) % (0x7f00 - 0x3280);  /* bf16 scales from ~1.5e-8 up */
            float sf = bf16_value(sb);
            float v = f_from_bits(next_u32(&st) & 0xdfffffffu);        /* exponent field < 192 */
            checked += check(v, sf, 1.0f / sf, &bad, &bad_bits, &bad_fast, &fallback);
        }
    }
    printf("checked %ld (v, sf) pairs, code mismatches %ld, quotient mismatches %ld, "
           "one-fma code mismatches %ld (fallbacks %ld)\n", checked, bad, bad_bits, bad_fast, fallback);
    return (bad != 0 || bad_bits != 0 || bad_fast != 0);
}
