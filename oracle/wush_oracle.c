/*
 * wush_oracle.c -- CPU restatement of the WUSH INT4 W4A4 path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * torch binding, the my_int4 package) links, loads or calls this file.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as
 * the checker.
 *
 * Build (see oracle/Makefile): gcc -O2 -ffp-contract=off -fno-fast-math
 * -fPIC -shared.  On x86-64 every float operation below is one SSE
 * instruction with round-to-nearest-even and denormals kept, which is the
 * arithmetic of the reference's eager torch CPU path.
 *
 * Each function cites the reference file:line it restates
 * (paths relative to the reference repository root).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* rtn_int4.py:19  C_CLIP = 0.35337862372398376 (fp32 bits 0x3EB4EE0B);
 * rtn_int4.py:44  "+ 1e-8" (fp32 bits 0x322BCC77). */
static const float C_CLIP = 0.35337862372398376f;
static const float EPS = 1e-8f;

static inline float bf16_to_f32(uint16_t b)
{
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even fp32 -> bf16, as torch's Tensor.to(torch.bfloat16)
 * (rtn_int4.py:47).  NaN maps to the quiet pattern 0x7FC0 with its sign. */
static inline uint16_t f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float half_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, u;
    if (e == 0) {
        if (m == 0) {
            u = sign;
        } else { /* subnormal half: normalise */
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; ++sh; }
            m &= 0x3ffu;
            u = sign | ((uint32_t)(127 - 15 - sh + 1) << 23) | (m << 13);
        }
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Code for one value: round-half-even of the IEEE quotient, clamp to
 * [-7, 7] (rtn_int4.py:50-51; quant_int4.cu:90-93).  NaN -> 0, which is what
 * the reference GPU kernel's __float2int_rn yields (quant_int4.cu:90). */
static inline int code_of(float v, float scale)
{
    float y = v / scale;
    if (y != y)
        return 0;
    float r = rintf(y);
    if (r > 7.0f) r = 7.0f;
    if (r < -7.0f) r = -7.0f;
    return (int)r;
}

/* One 32-element group: rtn_int4.py:22-55 / quant_int4.cu:59-100.
 *   s1 = sum x_i, s2 = sum x_i*x_i, i = 0..31 in order, every mul and add
 *   rounded separately (rtn_int4.py:22-30);
 *   mean = s1/32, var = s2/32 - mean*mean (rtn_int4.py:40-41);
 *   scale = var >= 0 ? sqrt(var)*C_CLIP + 1e-8 : 1.0 (rtn_int4.py:42-45);
 *   s = bf16(scale); codes from the bf16 value (rtn_int4.py:47-51);
 *   byte k = code[2k] & 0xF | (code[2k+1] & 0xF) << 4 (rtn_int4.py:53-55). */
static void quant_group(const float *v, uint8_t *q, uint16_t *s)
{
    float s1 = 0.0f, s2 = 0.0f;
    for (int i = 0; i < 32; ++i) {
        float p = v[i] * v[i];
        s1 = s1 + v[i];
        s2 = s2 + p;
    }
    float mean = s1 / 32.0f;
    float mm = mean * mean;
    float var = s2 / 32.0f - mm;
    float scale = 1.0f;
    if (var >= 0.0f) {
        float r = sqrtf(var);
        float t = r * C_CLIP;
        scale = t + EPS;
    }
    uint16_t sb = f32_to_bf16(scale);
    float sf = bf16_to_f32(sb);
    *s = sb;
    for (int k = 0; k < 16; ++k) {
        int c0 = code_of(v[2 * k], sf);
        int c1 = code_of(v[2 * k + 1], sf);
        q[k] = (uint8_t)((c0 & 0xF) | ((c1 & 0xF) << 4));
    }
}

/* rtn_int4.quant_int4 on fp32 input of n_groups*32 values. */
void oracle_quant_f32(const float *x, uint8_t *q, uint16_t *s, int64_t n_groups)
{
    for (int64_t g = 0; g < n_groups; ++g)
        quant_group(x + g * 32, q + g * 16, s + g);
}

/* Same on bf16 input (_C.quant_int4's dtype, quant_int4.cu:112); the bf16 ->
 * fp32 widening is exact (rtn_int4.py:36). */
void oracle_quant_bf16(const uint16_t *x, uint8_t *q, uint16_t *s, int64_t n_groups)
{
    float v[32];
    for (int64_t g = 0; g < n_groups; ++g) {
        for (int i = 0; i < 32; ++i)
            v[i] = bf16_to_f32(x[g * 32 + i]);
        quant_group(v, q + g * 16, s + g);
    }
}

/* Same on fp16 input (rtn_int4.py:36 upcasts any float dtype). */
void oracle_quant_f16(const uint16_t *x, uint8_t *q, uint16_t *s, int64_t n_groups)
{
    float v[32];
    for (int64_t g = 0; g < n_groups; ++g) {
        for (int i = 0; i < 32; ++i)
            v[i] = half_to_f32(x[g * 32 + i]);
        quant_group(v, q + g * 16, s + g);
    }
}

/* WUSH transform of one row: x'_j = sum_i x_i * T[c][j][i], i ascending,
 * mul then add, fp32, starting from 0 (test_sw2.py:12-24 ref_fused;
 * fused_tq_int4.cu:48-58).  x and t are bf16 bit patterns. */
void oracle_transform_bf16(const uint16_t *x, const uint16_t *t, float *xp,
                           int64_t rows, int64_t K)
{
    const int64_t C = K / 32;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < C; ++c) {
            const uint16_t *xg = x + r * K + c * 32;
            const uint16_t *tc = t + c * 1024;
            float xv[32];
            for (int i = 0; i < 32; ++i)
                xv[i] = bf16_to_f32(xg[i]);
            for (int j = 0; j < 32; ++j) {
                float acc = 0.0f;
                for (int i = 0; i < 32; ++i) {
                    float p = xv[i] * bf16_to_f32(tc[j * 32 + i]);
                    acc = acc + p;
                }
                xp[r * K + c * 32 + j] = acc;
            }
        }
    }
}

/* Fused transform + quant (fused_tq_int4.cu:27-85): the transform above, then
 * the group quantizer on the fp32 x' (no bf16 rounding of x'). */
void oracle_fused_tq_bf16(const uint16_t *x, const uint16_t *t, uint8_t *q, uint16_t *s,
                          int64_t rows, int64_t K)
{
    const int64_t C = K / 32;
    float xp[32];
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < C; ++c) {
            const uint16_t *xg = x + r * K + c * 32;
            const uint16_t *tc = t + c * 1024;
            float xv[32];
            for (int i = 0; i < 32; ++i)
                xv[i] = bf16_to_f32(xg[i]);
            for (int j = 0; j < 32; ++j) {
                float acc = 0.0f;
                for (int i = 0; i < 32; ++i) {
                    float p = xv[i] * bf16_to_f32(tc[j * 32 + i]);
                    acc = acc + p;
                }
                xp[j] = acc;
            }
            quant_group(xp, q + (r * C + c) * 16, s + r * C + c);
        }
    }
}

/* Nibble -> signed int (rtn_int4.py:60-65, "<<12 >>12" on int16). */
static inline int nib(uint8_t b, int hi)
{
    int v = hi ? (b >> 4) : (b & 0xF);
    return v >= 8 ? v - 16 : v;
}

/* dequant_int4 (rtn_int4.py:58-68): code * float(scale), exact in fp32. */
void oracle_dequant(const uint8_t *q, const uint16_t *s, float *out, int64_t n_groups)
{
    for (int64_t g = 0; g < n_groups; ++g) {
        float sf = bf16_to_f32(s[g]);
        for (int k = 0; k < 16; ++k) {
            uint8_t b = q[g * 16 + k];
            out[g * 32 + 2 * k] = (float)nib(b, 0) * sf;
            out[g * 32 + 2 * k + 1] = (float)nib(b, 1) * sf;
        }
    }
}

/* Exact int32 per-group dot products D[m][n][g] = sum_{k in g} qx*qw
 * (gemm_int4.cu:63-82; gemm_s4.cu:85 "Y = sum_g sx*sw*D"). */
void oracle_group_dots(const uint8_t *xq, const uint8_t *wq, int32_t *D,
                       int64_t M, int64_t N, int64_t K)
{
    const int64_t G = K / 32, K2 = K / 2;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n)
            for (int64_t g = 0; g < G; ++g) {
                int32_t acc = 0;
                for (int k = 0; k < 16; ++k) {
                    uint8_t a = xq[m * K2 + g * 16 + k], b = wq[n * K2 + g * 16 + k];
                    acc += nib(a, 0) * nib(b, 0) + nib(a, 1) * nib(b, 1);
                }
                D[(m * N + n) * G + g] = acc;
            }
}

/* fp64 evaluation of the dequantized product (test_p13.py:22):
 * Y[m][n] = sum_g double(sx)*double(sw)*D.  Each term is exact in double
 * (|D| < 2^11, bf16 scales have 8-bit significands) and equals
 * sum_{k in g} dq_x * dq_w, so this is dequant(x) @ dequant(w)^T in fp64. */
void oracle_gemm_f64(const uint8_t *xq, const uint16_t *xs, const uint8_t *wq, const uint16_t *ws,
                     double *Y, int64_t M, int64_t N, int64_t K)
{
    const int64_t G = K / 32, K2 = K / 2;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int64_t g = 0; g < G; ++g) {
                int32_t d = 0;
                for (int k = 0; k < 16; ++k) {
                    uint8_t a = xq[m * K2 + g * 16 + k], b = wq[n * K2 + g * 16 + k];
                    d += nib(a, 0) * nib(b, 0) + nib(a, 1) * nib(b, 1);
                }
                acc += (double)bf16_to_f32(xs[m * G + g]) * (double)bf16_to_f32(ws[n * G + g]) * (double)d;
            }
            Y[m * N + n] = acc;
        }
}

/* Per-tensor quant (fast_path.cu:17-39; bit mirror test_p12.py:21-26):
 * code = clamp(rint(x * inv_scale), -7, 7) with one fp32 multiply. */
void oracle_quant_tensor_scale_bf16(const uint16_t *x, uint8_t *q, int64_t n, float inv_scale)
{
    for (int64_t k = 0; k < n / 2; ++k) {
        int c[2];
        for (int h = 0; h < 2; ++h) {
            float y = bf16_to_f32(x[2 * k + h]) * inv_scale;
            if (y != y) {
                c[h] = 0;
                continue;
            }
            float r = rintf(y);
            if (r > 7.0f) r = 7.0f;
            if (r < -7.0f) r = -7.0f;
            c[h] = (int)r;
        }
        q[k] = (uint8_t)((c[0] & 0xF) | ((c[1] & 0xF) << 4));
    }
}

/* Per-tensor GEMM in fp64 (test_p12.py:94-105): alpha * sum_k qx*qw. */
void oracle_gemm_tensor_scale_f64(const uint8_t *xq, const uint8_t *wq, double alpha, double *Y,
                                  int64_t M, int64_t N, int64_t K)
{
    const int64_t K2 = K / 2;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            int64_t acc = 0;
            for (int64_t k = 0; k < K2; ++k) {
                uint8_t a = xq[m * K2 + k], b = wq[n * K2 + k];
                acc += nib(a, 0) * nib(b, 0) + nib(a, 1) * nib(b, 1);
            }
            Y[m * N + n] = alpha * (double)acc;
        }
}

/* The s4 fragment self-test's product (gemm_s4.cu:50-82): C = A(8x32) B(32x8)
 * in int32. */
void oracle_int_matmul_8x32x8(const int8_t *a, const int8_t *b, int32_t *c)
{
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 8; ++j) {
            int32_t acc = 0;
            for (int k = 0; k < 32; ++k)
                acc += (int32_t)a[i * 32 + k] * (int32_t)b[k * 8 + j];
            c[i * 8 + j] = acc;
        }
}
