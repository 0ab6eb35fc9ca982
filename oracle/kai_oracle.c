/*
 * CPU oracle for the GGUF dequant-fused quantized linear path.
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library and the timed CPU
 * baseline; see kai_oracle.h for what it restates and how it is pinned.
 */
#include "kai_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle_iq3s_grid.h"

#ifdef _OPENMP
#include <omp.h>
#endif

#define QK8_1 32
#define Q8_1_BYTES 36

int oracle_block_elems(int type) {
    switch (type) {
        case ORACLE_Q4_0: case ORACLE_Q8_0: case ORACLE_Q8_1: return 32;
        case ORACLE_Q2_K: case ORACLE_Q4_K: case ORACLE_Q6_K: case ORACLE_IQ3_S: return 256;
        default: return 0;
    }
}

/* Byte sizes: gguf_repack.py:20-34, triton/gemm/utils.py:28-47. */
int oracle_block_bytes(int type) {
    switch (type) {
        case ORACLE_Q4_0: return 18;
        case ORACLE_Q8_0: return 34;
        case ORACLE_Q8_1: return 36;
        case ORACLE_Q2_K: return 84;
        case ORACLE_Q4_K: return 144;
        case ORACLE_Q6_K: return 210;
        case ORACLE_IQ3_S: return 110;
        default: return 0;
    }
}

/* ---------------------------------------------------------------- fp16 / bf16 */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1f;
    const uint32_t mant = h & 0x3ffu;
    if (exp == 0) {
        /* zero or subnormal: mant * 2^-24, exact in float */
        const float v = (float)mant * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((uint32_t)(exp - 15 + 127) << 23) | (mant << 13));
}

/* IEEE binary32 -> binary16, round to nearest, ties to even; overflow -> inf. */
uint16_t oracle_float_to_half(float f) {
    const uint32_t u = f2u(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) { /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u | ((a >> 13) & 0x3ffu) : 0));
    }
    const int e = (int)(a >> 23) - 127;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {
        /* normal half: keep 10 mantissa bits, round the 13 dropped bits */
        uint32_t mant = a & 0x7fffffu;
        uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
        const uint32_t rest = mant & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1; /* may carry into exp: fine */
        return (uint16_t)(sign | h);
    }
    if (e < -25) return sign; /* below half of the smallest subnormal */
    /* subnormal half: value = m * 2^-24, m = round(a * 2^24) with ties to even */
    const uint32_t mant = (a & 0x7fffffu) | 0x800000u; /* value = mant * 2^(e-23) */
    const int shift = -e - 14 + 13;                    /* bits dropped to reach 2^-24 units */
    uint32_t h = mant >> shift;
    const uint32_t rest = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rest > half || (rest == half && (h & 1u))) h += 1;
    return (uint16_t)(sign | h);
}

float oracle_bf16_to_float(uint16_t b) { return u2f((uint32_t)b << 16); }

static float load_x(const void *x, int dtype, int64_t i) {
    switch (dtype) {
        case 0: return ((const float *)x)[i];
        case 1: return oracle_bf16_to_float(((const uint16_t *)x)[i]);
        default: return oracle_half_to_float(((const uint16_t *)x)[i]);
    }
}

/* ---------------------------------------------------------------- Q8_1 prep */

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

/* kai_dual_mmvq.cuh:399-403 and current_ggml_direct.cu:808-839. */
size_t oracle_activation_bytes(int64_t m, int64_t k, int two_pass) {
    const size_t pass = align256((size_t)m * (size_t)(k / QK8_1) * Q8_1_BYTES);
    return pass * (two_pass ? 2 : 1) + align256((size_t)m * sizeof(float));
}

/* C roundf: half-way cases away from zero (what CUDA's roundf does too). */
static void store_q8_1(uint8_t *blk, const int8_t *q, float d, int isum) {
    const uint16_t hd = oracle_float_to_half(d);
    const uint16_t hs = oracle_float_to_half(d * (float)isum);
    memcpy(blk, &hd, 2);
    memcpy(blk + 2, &hs, 2);
    memcpy(blk + 4, q, 32);
}

/*
 * kai_dual::prepare_dual (kai_dual_mmvq.cuh:147-254):
 *   row amax (fmaxf over |x|, :157-200); biased exponent e of amax;
 *   se = clamp(260 - e, 1, 253) for 0 < e < 255 else 127; scale = 2^(se-127),
 *   inverse = 2^(127-se) (:202-211);
 *   per 32 values: v = x*scale; a = max|v|; d = a/127; q = a == 0 ? 0 : roundf(v/d);
 *   ds = (half(d), half(d * sum q)) (:216-233);
 *   two_pass: v -= half(d)*q (contracted to one fused multiply-add, as CUDA does
 *   for `v[j] -= d1h * float(q1[j])`), then the same quantization (:235-253).
 */
int oracle_prepare(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                   void *activation, int two_pass) {
    if (!x || !activation || m < 1 || k <= 0 || k % QK8_1 || stride_x < k || x_dtype < 0 || x_dtype > 2)
        return -1;
    const int64_t nb = k / QK8_1;
    const size_t pass = align256((size_t)m * (size_t)nb * Q8_1_BYTES);
    uint8_t *y1 = (uint8_t *)activation;
    uint8_t *y2 = two_pass ? y1 + pass : NULL;
    float *inverse = (float *)(y1 + pass * (two_pass ? 2 : 1));
    for (int64_t row = 0; row < m; ++row) {
        float amax = 0.0f;
        for (int64_t i = 0; i < k; ++i) amax = fmaxf(amax, fabsf(load_x(x, x_dtype, row * stride_x + i)));
        const int biased = (int)((f2u(amax) >> 23) & 255u);
        int se = 127;
        if (biased != 0 && biased != 255) {
            se = 260 - biased;
            if (se < 1) se = 1;
            if (se > 253) se = 253;
        }
        const float scale = u2f((uint32_t)se << 23);
        inverse[row] = u2f((uint32_t)(254 - se) << 23);
        for (int64_t ib = 0; ib < nb; ++ib) {
            float v[32];
            float a1 = 0.0f;
            for (int j = 0; j < 32; ++j) {
                v[j] = load_x(x, x_dtype, row * stride_x + ib * 32 + j) * scale;
                a1 = fmaxf(a1, fabsf(v[j]));
            }
            const float d1 = a1 / 127.0f;
            int8_t q1[32];
            int isum1 = 0;
            for (int j = 0; j < 32; ++j) {
                q1[j] = (int8_t)(a1 == 0.0f ? 0.0f : roundf(v[j] / d1));
                isum1 += q1[j];
            }
            store_q8_1(y1 + (row * nb + ib) * Q8_1_BYTES, q1, d1, isum1);
            if (two_pass) {
                uint16_t hd;
                memcpy(&hd, y1 + (row * nb + ib) * Q8_1_BYTES, 2);
                const float d1h = oracle_half_to_float(hd);
                float a2 = 0.0f;
                for (int j = 0; j < 32; ++j) {
                    v[j] = fmaf(-d1h, (float)q1[j], v[j]);
                    a2 = fmaxf(a2, fabsf(v[j]));
                }
                const float d2 = a2 / 127.0f;
                int8_t q2[32];
                int isum2 = 0;
                for (int j = 0; j < 32; ++j) {
                    q2[j] = (int8_t)(a2 == 0.0f ? 0.0f : roundf(v[j] / d2));
                    isum2 += q2[j];
                }
                store_q8_1(y2 + (row * nb + ib) * Q8_1_BYTES, q2, d2, isum2);
            }
        }
    }
    return 0;
}

/* Sum of 32 values as the xor butterfly of gguf_kernel.cu:50-54 leaves it in lane 0:
 * pass h (16, 8, 4, 2, 1) adds value i + h to value i for i < h. fp32 addition is
 * commutative, so lane 0's `sum += shfl(sum, h)` is this sum whichever operand is first. */
static float butterfly_sum32(const float *v) {
    float t[32];
    memcpy(t, v, sizeof t);
    for (int h = 16; h >= 1; h >>= 1)
        for (int i = 0; i < h; ++i) t[i] = t[i] + t[i + h];
    return t[0];
}

/* quantize_q8_1 (gguf_kernel.cu:32-69): per 32 values d = amax / 127,
 * q = amax == 0 ? 0 : roundf(x / d) (:56-57), ds = (half(d), half(sum x)) (:67-68); no row
 * normalisation, so inverse = 1. */
int oracle_prepare_legacy(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                          void *activation) {
    if (!x || !activation || m < 1 || k <= 0 || k % QK8_1 || stride_x < k || x_dtype < 0 || x_dtype > 2)
        return -1;
    const int64_t nb = k / QK8_1;
    uint8_t *y = (uint8_t *)activation;
    float *inverse = (float *)(y + align256((size_t)m * (size_t)nb * Q8_1_BYTES));
    for (int64_t row = 0; row < m; ++row) {
        inverse[row] = 1.0f;
        for (int64_t ib = 0; ib < nb; ++ib) {
            float v[32];
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) {
                v[j] = load_x(x, x_dtype, row * stride_x + ib * 32 + j);
                amax = fmaxf(amax, fabsf(v[j]));
            }
            const float d = amax / 127.0f;
            int8_t q[32];
            for (int j = 0; j < 32; ++j) q[j] = (int8_t)(amax == 0.0f ? 0.0f : roundf(v[j] / d));
            uint8_t *blk = y + (row * nb + ib) * Q8_1_BYTES;
            const uint16_t hd = oracle_float_to_half(d), hs = oracle_float_to_half(butterfly_sum32(v));
            memcpy(blk, &hd, 2);
            memcpy(blk + 2, &hs, 2);
            memcpy(blk + 4, q, 32);
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- fused producers */

/* Round to nearest even; NaN -> quiet NaN with the sign and top payload bits kept. */
uint16_t oracle_float_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float round_to_dtype(float v, int dtype) {
    if (dtype == 1) return oracle_bf16_to_float(oracle_float_to_bf16(v));
    if (dtype == 2) return oracle_half_to_float(oracle_float_to_half(v));
    return v;
}

/*
 * e^x as the SwiGLU producer evaluates it (the exp of the reference's silu,
 * kai_prepare_ext.cuh:158, is CUDA's expf, whose bits are unspecified): Cody-Waite
 * reduction x = n ln2 + r with ln2 split as 0.693145751953125 (exact in 16 bits) +
 * 1.42860682030941723212e-6, e^r by its degree-7 Taylor polynomial in Horner form with
 * fused multiply-adds, scaled by 2^n. Every line is one IEEE operation.
 */
float oracle_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.97208404541015625f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.42860682030941723212e-6f, r);
    float p = 1.98412698e-4f;
    p = fmaf(p, r, 1.38888889e-3f);
    p = fmaf(p, r, 8.33333333e-3f);
    p = fmaf(p, r, 4.16666667e-2f);
    p = fmaf(p, r, 1.66666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/*
 * kai_dual::prepare_view (kai_prepare_ext.cuh:121-140, entry current_ggml_direct.cu:883-901):
 * stored column c of row j is x[j, ((c/s)%a)*b*s + (c/(a*s))*s + c%s], then the single-pass
 * Q8_1 preparation of those values (oracle_prepare with two_pass = 0).
 */
int oracle_prepare_view(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                        void *activation, int64_t a, int64_t b, int64_t s) {
    if (!x || !activation || m < 1 || k <= 0 || k % QK8_1 || stride_x < k || s <= 0 || s % QK8_1 ||
        a <= 0 || b <= 0 || a * b * s != k || x_dtype < 0 || x_dtype > 2)
        return -1;
    float *v = (float *)malloc((size_t)(m * k) * sizeof(float));
    if (!v) return -1;
    for (int64_t j = 0; j < m; ++j)
        for (int64_t c = 0; c < k; ++c)
            v[j * k + c] = load_x(x, x_dtype, j * stride_x + ((c / s) % a) * b * s + (c / (a * s)) * s + c % s);
    const int rc = oracle_prepare(v, 0, m, k, k, activation, 0);
    free(v);
    return rc;
}

/*
 * kai_dual::prepare_swiglu (kai_prepare_ext.cuh:142-183, entry current_ggml_direct.cu:903-919):
 * act[c] = rd(rd(g / (1 + exp(-g))) * u) with g = row[c], u = row[k + c], rd rounding to
 * the input dtype and exp = oracle_expf; then the single-pass Q8_1 preparation.
 */
int oracle_prepare_swiglu(const void *gate_up, int dtype, int64_t m, int64_t k, int64_t stride,
                          void *activation) {
    if (!gate_up || !activation || m < 1 || k <= 0 || k % QK8_1 || stride < 2 * k || dtype < 0 || dtype > 2)
        return -1;
    float *v = (float *)malloc((size_t)(m * k) * sizeof(float));
    if (!v) return -1;
    for (int64_t j = 0; j < m; ++j)
        for (int64_t c = 0; c < k; ++c) {
            const float g = load_x(gate_up, dtype, j * stride + c);
            const float u = load_x(gate_up, dtype, j * stride + k + c);
            v[j * k + c] = round_to_dtype(round_to_dtype(g / (1.0f + oracle_expf(-g)), dtype) * u, dtype);
        }
    const int rc = oracle_prepare(v, 0, m, k, k, activation, 0);
    free(v);
    return rc;
}

/*
 * kai_dual::norm_prepare (kai_prepare_ext.cuh:185-251, entry current_ggml_direct.cu:921-944):
 * v = x (+ r; v is stored to residual_out), y = bf16((v * rstd) * w32) with
 * rstd = 1 / sqrt(sum(v^2) / k + eps), and the single-pass Q8_1 preparation of y.
 * sum(v^2) is summed in the order the HIP producer uses (the reference's warp-shuffle order
 * differs, so its y may differ from this one by one bf16 ulp where the product sits on a
 * rounding boundary): 512 partial sums, partial t taking runs t, t + 512, ... of 8 values
 * in order by fused multiply-adds; a pairwise tree over each 64 consecutive partials;
 * the 8 tree sums added in order.
 */
int oracle_norm_prepare(const void *x, int x_dtype, int64_t stride_x, const void *residual,
                        int residual_dtype, int64_t stride_r, float *residual_out,
                        const float *weight32, float eps, uint16_t *y, int64_t m, int64_t k,
                        void *activation) {
    enum { THREADS = 512, LANES = 64 };
    if (!x || !y || !weight32 || !activation || m < 1 || k <= 0 || k % QK8_1 || stride_x < k ||
        (residual && (!residual_out || stride_r < k)) || x_dtype < 0 || x_dtype > 1 ||
        (residual && (residual_dtype < 0 || residual_dtype > 1)) || k / 8 > (int64_t)THREADS * 8)
        return -1;
    float *v = (float *)malloc((size_t)(m * k) * sizeof(float));
    if (!v) return -1;
    for (int64_t j = 0; j < m; ++j) {
        float *vr = v + j * k;
        for (int64_t c = 0; c < k; ++c) {
            vr[c] = load_x(x, x_dtype, j * stride_x + c);
            if (residual) {
                vr[c] += load_x(residual, residual_dtype, j * stride_r + c);
                residual_out[j * k + c] = vr[c];
            }
        }
        float part[THREADS];
        for (int t = 0; t < THREADS; ++t) {
            float ss = 0.0f;
            for (int64_t r = t; r < k / 8; r += THREADS)
                for (int e = 0; e < 8; ++e) ss = fmaf(vr[8 * r + e], vr[8 * r + e], ss);
            part[t] = ss;
        }
        for (int width = 1; width < LANES; width *= 2)
            for (int t = 0; t < THREADS; t += 2 * width) part[t] = part[t] + part[t + width];
        float total = part[0];
        for (int w = 1; w < THREADS / LANES; ++w) total += part[w * LANES];
        const float rstd = 1.0f / sqrtf(total / (float)k + eps);
        for (int64_t c = 0; c < k; ++c) {
            const uint16_t h = oracle_float_to_bf16(vr[c] * rstd * weight32[c]);
            y[j * k + c] = h;
            vr[c] = oracle_bf16_to_float(h);
        }
    }
    const int rc = oracle_prepare(v, 0, m, k, k, activation, 0);
    free(v);
    return rc;
}

/* ---------------------------------------------------------------- weight decoding */

static float rd_half(const uint8_t *p) { uint16_t h; memcpy(&h, p, 2); return oracle_half_to_float(h); }

/* Q4_K 6-bit scale/min unpack: gguf-py quants.py:480-502 (Q4_K.get_scale_min). */
static void q4k_scale_min(const uint8_t *s, uint8_t sc[8], uint8_t mn[8]) {
    for (int i = 0; i < 4; ++i) {
        sc[i] = s[i] & 63;
        mn[i] = s[4 + i] & 63;
        sc[4 + i] = (uint8_t)((s[8 + i] & 0x0f) | ((s[i] >> 2) & 0x30));
        mn[4 + i] = (uint8_t)((s[8 + i] >> 4) | ((s[4 + i] >> 2) & 0x30));
    }
}

/* Integer code of element e of a block (see each case for its layout). */
static int q6k_code(const uint8_t *b, int e) {
    /* quants.py:553-573: e = 128h + 32s + l; low 4 bits from ql[64h + 32(s%2) + l]
     * (nibble s/2), high 2 bits from qh[32h + l] bits 2s..2s+1; value code - 32. */
    const int h = e / 128, s = (e % 128) / 32, l = e % 32;
    const int lo = (b[64 * h + 32 * (s % 2) + l] >> (4 * (s / 2))) & 0x0f;
    const int hi = (b[128 + 32 * h + l] >> (2 * s)) & 3;
    return (lo | (hi << 4)) - 32;
}

static int q2k_code(const uint8_t *b, int e) {
    /* quants.py:407-429: e = 128h + 32s + l; code = (qs[32h + l] >> 2s) & 3, qs at byte 16. */
    const int h = e / 128, s = (e % 128) / 32, l = e % 32;
    return (b[16 + 32 * h + l] >> (2 * s)) & 3;
}

static int q4k_code(const uint8_t *b, int e) {
    /* quants.py:505-523: sub-block i = e/32; qs[32(i/2) + l] low nibble for even i,
     * high nibble for odd i; qs at byte 16. */
    const int i = e / 32, l = e % 32;
    return (b[16 + 32 * (i / 2) + l] >> (4 * (i % 2))) & 0x0f;
}

/* IQ3_S signed level of element e: quants.py:1097-1125. */
static int iq3s_value(const uint8_t *b, int e) {
    const int g = e / 32, t = e % 32, i = t / 4, j = t % 4;
    const int idx = b[2 + 8 * g + i] | (((b[66 + g] >> i) & 1) << 8);
    const int level = oracle_iq3s_levels[idx][j];
    const int neg = (b[74 + 4 * g + t / 8] >> (t % 8)) & 1;
    return neg ? -level : level;
}

static int iq3s_scale(const uint8_t *b, int g) { return (b[106 + g / 2] >> (4 * (g % 2))) & 0x0f; }

int oracle_dequantize_row(int type, const uint8_t *row, int64_t k, float *out) {
    const int qk = oracle_block_elems(type), bb = oracle_block_bytes(type);
    if (!qk || type == ORACLE_Q8_1 || k % qk) return -1;
    for (int64_t blk = 0; blk < k / qk; ++blk) {
        const uint8_t *b = row + blk * bb;
        float *o = out + blk * qk;
        switch (type) {
            case ORACLE_Q8_0: { /* quants.py:397-402 */
                const float d = rd_half(b);
                for (int e = 0; e < 32; ++e) o[e] = d * (float)(int8_t)b[2 + e];
                break;
            }
            case ORACLE_Q4_0: { /* quants.py:242-252 */
                const float d = rd_half(b);
                for (int e = 0; e < 16; ++e) {
                    o[e] = d * (float)((b[2 + e] & 0x0f) - 8);
                    o[e + 16] = d * (float)((b[2 + e] >> 4) - 8);
                }
                break;
            }
            case ORACLE_Q4_K: {
                const float d = rd_half(b), dmin = rd_half(b + 2);
                uint8_t sc[8], mn[8];
                q4k_scale_min(b + 4, sc, mn);
                for (int e = 0; e < 256; ++e)
                    o[e] = d * (float)sc[e / 32] * (float)q4k_code(b, e) - dmin * (float)mn[e / 32];
                break;
            }
            case ORACLE_Q6_K: {
                const float d = rd_half(b + 208);
                for (int e = 0; e < 256; ++e) o[e] = d * (float)(int8_t)b[192 + e / 16] * (float)q6k_code(b, e);
                break;
            }
            case ORACLE_Q2_K: {
                const float d = rd_half(b + 80), dmin = rd_half(b + 82);
                for (int e = 0; e < 256; ++e) {
                    const int s = b[e / 16];
                    o[e] = d * (float)(s & 0x0f) * (float)q2k_code(b, e) - dmin * (float)(s >> 4);
                }
                break;
            }
            case ORACLE_IQ3_S: {
                const float d = rd_half(b);
                for (int e = 0; e < 256; ++e)
                    o[e] = d * (float)(1 + 2 * iq3s_scale(b, e / 32)) * (float)iq3s_value(b, e);
                break;
            }
            default: return -1;
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- block dots */

typedef struct {
    const uint8_t *blocks; /* Q8_1 blocks of one activation row */
} q8row;

static float q8_d(const uint8_t *blk) { return rd_half(blk); }
static float q8_s(const uint8_t *blk) { return rd_half(blk + 2); }
static const int8_t *q8_q(const uint8_t *blk) { return (const int8_t *)(blk + 4); }

/*
 * One weight block against the matching Q8_1 blocks, in FP64 from exact integer sums.
 * Formulas (vecdotq.cuh in-tree b2899 text; upstream @0c1e570 has the same arithmetic):
 *   Q8_0  d_w * d8 * sum q_w q8                                   (:165-177, :852-867)
 *   Q4_0  d_w * (d8 * sum nib q8 - 8 * s8), s8 = stored half ds.y  (:46-66, :493-509)
 *   Q4_K  sum_i d8_i (d sc_i dot_i - dmin m_i sum q8_i)           (:328-351, :1159-1202)
 *   Q6_K  d * sum_g d8 sc_g dot(code - 32, q8) over 16-groups       (:447-465, :1417-1441)
 *   Q2_K  sum_g d8 (d sc_g dot(code, q8) - dmin m_g sum q8) per 16  (:204-230, :923-944)
 *   IQ3_S sum_i d d8_i (1 + 2 sc_i) dot(signed grid level, q8)      (:1649-1672; quants.py:1109)
 */
static double block_dot(int type, const uint8_t *b, const uint8_t *q8) {
    switch (type) {
        case ORACLE_Q8_0: {
            const int8_t *u = q8_q(q8);
            int64_t s = 0;
            for (int e = 0; e < 32; ++e) s += (int64_t)(int8_t)b[2 + e] * u[e];
            return (double)rd_half(b) * (double)q8_d(q8) * (double)s;
        }
        case ORACLE_Q4_0: {
            const int8_t *u = q8_q(q8);
            int64_t s = 0;
            for (int e = 0; e < 16; ++e) s += (int64_t)(b[2 + e] & 0x0f) * u[e] + (int64_t)(b[2 + e] >> 4) * u[e + 16];
            return (double)rd_half(b) * ((double)q8_d(q8) * (double)s - 8.0 * (double)q8_s(q8));
        }
        case ORACLE_Q4_K: {
            const double d = rd_half(b), dmin = rd_half(b + 2);
            uint8_t sc[8], mn[8];
            q4k_scale_min(b + 4, sc, mn);
            double acc = 0.0;
            for (int i = 0; i < 8; ++i) {
                const uint8_t *blk = q8 + i * Q8_1_BYTES;
                const int8_t *u = q8_q(blk);
                int64_t dot = 0, usum = 0;
                for (int l = 0; l < 32; ++l) {
                    dot += (int64_t)q4k_code(b, 32 * i + l) * u[l];
                    usum += u[l];
                }
                acc += (double)q8_d(blk) * (d * sc[i] * (double)dot - dmin * mn[i] * (double)usum);
            }
            return acc;
        }
        case ORACLE_Q6_K: {
            const double d = rd_half(b + 208);
            double acc = 0.0;
            for (int g = 0; g < 16; ++g) {
                const uint8_t *blk = q8 + (g / 2) * Q8_1_BYTES;
                const int8_t *u = q8_q(blk) + 16 * (g % 2);
                int64_t dot = 0;
                for (int l = 0; l < 16; ++l) dot += (int64_t)q6k_code(b, 16 * g + l) * u[l];
                acc += (double)q8_d(blk) * (double)(int8_t)b[192 + g] * (double)dot;
            }
            return d * acc;
        }
        case ORACLE_Q2_K: {
            const double d = rd_half(b + 80), dmin = rd_half(b + 82);
            double acc = 0.0;
            for (int g = 0; g < 16; ++g) {
                const uint8_t *blk = q8 + (g / 2) * Q8_1_BYTES;
                const int8_t *u = q8_q(blk) + 16 * (g % 2);
                int64_t dot = 0, usum = 0;
                for (int l = 0; l < 16; ++l) {
                    dot += (int64_t)q2k_code(b, 16 * g + l) * u[l];
                    usum += u[l];
                }
                acc += (double)q8_d(blk) * (d * (b[g] & 0x0f) * (double)dot - dmin * (b[g] >> 4) * (double)usum);
            }
            return acc;
        }
        case ORACLE_IQ3_S: {
            const double d = rd_half(b);
            double acc = 0.0;
            for (int g = 0; g < 8; ++g) {
                const uint8_t *blk = q8 + g * Q8_1_BYTES;
                const int8_t *u = q8_q(blk);
                int64_t dot = 0;
                for (int t = 0; t < 32; ++t) dot += (int64_t)iq3s_value(b, 32 * g + t) * u[t];
                acc += d * (double)q8_d(blk) * (double)(1 + 2 * iq3s_scale(b, g)) * (double)dot;
            }
            return acc;
        }
        default: return 0.0;
    }
}

static int mm_args_ok(int type, int64_t n, int64_t k, int64_t m, const void *w, const void *act) {
    const int qk = oracle_block_elems(type);
    return w && act && qk && type != ORACLE_Q8_1 && n > 0 && m > 0 && k > 0 && k % qk == 0;
}

static double row_dot(int type, const uint8_t *wrow, int64_t k, const uint8_t *arow) {
    const int qk = oracle_block_elems(type), bb = oracle_block_bytes(type);
    double acc = 0.0;
    for (int64_t blk = 0; blk < k / qk; ++blk)
        acc += block_dot(type, wrow + blk * bb, arow + blk * (qk / QK8_1) * Q8_1_BYTES);
    return acc;
}

int oracle_mul_mat(int type, const uint8_t *weight, int64_t n, int64_t k, int64_t m,
                   const void *activation, int two_pass, double *out, int threads) {
    if (!mm_args_ok(type, n, k, m, weight, activation) || !out) return -1;
    const int qk = oracle_block_elems(type), bb = oracle_block_bytes(type);
    const int64_t row_bytes = (k / qk) * bb;
    const int64_t nb = k / QK8_1;
    const size_t pass = align256((size_t)m * (size_t)nb * Q8_1_BYTES);
    const uint8_t *y1 = (const uint8_t *)activation;
    const uint8_t *y2 = two_pass ? y1 + pass : NULL;
    const float *inverse = (const float *)(y1 + pass * (two_pass ? 2 : 1));
    (void)threads;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t j = 0; j < m; ++j) {
            double acc = row_dot(type, weight + r * row_bytes, k, y1 + j * nb * Q8_1_BYTES);
            if (y2) acc += row_dot(type, weight + r * row_bytes, k, y2 + j * nb * Q8_1_BYTES);
            out[j * n + r] = (double)inverse[j] * acc;
        }
    }
    return 0;
}

/* Q4_K superblock against 8 legacy Q8_1 blocks as the legacy MMQ forms it
 * (vec_dot_q4_K_q8_1_impl_mmq, vecdotq.cuh:353-377):
 *   d * sum_i d8_i sc_i dot_i - dmin * sum_i s8_i m_i, s8 = the stored half(sum x). */
static double block_dot_q4k_mmq(const uint8_t *b, const uint8_t *q8) {
    const double d = rd_half(b), dmin = rd_half(b + 2);
    uint8_t sc[8], mn[8];
    q4k_scale_min(b + 4, sc, mn);
    double sum_d = 0.0, sum_m = 0.0;
    for (int i = 0; i < 8; ++i) {
        const uint8_t *blk = q8 + i * Q8_1_BYTES;
        const int8_t *u = q8_q(blk);
        int64_t dot = 0;
        for (int l = 0; l < 32; ++l) dot += (int64_t)q4k_code(b, 32 * i + l) * u[l];
        sum_d += (double)q8_d(blk) * sc[i] * (double)dot;
        sum_m += (double)q8_s(blk) * mn[i];
    }
    return d * sum_d - dmin * sum_m;
}

int oracle_mul_mat_legacy(int type, const uint8_t *weight, int64_t n, int64_t k, int64_t m,
                          const void *activation, int batched, double *out, int threads) {
    if (!mm_args_ok(type, n, k, m, weight, activation) || !out) return -1;
    if (!(batched && type == ORACLE_Q4_K)) return oracle_mul_mat(type, weight, n, k, m, activation, 0, out, threads);
    const int64_t row_bytes = (k / 256) * 144, nb = k / QK8_1;
    const uint8_t *y = (const uint8_t *)activation;
    const float *inverse = (const float *)(y + align256((size_t)m * (size_t)nb * Q8_1_BYTES));
    (void)threads;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t j = 0; j < m; ++j) {
            double acc = 0.0;
            for (int64_t blk = 0; blk < k / 256; ++blk)
                acc += block_dot_q4k_mmq(weight + r * row_bytes + blk * 144, y + (j * nb + blk * 8) * Q8_1_BYTES);
            out[j * n + r] = (double)inverse[j] * acc;
        }
    }
    return 0;
}

int oracle_mul_mat_f32(int type, const uint8_t *weight, int64_t n, int64_t k, int64_t m,
                       const void *activation, int two_pass, float *out, int64_t stride_out,
                       int threads) {
    if (!mm_args_ok(type, n, k, m, weight, activation) || !out || stride_out < n) return -1;
    const int qk = oracle_block_elems(type), bb = oracle_block_bytes(type);
    const int64_t row_bytes = (k / qk) * bb;
    const int64_t nb = k / QK8_1;
    const size_t pass = align256((size_t)m * (size_t)nb * Q8_1_BYTES);
    const uint8_t *y1 = (const uint8_t *)activation;
    const uint8_t *y2 = two_pass ? y1 + pass : NULL;
    const float *inverse = (const float *)(y1 + pass * (two_pass ? 2 : 1));
    (void)threads;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t j = 0; j < m; ++j) {
            double acc = row_dot(type, weight + r * row_bytes, k, y1 + j * nb * Q8_1_BYTES);
            if (y2) acc += row_dot(type, weight + r * row_bytes, k, y2 + j * nb * Q8_1_BYTES);
            out[j * stride_out + r] = (float)((double)inverse[j] * acc);
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- batched path (m > 8) */

#define MMQ_BLOCK_BYTES 144 /* block_q8_1_mmq: 16 header bytes + 128 codes */
#define MMQ_ROW_PADDING 512 /* MATRIX_ROW_PADDING, current_ggml_direct.cu:1136 */

/* Layout per type: GGML's mmq_get_q8_1_ds_layout (upstream mmq.cuh), as selected per
 * matrix by layout_index (current_ggml_direct.cu:1113-1116). */
int oracle_mmq_layout(int type) {
    switch (type) {
        case ORACLE_Q8_0: case ORACLE_Q6_K: case ORACLE_IQ3_S: return ORACLE_MMQ_D4;
        case ORACLE_Q4_0: case ORACLE_Q4_K: return ORACLE_MMQ_DS4;
        case ORACLE_Q2_K: return ORACLE_MMQ_D2S6;
        default: return -1;
    }
}

int64_t oracle_mmq_blocks128(int64_t k) {
    return (k + MMQ_ROW_PADDING - 1) / MMQ_ROW_PADDING * (MMQ_ROW_PADDING / 128);
}

size_t oracle_mmq_plane_bytes(int64_t m, int64_t k) {
    return (size_t)oracle_mmq_blocks128(k) * (size_t)m * MMQ_BLOCK_BYTES;
}

/* Row scale of row_scale (current_ggml_direct.cu:978-1022): the same closed form as the
 * decode preparation (kai_dual_mmvq.cuh:202-211). Returns scale, writes inverse. */
static float mmq_row_scale(const void *x, int x_dtype, int64_t row_off, int64_t k, float *inverse) {
    float amax = 0.0f;
    for (int64_t i = 0; i < k; ++i) amax = fmaxf(amax, fabsf(load_x(x, x_dtype, row_off + i)));
    const int biased = (int)((f2u(amax) >> 23) & 255u);
    int se = 127;
    if (biased != 0 && biased != 255) {
        se = 260 - biased;
        if (se < 1) se = 1;
        if (se > 253) se = 253;
    }
    *inverse = u2f((uint32_t)(254 - se) << 23);
    return u2f((uint32_t)se << 23);
}

/* float -> int8 as the reference's char4 store of roundf(...) converts it: NaN to 0,
 * out-of-range saturated (only reachable when d_inv overflows to inf). */
static int8_t mmq_code(float p) {
    if (p != p) return 0;
    const float r = roundf(p);
    if (r > 127.0f) return 127;
    if (r < -128.0f) return -128;
    return (int8_t)r;
}

/*
 * quantize_scaled (current_ggml_direct.cu:1025-1092) over one row, normalised values v
 * (zero past k). Per G-value group (G = 64 for D2S6, else 32): amax = fmaxf over |v|
 * (:1045-1052), d_inv = 127/amax (:1053), q = roundf(v*d_inv) (:1054-1058), d = 1/d_inv
 * (:1059); sums d*float(sum q) over 32 (DS4) or 16 (D2S6) values (:1061-1068); stores
 * (:1070-1090): D4 d4[i/32] = d; DS4 ds4[i/32] = half2_rn(d, sum); D2S6 d2s6[i/64] = half(d),
 * d2s6[2 + i/16] = half(sum) for i < 96.
 */
static void mmq_quantize_row(const float *v, int64_t kpad, int layout, int64_t m, int64_t row, uint8_t *plane) {
    const int g = layout == ORACLE_MMQ_D2S6 ? 64 : 32;
    for (int64_t b = 0; b < kpad / 128; ++b) {
        uint8_t *blk = plane + ((size_t)b * (size_t)m + (size_t)row) * MMQ_BLOCK_BYTES;
        int8_t *qs = (int8_t *)(blk + 16);
        for (int gi = 0; gi < 128 / g; ++gi) {
            const float *vg = v + b * 128 + gi * g;
            float amax = 0.0f;
            for (int i = 0; i < g; ++i) amax = fmaxf(amax, fabsf(vg[i]));
            const float d_inv = 127.0f / amax;
            const float d = 1.0f / d_inv;
            int8_t *q = qs + gi * g;
            for (int i = 0; i < g; ++i) q[i] = mmq_code(vg[i] * d_inv);
            if (layout == ORACLE_MMQ_D4) {
                memcpy(blk + 4 * gi, &d, 4);
            } else if (layout == ORACLE_MMQ_DS4) {
                int s = 0;
                for (int i = 0; i < 32; ++i) s += q[i];
                const uint16_t hd = oracle_float_to_half(d), hs = oracle_float_to_half(d * (float)s);
                memcpy(blk + 4 * gi, &hd, 2);
                memcpy(blk + 4 * gi + 2, &hs, 2);
            } else {
                const uint16_t hd = oracle_float_to_half(d);
                memcpy(blk + 2 * gi, &hd, 2);
                for (int h = 0; h < 4; ++h) {
                    const int slot = 4 * gi + h; /* 16-value group within the 128 */
                    if (slot >= 6) continue;
                    int s = 0;
                    for (int i = 0; i < 16; ++i) s += q[16 * h + i];
                    const uint16_t hs = oracle_float_to_half(d * (float)s);
                    memcpy(blk + 4 + 2 * slot, &hs, 2);
                }
            }
        }
    }
}

int oracle_prepare_mmq(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                       int layout, uint8_t *plane, float *inverse) {
    if (!x || !plane || !inverse || m < 1 || k <= 0 || k % 4 || stride_x < k || x_dtype < 0 || x_dtype > 2 ||
        layout < 0 || layout > 2)
        return -1;
    const int64_t kpad = oracle_mmq_blocks128(k) * 128;
    float *v = (float *)malloc((size_t)kpad * sizeof(float));
    if (!v) return -1;
    for (int64_t row = 0; row < m; ++row) {
        const float scale = mmq_row_scale(x, x_dtype, row * stride_x, k, inverse + row);
        for (int64_t i = 0; i < kpad; ++i) v[i] = i < k ? load_x(x, x_dtype, row * stride_x + i) * scale : 0.0f;
        mmq_quantize_row(v, kpad, layout, m, row, plane);
    }
    free(v);
    return 0;
}

static float h2f_bits(const uint8_t *p) { return rd_half(p); }
static double half_round(double v) { return (double)oracle_half_to_float(oracle_float_to_half((float)v)); }

/*
 * One weight block against its activation in a plane (row j of m), FP64 from exact
 * integer dots. GGML MMQ (upstream mmq.cuh @0c1e570, not vendored) on int8 tensor cores,
 * restated from its published tile loaders and dots:
 *   Q8_0  (D4)   d_w * d4 * sum q_w q                      load_tiles_q8_0, vec_dot_q8_0_q8_1_mma
 *   Q4_0  (DS4)  d_w * d8 * sum (nib - 8) q                 load_tiles_q4_0 (codes - 8), same dot on ds.x
 *   Q4_K  (DS4)  sum_i half(d sc_i) d8_i dot_i - half(dmin m_i) s8_i
 *                                                           load_tiles_q4_K (x_dm = dm*(sc, m) in half),
 *                                                           vec_dot_q8_1_q8_1_mma (s8 = stored ds.y)
 *   Q6_K  (D4)   d * sum_i d4_i (sc_2i dot_2i + sc_2i+1 dot_2i+1)   vec_dot_q6_K_q8_1_mma
 *   Q2_K  (D2S6) sum_g half(d sc_g) d64 dot_g - half(dmin m_g) S_g with S_g the stored half
 *                sum for the first 96 values of a 128-block and d64 * sum q for the last 32
 *                                                           load_tiles_q2_K, vec_dot_q2_K_q8_1_mma
 *   IQ3_S (D4)   sum_i d (1 + 2 sc_i) d4_i dot_i            load_tiles_iq3_s, vec_dot_q8_0_q8_1_mma
 * The value formulas are those of vecdotq.cuh (cited at block_dot); only the activation's
 * scales and sums and the half rounding of the K-quant weight scales differ.
 */
static double mmq_block_dot(int type, const uint8_t *b, const uint8_t *plane, int64_t m, int64_t j, int64_t e0) {
    /* activation values [e0, e0 + qk) of row j: 128-block e/128, position e%128 */
#define ABLK(e) (plane + ((size_t)((e) / 128) * (size_t)m + (size_t)j) * MMQ_BLOCK_BYTES)
#define ACODE(e) (((const int8_t *)(ABLK(e) + 16))[(e) % 128])
    switch (type) {
        case ORACLE_Q8_0: {
            float d4;
            memcpy(&d4, ABLK(e0) + 4 * ((e0 % 128) / 32), 4);
            int64_t s = 0;
            for (int e = 0; e < 32; ++e) s += (int64_t)(int8_t)b[2 + e] * ACODE(e0 + e);
            return (double)rd_half(b) * (double)d4 * (double)s;
        }
        case ORACLE_Q4_0: {
            const double d8 = h2f_bits(ABLK(e0) + 4 * ((e0 % 128) / 32));
            int64_t s = 0;
            for (int e = 0; e < 16; ++e)
                s += (int64_t)((b[2 + e] & 0x0f) - 8) * ACODE(e0 + e) + (int64_t)((b[2 + e] >> 4) - 8) * ACODE(e0 + e + 16);
            return (double)rd_half(b) * d8 * (double)s;
        }
        case ORACLE_Q4_K: {
            const float d = rd_half(b), dmin = rd_half(b + 2);
            uint8_t sc[8], mn[8];
            q4k_scale_min(b + 4, sc, mn);
            double acc = 0.0;
            for (int i = 0; i < 8; ++i) {
                const int64_t e = e0 + 32 * i;
                const uint8_t *hdr = ABLK(e) + 4 * ((e % 128) / 32);
                const double d8 = h2f_bits(hdr), s8 = h2f_bits(hdr + 2);
                int64_t dot = 0;
                for (int l = 0; l < 32; ++l) dot += (int64_t)q4k_code(b, 32 * i + l) * ACODE(e + l);
                acc += half_round((double)d * sc[i]) * d8 * (double)dot - half_round((double)dmin * mn[i]) * s8;
            }
            return acc;
        }
        case ORACLE_Q6_K: {
            const double d = rd_half(b + 208);
            double acc = 0.0;
            for (int g = 0; g < 16; ++g) {
                const int64_t e = e0 + 16 * g;
                float d4;
                memcpy(&d4, ABLK(e) + 4 * ((e % 128) / 32), 4);
                int64_t dot = 0;
                for (int l = 0; l < 16; ++l) dot += (int64_t)q6k_code(b, 16 * g + l) * ACODE(e + l);
                acc += (double)d4 * (double)(int8_t)b[192 + g] * (double)dot;
            }
            return d * acc;
        }
        case ORACLE_Q2_K: {
            const float d = rd_half(b + 80), dmin = rd_half(b + 82);
            double acc = 0.0;
            for (int g = 0; g < 16; ++g) {
                const int64_t e = e0 + 16 * g;
                const uint8_t *hdr = ABLK(e);
                const int slot = (int)((e % 128) / 16);
                const double d64 = h2f_bits(hdr + 2 * (slot / 4));
                int64_t dot = 0, qsum = 0;
                for (int l = 0; l < 16; ++l) {
                    dot += (int64_t)q2k_code(b, 16 * g + l) * ACODE(e + l);
                    qsum += ACODE(e + l);
                }
                const double s = slot < 6 ? (double)h2f_bits(hdr + 4 + 2 * slot) : d64 * (double)qsum;
                acc += half_round((double)d * (b[g] & 0x0f)) * d64 * (double)dot - half_round((double)dmin * (b[g] >> 4)) * s;
            }
            return acc;
        }
        case ORACLE_IQ3_S: {
            const double d = rd_half(b);
            double acc = 0.0;
            for (int g = 0; g < 8; ++g) {
                const int64_t e = e0 + 32 * g;
                float d4;
                memcpy(&d4, ABLK(e) + 4 * ((e % 128) / 32), 4);
                int64_t dot = 0;
                for (int t = 0; t < 32; ++t) dot += (int64_t)iq3s_value(b, 32 * g + t) * ACODE(e + t);
                acc += d * (double)(1 + 2 * iq3s_scale(b, g)) * (double)d4 * (double)dot;
            }
            return acc;
        }
        default: return 0.0;
    }
#undef ACODE
#undef ABLK
}

int oracle_mul_mat_mmq(int type, const uint8_t *weight, int64_t n, int64_t k, int64_t m,
                       const uint8_t *plane, const float *inverse, double *out, int threads) {
    if (!mm_args_ok(type, n, k, m, weight, plane) || !inverse || !out || oracle_mmq_layout(type) < 0) return -1;
    const int qk = oracle_block_elems(type), bb = oracle_block_bytes(type);
    const int64_t row_bytes = (k / qk) * bb;
    (void)threads;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t j = 0; j < m; ++j) {
            double acc = 0.0;
            for (int64_t blk = 0; blk < k / qk; ++blk)
                acc += mmq_block_dot(type, weight + r * row_bytes + blk * bb, plane, m, j, blk * qk);
            out[j * n + r] = (double)inverse[j] * acc;
        }
    }
    return 0;
}

const char *oracle_build_info(void) {
#ifdef _OPENMP
    return "kai_oracle C99 restatement, OpenMP";
#else
    return "kai_oracle C99 restatement, serial";
#endif
}
