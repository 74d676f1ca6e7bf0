/*
 * mcpm_oracle.c -- CPU oracle for the MiniCPM5 batch-1 decode path.
 * TEST INFRASTRUCTURE ONLY (see mcpm_oracle.h).  Built with -ffp-contract=off:
 * every multiply-add that is fused is written as fmaf().
 */
#include "mcpm_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ formats */

/* IEEE binary16 -> binary32 (include/ops.h:14-31), subnormals normalised. */
float or_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = -1;
            do { mant <<= 1; e++; } while (!(mant & 0x400u));
            bits = sign | ((uint32_t)(112 - e) << 23) | ((mant & 0x3ffu) << 13);
        }
    } else {
        bits = sign | ((uint32_t)(exp + 112) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* 6-bit scale/min unpack of a Q4_K block (include/ops.h:77-97). */
void or_q4k_scales_mins(const uint8_t *q, uint8_t *sc, uint8_t *mn) {
    for (int j = 0; j < 4; ++j) {
        sc[j] = q[j] & 63;
        mn[j] = q[j + 4] & 63;
    }
    for (int j = 4; j < 8; ++j) {
        sc[j] = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        mn[j] = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/*
 * exp(x) for fp32, from the mathematics: x = k*ln2 + r with k = nearest
 * integer to x/ln2 and r reduced by a two-part (Cody-Waite) ln2; exp(r) by its
 * Taylor series to degree 7 in Horner form (|r| <= 0.3466 gives a truncation
 * error below 8e-9 relative); the result scaled by 2^k.  The HIP kernels use
 * the same operation sequence, so both sides round identically.  Stands in for
 * std::exp in ops.cpp:740 (SiLU) and ops.cpp:601 (softmax).
 */
float or_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.972084045410156f) return 0.0f;
    const float inv_ln2 = 1.44269502162933349609375f;
    const float ln2_hi = 0.693145751953125f;
    const float ln2_lo = 1.428606765330187045e-06f;
    float k = rintf(x * inv_ln2);
    float r = fmaf(-k, ln2_hi, x);
    r = fmaf(-k, ln2_lo, r);
    float p = 1.98412698412698412526e-4f;      /* 1/5040 */
    p = fmaf(p, r, 1.38888888888888894189e-3f); /* 1/720 */
    p = fmaf(p, r, 8.33333333333333321769e-3f); /* 1/120 */
    p = fmaf(p, r, 4.16666666666666643537e-2f); /* 1/24 */
    p = fmaf(p, r, 1.66666666666666657415e-1f); /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

/* ------------------------------------------------------------------- Q8_K */

/*
 * quantize_row_q8_K_avx2 (ops_avx2.cpp:85-144) and the quantizing halves of
 * rmsnorm_and_quantize_q8k / swiglu_and_quantize_q8k (ops.cpp:704-722,746-764):
 * amax = max|x|; amax == 0 -> zero block; d = amax/127; v = x*(127/amax);
 * q = clamp(round(v), -127, 127); bsums[g] = sum of qs[16g..16g+15].
 */
static void quantize_block(const float *x, or_block_q8_K *dst, int ties_away) {
    float amax = 0.0f;
    for (int i = 0; i < OR_QK_K; ++i) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    if (amax == 0.0f) {
        memset(dst, 0, sizeof(*dst));
        return;
    }
    /* The source reads amax / 127.0f; the reference's -ffast-math build
     * (-freciprocal-math) evaluates it as amax * (1/127.0f).  Pinned against
     * the compiled reference in tests/test_oracle.py (test_quantize_golden,
     * test_quantize_row_q8k). */
    dst->d = amax * (1.0f / 127.0f);
    const float mul = 127.0f / amax;
    for (int i = 0; i < OR_QK_K; ++i) {
        float v = x[i] * mul;
        float r = ties_away ? roundf(v) : rintf(v);
        if (r > 127.0f) r = 127.0f;
        if (r < -127.0f) r = -127.0f;
        dst->qs[i] = (int8_t)r;
    }
    for (int g = 0; g < 16; ++g) {
        int s = 0;
        for (int i = 0; i < 16; ++i) s += dst->qs[16 * g + i];
        dst->bsums[g] = (int16_t)s;
    }
}

void or_quantize_row_q8_K(const float *x, int n, or_block_q8_K *y, int ties_away) {
    for (int b = 0; b < n / OR_QK_K; ++b) quantize_block(x + (size_t)b * OR_QK_K, y + b, ties_away);
}

/* ------------------------------------------------------------- dequantize */

static void dequant_q4_K_block(const or_block_q4_K *b, float *out) {
    uint8_t sc[8], mn[8];
    or_q4k_scales_mins(b->scales, sc, mn);
    const float d = or_fp16_to_fp32(b->d), dmin = or_fp16_to_fp32(b->dmin);
    for (int c = 0; c < 4; ++c) {
        /* ops.cpp:655-664: w = (d*sc)*q - dmin*mn; both products are exact. */
        const float d1 = d * (float)sc[2 * c], m1 = dmin * (float)mn[2 * c];
        const float d2 = d * (float)sc[2 * c + 1], m2 = dmin * (float)mn[2 * c + 1];
        for (int l = 0; l < 32; ++l) {
            const uint8_t q = b->qs[32 * c + l];
            out[64 * c + l] = d1 * (float)(q & 0x0f) - m1;
            out[64 * c + 32 + l] = d2 * (float)(q >> 4) - m2;
        }
    }
}

static int q6_code(const or_block_q6_K *b, int e) {
    const int h = e / 128, r = e % 128, g = r / 32, l = r % 32;
    const uint8_t qh = b->qh[32 * h + l];
    const uint8_t ql = b->ql[64 * h + 32 * (g & 1) + l];
    const int lo = (g < 2) ? (ql & 0x0f) : (ql >> 4);
    return lo | (((qh >> (2 * g)) & 3) << 4);
}

static void dequant_q6_K_block(const or_block_q6_K *b, float *out) {
    const float d = or_fp16_to_fp32(b->d);
    for (int e = 0; e < OR_QK_K; ++e) {
        /* ops.cpp:194-228: (d*sc)*(q-32). */
        out[e] = (d * (float)b->scales[e / 16]) * (float)(q6_code(b, e) - 32);
    }
}

void or_dequant_row(int type, const void *blocks, int n, float *out) {
    if (type == OR_F32) {
        memcpy(out, blocks, (size_t)n * 4);
    } else if (type == OR_Q8_0) {
        const or_block_q8_0 *b = (const or_block_q8_0 *)blocks;
        for (int i = 0; i < n / OR_QK8_0; ++i) {
            const float d = or_fp16_to_fp32(b[i].d);
            for (int j = 0; j < OR_QK8_0; ++j) out[OR_QK8_0 * i + j] = d * (float)b[i].qs[j];
        }
    } else if (type == OR_Q4_K) {
        const or_block_q4_K *b = (const or_block_q4_K *)blocks;
        for (int i = 0; i < n / OR_QK_K; ++i) dequant_q4_K_block(b + i, out + OR_QK_K * i);
    } else if (type == OR_Q6_K) {
        const or_block_q6_K *b = (const or_block_q6_K *)blocks;
        for (int i = 0; i < n / OR_QK_K; ++i) dequant_q6_K_block(b + i, out + OR_QK_K * i);
    }
}

/* -------------------------------------------------------- Q4_K/Q6_K dots */

/*
 * Integer lane m (0..7) of dot_row_q4_K_q8_K_avx2 (ops_avx2.cpp:161-181): the
 * maddubs/madd pair folds bytes 4m..4m+3 of each 32-byte chunk, so
 *   isum[m] = sum_j sc[2j]*sum_{l=4m}^{4m+3} lo(qs[32j+l])*x[64j+l]
 *                + sc[2j+1]*sum_l hi(qs[32j+l])*x[64j+32+l]
 * minsum = sum_g mn[g]*(bsums[2g]+bsums[2g+1])   (ops_avx2.cpp:187-191)
 */
void or_q4k_block_lanes(const or_block_q4_K *w, const or_block_q8_K *a, int32_t isum[8], int32_t *minsum) {
    uint8_t sc[8], mn[8];
    or_q4k_scales_mins(w->scales, sc, mn);
    /* Integer sums are exact, so they are formed per byte column l and folded
     * into lane l/4 afterwards. */
    int32_t col[32] = {0};
    for (int j = 0; j < 4; ++j) {
        const int32_t s_lo = sc[2 * j], s_hi = sc[2 * j + 1];
        for (int l = 0; l < 32; ++l) {
            const int32_t q = w->qs[32 * j + l];
            col[l] += s_lo * (q & 0x0f) * a->qs[64 * j + l] + s_hi * (q >> 4) * a->qs[64 * j + 32 + l];
        }
    }
    for (int m = 0; m < 8; ++m) isum[m] = col[4 * m] + col[4 * m + 1] + col[4 * m + 2] + col[4 * m + 3];
    int32_t ms = 0;
    for (int g = 0; g < 8; ++g) ms += (int32_t)mn[g] * ((int32_t)a->bsums[2 * g] + (int32_t)a->bsums[2 * g + 1]);
    *minsum = ms;
}

/*
 * Integer lane m of dot_row_q6_K_q8_K_avx2 (ops_avx2.cpp:224-270): elements
 * 128h+32g+l with l in [4m,4m+4), scale index 8h+2g+(l>=16), codes kept in
 * [0,63]; then minus 32*(bsums[2m]*sc[2m] + bsums[2m+1]*sc[2m+1]).
 */
void or_q6k_block_lanes(const or_block_q6_K *w, const or_block_q8_K *a, int32_t isum[8]) {
    int32_t col[32] = {0};
    for (int h = 0; h < 2; ++h) {
        const uint8_t *ql = w->ql + 64 * h, *qh = w->qh + 32 * h;
        const int8_t *x = a->qs + 128 * h;
        for (int l = 0; l < 32; ++l) {
            const int32_t H = qh[l], A0 = ql[l], A1 = ql[32 + l];
            const int hi = l >= 16;
            const int32_t q0 = (A0 & 15) | ((H & 3) << 4), q1 = (A1 & 15) | (((H >> 2) & 3) << 4);
            const int32_t q2 = (A0 >> 4) | (((H >> 4) & 3) << 4), q3 = (A1 >> 4) | (((H >> 6) & 3) << 4);
            col[l] += w->scales[8 * h + 0 + hi] * q0 * x[l] + w->scales[8 * h + 2 + hi] * q1 * x[32 + l] +
                      w->scales[8 * h + 4 + hi] * q2 * x[64 + l] + w->scales[8 * h + 6 + hi] * q3 * x[96 + l];
        }
    }
    for (int m = 0; m < 8; ++m) {
        const int32_t off = (int32_t)a->bsums[2 * m] * w->scales[2 * m] +
                            (int32_t)a->bsums[2 * m + 1] * w->scales[2 * m + 1];
        isum[m] = col[4 * m] + col[4 * m + 1] + col[4 * m + 2] + col[4 * m + 3] - 32 * off;
    }
}

/* hsum_f32_8 (ops_avx2.cpp:43-48): ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). */
static float hsum8(const float a[8]) {
    const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s2) + (s1 + s3);
}

/*
 * dot_row_q4_K_q8_K_avx2 float path (ops_avx2.cpp:183-195): per block,
 * acc[m] = fma(d_x*d_w, float(isum[m]), acc[m]); acc_min = fma(-(d_x*dmin_w),
 * float(minsum), acc_min) (the compiled reference contracts this line);
 * result = hsum8(acc) + acc_min.
 */
float or_dot_q4_K_q8_K(const or_block_q4_K *w, const or_block_q8_K *a, int nb) {
    float acc[8] = {0};
    float acc_min = 0.0f;
    for (int b = 0; b < nb; ++b) {
        int32_t isum[8], minsum;
        or_q4k_block_lanes(w + b, a + b, isum, &minsum);
        const float ds = a[b].d * or_fp16_to_fp32(w[b].d);
        for (int m = 0; m < 8; ++m) acc[m] = fmaf(ds, (float)isum[m], acc[m]);
        const float dm = a[b].d * or_fp16_to_fp32(w[b].dmin);
        acc_min = fmaf(-dm, (float)minsum, acc_min);
    }
    return hsum8(acc) + acc_min;
}

/* dot_row_q6_K_q8_K_avx2 float path (ops_avx2.cpp:270-275). */
float or_dot_q6_K_q8_K(const or_block_q6_K *w, const or_block_q8_K *a, int nb) {
    float acc[8] = {0};
    for (int b = 0; b < nb; ++b) {
        int32_t isum[8];
        or_q6k_block_lanes(w + b, a + b, isum);
        const float ds = a[b].d * or_fp16_to_fp32(w[b].d);
        for (int m = 0; m < 8; ++m) acc[m] = fmaf(ds, (float)isum[m], acc[m]);
    }
    return hsum8(acc);
}

/* gemv_q4_K_q8_K_avx2 / gemv_q6_K_q8_K_avx2 (ops_avx2.cpp:278-298). */
void or_gemv_q4_K_q8_K(const void *w, const or_block_q8_K *xq, float *out, int rows, int cols) {
    const or_block_q4_K *bw = (const or_block_q4_K *)w;
    const int nb = cols / OR_QK_K;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) out[r] = or_dot_q4_K_q8_K(bw + (size_t)r * nb, xq, nb);
}

void or_gemv_q6_K_q8_K(const void *w, const or_block_q8_K *xq, float *out, int rows, int cols) {
    const or_block_q6_K *bw = (const or_block_q6_K *)w;
    const int nb = cols / OR_QK_K;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) out[r] = or_dot_q6_K_q8_K(bw + (size_t)r * nb, xq, nb);
}

/* gemv_qkv_q4_K_q8_K_avx2 / gemv_qkv_q4_q4_q6_q8_K_avx2 (ops_avx2.cpp:320-374):
 * q and k rows are Q4_K, v rows follow v_type. */
void or_gemv_qkv_q8_K(const void *wq, const void *wk, const void *wv, int v_type, const or_block_q8_K *xq,
                      float *q, float *k, float *v, int q_rows, int kv_rows, int cols) {
    or_gemv_q4_K_q8_K(wq, xq, q, q_rows, cols);
    or_gemv_q4_K_q8_K(wk, xq, k, kv_rows, cols);
    if (v_type == OR_Q6_K) or_gemv_q6_K_q8_K(wv, xq, v, kv_rows, cols);
    else or_gemv_q4_K_q8_K(wv, xq, v, kv_rows, cols);
}

/* gemv_gate_up_q4_K_q8_K_avx2 (ops_avx2.cpp:378-460): two independent row dots. */
void or_gemv_gate_up_q4_K_q8_K(const void *wg, const void *wu, const or_block_q8_K *xq, float *gate,
                               float *up, int rows, int cols) {
    or_gemv_q4_K_q8_K(wg, xq, gate, rows, cols);
    or_gemv_q4_K_q8_K(wu, xq, up, rows, cols);
}

/*
 * gemv_f32 (ops.cpp:32-43).  Order: 64 strided partial sums
 * p[t] = sum over c = t, t+64, ... of w*x (multiply, then add), then the
 * 64-slot pairwise tree (p[t] += p[t+s] for s = 32..1).
 */
static float tree_sum(float *p, int n) {
    for (int s = n / 2; s >= 1; s /= 2)
        for (int t = 0; t < s; ++t) p[t] = p[t] + p[t + s];
    return p[0];
}

void or_gemv_f32(const float *w, const float *x, float *out, int rows, int cols) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        float p[64];
        for (int t = 0; t < 64; ++t) {
            float s = 0.0f;
            for (int c = t; c < cols; c += 64) s = s + w[(size_t)r * cols + c] * x[c];
            p[t] = s;
        }
        out[r] = tree_sum(p, 64);
    }
}

/* gemv_q8_0 (ops.cpp:58-79): per block s = sum_i float(qs_i)*x_i (i ascending,
 * multiply then add); row = row + s*d (blocks ascending). */
void or_gemv_q8_0(const void *w, const float *x, float *out, int rows, int cols) {
    const or_block_q8_0 *b = (const or_block_q8_0 *)w;
    const int nb = cols / OR_QK8_0;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        float row = 0.0f;
        for (int i = 0; i < nb; ++i) {
            const or_block_q8_0 *blk = b + (size_t)r * nb + i;
            float s = 0.0f;
            for (int j = 0; j < OR_QK8_0; ++j) s = s + (float)blk->qs[j] * x[OR_QK8_0 * i + j];
            row = row + s * or_fp16_to_fp32(blk->d);
        }
        out[r] = row;
    }
}

/* gemv_q4_K_scalar / gemv_q6_K_scalar (ops.cpp:95-147, 171-238): fp32
 * activations, no Q8_K (non-AVX2 builds).  Accumulators as in the source
 * (two for Q4_K, four for Q6_K), multiply then add. */
void or_gemv_q4_K_f32act(const void *w, const float *x, float *out, int rows, int cols) {
    const or_block_q4_K *bw = (const or_block_q4_K *)w;
    const int nb = cols / OR_QK_K;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        float s1 = 0.0f, s2 = 0.0f;
        for (int b = 0; b < nb; ++b) {
            const or_block_q4_K *blk = bw + (size_t)r * nb + b;
            uint8_t sc[8], mn[8];
            or_q4k_scales_mins(blk->scales, sc, mn);
            const float d = or_fp16_to_fp32(blk->d), dmin = or_fp16_to_fp32(blk->dmin);
            for (int c = 0; c < 4; ++c) {
                const float d1 = d * (float)sc[2 * c], m1 = dmin * (float)mn[2 * c];
                const float d2 = d * (float)sc[2 * c + 1], m2 = dmin * (float)mn[2 * c + 1];
                for (int l = 0; l < 32; ++l) {
                    const uint8_t q = blk->qs[32 * c + l];
                    const float w1 = d1 * (float)(q & 0x0f) - m1;
                    const float w2 = d2 * (float)(q >> 4) - m2;
                    s1 = s1 + w1 * x[b * OR_QK_K + 64 * c + l];
                    s2 = s2 + w2 * x[b * OR_QK_K + 64 * c + 32 + l];
                }
            }
        }
        out[r] = s1 + s2;
    }
}

void or_gemv_q6_K_f32act(const void *w, const float *x, float *out, int rows, int cols) {
    const or_block_q6_K *bw = (const or_block_q6_K *)w;
    const int nb = cols / OR_QK_K;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int b = 0; b < nb; ++b) {
            const or_block_q6_K *blk = bw + (size_t)r * nb + b;
            const float d = or_fp16_to_fp32(blk->d);
            for (int h = 0; h < 2; ++h) {
                for (int l = 0; l < 32; ++l) {
                    for (int g = 0; g < 4; ++g) {
                        const int e = 128 * h + 32 * g + l;
                        /* ops.cpp:194-228: (d*sc)*q then times x. */
                        const float sg = d * (float)blk->scales[8 * h + 2 * g + (l >= 16)];
                        s[g] = s[g] + sg * (float)(q6_code(blk, e) - 32) * x[b * OR_QK_K + e];
                    }
                }
            }
        }
        out[r] = s[0] + s[1] + s[2] + s[3];
    }
}

/* ------------------------------------------------------------- dispatchers */

int or_matmul(int type, const void *w, const float *x, float *out, int rows, int cols) {
    if (type == OR_F32) {
        or_gemv_f32((const float *)w, x, out, rows, cols);
    } else if (type == OR_Q8_0) {
        or_gemv_q8_0(w, x, out, rows, cols);
    } else if (type == OR_Q4_K || type == OR_Q6_K) {
        /* gemv_q4_K_avx2 / gemv_q6_K_avx2 (ops_avx2.cpp:462-476): quantize x
         * with ties-to-even, then the Q8_K GEMV. */
        or_block_q8_K *xq = (or_block_q8_K *)malloc(sizeof(or_block_q8_K) * (size_t)(cols / OR_QK_K));
        or_quantize_row_q8_K(x, cols, xq, 0);
        if (type == OR_Q4_K) or_gemv_q4_K_q8_K(w, xq, out, rows, cols);
        else or_gemv_q6_K_q8_K(w, xq, out, rows, cols);
        free(xq);
    } else {
        for (int r = 0; r < rows; ++r) out[r] = 0.001f;
        return -1;
    }
    return 0;
}

int or_matmul_q8k(int type, const void *w, const or_block_q8_K *xq, float *out, int rows, int cols) {
    if (type == OR_Q4_K) or_gemv_q4_K_q8_K(w, xq, out, rows, cols);
    else if (type == OR_Q6_K) or_gemv_q6_K_q8_K(w, xq, out, rows, cols);
    else {
        for (int r = 0; r < rows; ++r) out[r] = 0.0f;
        return -1;
    }
    return 0;
}

/* ------------------------------------------------------ norms, activations */

/*
 * rms = 1/sqrt(sum(x^2)/dim + eps) (ops.cpp:470-475, 681-686).  Order of the
 * sum of squares: 256 strided partials p[t] = sum over i = t, t+256, ... of
 * x_i*x_i (multiply, then add), then the 256-slot pairwise tree.
 */
float or_rms_scale(const float *x, int dim, float eps) {
    float p[256];
    for (int t = 0; t < 256; ++t) {
        float s = 0.0f;
        for (int i = t; i < dim; i += 256) s = s + x[i] * x[i];
        p[t] = s;
    }
    const float sum = tree_sum(p, 256);
    return 1.0f / sqrtf(sum / (float)dim + eps);
}

/* rmsnorm (ops.cpp:468-481): out = (x*rms)*w. */
void or_rmsnorm(float *out, const float *x, const float *w, int dim, float eps) {
    const float rms = or_rms_scale(x, dim, eps);
    for (int i = 0; i < dim; ++i) out[i] = x[i] * rms * w[i];
}

/* rmsnorm_and_quantize_q8k (ops.cpp:676-723): (x*rms)*w, then Q8_K, lround. */
void or_rmsnorm_and_quantize_q8k(or_block_q8_K *out, const float *x, const float *w, int dim, float eps) {
    float *tmp = (float *)malloc(sizeof(float) * (size_t)dim);
    or_rmsnorm(tmp, x, w, dim, eps);
    or_quantize_row_q8_K(tmp, dim, out, 1);
    free(tmp);
}

/* SwiGLU (ops.cpp:738-742): g/(1+exp(-g)) * u. */
void or_swiglu(float *h, const float *gate, const float *up, int dim) {
    for (int i = 0; i < dim; ++i) {
        const float g = gate[i];
        const float silu = g / (1.0f + or_expf(-g));
        h[i] = silu * up[i];
    }
}

void or_swiglu_and_quantize_q8k(or_block_q8_K *out, const float *gate, const float *up, int dim) {
    float *tmp = (float *)malloc(sizeof(float) * (size_t)dim);
    or_swiglu(tmp, gate, up, dim);
    or_quantize_row_q8_K(tmp, dim - dim % OR_QK_K, out, 1);
    free(tmp);
}

/* apply_rope over all heads (ops.cpp:502-516; loop model.cpp:187-192):
 * theta = 1/powf(base, i/hd), a = pos*theta, adjacent pairs rotated. */
void or_apply_rope(float *vec, int pos, int n_heads, int head_dim, float base) {
    for (int h = 0; h < n_heads; ++h) {
        for (int i = 0; i < head_dim; i += 2) {
            const int idx = h * head_dim + i;
            const float theta = 1.0f / powf(base, (float)i / (float)head_dim);
            const float a = (float)pos * theta;
            const float c = cosf(a), s = sinf(a);
            const float v0 = vec[idx], v1 = vec[idx + 1];
            vec[idx] = v0 * c - v1 * s;
            vec[idx + 1] = v0 * s + v1 * c;
        }
    }
}

/*
 * execute_attention (ops.cpp:537-628): append k,v at pos; per query head h
 * (kv head h / (n_heads/n_kv_heads)) softmax(q.k_t/sqrt(hd)) over t = 0..pos,
 * output sum_t p_t v_t.  The reference's two-pass softmax is evaluated here as
 * split softmax over chunks of OR_ATTN_CHUNK positions:
 *   s_t  = (sum_i q_i*k_ti, a sequential fmaf chain over i from 0) * scale
 *   per chunk c:  m_c = max(-1e9, s_t);  e_t = exp(s_t - m_c);
 *                 z_c = 64-slot pairwise tree of e_t (absent slots 0);
 *                 o_c[i] = sequential fmaf chain over t of e_t*v_ti from 0
 *   m = max_c m_c; f_c = exp(m_c - m), chunks ascending:
 *                 Z = fmaf(z_c, f_c, Z); O[i] = fmaf(o_c[i], f_c, O[i])
 *   out[i] = O[i] / Z
 */
int or_attention(float *out, const float *q, const float *k_cur, const float *v_cur, float *k_cache,
                 float *v_cache, int pos, int max_seq_len, int n_heads, int n_kv_heads, int head_dim) {
    if (pos >= max_seq_len) return -1;
    const int kvd = n_kv_heads * head_dim;
    memcpy(k_cache + (size_t)pos * kvd, k_cur, sizeof(float) * (size_t)kvd);
    memcpy(v_cache + (size_t)pos * kvd, v_cur, sizeof(float) * (size_t)kvd);
    const float scale = 1.0f / sqrtf((float)head_dim);
    const int group = n_heads / n_kv_heads;
    const int T = pos + 1;
    const int nch = (T + OR_ATTN_CHUNK - 1) / OR_ATTN_CHUNK;
    float *mc = (float *)malloc(sizeof(float) * (size_t)nch);
    float *zc = (float *)malloc(sizeof(float) * (size_t)nch);
    float *oc = (float *)malloc(sizeof(float) * (size_t)nch * head_dim);
    for (int h = 0; h < n_heads; ++h) {
        const int kvh = h / group;
        const float *qh = q + (size_t)h * head_dim;
        for (int c = 0; c < nch; ++c) {
            float s[OR_ATTN_CHUNK], e[OR_ATTN_CHUNK];
            const int t0 = c * OR_ATTN_CHUNK;
            float m = -1e9f;
            for (int j = 0; j < OR_ATTN_CHUNK; ++j) {
                const int t = t0 + j;
                if (t >= T) { s[j] = 0.0f; continue; }
                const float *kt = k_cache + (size_t)t * kvd + (size_t)kvh * head_dim;
                float dot = 0.0f;
                for (int i = 0; i < head_dim; ++i) dot = fmaf(qh[i], kt[i], dot);
                s[j] = dot * scale;
                if (s[j] > m) m = s[j];
            }
            for (int j = 0; j < OR_ATTN_CHUNK; ++j) e[j] = (t0 + j < T) ? or_expf(s[j] - m) : 0.0f;
            float tmp[OR_ATTN_CHUNK];
            memcpy(tmp, e, sizeof(tmp));
            mc[c] = m;
            zc[c] = tree_sum(tmp, OR_ATTN_CHUNK);
            for (int i = 0; i < head_dim; ++i) {
                float o = 0.0f;
                for (int j = 0; j < OR_ATTN_CHUNK && t0 + j < T; ++j) {
                    const float *vt = v_cache + (size_t)(t0 + j) * kvd + (size_t)kvh * head_dim;
                    o = fmaf(e[j], vt[i], o);
                }
                oc[(size_t)c * head_dim + i] = o;
            }
        }
        float m = mc[0];
        for (int c = 1; c < nch; ++c) if (mc[c] > m) m = mc[c];
        float Z = 0.0f;
        for (int c = 0; c < nch; ++c) Z = fmaf(zc[c], or_expf(mc[c] - m), Z);
        for (int i = 0; i < head_dim; ++i) {
            float O = 0.0f;
            for (int c = 0; c < nch; ++c) O = fmaf(oc[(size_t)c * head_dim + i], or_expf(mc[c] - m), O);
            out[(size_t)h * head_dim + i] = O / Z;
        }
    }
    free(mc);
    free(zc);
    free(oc);
    return 0;
}

/* get_embedding (ops.cpp:631-673), extended to Q6_K rows (tied embedding). */
int or_get_embedding(float *out, int type, const void *embd, int dim, int token) {
    if (type == OR_Q4_K) {
        or_dequant_row(type, (const or_block_q4_K *)embd + (size_t)token * (dim / OR_QK_K), dim, out);
    } else if (type == OR_Q6_K) {
        or_dequant_row(type, (const or_block_q6_K *)embd + (size_t)token * (dim / OR_QK_K), dim, out);
    } else {
        memset(out, 0, sizeof(float) * (size_t)dim);
        return -1;
    }
    return 0;
}

/* Greedy decoding: first index of the maximum. */
void or_set_threads(int n) {
    omp_set_dynamic(0);
    omp_set_num_threads(n);
}

int or_argmax(const float *x, int n) {
    int best = 0;
    for (int i = 1; i < n; ++i) if (x[i] > x[best]) best = i;
    return best;
}

/* ------------------------------------------------------------------ model */

struct or_model {
    or_config c;
    const void *embd;
    int embd_type;
    const float *out_norm;
    const void *out_w;
    int out_type;
    or_layer *layers;
    int max_seq;
    float **kc, **vc;
    float *x, *xn, *q, *k, *v, *att, *o, *gate, *up, *dn;
    or_block_q8_K *xq, *hq;
};

or_model *or_model_create(const or_config *cfg, const void *embd, int embd_type, const float *out_norm,
                          const void *out_w, int out_type, const or_layer *layers) {
    or_model *m = (or_model *)calloc(1, sizeof(or_model));
    m->c = *cfg;
    m->embd = embd;
    m->embd_type = embd_type;
    m->out_norm = out_norm;
    m->out_w = out_w;
    m->out_type = out_type;
    m->layers = (or_layer *)malloc(sizeof(or_layer) * (size_t)cfg->n_layers);
    memcpy(m->layers, layers, sizeof(or_layer) * (size_t)cfg->n_layers);
    const int qd = cfg->n_heads * cfg->head_dim, kvd = cfg->n_kv_heads * cfg->head_dim;
    m->x = (float *)calloc((size_t)cfg->dim, 4);
    m->xn = (float *)calloc((size_t)cfg->dim, 4);
    m->q = (float *)calloc((size_t)qd, 4);
    m->k = (float *)calloc((size_t)kvd, 4);
    m->v = (float *)calloc((size_t)kvd, 4);
    m->att = (float *)calloc((size_t)qd, 4);
    m->o = (float *)calloc((size_t)cfg->dim, 4);
    m->gate = (float *)calloc((size_t)cfg->ffn_pad, 4);
    m->up = (float *)calloc((size_t)cfg->ffn_pad, 4);
    m->dn = (float *)calloc((size_t)cfg->dim, 4);
    m->xq = (or_block_q8_K *)calloc((size_t)(cfg->dim / OR_QK_K), sizeof(or_block_q8_K));
    m->hq = (or_block_q8_K *)calloc((size_t)(cfg->ffn_pad / OR_QK_K), sizeof(or_block_q8_K));
    return m;
}

int or_model_init_kv(or_model *m, int max_seq_len) {
    const size_t kvd = (size_t)m->c.n_kv_heads * m->c.head_dim;
    if (m->kc) {
        for (int l = 0; l < m->c.n_layers; ++l) { free(m->kc[l]); free(m->vc[l]); }
        free(m->kc);
        free(m->vc);
    }
    m->kc = (float **)calloc((size_t)m->c.n_layers, sizeof(float *));
    m->vc = (float **)calloc((size_t)m->c.n_layers, sizeof(float *));
    for (int l = 0; l < m->c.n_layers; ++l) {
        m->kc[l] = (float *)calloc((size_t)max_seq_len * kvd, 4);
        m->vc[l] = (float *)calloc((size_t)max_seq_len * kvd, 4);
        if (!m->kc[l] || !m->vc[l]) return -1;
    }
    m->max_seq = max_seq_len;
    return 0;
}

/* MiniCPM5Engine::forward (src/model.cpp:142-242) with explicit shapes. */
/* Every layer of one token (src/model.cpp:142-227); the hidden state is left
 * in m->x.  Returns 0, or -1 when pos is past the KV capacity. */
static int or_model_layers(or_model *m, int token, int pos) {
    const or_config *c = &m->c;
    const int qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
    or_get_embedding(m->x, m->embd_type, m->embd, c->dim, token);
    for (int l = 0; l < c->n_layers; ++l) {
        const or_layer *L = &m->layers[l];
        or_rmsnorm_and_quantize_q8k(m->xq, m->x, L->attn_norm, c->dim, c->eps);
        or_gemv_qkv_q8_K(L->wq, L->wk, L->wv, L->wv_type, m->xq, m->q, m->k, m->v, qd, kvd, c->dim);
        or_apply_rope(m->q, pos, c->n_heads, c->head_dim, c->rope_base);
        or_apply_rope(m->k, pos, c->n_kv_heads, c->head_dim, c->rope_base);
        if (or_attention(m->att, m->q, m->k, m->v, m->kc[l], m->vc[l], pos, m->max_seq, c->n_heads,
                         c->n_kv_heads, c->head_dim) != 0)
            return -1;
        or_matmul(L->wo_type, L->wo, m->att, m->o, c->dim, qd);
        for (int i = 0; i < c->dim; ++i) m->x[i] = m->x[i] + m->o[i];
        or_rmsnorm_and_quantize_q8k(m->xq, m->x, L->ffn_norm, c->dim, c->eps);
        or_gemv_gate_up_q4_K_q8_K(L->wg, L->wu, m->xq, m->gate, m->up, c->ffn, c->dim);
        or_swiglu_and_quantize_q8k(m->hq, m->gate, m->up, c->ffn_pad);
        or_matmul_q8k(L->wd_type, L->wd, m->hq, m->dn, c->dim, c->ffn_pad);
        for (int i = 0; i < c->dim; ++i) m->x[i] = m->x[i] + m->dn[i];
    }
    return 0;
}

/* A prompt token whose logits nobody reads: the layers (so its K and V rows
 * reach the cache) without the LM head. */
int or_model_forward_kv(or_model *m, int token, int pos) { return or_model_layers(m, token, pos); }

int or_model_forward(or_model *m, int token, int pos, float *logits) {
    const or_config *c = &m->c;
    if (or_model_layers(m, token, pos) != 0) return -1;
    or_rmsnorm(m->xn, m->x, m->out_norm, c->dim, c->eps);
    float *lg = logits ? logits : (float *)malloc(sizeof(float) * (size_t)c->vocab);
    or_matmul(m->out_type, m->out_w, m->xn, lg, c->vocab, c->dim);
    const int best = or_argmax(lg, c->vocab);
    if (!logits) free(lg);
    return best;
}

const float *or_model_hidden(const or_model *m) { return m->x; }

int or_model_read_kv(const or_model *m, int layer, int pos0, int n, float *k, float *v) {
    const size_t kvd = (size_t)m->c.n_kv_heads * (size_t)m->c.head_dim;
    if (!m->kc || layer < 0 || layer >= m->c.n_layers || pos0 < 0 || n < 0 || pos0 + n > m->max_seq) return -1;
    if (k) memcpy(k, m->kc[layer] + (size_t)pos0 * kvd, (size_t)n * kvd * sizeof(float));
    if (v) memcpy(v, m->vc[layer] + (size_t)pos0 * kvd, (size_t)n * kvd * sizeof(float));
    return 0;
}

void or_model_free(or_model *m) {
    if (!m) return;
    if (m->kc) {
        for (int l = 0; l < m->c.n_layers; ++l) { free(m->kc[l]); free(m->vc[l]); }
        free(m->kc);
        free(m->vc);
    }
    free(m->layers);
    free(m->x); free(m->xn); free(m->q); free(m->k); free(m->v); free(m->att); free(m->o);
    free(m->gate); free(m->up); free(m->dn); free(m->xq); free(m->hq);
    free(m);
}

/* ---------------------------------------------------------------- sampler */

void or_mt_seed(or_mt19937 *g, uint32_t seed) {
    g->mt[0] = seed;
    for (int i = 1; i < 624; ++i) g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + (uint32_t)i;
    g->idx = 624;
}

uint32_t or_mt_next(or_mt19937 *g) {
    if (g->idx >= 624) {
        for (int i = 0; i < 624; ++i) {
            const uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
            g->mt[i] = g->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        }
        g->idx = 0;
    }
    uint32_t y = g->mt[g->idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

/* std::uniform_real_distribution<float>(0,1) over std::mt19937 in libstdc++:
 * generate_canonical<float,24> = float(g()) / 2^32, clamped below 1. */
float or_mt_uniform01(or_mt19937 *g) {
    float r = (float)or_mt_next(g) / 4294967296.0f;
    if (r >= 1.0f) r = nextafterf(1.0f, 0.0f);
    return r;
}

typedef struct { float p; int id; } or_pi;

static int cmp_pi(const void *a, const void *b) {
    const or_pi *x = (const or_pi *)a, *y = (const or_pi *)b;
    if (x->p > y->p) return -1;
    if (x->p < y->p) return 1;
    return (x->id > y->id) - (x->id < y->id);
}

/* Sampler::sample (src/sampler.cpp:8-73) for a given uniform draw r.  Equal
 * probabilities are ordered by token id (std::sort leaves them unspecified). */
int or_sample(const float *logits, int n, float temperature, float top_p, float r) {
    const float inv_temp = (temperature > 0.0f) ? (1.0f / temperature) : 1.0f;
    const int apply_temp = (temperature != 1.0f && temperature > 0.0f);
    float maxl = -1e9f;
    for (int i = 0; i < n; ++i) {
        const float v = apply_temp ? logits[i] * inv_temp : logits[i];
        if (v > maxl) maxl = v;
    }
    or_pi *pr = (or_pi *)malloc(sizeof(or_pi) * (size_t)n);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float v = apply_temp ? logits[i] * inv_temp : logits[i];
        pr[i].p = or_expf(v - maxl);
        pr[i].id = i;
        sum = sum + pr[i].p;
    }
    for (int i = 0; i < n; ++i) pr[i].p = pr[i].p / sum;
    int cnt = n;
    if (top_p > 0.0f && top_p < 1.0f) {
        qsort(pr, (size_t)n, sizeof(or_pi), cmp_pi);
        float cum = 0.0f;
        int last = 0;
        for (int i = 0; i < n; ++i) {
            cum = cum + pr[i].p;
            last = i;
            if (cum >= top_p) break;
        }
        cnt = last + 1;
        for (int i = 0; i < cnt; ++i) pr[i].p = pr[i].p / cum;
    }
    float cur = 0.0f;
    int out = pr[cnt - 1].id;
    for (int i = 0; i < cnt; ++i) {
        cur = cur + pr[i].p;
        if (r <= cur) { out = pr[i].id; break; }
    }
    free(pr);
    return out;
}

/* The device sampler's arithmetic (mcpm_sample_device and the engine's
 * sampled decode).  Sampler::sample (src/sampler.cpp:8-73) step for step --
 * temperature, softmax with the max subtracted, the (p desc, id asc) order
 * when 0 < top_p < 1, the top-p cut, the walk over the running sum -- with
 * every running sum taken in double over blocks of OR_SB positions: in order
 * within a block, the blocks in order, a position's running sum being the
 * sum of the blocks before it plus its in-block running sum.  The walk
 * compares r*C with the running sum of p (C = the running sum at the cut),
 * which is the reference's comparison of r with the running sum of p/cum
 * without the per-term division.  Deviation from the reference: rounding
 * only (its sums run sequentially in float, which a GPU cannot split).
 * Positions past the cut never enter a sum that decides anything. */
#define OR_SB 256

int or_sample_blocked(const float *logits, int n, float temperature, float top_p, float r) {
    const float inv_temp = (temperature > 0.0f) ? (1.0f / temperature) : 1.0f;
    const int apply_temp = (temperature != 1.0f && temperature > 0.0f);
    float maxl = -1e9f;
    for (int i = 0; i < n; ++i) {
        const float v = apply_temp ? logits[i] * inv_temp : logits[i];
        if (v > maxl) maxl = v;
    }
    or_pi *pr = (or_pi *)malloc(sizeof(or_pi) * (size_t)n);
    double total = 0.0, blk = 0.0;
    for (int i = 0; i < n; ++i) {
        const float v = apply_temp ? logits[i] * inv_temp : logits[i];
        pr[i].p = or_expf(v - maxl);
        pr[i].id = i;
        blk = blk + (double)pr[i].p;
        if (i % OR_SB == OR_SB - 1 || i == n - 1) {
            total = total + blk;
            blk = 0.0;
        }
    }
    const float sum = (float)total;
    for (int i = 0; i < n; ++i) pr[i].p = pr[i].p / sum;
    const int topp = (top_p > 0.0f && top_p < 1.0f);
    if (topp) qsort(pr, (size_t)n, sizeof(or_pi), cmp_pi);
    /* the cut: first k whose running sum, rounded to float, reaches top_p */
    int cnt = n;
    double off = 0.0, pre = 0.0, C = 0.0;
    for (int k = 0; k < n; ++k) {
        pre = pre + (double)pr[k].p;
        C = off + pre;
        if (topp && (float)C >= top_p) {
            cnt = k + 1;
            break;
        }
        if (k % OR_SB == OR_SB - 1) {
            off = off + pre;
            pre = 0.0;
        }
    }
    /* the walk: first k < cnt whose running sum reaches r*C */
    const double t = (double)r * C;
    int out = pr[cnt - 1].id;
    off = 0.0;
    pre = 0.0;
    for (int k = 0; k < cnt; ++k) {
        pre = pre + (double)pr[k].p;
        if (t <= off + pre) {
            out = pr[k].id;
            break;
        }
        if (k % OR_SB == OR_SB - 1) {
            off = off + pre;
            pre = 0.0;
        }
    }
    free(pr);
    return out;
}
