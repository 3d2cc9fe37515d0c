/*
 * TEST INFRASTRUCTURE ONLY -- the checker, never the product.
 *
 * A plain-C restatement of inference.rs's CPU QMatMul arithmetic for the GGUF
 * Q8_0 / Q4_K / Q6_K weight types and the Q8_0 / Q8_K activation blocks.  The
 * HIP library is compared against it; tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py are its only users.  Built with
 * -ffp-contract=off: the reference's llama.cpp-style quantizer (utils.rs:37-45,
 * `Quantizer::LlamaCpp`) rounds every product before the sum.
 *
 * Citations are file:line in the inference.rs repository.
 *
 * What pins each part (tests/test_oracle.py):
 *   f16 conversion       numpy's IEEE binary16 cast on every f16 bit pattern and random floats
 *   quantize_block32     the reference's own known-answer blocks (quantized/mod.rs:1650-1686)
 *   Q8_K quantizer       closed form on special blocks (zero, tied maxima, signs); bsums == sums of qs
 *   Q4_K / Q5_K / Q6_K   exact-grid known answers, float64 re-derivations of the candidate-scale searches, a
 *   weights              byte-identical second float32 reading in numpy, planted mistakes (tests/test_weight_quantizers.py)
 *   dequantize           closed forms against hand-built blocks
 *   vec_dot / matmul     float64 brute force over the dequantized operands; a planted-error check
 *   MoE                  brute force per route over oracle_matmul
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- f16 (IEEE binary16, RNE) */

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) { /* inf / nan: keep a quiet nan payload bit */
        if (man == 0) return sign | 0x7c00u;
        return (uint16_t)(sign | 0x7e00u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return sign | 0x7c00u; /* overflow to inf */
    if (e <= 0) {
        /* subnormal or zero in f16 */
        if (e < -10) return sign; /* rounds to zero */
        uint32_t m = man | 0x800000u;           /* implicit bit */
        uint32_t shift = (uint32_t)(14 - e);    /* 24-bit mantissa -> 10-bit subnormal */
        uint32_t half_bits = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (half_bits & 1u))) half_bits++;
        return (uint16_t)(sign | half_bits);
    }
    uint32_t half_bits = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half_bits & 1u))) half_bits++; /* may carry into exp: correct */
    return (uint16_t)(sign | half_bits);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    if (exp == 31) return bits_f32(sign | 0x7f800000u | (man << 13));
    return bits_f32(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

/* ---------------------------------------------------------------- type table */

/* the IQ4_NL / IQ4_XS value table (crates/inference-quant/src/gguf/raw.rs:13-15) */
const int8_t oracle_kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

size_t oracle_type_size(int type) {
    switch (type) {
    case OR_Q8_0: return sizeof(or_block_q8_0);
    case OR_Q4K: return sizeof(or_block_q4k);
    case OR_Q6K: return sizeof(or_block_q6k);
    case OR_Q8K: return sizeof(or_block_q8k);
    case OR_Q4_0: return sizeof(or_block_q4_0);
    case OR_Q5_0: return sizeof(or_block_q5_0);
    case OR_Q5K: return sizeof(or_block_q5k);
    case OR_IQ4XS: return sizeof(or_block_iq4xs);
    default: return 0;
    }
}

size_t oracle_block_size(int type) {
    switch (type) {
    case OR_Q8_0: case OR_Q4_0: case OR_Q5_0: return 32;
    case OR_Q4K: case OR_Q6K: case OR_Q8K: case OR_Q5K: case OR_IQ4XS: return 256;
    default: return 0;
    }
}

/* ---------------------------------------------------------------- planted mistakes
 * Built with -DORACLE_PLANT=n (tests/test_weight_quantizers.py only, into a temporary library), the weight quantizers
 * carry one deliberate mistake each, so the tests can show that their checks catch it:
 *   1 make_qkx2_quants fuses its multiply-adds (the ik_llama.cpp build's madd, not the LlamaCpp one)
 *   2 Q4_K searches from rmin -0.5 instead of -1
 *   3 Q4_K stores dmin = max_min / 64
 *   4 make_qx_quants tries candidate scales around nmax - 1
 *   5 Q6_K scales its sub-block scales by -127 / max_scale
 *   6 Q5_K searches 20 steps instead of 15
 *   7 make_qkx2_quants scores candidates by absolute error
 *   8 make_qkx2_quants refits a positive min as sum_xl / sum_l
 * The default build (ORACLE_PLANT undefined) is the restatement. */
#ifndef ORACLE_PLANT
#define ORACLE_PLANT 0
#endif

/* ---------------------------------------------------------------- rounding helpers (utils.rs) */

/* utils.rs:3-4, 32-35: add 1.5*2^23, read the low mantissa bits: round to nearest, ties to even */
static int32_t nearest_int(float v) {
    volatile float t = v + 12582912.0f;
    return (int32_t)(f32_bits(t) & 0x007fffffu) - 0x00400000;
}

/* utils.rs:70-73 with Quantizer::LlamaCpp: the product rounded before the magic add */
static int32_t nearest_int_mul(float a, float b) {
    volatile float p = a * b;
    return nearest_int(p);
}

static int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Rust's `f32 as i8`: saturating, NaN -> 0 */
static int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* Rust's `f32 as u8`: saturating, truncating toward zero, NaN -> 0 */
static uint8_t sat_u8(float v) {
    if (!(v > 0.0f)) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)v;
}

/* ---------------------------------------------------------------- Q8_0 (mod.rs:41-56, k_quants.rs:899-1000) */

float oracle_quantize_block32(const float *x, int8_t *qs) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i])); /* fold(0, max(|v|)) */
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int i = 0; i < 32; i++) qs[i] = sat_i8(roundf(x[i] * id)); /* round: half away from zero */
    return d;
}

void oracle_quantize_q8_0(const float *x, int64_t n, or_block_q8_0 *y) {
    for (int64_t b = 0; b < n / 32; b++) y[b].d = oracle_f32_to_f16(oracle_quantize_block32(x + 32 * b, y[b].qs));
}

/* ---------------------------------------------------------------- Q8_K (k_quants.rs:2721-2760) */

void oracle_quantize_q8k(const float *x, int64_t n, or_block_q8k *y) {
    for (int64_t b = 0; b < n / 256; b++) {
        const float *xs = x + 256 * b;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; j++) {
            if (amax < fabsf(xs[j])) { amax = fabsf(xs[j]); max = xs[j]; } /* first of the largest |x| */
        }
        if (amax == 0.0f) {
            y[b].d = 0.0f;
            memset(y[b].qs, 0, sizeof y[b].qs);
            memset(y[b].bsums, 0, sizeof y[b].bsums);
            continue;
        }
        float iscale = -127.0f / max;
        for (int j = 0; j < 256; j++) {
            /* clamp(-128, 127) then `as i8`: saturating, a NaN (clamp keeps it) becomes 0 */
            y[b].qs[j] = sat_i8(roundf(iscale * xs[j]));
        }
        for (int j = 0; j < 16; j++) {
            int32_t s = 0;
            for (int i = 0; i < 16; i++) s += y[b].qs[16 * j + i];
            y[b].bsums[j] = (int16_t)s;
        }
        y[b].d = 1.0f / iscale;
    }
}

/* ---------------------------------------------------------------- Q4_K weights */

/* utils.rs:119-129 */
static void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* utils.rs:268-361, make_qkx2_quants with Quantizer::LlamaCpp (every product rounded, -ffp-contract=off) and
 * k_quants.rs:245-250 Q4K_SEARCH {rmin -1, rdelta 0.1, nstep 20, mad false}; returns scale, *neg_min = -min */
static float make_qkx2_quants(int nmax, const float *x, const float *weights, float rmin, float rdelta, int nstep,
                              int use_mad, uint8_t *l, float *neg_min) {
    const int n = 32;
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; i++) {
        min = fminf(min, x[i]);
        max = fmaxf(max, x[i]);
        sum_w += weights[i];
        sum_x = weights[i] * x[i] + sum_x;
    }
    if (min > 0.0f) min = 0.0f;
    if (max == min) {
        memset(l, 0, (size_t)n);
        *neg_min = -min;
        return 0.0f;
    }
    if (ORACLE_PLANT == 7) use_mad = 1;
    float iscale = (float)nmax / (max - min);
    float scale = 1.0f / iscale;
    float best_error = 0.0f;
    for (int i = 0; i < n; i++) {
        int32_t li = clampi(nearest_int_mul(iscale, x[i] - min), 0, nmax);
        l[i] = (uint8_t)li;
        float diff = scale * (float)li + min - x[i];
        float e = use_mad ? fabsf(diff) : diff * diff;
        best_error = ORACLE_PLANT == 1 ? fmaf(weights[i], e, best_error) : weights[i] * e + best_error;
    }
    if (nstep == 0) { *neg_min = -min; return scale; }
    int32_t laux[32];
    for (int is = 0; is <= nstep; is++) {
        iscale = (rdelta * (float)is + rmin + (float)nmax) / (max - min);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        for (int i = 0; i < n; i++) {
            int32_t li = clampi(nearest_int_mul(iscale, x[i] - min), 0, nmax);
            laux[i] = li;
            float w = weights[i], lf = (float)li;
            float wl = w * lf;
            sum_l += wl;
            sum_l2 = ORACLE_PLANT == 1 ? fmaf(wl, lf, sum_l2) : wl * lf + sum_l2;
            sum_xl = ORACLE_PLANT == 1 ? fmaf(wl, x[i], sum_xl) : wl * x[i] + sum_xl;
        }
        float d = sum_w * sum_l2 - sum_l * sum_l;
        if (d > 0.0f) {
            float this_scale = -(sum_x * sum_l - sum_w * sum_xl) / d;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / d;
            if (this_min > 0.0f) {
                this_min = 0.0f;
                this_scale = ORACLE_PLANT == 8 ? sum_xl / sum_l : sum_xl / sum_l2;
            }
            float cur_error = 0.0f;
            for (int i = 0; i < n; i++) {
                float diff = this_scale * (float)laux[i] + this_min - x[i];
                float e = use_mad ? fabsf(diff) : diff * diff;
                cur_error = ORACLE_PLANT == 1 ? fmaf(weights[i], e, cur_error) : weights[i] * e + cur_error;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; i++) l[i] = (uint8_t)laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *neg_min = -min;
    return scale;
}

/* k_quants.rs:1930-2001 (the plain, no-imatrix branch) and k_quants.rs:302-305 (qkx2_weights) */
static void quantize_q4k_block(const float *x, or_block_q4k *blk) {
    uint8_t l[256];
    float mins[8], scales[8];
    memset(blk, 0, sizeof *blk);
    for (int j = 0; j < 8; j++) {
        const float *xs = x + 32 * j;
        float ss = 0.0f;
        for (int i = 0; i < 32; i++) ss = ss + xs[i] * xs[i];
        float av_x = sqrtf(ss / 32.0f);
        float w[32];
        for (int i = 0; i < 32; i++) w[i] = av_x + fabsf(xs[i]);
        scales[j] = make_qkx2_quants(15, xs, w, ORACLE_PLANT == 2 ? -0.5f : -1.0f, 0.1f, 20, 0, l + 32 * j, &mins[j]);
    }
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        max_scale = fmaxf(scales[j], max_scale);
        max_min = fmaxf(mins[j], max_min);
    }
    float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    for (int j = 0; j < 8; j++) {
        int32_t lsi = nearest_int_mul(inv_scale, scales[j]);
        int32_t lmi = nearest_int_mul(inv_min, mins[j]);
        uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
        uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
        if (j < 4) {
            blk->scales[j] = ls;
            blk->scales[j + 4] = lm;
        } else {
            blk->scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            blk->scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
            blk->scales[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    blk->d = oracle_f32_to_f16(max_scale / 63.0f);
    blk->dmin = oracle_f32_to_f16(max_min / (ORACLE_PLANT == 3 ? 64.0f : 63.0f));
    for (int j = 0; j < 8; j++) {
        uint8_t sc, m;
        get_scale_min_k4(j, blk->scales, &sc, &m);
        float d = oracle_f16_to_f32(blk->d) * (float)sc;
        if (d != 0.0f) {
            float dm = oracle_f16_to_f32(blk->dmin) * (float)m;
            for (int ii = 0; ii < 32; ii++) {
                int32_t lv = nearest_int((x[32 * j + ii] + dm) / d);
                l[32 * j + ii] = (uint8_t)clampi(lv, 0, 15);
            }
        }
    }
    for (int j = 0; j < 256; j += 64)
        for (int lv = 0; lv < 32; lv++) blk->qs[(j / 64) * 32 + lv] = (uint8_t)(l[j + lv] | (l[j + lv + 32] << 4));
}

void oracle_quantize_q4k(const float *x, int64_t n, or_block_q4k *y) {
    int64_t nb = n / 256;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nb; b++) quantize_q4k_block(x + 256 * b, y + b);
}

/* ---------------------------------------------------------------- Q6_K weights */

/* utils.rs:135-264, make_qx_quants with Quantizer::LlamaCpp, qw = null; n = 16 */
static float make_qx_quants(int n, int nmax, const float *x, int8_t *ls, int rmse_type) {
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); max = x[i]; }
    }
    if (amax < 1e-15f) {
        memset(ls, 0, (size_t)n);
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    if (rmse_type == 0) {
        for (int i = 0; i < n; i++) ls[i] = (int8_t)(nmax + clampi(nearest_int_mul(iscale, x[i]), -nmax, nmax - 1));
        return 1.0f / iscale;
    }
    int return_early = rmse_type < 0;
    rmse_type = rmse_type < 0 ? -rmse_type : rmse_type;
    float wts[32];
    for (int i = 0; i < n; i++) {
        switch (rmse_type) {
        case 1: wts[i] = x[i] * x[i]; break;
        case 2: wts[i] = 1.0f; break;
        case 3: wts[i] = fabsf(x[i]); break;
        default: wts[i] = sqrtf(fabsf(x[i])); break;
        }
    }
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        float lf = (float)clampi(nearest_int_mul(iscale, x[i]), -nmax, nmax - 1);
        float w = wts[i];
        sumlx = (w * x[i]) * lf + sumlx;
        suml2 = (w * lf) * lf + suml2;
    }
    for (int i = 0; i < n; i++) ls[i] = (int8_t)(nmax + clampi(nearest_int_mul(iscale, x[i]), -nmax, nmax - 1));
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    if (return_early) return suml2 > 0.0f ? 0.5f * (scale + 1.0f / iscale) : 1.0f / iscale;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; is++) {
        if (is == 0) continue;
        float tenths = (float)is;
        iscale = -(0.1f * tenths + (float)(ORACLE_PLANT == 4 ? nmax - 1 : nmax)) / max;
        sumlx = 0.0f;
        suml2 = 0.0f;
        for (int i = 0; i < n; i++) {
            float lf = (float)clampi(nearest_int_mul(iscale, x[i]), -nmax, nmax - 1);
            float w = wts[i];
            sumlx = (w * x[i]) * lf + sumlx;
            suml2 = (w * lf) * lf + suml2;
        }
        if (suml2 > 0.0f && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; i++)
                ls[i] = (int8_t)(nmax + clampi(nearest_int_mul(iscale, x[i]), -nmax, nmax - 1));
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

/* k_quants.rs:2590-2646 (no imatrix) */
static void quantize_q6k_block(const float *x, or_block_q6k *y) {
    int8_t l[256];
    float scales[16];
    float max_scale = 0.0f, max_abs_scale = 0.0f;
    for (int ib = 0; ib < 16; ib++) {
        float scale = make_qx_quants(16, 32, x + 16 * ib, l + 16 * ib, 1);
        scales[ib] = scale;
        if (fabsf(scale) > max_abs_scale) { max_abs_scale = fabsf(scale); max_scale = scale; }
    }
    float iscale = (ORACLE_PLANT == 5 ? -127.0f : -128.0f) / max_scale;
    y->d = oracle_f32_to_f16(1.0f / iscale);
    for (int j = 0; j < 16; j++) {
        int32_t v = nearest_int_mul(iscale, scales[j]);
        y->scales[j] = (int8_t)(v < 127 ? v : 127);
    }
    for (int j = 0; j < 16; j++) {
        float d = oracle_f16_to_f32(y->d) * (float)y->scales[j];
        if (d == 0.0f) continue;
        for (int ii = 0; ii < 16; ii++) l[16 * j + ii] = (int8_t)(clampi(nearest_int(x[16 * j + ii] / d), -32, 31) + 32);
    }
    for (int h = 0; h < 2; h++) {
        int j = 128 * h;
        uint8_t *ql = y->ql + 64 * h;
        uint8_t *qh = y->qh + 32 * h;
        for (int i = 0; i < 32; i++) {
            int8_t q1 = l[j + i], q2 = l[j + i + 32], q3 = l[j + i + 64], q4 = l[j + i + 96];
            ql[i] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
            ql[i + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
            qh[i] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    }
}

void oracle_quantize_q6k(const float *x, int64_t n, or_block_q6k *y) {
    int64_t nb = n / 256;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nb; b++) quantize_q6k_block(x + 256 * b, y + b);
}

/* The sub-block searches on their own, for the tests that pin them: make_qkx2_quants over 32 values (returns the
 * scale, *neg_min = the subtracted min negated, as the reference returns it) and make_qx_quants over n <= 32. */
float oracle_make_qkx2_quants(int nmax, const float *x, const float *weights, float rmin, float rdelta, int nstep,
                              int use_mad, uint8_t *l, float *neg_min) {
    return make_qkx2_quants(nmax, x, weights, rmin, rdelta, nstep, use_mad, l, neg_min);
}
float oracle_make_qx_quants(int n, int nmax, const float *x, int8_t *ls, int rmse_type) {
    return n >= 1 && n <= 32 ? make_qx_quants(n, nmax, x, ls, rmse_type) : 0.0f;
}

/* ---------------------------------------------------------------- Q5_K weights */

/* k_quants.rs:2256-2334 (the plain, no-imatrix branch): Q4_K's search with 31 levels and Q5K_SEARCH
 * {rmin -0.5, rdelta 0.1, nstep 15, mad false} (k_quants.rs:254-259), the fifth bits moved to qh */
static void quantize_q5k_block(const float *x, or_block_q5k *blk) {
    uint8_t l[256];
    float mins[8], scales[8];
    memset(blk, 0, sizeof *blk);
    for (int j = 0; j < 8; j++) {
        const float *xs = x + 32 * j;
        float ss = 0.0f;
        for (int i = 0; i < 32; i++) ss = ss + xs[i] * xs[i];
        float av_x = sqrtf(ss / 32.0f);
        float w[32];
        for (int i = 0; i < 32; i++) w[i] = av_x + fabsf(xs[i]);
        scales[j] = make_qkx2_quants(31, xs, w, -0.5f, 0.1f, ORACLE_PLANT == 6 ? 20 : 15, 0, l + 32 * j, &mins[j]);
    }
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        max_scale = fmaxf(scales[j], max_scale);
        max_min = fmaxf(mins[j], max_min);
    }
    float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    for (int j = 0; j < 8; j++) {
        int32_t lsi = nearest_int_mul(inv_scale, scales[j]);
        int32_t lmi = nearest_int_mul(inv_min, mins[j]);
        uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
        uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
        if (j < 4) {
            blk->scales[j] = ls;
            blk->scales[j + 4] = lm;
        } else {
            blk->scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            blk->scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
            blk->scales[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    blk->d = oracle_f32_to_f16(max_scale / 63.0f);
    blk->dmin = oracle_f32_to_f16(max_min / 63.0f);
    for (int j = 0; j < 8; j++) {
        uint8_t sc, m;
        get_scale_min_k4(j, blk->scales, &sc, &m);
        float d = oracle_f16_to_f32(blk->d) * (float)sc;
        if (d == 0.0f) continue;
        float dm = oracle_f16_to_f32(blk->dmin) * (float)m;
        for (int ii = 0; ii < 32; ii++) l[32 * j + ii] = (uint8_t)clampi(nearest_int((x[32 * j + ii] + dm) / d), 0, 31);
    }
    uint8_t m1 = 1, m2 = 2;
    for (int nn = 0; nn < 256; nn += 64) {
        const int off = nn / 64 * 32;
        for (int j = 0; j < 32; j++) {
            uint8_t l1 = l[nn + j], l2 = l[nn + j + 32];
            if (l1 > 15) { l1 -= 16; blk->qh[j] |= m1; }
            if (l2 > 15) { l2 -= 16; blk->qh[j] |= m2; }
            blk->qs[off + j] = (uint8_t)(l1 | (l2 << 4));
        }
        m1 <<= 2;
        m2 <<= 2;
    }
}

void oracle_quantize_q5k(const float *x, int64_t n, or_block_q5k *y) {
    int64_t nb = n / 256;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nb; b++) quantize_q5k_block(x + 256 * b, y + b);
}

/* ---------------------------------------------------------------- Q4_0 / Q5_0 weights */

/* the signed value of largest magnitude, the first one on a tie (k_quants.rs:393-401, 694-701) */
static float signed_absmax32(const float *x) {
    float amax = 0.0f, max = 0.0f;
    for (int i = 0; i < 32; i++)
        if (amax < fabsf(x[i])) { amax = fabsf(x[i]); max = x[i]; }
    return max;
}

/* k_quants.rs:380-418: d = max / -8, q = min(15, (x / d + 8.5) as u8) */
void oracle_quantize_q4_0(const float *x, int64_t n, or_block_q4_0 *y) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float *xs = x + 32 * b;
        float d = signed_absmax32(xs) / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = oracle_f32_to_f16(d);
        for (int j = 0; j < 16; j++) {
            uint8_t q0 = sat_u8(xs[j] * id + 8.5f), q1 = sat_u8(xs[16 + j] * id + 8.5f);
            q0 = q0 < 15 ? q0 : 15;
            q1 = q1 < 15 ? q1 : 15;
            y[b].qs[j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

/* k_quants.rs:681-717: d = max / -16, q = min(31, (x / d + 16.5) as i8) as u8, fifth bits into qh */
void oracle_quantize_q5_0(const float *x, int64_t n, or_block_q5_0 *y) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float *xs = x + 32 * b;
        float d = signed_absmax32(xs) / -16.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = oracle_f32_to_f16(d);
        uint32_t qh = 0;
        for (int j = 0; j < 16; j++) {
            int8_t a = sat_i8(xs[j] * id + 16.5f), c = sat_i8(xs[16 + j] * id + 16.5f);
            uint8_t q0 = (uint8_t)(a < 31 ? a : 31), q1 = (uint8_t)(c < 31 ? c : 31);
            y[b].qs[j] = (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
            qh |= (uint32_t)((q0 & 0x10) >> 4) << j;
            qh |= (uint32_t)((q1 & 0x10) >> 4) << (j + 16);
        }
        memcpy(y[b].qh, &qh, 4); /* little-endian */
    }
}

int oracle_quantize(int type, const float *x, int64_t n, void *out) {
    size_t bs = oracle_block_size(type);
    if (bs == 0 || n % (int64_t)bs != 0) return -1;
    switch (type) {
    case OR_Q8_0: oracle_quantize_q8_0(x, n, (or_block_q8_0 *)out); return 0;
    case OR_Q4K: oracle_quantize_q4k(x, n, (or_block_q4k *)out); return 0;
    case OR_Q6K: oracle_quantize_q6k(x, n, (or_block_q6k *)out); return 0;
    case OR_Q8K: oracle_quantize_q8k(x, n, (or_block_q8k *)out); return 0;
    case OR_Q4_0: oracle_quantize_q4_0(x, n, (or_block_q4_0 *)out); return 0;
    case OR_Q5_0: oracle_quantize_q5_0(x, n, (or_block_q5_0 *)out); return 0;
    case OR_Q5K: oracle_quantize_q5k(x, n, (or_block_q5k *)out); return 0;
    default: return -1;
    }
}

/* ---------------------------------------------------------------- dequantize */

/* Q8_0: k_quants.rs:905-921; Q4_K: 2096-2123; Q6_K: 2649-2680; Q8_K: 2762-2773; Q4_0: 313-330; Q5_0: 720-743;
 * Q5_K: 2433-2467; IQ4_XS: crates/inference-quant/src/gguf/raw.rs:773-808 */
void oracle_dequantize(int type, const void *blocks, int64_t n, float *y) {
    if (type == OR_Q8_0) {
        const or_block_q8_0 *b = (const or_block_q8_0 *)blocks;
        for (int64_t i = 0; i < n / 32; i++) {
            float d = oracle_f16_to_f32(b[i].d);
            for (int j = 0; j < 32; j++) y[32 * i + j] = (float)b[i].qs[j] * d;
        }
    } else if (type == OR_Q4K) {
        const or_block_q4k *b = (const or_block_q4k *)blocks;
        for (int64_t i = 0; i < n / 256; i++) {
            float d = oracle_f16_to_f32(b[i].d), min = oracle_f16_to_f32(b[i].dmin);
            float *out = y + 256 * i;
            int is = 0, idx = 0;
            for (int j = 0; j < 256; j += 64) {
                const uint8_t *q = b[i].qs + j / 2;
                uint8_t sc, m;
                get_scale_min_k4(is, b[i].scales, &sc, &m);
                float d1 = d * (float)sc, m1 = min * (float)m;
                get_scale_min_k4(is + 1, b[i].scales, &sc, &m);
                float d2 = d * (float)sc, m2 = min * (float)m;
                for (int l = 0; l < 32; l++) out[idx++] = d1 * (float)(q[l] & 0xF) - m1;
                for (int l = 0; l < 32; l++) out[idx++] = d2 * (float)(q[l] >> 4) - m2;
                is += 2;
            }
        }
    } else if (type == OR_Q6K) {
        const or_block_q6k *b = (const or_block_q6k *)blocks;
        for (int64_t i = 0; i < n / 256; i++) {
            float d = oracle_f16_to_f32(b[i].d);
            for (int nn = 0; nn < 256; nn += 128) {
                int idx = nn / 128;
                float *ys = y + 256 * i + nn;
                const int8_t *sc = b[i].scales + 8 * idx;
                const uint8_t *ql = b[i].ql + 64 * idx;
                const uint8_t *qh = b[i].qh + 32 * idx;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int8_t q1 = (int8_t)(((ql[l] & 0xF) | ((qh[l] & 3) << 4))) - 32;
                    int8_t q2 = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4))) - 32;
                    int8_t q3 = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4))) - 32;
                    int8_t q4 = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4))) - 32;
                    ys[l] = d * (float)sc[is] * (float)q1;
                    ys[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    ys[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    ys[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
        }
    } else if (type == OR_Q8K) {
        const or_block_q8k *b = (const or_block_q8k *)blocks;
        for (int64_t i = 0; i < n / 256; i++)
            for (int j = 0; j < 256; j++) y[256 * i + j] = b[i].d * (float)b[i].qs[j];
    } else if (type == OR_Q4_0) {
        const or_block_q4_0 *b = (const or_block_q4_0 *)blocks;
        for (int64_t i = 0; i < n / 32; i++) {
            float d = oracle_f16_to_f32(b[i].d);
            for (int j = 0; j < 16; j++) {
                y[32 * i + j] = (float)((int)(b[i].qs[j] & 0x0F) - 8) * d;
                y[32 * i + j + 16] = (float)((int)(b[i].qs[j] >> 4) - 8) * d;
            }
        }
    } else if (type == OR_Q5_0) {
        const or_block_q5_0 *b = (const or_block_q5_0 *)blocks;
        for (int64_t i = 0; i < n / 32; i++) {
            float d = oracle_f16_to_f32(b[i].d);
            uint32_t qh;
            memcpy(&qh, b[i].qh, 4);
            for (int j = 0; j < 16; j++) {
                int h0 = (int)(((qh >> j) << 4) & 0x10), h1 = (int)((qh >> (j + 12)) & 0x10);
                y[32 * i + j] = (float)(((int)(b[i].qs[j] & 0x0F) | h0) - 16) * d;
                y[32 * i + j + 16] = (float)(((int)(b[i].qs[j] >> 4) | h1) - 16) * d;
            }
        }
    } else if (type == OR_Q5K) {
        const or_block_q5k *b = (const or_block_q5k *)blocks;
        for (int64_t i = 0; i < n / 256; i++) {
            float d = oracle_f16_to_f32(b[i].d), min = oracle_f16_to_f32(b[i].dmin);
            float *out = y + 256 * i;
            uint8_t u1 = 1, u2 = 2;
            for (int j = 0, is = 0; j < 256; j += 64, is += 2) {
                const uint8_t *ql = b[i].qs + j / 2;
                uint8_t sc, m;
                get_scale_min_k4(is, b[i].scales, &sc, &m);
                float d1 = d * (float)sc, m1 = min * (float)m;
                get_scale_min_k4(is + 1, b[i].scales, &sc, &m);
                float d2 = d * (float)sc, m2 = min * (float)m;
                for (int l = 0; l < 32; l++)
                    out[j + l] = d1 * ((float)(ql[l] & 0xF) + ((b[i].qh[l] & u1) ? 16.0f : 0.0f)) - m1;
                for (int l = 0; l < 32; l++)
                    out[j + 32 + l] = d2 * ((float)(ql[l] >> 4) + ((b[i].qh[l] & u2) ? 16.0f : 0.0f)) - m2;
                u1 <<= 2;
                u2 <<= 2;
            }
        }
    } else if (type == OR_IQ4XS) {
        const or_block_iq4xs *b = (const or_block_iq4xs *)blocks;
        for (int64_t i = 0; i < n / 256; i++) {
            float d = oracle_f16_to_f32(b[i].d);
            for (int ib = 0; ib < 8; ib++) {
                int ls = ((b[i].scales_l[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((b[i].scales_h >> (2 * ib)) & 3) << 4);
                float scale = d * (float)(ls - 32);
                const uint8_t *qs = b[i].qs + 16 * ib;
                float *out = y + 256 * i + 32 * ib;
                for (int j = 0; j < 16; j++) {
                    out[j] = scale * (float)oracle_kvalues_iq4nl[qs[j] & 0xF];
                    out[j + 16] = scale * (float)oracle_kvalues_iq4nl[qs[j] >> 4];
                }
            }
        }
    }
}

/* ---------------------------------------------------------------- vec_dot_unopt */

float oracle_vec_dot_q8_0_q8_0(int64_t n, const or_block_q8_0 *x, const or_block_q8_0 *y) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / 32; b++) {
        int32_t sum_i = 0;
        for (int j = 0; j < 32; j++) sum_i += (int32_t)x[b].qs[j] * (int32_t)y[b].qs[j];
        sumf += (float)sum_i * oracle_f16_to_f32(x[b].d) * oracle_f16_to_f32(y[b].d);
    }
    return sumf;
}

float oracle_vec_dot_q4k_q8k(int64_t n, const or_block_q4k *xs, const or_block_q8k *ys) {
    const uint32_t kmask1 = 0x3f3f3f3fu, kmask2 = 0x0f0f0f0fu, kmask3 = 0x03030303u;
    float sums[8] = {0};
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / 256; b++) {
        const or_block_q4k *x = xs + b;
        const or_block_q8k *y = ys + b;
        int8_t aux8[256];
        int32_t aux32[8] = {0};
        for (int c = 0; c < 4; c++) {
            for (int l = 0; l < 32; l++) aux8[64 * c + l] = (int8_t)(x->qs[32 * c + l] & 0xF);
            for (int l = 0; l < 32; l++) aux8[64 * c + 32 + l] = (int8_t)(x->qs[32 * c + l] >> 4);
        }
        uint32_t utmp[4];
        memcpy(utmp, x->scales, 12); /* little-endian words */
        utmp[3] = ((utmp[2] >> 4) & kmask2) | (((utmp[1] >> 6) & kmask3) << 4);
        uint32_t uaux = utmp[1] & kmask1;
        utmp[1] = (utmp[2] & kmask2) | (((utmp[0] >> 6) & kmask3) << 4);
        utmp[2] = uaux;
        utmp[0] &= kmask1;
        uint8_t scales[8], mins[8];
        memcpy(scales, utmp, 8);
        memcpy(mins, utmp + 2, 8);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += (int32_t)y->bsums[j] * (int32_t)mins[j / 2];
        const int8_t *a = aux8;
        const int8_t *q8 = y->qs;
        for (int s = 0; s < 8; s++) {
            int32_t scale = scales[s];
            for (int r = 0; r < 4; r++) {
                for (int l = 0; l < 8; l++) aux32[l] += scale * (int32_t)(int16_t)((int16_t)q8[l] * (int16_t)a[l]);
                q8 += 8;
                a += 8;
            }
        }
        float d = oracle_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        float dmin = oracle_f16_to_f32(x->dmin) * y->d;
        sumf -= dmin * (float)sumi;
    }
    float s = 0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return sumf + s;
}

float oracle_vec_dot_q6k_q8k(int64_t n, const or_block_q6k *xs, const or_block_q8k *ys) {
    float sums[8] = {0};
    for (int64_t b = 0; b < n / 256; b++) {
        const or_block_q6k *x = xs + b;
        const or_block_q8k *y = ys + b;
        int8_t aux8[256];
        float aux32[8] = {0};
        for (int j = 0; j < 256; j += 128) {
            int8_t *a = aux8 + j;
            const uint8_t *q4 = x->ql + j / 2;
            const uint8_t *qh = x->qh + j / 4;
            for (int l = 0; l < 32; l++) {
                a[l] = (int8_t)((int32_t)((q4[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
                a[l + 32] = (int8_t)((int32_t)((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                a[l + 64] = (int8_t)((int32_t)((q4[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                a[l + 96] = (int8_t)((int32_t)((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
            }
        }
        for (int j = 0; j < 16; j++) {
            float scale = (float)x->scales[j];
            const int8_t *q8 = y->qs + 16 * j;
            const int8_t *a = aux8 + 16 * j;
            for (int h = 0; h < 2; h++)
                for (int l = 0; l < 8; l++) aux32[l] += scale * (float)(int16_t)((int16_t)q8[8 * h + l] * (int16_t)a[8 * h + l]);
        }
        float d = oracle_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += aux32[l] * d;
    }
    float s = 0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return s;
}

float oracle_vec_dot_q4_0_q8_0(int64_t n, const or_block_q4_0 *x, const or_block_q8_0 *y) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / 32; b++) {
        int32_t sum_i = 0;
        for (int j = 0; j < 16; j++)
            sum_i += ((int32_t)(x[b].qs[j] & 0x0F) - 8) * y[b].qs[j] + ((int32_t)(x[b].qs[j] >> 4) - 8) * y[b].qs[j + 16];
        sumf += (float)sum_i * oracle_f16_to_f32(x[b].d) * oracle_f16_to_f32(y[b].d);
    }
    return sumf;
}

float oracle_vec_dot_q5_0_q8_0(int64_t n, const or_block_q5_0 *x, const or_block_q8_0 *y) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / 32; b++) {
        uint32_t qh;
        memcpy(&qh, x[b].qh, 4);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) {
            int32_t h0 = (int32_t)(((qh & (1u << j)) >> j) << 4);
            int32_t h1 = (int32_t)((qh & (1u << (j + 16))) >> (j + 12));
            int32_t x0 = ((int32_t)(x[b].qs[j] & 0x0F) | h0) - 16;
            int32_t x1 = ((int32_t)(x[b].qs[j] >> 4) | h1) - 16;
            sumi += x0 * y[b].qs[j] + x1 * y[b].qs[j + 16];
        }
        sumf += (float)sumi * oracle_f16_to_f32(x[b].d) * oracle_f16_to_f32(y[b].d);
    }
    return sumf;
}

float oracle_vec_dot_q5k_q8k(int64_t n, const or_block_q5k *xs, const or_block_q8k *ys) {
    const uint32_t kmask1 = 0x3f3f3f3fu, kmask2 = 0x0f0f0f0fu, kmask3 = 0x03030303u;
    float sums[8] = {0};
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / 256; b++) {
        const or_block_q5k *x = xs + b;
        const or_block_q8k *y = ys + b;
        int8_t aux8[256];
        int32_t aux32[8] = {0};
        uint8_t m = 1;
        for (int c = 0; c < 4; c++) {
            const uint8_t *q5 = x->qs + 32 * c;
            for (int l = 0; l < 32; l++) aux8[64 * c + l] = (int8_t)((q5[l] & 0xF) + ((x->qh[l] & m) ? 16 : 0));
            m <<= 1;
            for (int l = 0; l < 32; l++) aux8[64 * c + 32 + l] = (int8_t)((q5[l] >> 4) + ((x->qh[l] & m) ? 16 : 0));
            m <<= 1;
        }
        uint32_t utmp[4];
        memcpy(utmp, x->scales, 12);
        utmp[3] = ((utmp[2] >> 4) & kmask2) | (((utmp[1] >> 6) & kmask3) << 4);
        uint32_t uaux = utmp[1] & kmask1;
        utmp[1] = (utmp[2] & kmask2) | (((utmp[0] >> 6) & kmask3) << 4);
        utmp[2] = uaux;
        utmp[0] &= kmask1;
        uint8_t scales[8], mins[8];
        memcpy(scales, utmp, 8);
        memcpy(mins, utmp + 2, 8);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += (int32_t)y->bsums[j] * (int32_t)mins[j / 2];
        const int8_t *a = aux8;
        const int8_t *q8 = y->qs;
        for (int s = 0; s < 8; s++) {
            int32_t scale = scales[s];
            for (int r = 0; r < 4; r++) {
                for (int l = 0; l < 8; l++) aux32[l] += scale * (int32_t)(int16_t)((int16_t)q8[l] * (int16_t)a[l]);
                q8 += 8;
                a += 8;
            }
        }
        float d = oracle_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        float dmin = oracle_f16_to_f32(x->dmin) * y->d;
        sumf -= dmin * (float)sumi;
    }
    float s = 0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return sumf + s;
}

float oracle_vec_dot_iq4xs_q8k(int64_t n, const or_block_iq4xs *xs, const or_block_q8k *ys) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / 256; b++) {
        const or_block_iq4xs *x = xs + b;
        const or_block_q8k *y = ys + b;
        float d = oracle_f16_to_f32(x->d) * y->d;
        for (int ib = 0; ib < 8; ib++) {
            const uint8_t *qs = x->qs + 16 * ib;
            const int8_t *q8 = y->qs + 32 * ib;
            int32_t sumi = 0;
            for (int j = 0; j < 16; j++)
                sumi += (int32_t)q8[j] * oracle_kvalues_iq4nl[qs[j] & 0xF] + (int32_t)q8[j + 16] * oracle_kvalues_iq4nl[qs[j] >> 4];
            int32_t ls = (int32_t)(((x->scales_l[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((x->scales_h >> (2 * ib)) & 3) << 4)) - 32;
            sumf += d * (float)(ls * sumi);
        }
    }
    return sumf;
}

/* ---------------------------------------------------------------- matmul (k_quants.rs:2776-2894) */

/* GgmlType::VecDotType: Q8_0 for the 32-value types, Q8_K for the super-block types (IQ4_XS: cpu_dot.rs:67-68) */
static int vec_dot_type(int type) { return oracle_block_size(type) == 32 ? OR_Q8_0 : OR_Q8K; }

static float vec_dot_any(int type, int64_t k, const void *w_row, const void *a_row) {
    switch (type) {
    case OR_Q8_0: return oracle_vec_dot_q8_0_q8_0(k, (const or_block_q8_0 *)w_row, (const or_block_q8_0 *)a_row);
    case OR_Q4K: return oracle_vec_dot_q4k_q8k(k, (const or_block_q4k *)w_row, (const or_block_q8k *)a_row);
    case OR_Q6K: return oracle_vec_dot_q6k_q8k(k, (const or_block_q6k *)w_row, (const or_block_q8k *)a_row);
    case OR_Q4_0: return oracle_vec_dot_q4_0_q8_0(k, (const or_block_q4_0 *)w_row, (const or_block_q8_0 *)a_row);
    case OR_Q5_0: return oracle_vec_dot_q5_0_q8_0(k, (const or_block_q5_0 *)w_row, (const or_block_q8_0 *)a_row);
    case OR_Q5K: return oracle_vec_dot_q5k_q8k(k, (const or_block_q5k *)w_row, (const or_block_q8k *)a_row);
    case OR_IQ4XS: return oracle_vec_dot_iq4xs_q8k(k, (const or_block_iq4xs *)w_row, (const or_block_q8k *)a_row);
    default: return 0.0f;
    }
}

static int set_threads(int threads) {
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

int oracle_matmul_preq(int type, int64_t m, int64_t k, int64_t n, const void *lhs_q, const void *rhs, float *dst,
                       int threads) {
    size_t bs = oracle_block_size(type), ts = oracle_type_size(type);
    if (bs == 0 || type == OR_Q8K || k % (int64_t)bs != 0) return -1;
    int64_t kb = k / (int64_t)bs;
    size_t a_ts = oracle_type_size(vec_dot_type(type));
    int nt = set_threads(threads);
    (void)nt;
    for (int64_t r = 0; r < m; r++) {
        const char *a_row = (const char *)lhs_q + (size_t)(r * kb) * a_ts;
#pragma omp parallel for schedule(static) num_threads(nt)
        for (int64_t c = 0; c < n; c++)
            dst[r * n + c] = vec_dot_any(type, k, (const char *)rhs + (size_t)(c * kb) * ts, a_row);
    }
    return 0;
}

int oracle_matmul(int type, int64_t m, int64_t k, int64_t n, const float *lhs, const void *rhs, float *dst,
                  int threads) {
    size_t bs = oracle_block_size(type);
    if (bs == 0 || type == OR_Q8K || k % (int64_t)bs != 0) return -1;
    int vt = vec_dot_type(type);
    size_t a_ts = oracle_type_size(vt);
    int64_t kb = k / (int64_t)bs;
    void *lhs_q = malloc((size_t)(m * kb) * a_ts + 1);
    if (!lhs_q) return -1;
    for (int64_t r = 0; r < m; r++) oracle_quantize(vt, lhs + r * k, k, (char *)lhs_q + (size_t)(r * kb) * a_ts);
    int rc = oracle_matmul_preq(type, m, k, n, lhs_q, rhs, dst, threads);
    free(lhs_q);
    return rc;
}

/* The values (weight q - offset) and f16 scale of 32-value block b of a Q8_0 / Q4_0 / Q5_0 row */
static uint16_t b32_values(int type, const void *row, int64_t b, int32_t v[32]) {
    if (type == OR_Q8_0) {
        const or_block_q8_0 *x = (const or_block_q8_0 *)row + b;
        for (int j = 0; j < 32; j++) v[j] = x->qs[j];
        return x->d;
    }
    if (type == OR_Q4_0) {
        const or_block_q4_0 *x = (const or_block_q4_0 *)row + b;
        for (int j = 0; j < 16; j++) {
            v[j] = (int32_t)(x->qs[j] & 0x0F) - 8;
            v[j + 16] = (int32_t)(x->qs[j] >> 4) - 8;
        }
        return x->d;
    }
    const or_block_q5_0 *x = (const or_block_q5_0 *)row + b;
    uint32_t qh;
    memcpy(&qh, x->qh, 4);
    for (int j = 0; j < 16; j++) {
        v[j] = ((int32_t)(x->qs[j] & 0x0F) | (int32_t)(((qh >> j) & 1u) << 4)) - 16;
        v[j + 16] = ((int32_t)(x->qs[j] >> 4) | (int32_t)(((qh >> (j + 16)) & 1u) << 4)) - 16;
    }
    return x->d;
}

int oracle_matmul_q8k_act(int type, int64_t m, int64_t k, int64_t n, const float *lhs, const void *rhs, float *dst,
                          int threads) {
    if (type != OR_Q8_0 && type != OR_Q4_0 && type != OR_Q5_0) return oracle_matmul(type, m, k, n, lhs, rhs, dst, threads);
    if (k % 32 != 0) return -1;
    const int64_t kp = (k + 255) / 256 * 256, nb = k / 32;
    const size_t row_bytes = (size_t)nb * oracle_type_size(type);
    float *xp = (float *)calloc((size_t)kp, sizeof(float));
    or_block_q8k *a = (or_block_q8k *)malloc((size_t)(kp / 256) * sizeof(or_block_q8k));
    if (!xp || !a) {
        free(xp);
        free(a);
        return -1;
    }
    for (int64_t r = 0; r < m; r++) {
        memcpy(xp, lhs + r * k, (size_t)k * sizeof(float));
        oracle_quantize_q8k(xp, kp, a);
        for (int64_t c = 0; c < n; c++) {
            const void *wrow = (const char *)rhs + (size_t)c * row_bytes;
            float sumf = 0.0f;
            for (int64_t b = 0; b < nb; b++) {
                int32_t v[32];
                const uint16_t dw = b32_values(type, wrow, b, v);
                const or_block_q8k *y = a + b / 8;
                int32_t sumi = 0;
                for (int j = 0; j < 32; j++) sumi += v[j] * y->qs[32 * (b % 8) + j];
                sumf += (float)sumi * oracle_f16_to_f32(dw) * y->d;
            }
            dst[r * n + c] = sumf;
        }
    }
    free(xp);
    free(a);
    return 0;
}

/* ---------------------------------------------------------------- MoE */

int oracle_indexed_moe(int type, int64_t n_experts, int64_t n, int64_t k, const void *w, const float *x,
                       int64_t batch, int64_t xdim1, int64_t topk, const uint32_t *ids, float *y, int threads) {
    size_t bs = oracle_block_size(type), ts = oracle_type_size(type);
    if (bs == 0 || k % (int64_t)bs != 0 || (xdim1 != 1 && xdim1 != topk)) return -1;
    size_t expert_bytes = (size_t)(n * (k / (int64_t)bs)) * ts;
    for (int64_t b = 0; b < batch; b++) {
        for (int64_t s = 0; s < topk; s++) {
            uint32_t e = ids[b * topk + s];
            if ((int64_t)e >= n_experts) return -1;
            const float *xr = x + (b * xdim1 + (xdim1 == 1 ? 0 : s)) * k;
            int rc = oracle_matmul(type, 1, k, n, xr, (const char *)w + e * expert_bytes, y + (b * topk + s) * n, threads);
            if (rc) return rc;
        }
    }
    return 0;
}

int oracle_moe_dispatch(const int32_t *topk_ids, int32_t total, int32_t n_experts, int32_t topk,
                        int32_t *expert_bounds, int32_t *sorted_token_ids, int32_t *sorted_source_ids) {
    for (int32_t e = 0; e <= n_experts; e++) expert_bounds[e] = 0;
    for (int32_t i = 0; i < total; i++) {
        if (topk_ids[i] < 0 || topk_ids[i] >= n_experts) return -1;
        expert_bounds[topk_ids[i] + 1]++;
    }
    for (int32_t e = 0; e < n_experts; e++) expert_bounds[e + 1] += expert_bounds[e];
    int32_t *cursor = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n_experts > 0 ? n_experts : 1));
    if (!cursor) return -1;
    for (int32_t e = 0; e < n_experts; e++) cursor[e] = expert_bounds[e];
    for (int32_t i = 0; i < total; i++) {
        int32_t pos = cursor[topk_ids[i]]++;
        sorted_token_ids[pos] = i;
        sorted_source_ids[pos] = i / topk;
    }
    free(cursor);
    return 0;
}

void oracle_moe_weighted_reduce(const float *in, const float *w, float *out, int32_t tokens, int32_t hidden,
                                int32_t topk) {
    for (int32_t t = 0; t < tokens; t++)
        for (int32_t h = 0; h < hidden; h++) {
            float acc = 0.0f;
            for (int32_t s = 0; s < topk; s++) {
                float ws = w[t * topk + s];
                if (ws != 0.0f) acc += in[((size_t)t * topk + s) * hidden + h] * ws; /* zero-weight routes skipped */
            }
            out[(size_t)t * hidden + h] = acc;
        }
}
