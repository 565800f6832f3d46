/*
 * hx_oracle.c — CPU restatement of the reference numerics (the oracle).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg, never by the product library. Build flags keep
 * float math canonical: -ffp-contract=off, no -ffast-math (see Makefile).
 * Citations are to the reference tree; the header lists what each part follows.
 */
#define _GNU_SOURCE
#include "hx_oracle.h"

#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define QK 64
#define CANON_NAN 0x7fc00000u

typedef struct { uint16_t d; int8_t q[64]; } __attribute__((packed)) blk_q8;   /* FORMAT.md §6, 66 B */
typedef struct { uint16_t d; uint8_t qs[32]; } __attribute__((packed)) blk_q4;  /* 34 B */
typedef struct { float d; int32_t sum; int8_t q[64]; } act_q8;                   /* 72 B */

static float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float canon(float v) { return v != v ? bits_f(CANON_NAN) : v; }

/* ------------------------------------------------------------ binary16 / bfloat16 */

/* IEEE binary16 -> binary32, exact; NaNs come back quiet with their payload
 * (platform_common.inc:19-37). */
float ho_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, mant = h & 1023u;
    if (e == 31u) return bits_f(sign | 0x7f800000u | (mant << 13) | (mant ? 0x400000u : 0u));
    if (e) return bits_f(sign | ((e + 112u) << 23) | (mant << 13));
    if (!mant) return bits_f(sign);
    /* subnormal: mant * 2^-24 is exact in binary32 */
    return bits_f(sign | f_bits((float)mant * 5.9604644775390625e-8f));
}

/* binary32 -> binary16, round to nearest even, overflow to inf, NaN quiet
 * (platform_common.inc:39-65). Written from the IEEE definition. */
uint16_t ho_f32_to_f16(float f) {
    const uint32_t x = f_bits(f), sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* rounds to >= 65536 */
    if (ax >= 0x38800000u) {                                            /* normal binary16 */
        uint32_t r = ax - 0x38000000u;                                  /* rebias 127 -> 15 */
        r = r + 0x0fffu + ((r >> 13) & 1u);
        return (uint16_t)(sign | (r >> 13));
    }
    if (ax <= 0x33000000u) return (uint16_t)sign;                       /* <= 2^-25 */
    {
        const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, sh = 126u - e;
        uint32_t q = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
}

uint16_t ho_f32_to_bf16(float f) {
    uint32_t x = f_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x = x + 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

static float bf16_to_f32(uint16_t h) { return bits_f((uint32_t)h << 16); }

/* ------------------------------------------------------------ exponential */

static int g_exp_mode = HO_EXP_LIBM;
void ho_set_exp_mode(int mode) { g_exp_mode = mode == HO_EXP_PORTABLE || mode == HO_EXP_GLIBC ? mode : HO_EXP_LIBM; }
int ho_get_exp_mode(void) { return g_exp_mode; }

/* exp in IEEE double from basic operations only (Cody & Waite, "Software Manual for
 * the Elementary Functions", 1980: x = n ln2 + r with ln2 split in a 32-bit head and
 * a tail, then exp(r) by its Taylor series to degree 13, |r| <= ln2/2, truncation
 * < 5e-18). The scale 2^n is applied in two exact steps so subnormal results round
 * once. Identical on every IEEE-754 machine when compiled without FMA contraction. */
double ho_exp_port_d(double x) {
    const double inv_ln2 = 1.44269504088896338700e+00;
    const double ln2_hi = 6.93147180369123816490e-01;   /* 0x3fe62e42fee00000: 32 significant bits */
    const double ln2_lo = 1.90821492927058770002e-10;   /* ln2 - ln2_hi */
    const double shifter = 6755399441055744.0;          /* 1.5 * 2^52: round to integer */
    double t, nd, r, p;
    int64_t n;
    uint64_t b1, b2;
    double s1, s2;
    if (x != x) return x;
    if (x > 709.79) return 1.0 / 0.0;
    if (x < -745.2) return 0.0;
    t = x * inv_ln2;
    nd = (t + shifter) - shifter;
    n = (int64_t)nd;
    r = (x - nd * ln2_hi) - nd * ln2_lo;
    p = 1.0 / 6227020800.0;                              /* 1/13! */
    p = p * r + 1.0 / 479001600.0;
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    /* 2^n = 2^n1 * 2^n2 with both factors normal; the first product is exact */
    {
        int64_t n1 = n < -1000 ? n + 600 : (n > 1000 ? n - 600 : n), n2 = n - n1;
        b1 = (uint64_t)(n1 + 1023) << 52;
        b2 = (uint64_t)(n2 + 1023) << 52;
        memcpy(&s1, &b1, 8);
        memcpy(&s2, &b2, 8);
    }
    return (p * s1) * s2;
}

float ho_exp_port_f(float x) { return (float)ho_exp_port_d((double)x); }

static __attribute__((noinline)) float libm_expf(float x) { return expf(x); }

/* glibc's expf (glibc 2.28 and later, sysdeps/ieee754/flt-32/e_expf.c, the algorithm of
 * Szabolcs Nagy's optimized-routines: exp(x) = 2^(k/32) 2^(r/32) with a 32-entry table of
 * 2^(i/32) and a cubic in double), as its x86-64 FMA build evaluates it: the compiler
 * fuses every multiply that feeds an add, so k and r come from the exact product
 * x * 32/ln2 (fma) and the cubic is three fmas. The reference engine calls the platform
 * libm's expf (docs/NUMERICS.md), which on this image is that build; the restatement is
 * checked against it on every one of the 2^32 inputs (tests/test_oracle.py). The table
 * entries are the correctly rounded doubles of 2^(i/32) minus i << 47 (checked against
 * a 80-digit computation in the same test). */
static const uint64_t EXP2F_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

float ho_exp_glibc_f(float x) {
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32.0;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double shift = 0x1.8p+52;
    const uint32_t ux = f_bits(x), abstop = (ux >> 20) & 0x7ff;
    if (abstop >= (f_bits(88.0f) >> 20)) {        /* |x| >= 88 or NaN */
        if (ux == f_bits(-1.0f / 0.0f)) return 0.0f;
        if (abstop >= (f_bits(1.0f / 0.0f) >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return 1.0f / 0.0f;   /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;         /* underflow */
    }
    const double xd = (double)x;
    double kd = fma(inv_ln2_32, xd, shift);
    uint64_t ki, t;
    memcpy(&ki, &kd, 8);
    kd = kd - shift;
    const double r = fma(inv_ln2_32, xd, -kd);
    t = EXP2F_TAB[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double z = fma(c0, r, c1), r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

float ho_expf(float x) {
    if (g_exp_mode == HO_EXP_PORTABLE) return ho_exp_port_f(x);
    if (g_exp_mode == HO_EXP_GLIBC) return ho_exp_glibc_f(x);
    return libm_expf(x);
}

/* Inputs u in [lo, hi) (float bit patterns) where ho_exp_glibc_f and the platform libm's
 * expf differ (NaN results compare equal), on nthreads threads. */
typedef struct { uint64_t lo, hi, bad; } expchk;
static void *expchk_run(void *p) {
    expchk *j = (expchk *)p;
    j->bad = 0;
    for (uint64_t u = j->lo; u < j->hi; u++) {
        const float x = bits_f((uint32_t)u), a = libm_expf(x), b = ho_exp_glibc_f(x);
        if (f_bits(a) != f_bits(b) && !(a != a && b != b)) j->bad++;
    }
    return NULL;
}

uint64_t ho_exp_glibc_mismatches(uint64_t lo, uint64_t hi, int nthreads) {
    expchk jobs[64];
    pthread_t th[64];
    int nt = nthreads < 1 ? 1 : (nthreads > 64 ? 64 : nthreads);
    for (int i = 0; i < nt; i++) {
        jobs[i].lo = lo + (hi - lo) * (uint64_t)i / (uint64_t)nt;
        jobs[i].hi = lo + (hi - lo) * (uint64_t)(i + 1) / (uint64_t)nt;
    }
    for (int i = 1; i < nt; i++) pthread_create(&th[i], NULL, expchk_run, &jobs[i]);
    expchk_run(&jobs[0]);
    uint64_t bad = jobs[0].bad;
    for (int i = 1; i < nt; i++) {
        pthread_join(th[i], NULL);
        bad += jobs[i].bad;
    }
    return bad;
}

/* ------------------------------------------------------------ canonical helpers (NUMERICS §1, §4) */

float ho_sum16(const float *a, int64_t n) {
    float L[16] = {0};
    for (int64_t i = 0; i < n; i++) L[i & 15] = L[i & 15] + a[i];
    for (int s = 8; s >= 1; s >>= 1)
        for (int j = 0; j < s; j++) L[j] = L[j] + L[j + s];
    return L[0];
}

float ho_dot16(const float *a, const float *b, int64_t n) {
    float L[16] = {0};
    for (int64_t i = 0; i < n; i++) L[i & 15] = L[i & 15] + a[i] * b[i];
    for (int s = 8; s >= 1; s >>= 1)
        for (int j = 0; j < s; j++) L[j] = L[j] + L[j + s];
    return L[0];
}

static int g_attn_mode = HO_ATTN_CANONICAL;
void ho_set_attn_mode(int mode) { g_attn_mode = mode == HO_ATTN_CHUNKED ? mode : HO_ATTN_CANONICAL; }
int ho_get_attn_mode(void) { return g_attn_mode; }

static void rmsnorm(float *y, const float *x, const float *w, int64_t n, float eps) {
    const float ms = ho_dot16(x, x, n) / (float)n;
    const float r = 1.0f / sqrtf(ms + eps);
    for (int64_t i = 0; i < n; i++) y[i] = (x[i] * r) * w[i];
}

static void softmax(float *x, int64_t n) {
    float m = x[0], s;
    for (int64_t i = 1; i < n; i++) m = x[i] > m ? x[i] : m;
    for (int64_t i = 0; i < n; i++) x[i] = ho_expf(x[i] - m);
    s = ho_sum16(x, n);
    for (int64_t i = 0; i < n; i++) x[i] = x[i] / s;
}

static float sigmoidf_(float x) { return 1.0f / (1.0f + ho_expf(-x)); }

static __attribute__((noinline)) float o_cosf(float x) { return cosf(x); }
static __attribute__((noinline)) float o_sinf(float x) { return sinf(x); }

/* ------------------------------------------------------------ quantizers (NUMERICS §6) */

size_t ho_row_bytes(int dtype, int64_t n) {
    if (n <= 0 || n > ((int64_t)1 << 40)) return 0;
    switch (dtype) {
    case HO_F32: case HO_I32: return (size_t)n * 4;
    case HO_F16: case HO_BF16: return (size_t)n * 2;
    case HO_U8: return (size_t)n;
    case HO_Q8: return n % QK ? 0 : (size_t)(n / QK) * 66;
    case HO_Q4: return n % QK ? 0 : (size_t)(n / QK) * 34;
    default: return 0;
    }
}

static float nan0(float v) { return v == v ? v : 0.0f; }
static float rne(float v) { return (v + 12582912.0f) - 12582912.0f; }   /* |v| < 2^22 */

/* f16 scale; an overflow saturates to the largest finite binary16 (quant.c:67-72). */
static uint16_t scale_f16(float d) {
    uint16_t h = ho_f32_to_f16(d);
    if ((h & 0x7c00u) == 0x7c00u) h = (uint16_t)((h & 0x8000u) | 0x7bffu);
    return h;
}

/* Q8: d = amax/127 stored as f16, q = rint(x / f16(d)) clamped to [-127, 127];
 * NaN counts as 0 (quant.c:99-116). */
static void quant_q8_row(const float *x, blk_q8 *out, int64_t nb) {
    for (int64_t b = 0; b < nb; b++, x += QK) {
        float amax = 0.0f, d;
        for (int i = 0; i < QK; i++) {
            const float a = fabsf(nan0(x[i]));
            if (a > amax) amax = a;
        }
        out[b].d = scale_f16(amax / 127.0f);
        d = ho_f16_to_f32(out[b].d);
        for (int i = 0; i < QK; i++) {
            float v = d != 0.0f ? nan0(x[i]) / d : 0.0f;
            v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
            out[b].q[i] = (int8_t)rne(v);
        }
    }
}

/* Q4 scale search as documented at quant.c:118-138: xm = first element of largest
 * magnitude; candidates f16(xm / m) for the 20 divisors below in order, each scored
 * once by err = sx2 - 2 d sxq + d^2 sqq in double (x*q exact, 4 fixed lanes), lowest
 * error wins (earlier on ties); then up to 3 least-squares refits d' = f16(sxq/sqq)
 * while they strictly lower the error; nibbles store q + 8 (byte j: element j low,
 * element j + 32 high). */
static const float q4_divisors[20] = {
    -8.0f, -7.75f, -8.25f, -7.5f, -8.5f, -7.25f, -8.75f, -7.0f, -9.0f, -9.25f,
    -9.5f, -9.75f, -10.0f, -10.5f, -11.0f, -12.0f, 7.0f, 7.5f, 7.75f, 8.0f,
};

static float q4_level(float x, float id) {
    float v = x * id;
    v = v < -8.0f ? -8.0f : v;
    v = v > 7.0f ? 7.0f : v;
    return rne(v);
}

static double q4_err(const float *x, const double *xd, double sx2, uint16_t h, double *sxq, double *sqq) {
    const float d = ho_f16_to_f32(h), id = d != 0.0f ? 1.0f / d : 0.0f;
    const double dd = (double)d;
    double lane[4] = {0.0, 0.0, 0.0, 0.0};
    int32_t qq = 0;
    for (int i = 0; i < QK; i += 4) {
        for (int j = 0; j < 4; j++) {
            const int q = (int)q4_level(x[i + j], id);
            lane[j] = lane[j] + xd[i + j] * q;
            qq += q * q;
        }
    }
    *sxq = (lane[0] + lane[1]) + (lane[2] + lane[3]);
    *sqq = (double)qq;
    return (sx2 - (2.0 * dd) * *sxq) + (dd * dd) * (double)qq;
}

static void quant_q4_row(const float *src, blk_q4 *out, int64_t nb) {
    for (int64_t b = 0; b < nb; b++, src += QK) {
        float x[QK], xm = 0.0f, amax = 0.0f;
        double xd[QK], sx2 = 0.0, best_err = 0.0, best_sxq = 0.0, best_sqq = 0.0;
        uint16_t best = 0, seen[20];
        int nseen = 0;
        for (int i = 0; i < QK; i++) {
            x[i] = nan0(src[i]);
            const float a = fabsf(x[i]);
            if (a > amax) { amax = a; xm = x[i]; }
            xd[i] = (double)x[i];
            sx2 = sx2 + xd[i] * xd[i];
        }
        if (amax > 0.0f) {
            for (int k = 0; k < 20; k++) {
                double sxq, sqq, err;
                const uint16_t h = scale_f16(xm / q4_divisors[k]);
                int dup = 0;
                for (int j = 0; j < nseen; j++) dup |= seen[j] == h;
                if (dup) continue;
                seen[nseen++] = h;
                err = q4_err(x, xd, sx2, h, &sxq, &sqq);
                if (k == 0 || err < best_err) { best = h; best_err = err; best_sxq = sxq; best_sqq = sqq; }
            }
            for (int it = 0; it < 3 && best_sqq > 0.0; it++) {
                double sxq, sqq, err;
                const uint16_t h = scale_f16((float)(best_sxq / best_sqq));
                if (h == best) break;
                err = q4_err(x, xd, sx2, h, &sxq, &sqq);
                if (!(err < best_err)) break;
                best = h; best_err = err; best_sxq = sxq; best_sqq = sqq;
            }
        }
        out[b].d = best;
        {
            const float d = ho_f16_to_f32(best), id = d != 0.0f ? 1.0f / d : 0.0f;
            int8_t q[QK];
            for (int i = 0; i < QK; i++) q[i] = (int8_t)q4_level(x[i], id);
            for (int j = 0; j < 32; j++) out[b].qs[j] = (uint8_t)((q[j] + 8) | ((q[j + 32] + 8) << 4));
        }
    }
}

static void quant_row(int dtype, const float *src, uint8_t *dst, int64_t n) {
    switch (dtype) {
    case HO_F32: memcpy(dst, src, (size_t)n * 4); break;
    case HO_F16: for (int64_t i = 0; i < n; i++) ((uint16_t *)dst)[i] = ho_f32_to_f16(src[i]); break;
    case HO_BF16: for (int64_t i = 0; i < n; i++) ((uint16_t *)dst)[i] = ho_f32_to_bf16(src[i]); break;
    case HO_Q8: quant_q8_row(src, (blk_q8 *)dst, n / QK); break;
    case HO_Q4: quant_q4_row(src, (blk_q4 *)dst, n / QK); break;
    default: break;
    }
}

int ho_quantize(int dtype, const float *src, int64_t rows, int64_t cols, void *dst) {
    const size_t rb = ho_row_bytes(dtype, cols);
    if (dtype < HO_F32 || dtype > HO_Q4 || !rb || rows < 0) return -1;
    for (int64_t r = 0; r < rows; r++) quant_row(dtype, src + (size_t)r * cols, (uint8_t *)dst + (size_t)r * rb, cols);
    return 0;
}

static void dequant_row(int dtype, const uint8_t *src, float *dst, int64_t n) {
    switch (dtype) {
    case HO_F32: memcpy(dst, src, (size_t)n * 4); break;
    case HO_F16: for (int64_t i = 0; i < n; i++) dst[i] = ho_f16_to_f32(((const uint16_t *)src)[i]); break;
    case HO_BF16: for (int64_t i = 0; i < n; i++) dst[i] = bf16_to_f32(((const uint16_t *)src)[i]); break;
    case HO_Q8: {
        const blk_q8 *b = (const blk_q8 *)src;
        for (int64_t k = 0; k < n / QK; k++) {
            const float d = ho_f16_to_f32(b[k].d);
            for (int i = 0; i < QK; i++) dst[k * QK + i] = d * (float)b[k].q[i];
        }
        break;
    }
    case HO_Q4: {
        const blk_q4 *b = (const blk_q4 *)src;
        for (int64_t k = 0; k < n / QK; k++) {
            const float d = ho_f16_to_f32(b[k].d);
            for (int j = 0; j < 32; j++) {
                dst[k * QK + j] = d * (float)((int)(b[k].qs[j] & 15) - 8);
                dst[k * QK + j + 32] = d * (float)((int)(b[k].qs[j] >> 4) - 8);
            }
        }
        break;
    }
    case HO_I32: for (int64_t i = 0; i < n; i++) dst[i] = (float)((const int32_t *)src)[i]; break;
    case HO_U8: for (int64_t i = 0; i < n; i++) dst[i] = (float)src[i]; break;
    default: break;
    }
}

int ho_dequantize(int dtype, const void *src, int64_t rows, int64_t cols, float *dst) {
    const size_t rb = ho_row_bytes(dtype, cols);
    if (!rb || rows < 0) return -1;
    for (int64_t r = 0; r < rows; r++) dequant_row(dtype, (const uint8_t *)src + (size_t)r * rb, dst + (size_t)r * cols, cols);
    return 0;
}

/* ------------------------------------------------------------ activations and matmul (NUMERICS §2, §3) */

void ho_act_quant(const float *x, int64_t n, void *outv) {
    act_q8 *out = (act_q8 *)outv;
    for (int64_t b = 0; b < n / QK; b++, x += QK) {
        float amax = 0.0f, d, id;
        int32_t sum = 0;
        for (int i = 0; i < QK; i++) {
            const float a = fabsf(x[i]);
            if (a > amax) amax = a;
        }
        d = amax / 127.0f;
        id = d != 0.0f ? 1.0f / d : 0.0f;
        for (int i = 0; i < QK; i++) {
            float v = x[i] * id;
            if (v != v) v = 0.0f;
            v = v > 127.0f ? 127.0f : v;
            v = v < -127.0f ? -127.0f : v;
            const int q = (int)rne(v);
            out[b].q[i] = (int8_t)q;
            sum += q;
        }
        out[b].d = d;
        out[b].sum = sum;
    }
}

static float row_quant(int dtype, const uint8_t *row, const act_q8 *a, int64_t nb) {
    float acc = 0.0f;
    for (int64_t g = 0; g < nb; g++) {
        int32_t isum = 0;
        float dw;
        if (dtype == HO_Q8) {
            const blk_q8 *w = (const blk_q8 *)row + g;
            for (int i = 0; i < QK; i++) isum += (int32_t)w->q[i] * (int32_t)a[g].q[i];
            dw = ho_f16_to_f32(w->d);
        } else {
            const blk_q4 *w = (const blk_q4 *)row + g;
            for (int j = 0; j < 32; j++) {
                isum += ((int32_t)(w->qs[j] & 15) - 8) * (int32_t)a[g].q[j];
                isum += ((int32_t)(w->qs[j] >> 4) - 8) * (int32_t)a[g].q[j + 32];
            }
            dw = ho_f16_to_f32(w->d);
        }
        acc = acc + (float)isum * (dw * a[g].d);
    }
    return canon(acc);
}

static float row_float(int dtype, const uint8_t *row, const float *x, int64_t n) {
    float L[16] = {0};
    for (int64_t i = 0; i < n; i++) {
        float w;
        if (dtype == HO_F32) w = ((const float *)row)[i];
        else if (dtype == HO_F16) w = ho_f16_to_f32(((const uint16_t *)row)[i]);
        else w = bf16_to_f32(((const uint16_t *)row)[i]);
        L[i & 15] = L[i & 15] + w * x[i];
    }
    for (int s = 8; s >= 1; s >>= 1)
        for (int j = 0; j < s; j++) L[j] = L[j] + L[j + s];
    return canon(L[0]);
}

/* A matrix-vector product over a row range, T activations. */
typedef struct mv_job {
    int dtype;
    const uint8_t *W;
    int64_t cols, r0, r1;
    const void *act;       /* act_q8 [T][nb] or float [T][cols] */
    int T;
    float *Y;              /* Y[t * ldy + r - ybase] */
    int64_t ldy, ybase;
} mv_job;

static void *mv_run(void *p) {
    const mv_job *j = (const mv_job *)p;
    const size_t rb = ho_row_bytes(j->dtype, j->cols);
    const int64_t nb = j->cols / QK;
    for (int64_t r = j->r0; r < j->r1; r++) {
        const uint8_t *row = j->W + (size_t)r * rb;
        for (int t = 0; t < j->T; t++) {
            float y;
            if (j->dtype == HO_Q8 || j->dtype == HO_Q4) y = row_quant(j->dtype, row, (const act_q8 *)j->act + (size_t)t * nb, nb);
            else y = row_float(j->dtype, row, (const float *)j->act + (size_t)t * j->cols, j->cols);
            j->Y[(size_t)t * j->ldy + (r - j->ybase)] = y;
        }
    }
    return NULL;
}

/* Rows [r0, r1) of W . X for T inputs x (f32 [T][cols]) into Y[t*ldy + r - r0],
 * on up to nthreads threads (every element is computed by one call, so the thread
 * count cannot change a result). */
static void matvec(int dtype, const uint8_t *W, int64_t cols, const float *X, int T, float *Y, int64_t ldy,
                   int64_t r0, int64_t r1, int nthreads) {
    void *act = NULL;
    const void *a = X;
    if (dtype == HO_Q8 || dtype == HO_Q4) {
        act = malloc(sizeof(act_q8) * (size_t)(cols / QK) * (size_t)T);
        for (int t = 0; t < T; t++) ho_act_quant(X + (size_t)t * cols, cols, (act_q8 *)act + (size_t)t * (cols / QK));
        a = act;
    }
    int64_t rows = r1 - r0;
    int nt = nthreads < 1 ? 1 : nthreads;
    {   /* at least ~2M multiply-adds per thread: thread start-up costs more below that */
        const double work = (double)rows * (double)cols * T / 2e6;
        if (work < nt) nt = work < 1.0 ? 1 : (int)work;
    }
    if (nt > rows) nt = (int)(rows > 0 ? rows : 1);
    mv_job jobs[64];
    pthread_t th[64];
    if (nt > 64) nt = 64;
    for (int i = 0; i < nt; i++) {
        jobs[i].dtype = dtype; jobs[i].W = W; jobs[i].cols = cols; jobs[i].act = a; jobs[i].T = T;
        jobs[i].Y = Y; jobs[i].ldy = ldy; jobs[i].ybase = r0;
        jobs[i].r0 = r0 + rows * i / nt;
        jobs[i].r1 = r0 + rows * (i + 1) / nt;
    }
    for (int i = 1; i < nt; i++) pthread_create(&th[i], NULL, mv_run, &jobs[i]);
    mv_run(&jobs[0]);
    for (int i = 1; i < nt; i++) pthread_join(th[i], NULL);
    free(act);
}

int ho_matmul(int dtype, const void *W, int64_t rows, int64_t cols, const float *X, int T, float *Y) {
    if (dtype < HO_F32 || dtype > HO_Q4 || !ho_row_bytes(dtype, cols) || rows < 0 || T < 0) return -1;
    if (!rows || !T) return 0;
    matvec(dtype, (const uint8_t *)W, cols, X, T, Y, rows, 0, rows, 1);
    return 0;
}

/* ------------------------------------------------------------ container reader (FORMAT.md) */

typedef struct tens {
    char name[80];
    int dtype, ndim;
    int64_t shape[4];
    uint64_t off, nbytes;
    const uint8_t *data;
} tens;

typedef struct expent { uint64_t off, nbytes; uint32_t dtype, flags; } expent;

typedef struct cfg {
    char arch[32];
    int n_layers, d_model, vocab, max_seq;
    float eps;
    int attn_kind, n_heads, n_kv_heads, head_dim, qk_norm, qkv_bias;
    int q_lora, kv_lora, nope, rope_qk, v_head, rope_dim, rope_style;
    float rope_factor, attn_scale;
    int dense_ffn, n_experts, top_k, expert_ffn, shared_ffn, shared_gate;
    int score_fn, score_bias, n_group, topk_group, norm_topk;
    float routed_scale, emb_scale, resid_scale, logit_scale;
    int tie;
    uint8_t layer_kind[512];
    int n_moe;
} cfg;

struct ho_model {
    char dump_dir[512];
    uint8_t *map;
    size_t size;
    cfg c;
    tens *t;
    int nt;
    expent *ex;
    const float *inv_freq;
    int cap, pos, nthreads;
    float *kv;            /* per layer: GQA K [cap][kvd], V [cap][kvd]; MLA c [cap][C], kpe [cap][r] */
    size_t per_layer;
    int *moe_ord;
    uint16_t *replay;     /* route replay [rows][n_moe][K], or NULL */
    int64_t replay_rows;
    int cur_pos;          /* position of the token being evaluated (replay row) */
    float *margins;       /* ho_set_margins: routing margins [tokens][n_moe] of the next eval */
    float *cur_margin;    /* where route() writes the margin of the current token and layer */
};

/* appends n floats to <dump_dir>/l<layer>_<name>.bin (debug comparisons) */
static void dump(const ho_model *m, const char *name, int layer, const void *v, int n, int elem) {
    char path[700];
    FILE *f;
    if (!m->dump_dir[0]) return;
    snprintf(path, sizeof path, "%s/l%d_%s.bin", m->dump_dir, layer, name);
    f = fopen(path, "ab");
    if (f) { fwrite(v, (size_t)elem, (size_t)n, f); fclose(f); }
}

void ho_set_dump(ho_model *m, const char *dir) {
    snprintf(m->dump_dir, sizeof m->dump_dir, "%s", dir ? dir : "");
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
static uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }
static float rdf(const uint8_t *p) { return bits_f(rd32(p)); }

static int fail(char *err, size_t n, const char *fmt, ...) {
    va_list ap;
    if (err && n) {
        va_start(ap, fmt);
        vsnprintf(err, n, fmt, ap);
        va_end(ap);
    }
    return 0;
}

typedef struct { const char *key; const uint8_t *p; uint32_t n; int type; } mkv;

static const mkv *meta_find(const mkv *kv, int nkv, const char *key) {
    const mkv *r = NULL;
    for (int i = 0; i < nkv; i++)
        if (!strcmp(kv[i].key, key)) r = &kv[i];   /* later duplicates win */
    return r;
}
static int mu32(const mkv *kv, int n, const char *k, int def) { const mkv *e = meta_find(kv, n, k); return e && e->type == 1 ? (int)rd32(e->p) : def; }
static float mf32(const mkv *kv, int n, const char *k, float def) { const mkv *e = meta_find(kv, n, k); return e && e->type == 2 ? rdf(e->p) : def; }

static const tens *find_tensor(const ho_model *m, int layer, const char *suffix) {
    char name[96];
    if (layer < 0) snprintf(name, sizeof name, "%s", suffix);
    else snprintf(name, sizeof name, "blk.%d.%s", layer, suffix);
    for (int i = 0; i < m->nt; i++)
        if (!strcmp(m->t[i].name, name)) return &m->t[i];
    return NULL;
}

static int parse(ho_model *m, char *err, size_t el) {
    const uint8_t *b = m->map;
    if (m->size < 64 || rd32(b) != 0x48545248u || rd32(b + 4) != 1) return fail(err, el, "not a .hearth v1 container");
    const uint64_t meta_off = rd64(b + 8), meta_bytes = rd64(b + 16), tdir = rd64(b + 24), nt = rd64(b + 32);
    const uint64_t edir = rd64(b + 40), ne = rd64(b + 48);
    if (meta_off + meta_bytes > m->size || tdir + nt * 128 > m->size || edir + ne * 32 > m->size)
        return fail(err, el, "directory outside the file");
    /* metadata */
    mkv kv[256];
    int nkv = 0;
    char keys[256][64];
    uint64_t p = 0;
    const uint8_t *mb = b + meta_off;
    while (p < meta_bytes && nkv < 256) {
        uint32_t klen = rd16(mb + p);
        p += 2;
        if (klen > 63) klen = 63;
        memcpy(keys[nkv], mb + p, klen);
        keys[nkv][klen] = 0;
        p += rd16(mb + p - 2);
        int type = mb[p++];
        uint32_t cnt = 0;
        uint64_t plen;
        if (type == 1 || type == 2) plen = 4;
        else if (type == 3) plen = 8;
        else { cnt = rd32(mb + p); p += 4; plen = (uint64_t)cnt * ((type == 4 || type == 7) ? 1 : 4); }
        kv[nkv].key = keys[nkv];
        kv[nkv].p = mb + p;
        kv[nkv].n = cnt;
        kv[nkv].type = type;
        nkv++;
        p += plen;
    }
    cfg *c = &m->c;
    memset(c, 0, sizeof *c);
    const mkv *a = meta_find(kv, nkv, "arch");
    if (a && a->type == 4) memcpy(c->arch, a->p, a->n < 31 ? a->n : 31);
    c->n_layers = mu32(kv, nkv, "n_layers", 0);
    c->d_model = mu32(kv, nkv, "d_model", 0);
    c->vocab = mu32(kv, nkv, "vocab_size", 0);
    c->max_seq = mu32(kv, nkv, "max_seq", 4096);
    c->eps = mf32(kv, nkv, "norm_eps", 1e-6f);
    c->attn_kind = mu32(kv, nkv, "attn_kind", 0);
    c->n_heads = mu32(kv, nkv, "n_heads", 0);
    if (c->n_layers < 1 || c->n_layers > 512 || c->d_model < 1 || c->vocab < 1 || c->n_heads < 1)
        return fail(err, el, "bad required metadata");
    c->n_kv_heads = mu32(kv, nkv, "n_kv_heads", c->n_heads);
    c->head_dim = mu32(kv, nkv, "head_dim", c->d_model / c->n_heads);
    c->qk_norm = mu32(kv, nkv, "qk_norm", 0);
    c->qkv_bias = mu32(kv, nkv, "qkv_bias", 0);
    c->q_lora = mu32(kv, nkv, "q_lora_rank", 0);
    c->kv_lora = mu32(kv, nkv, "kv_lora_rank", 0);
    c->nope = mu32(kv, nkv, "qk_nope_dim", 0);
    c->rope_qk = mu32(kv, nkv, "qk_rope_dim", 0);
    c->v_head = mu32(kv, nkv, "v_head_dim", 0);
    const int mla = c->attn_kind == 1;
    const int qk_dim = mla ? c->nope + c->rope_qk : c->head_dim;
    c->rope_dim = mu32(kv, nkv, "rope_dim", mla ? c->rope_qk : c->head_dim);
    c->rope_style = mu32(kv, nkv, "rope_style", 0);
    c->rope_factor = mf32(kv, nkv, "rope_attn_factor", 1.0f);
    c->attn_scale = mf32(kv, nkv, "attn_scale", 1.0f / sqrtf((float)qk_dim));
    c->dense_ffn = mu32(kv, nkv, "dense_ffn_dim", 0);
    c->n_experts = mu32(kv, nkv, "n_experts", 0);
    c->top_k = mu32(kv, nkv, "top_k", 0);
    c->expert_ffn = mu32(kv, nkv, "expert_ffn_dim", 0);
    c->shared_ffn = mu32(kv, nkv, "shared_ffn_dim", 0);
    c->shared_gate = mu32(kv, nkv, "shared_gate", 0);
    c->score_fn = mu32(kv, nkv, "score_fn", 0);
    c->score_bias = mu32(kv, nkv, "score_bias", 0);
    c->n_group = mu32(kv, nkv, "n_group", 1);
    c->topk_group = mu32(kv, nkv, "topk_group", 1);
    c->norm_topk = mu32(kv, nkv, "norm_topk_prob", 0);
    c->routed_scale = mf32(kv, nkv, "routed_scale", 1.0f);
    c->emb_scale = mf32(kv, nkv, "emb_scale", 1.0f);
    c->resid_scale = mf32(kv, nkv, "residual_scale", 1.0f);
    c->logit_scale = mf32(kv, nkv, "logit_scale", 1.0f);
    c->tie = mu32(kv, nkv, "tie_embeddings", 0);
    const mkv *lk = meta_find(kv, nkv, "layer_kind");
    for (int i = 0; i < c->n_layers; i++)
        c->layer_kind[i] = lk && lk->type == 7 && lk->n == (uint32_t)c->n_layers ? lk->p[i] : (c->n_experts > 0);
    c->n_moe = 0;
    for (int i = 0; i < c->n_layers; i++) c->n_moe += c->layer_kind[i];
    if (c->n_moe == 0) { c->n_experts = 0; c->top_k = 0; c->shared_ffn = 0; }
    /* tensors */
    m->nt = (int)nt;
    m->t = (tens *)calloc(nt ? nt : 1, sizeof(tens));
    for (uint64_t i = 0; i < nt; i++) {
        const uint8_t *e = b + tdir + 128 * i;
        tens *t = &m->t[i];
        memcpy(t->name, e, 79);
        t->name[79] = 0;
        t->dtype = (int)rd32(e + 80);
        t->ndim = (int)rd32(e + 84);
        for (int k = 0; k < 4; k++) t->shape[k] = rd32(e + 88 + 4 * k);
        t->off = rd64(e + 104);
        t->nbytes = rd64(e + 112);
        if (t->off + t->nbytes > m->size) return fail(err, el, "tensor %s outside the file", t->name);
        t->data = b + t->off;
    }
    m->ex = (expent *)calloc(ne ? ne : 1, sizeof(expent));
    for (uint64_t i = 0; i < ne; i++) {
        const uint8_t *e = b + edir + 32 * i;
        m->ex[i].off = rd64(e);
        m->ex[i].nbytes = rd64(e + 8);
        m->ex[i].dtype = rd32(e + 16);
        m->ex[i].flags = rd32(e + 20);
        if (m->ex[i].off + m->ex[i].nbytes > m->size) return fail(err, el, "slab outside the file");
    }
    if (c->n_moe && ne != (uint64_t)c->n_layers * (uint64_t)c->n_experts) return fail(err, el, "expert directory size");
    const tens *inv = find_tensor(m, -1, "rope_inv_freq");
    m->inv_freq = inv ? (const float *)inv->data : NULL;
    if (c->rope_dim / 2 && !m->inv_freq) return fail(err, el, "rope_inv_freq missing");
    return 1;
}

ho_model *ho_open(const char *path, int cap, char *err, size_t errlen) {
    ho_model *m = (ho_model *)calloc(1, sizeof *m);
    struct stat st;
    const int fd = open(path, O_RDONLY);
    if (fd < 0 || fstat(fd, &st) != 0) {
        if (fd >= 0) close(fd);
        free(m);
        fail(err, errlen, "cannot open %s", path);
        return NULL;
    }
    m->size = (size_t)st.st_size;
    m->map = (uint8_t *)mmap(NULL, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m->map == MAP_FAILED) { free(m); fail(err, errlen, "mmap failed"); return NULL; }
    if (!parse(m, err, errlen)) { ho_close(m); return NULL; }
    const cfg *c = &m->c;
    m->cap = cap > 0 ? (cap < c->max_seq ? cap : c->max_seq) : (c->max_seq < 4096 ? c->max_seq : 4096);
    m->nthreads = 1;
    if (c->attn_kind == 1) m->per_layer = (size_t)m->cap * (size_t)(c->kv_lora + c->rope_qk);
    else m->per_layer = (size_t)m->cap * (size_t)c->n_kv_heads * (size_t)c->head_dim * 2;
    m->kv = (float *)calloc(m->per_layer * (size_t)c->n_layers, sizeof(float));
    m->moe_ord = (int *)calloc((size_t)c->n_layers, sizeof(int));
    for (int l = 0, k = 0; l < c->n_layers; l++) m->moe_ord[l] = c->layer_kind[l] ? k++ : -1;
    if (!m->kv) { ho_close(m); fail(err, errlen, "out of memory for the KV cache"); return NULL; }
    return m;
}

void ho_close(ho_model *m) {
    if (!m) return;
    if (m->map && m->map != MAP_FAILED) munmap(m->map, m->size);
    free(m->t);
    free(m->ex);
    free(m->kv);
    free(m->moe_ord);
    free(m->replay);
    free(m);
}

void ho_set_threads(ho_model *m, int n) { if (m) m->nthreads = n < 1 ? 1 : n; }

void ho_info(const ho_model *m, int *o) {
    const cfg *c = &m->c;
    o[0] = c->n_layers; o[1] = c->d_model; o[2] = c->vocab; o[3] = c->n_heads; o[4] = c->n_kv_heads;
    o[5] = c->head_dim; o[6] = c->n_experts; o[7] = c->top_k; o[8] = c->expert_ffn; o[9] = c->n_moe;
    o[10] = m->cap; o[11] = c->attn_kind;
}

int ho_pos(const ho_model *m) { return m->pos; }

/* Route replay (model.c:1885-1960 loads and checks the trace): ids [rows][n_moe][K],
 * checked by the caller; NULL or rows 0 turns it off. */
int ho_set_replay(ho_model *m, const uint16_t *ids, int64_t rows) {
    free(m->replay);
    m->replay = NULL;
    m->replay_rows = 0;
    if (!ids || rows <= 0) return 0;
    const size_t n = (size_t)rows * (size_t)m->c.n_moe * (size_t)m->c.top_k;
    m->replay = (uint16_t *)malloc(n * sizeof(uint16_t));
    if (!m->replay) return -5;
    memcpy(m->replay, ids, n * sizeof(uint16_t));
    m->replay_rows = rows;
    return 0;
}

int ho_rewind(ho_model *m, int pos) {
    if (pos < 0 || pos > m->pos) return -3;
    m->pos = pos;
    return 0;
}

/* ------------------------------------------------------------ forward (NUMERICS §5) */

static void lin(ho_model *m, int layer, const char *name, const float *x, float *y) {
    const tens *t = find_tensor(m, layer, name);
    matvec(t->dtype, t->data, t->shape[1], x, 1, y, t->shape[0], 0, t->shape[0], m->nthreads);
}

static const float *vec(ho_model *m, int layer, const char *name) {
    const tens *t = find_tensor(m, layer, name);
    return t ? (const float *)t->data : NULL;
}

static void rope(float *x, const ho_model *m, int pos) {
    const cfg *c = &m->c;
    const int half = c->rope_dim / 2;
    for (int j = 0; j < half; j++) {
        const float th = (float)pos * m->inv_freq[j];
        const float cs = o_cosf(th) * c->rope_factor, sn = o_sinf(th) * c->rope_factor;
        const int ia = c->rope_style ? 2 * j : j, ib = c->rope_style ? 2 * j + 1 : j + half;
        const float a = x[ia], b = x[ib];
        x[ia] = a * cs - b * sn;
        x[ib] = b * cs + a * sn;
    }
}

/* Heads [0, H) of one token's attention on up to nthreads threads: fn(ctx, h, scratch)
 * computes head h alone and writes only its own outputs, so the thread count cannot
 * change a result; each thread has its own scratch of `scratch_floats` floats. */
typedef void (*head_fn)(void *ctx, int h, float *scratch);
typedef struct {
    head_fn fn;
    void *ctx;
    int h0, h1;
    size_t scratch_floats;
} head_job;

static void *head_run(void *p) {
    head_job *j = (head_job *)p;
    float *scr = malloc(sizeof(float) * (j->scratch_floats ? j->scratch_floats : 1));
    for (int h = j->h0; h < j->h1; h++) j->fn(j->ctx, h, scr);
    free(scr);
    return NULL;
}

static void par_heads(int H, int nthreads, head_fn fn, void *ctx, size_t scratch_floats) {
    int nt = nthreads < 1 ? 1 : (nthreads > 64 ? 64 : nthreads);
    if (nt > H) nt = H > 0 ? H : 1;
    head_job jobs[64];
    pthread_t th[64];
    for (int i = 0; i < nt; i++) {
        jobs[i].fn = fn; jobs[i].ctx = ctx; jobs[i].scratch_floats = scratch_floats;
        jobs[i].h0 = H * i / nt;
        jobs[i].h1 = H * (i + 1) / nt;
    }
    for (int i = 1; i < nt; i++) pthread_create(&th[i], NULL, head_run, &jobs[i]);
    head_run(&jobs[0]);
    for (int i = 1; i < nt; i++) pthread_join(th[i], NULL);
}

/* o_h = sum_i p_i v_{rows[i]} with each element summed over i in order from 0.0f
 * (model.c:552-575); v row r at base + rows[i] * stride, width n */
static void value_sum(const float *p, const int *rows, int nr, const float *base, size_t stride, int n, float *o) {
    for (int d = 0; d < n; d++) o[d] = 0.0f;
    for (int i = 0; i < nr; i++) {
        const float *v = base + (size_t)rows[i] * stride;
        for (int d = 0; d < n; d++) o[d] = o[d] + p[i] * v[d];
    }
}

typedef struct {
    const cfg *c;
    const float *q, *K, *Vc;
    float *o;
    const int *rows;
    int nr, kd;
} gqa_ctx;

/* the larger of a and b, NaN if either is NaN */
static float nanmax(float a, float b) { return a != a || b != b ? a + b : (b > a ? b : a); }

/* HO_ATTN_CHUNKED for one head (the steps ho_set_attn_mode lists); scratch: sc [nr],
 * oc [n], mc [nc] */
static void chunked_head(const float *q, const int *rows, int nr, const float *K, const float *Vc, size_t stride,
                         int n, float scale, float *sc, float *oc, float *mc, float *out) {
    const int CH = HO_ATTN_CHUNK, nc = (nr + CH - 1) / CH;
    for (int i = 0; i < nr; i++) {
        const float *k = K + (size_t)rows[i] * stride;
        float acc = 0.0f;
        for (int d = 0; d < n; d++) acc = fmaf(q[d], k[d], acc);
        sc[i] = scale * acc;
    }
    float M = 0.0f;
    for (int c = 0; c < nc; c++) {
        const int i0 = c * CH, i1 = i0 + CH < nr ? i0 + CH : nr;
        float m = sc[i0];
        for (int i = i0 + 1; i < i1; i++) m = nanmax(m, sc[i]);
        mc[c] = m;
        M = c ? nanmax(M, m) : m;
    }
    float L = 0.0f;
    for (int d = 0; d < n; d++) out[d] = 0.0f;
    for (int c = 0; c < nc; c++) {
        const int i0 = c * CH, i1 = i0 + CH < nr ? i0 + CH : nr;
        float a[HO_ATTN_CHUNK];
        for (int j = 0; j < CH; j++) a[j] = i0 + j < i1 ? ho_expf(sc[i0 + j] - mc[c]) : 0.0f;
        for (int d = 0; d < n; d++) oc[d] = 0.0f;
        for (int i = i0; i < i1; i++) {
            const float *v = Vc + (size_t)rows[i] * stride;
            for (int d = 0; d < n; d++) oc[d] = fmaf(a[i - i0], v[d], oc[d]);
        }
        for (int w = 1; w < CH; w *= 2)
            for (int k = 0; k < CH; k += 2 * w) a[k] = a[k] + a[k + w];
        const float wc = ho_expf(mc[c] - M);
        L = fmaf(a[0], wc, L);
        for (int d = 0; d < n; d++) out[d] = fmaf(oc[d], wc, out[d]);
    }
    for (int d = 0; d < n; d++) out[d] = out[d] / L;
}

int ho_attn_head(const float *q, const float *K, const float *V, size_t stride, const int32_t *rows, int nr, int n,
                 float scale, float *out) {
    if (!q || !K || !V || !rows || !out || nr < 1 || n < 1) return -1;
    float *sc = malloc(sizeof(float) * ((size_t)nr + (size_t)n + (size_t)nr));
    if (!sc) return -5;
    if (g_attn_mode == HO_ATTN_CHUNKED) {
        chunked_head(q, (const int *)rows, nr, K, V, stride, n, scale, sc, sc + nr, sc + nr + n, out);
    } else {
        for (int i = 0; i < nr; i++) sc[i] = scale * ho_dot16(q, K + (size_t)rows[i] * stride, n);
        softmax(sc, nr);
        value_sum(sc, (const int *)rows, nr, V, stride, n, out);
    }
    free(sc);
    return 0;
}

static void gqa_head(void *p, int h, float *sc) {
    const gqa_ctx *a = (const gqa_ctx *)p;
    const cfg *c = a->c;
    const int hd = c->head_dim, g = h / (c->n_heads / c->n_kv_heads);
    if (g_attn_mode == HO_ATTN_CHUNKED) {
        float *oc = sc + a->nr, *mc = oc + hd;
        chunked_head(a->q + h * hd, a->rows, a->nr, a->K + g * hd, a->Vc + g * hd, (size_t)a->kd, hd, c->attn_scale,
                     sc, oc, mc, a->o + h * hd);
        return;
    }
    for (int i = 0; i < a->nr; i++)
        sc[i] = c->attn_scale * ho_dot16(a->q + h * hd, a->K + (size_t)a->rows[i] * a->kd + g * hd, hd);
    softmax(sc, a->nr);
    value_sum(sc, a->rows, a->nr, a->Vc + g * hd, (size_t)a->kd, hd, a->o + h * hd);
}

/* One token's attention. rows[0..nr) are the cache slots it attends to in order
 * (its causal prefix for a chain; context then ancestors for a tree node); the token's
 * own K/V go to slot `slot` before the scores are computed. */
static void attn_gqa(ho_model *m, int l, const float *x, int pos, int slot, const int *rows, int nr, float *out) {
    const cfg *c = &m->c;
    const int H = c->n_heads, Hkv = c->n_kv_heads, hd = c->head_dim, qd = H * hd, kd = Hkv * hd;
    float *q = malloc(sizeof(float) * qd), *k = malloc(sizeof(float) * kd), *v = malloc(sizeof(float) * kd);
    float *o = malloc(sizeof(float) * qd);
    float *K = m->kv + (size_t)l * m->per_layer, *Vc = K + (size_t)m->cap * kd;
    lin(m, l, "attn_q", x, q);
    lin(m, l, "attn_k", x, k);
    lin(m, l, "attn_v", x, v);
    if (c->qkv_bias) {
        const float *bq = vec(m, l, "attn_q_bias"), *bk = vec(m, l, "attn_k_bias"), *bv = vec(m, l, "attn_v_bias");
        for (int i = 0; i < qd; i++) q[i] = q[i] + bq[i];
        for (int i = 0; i < kd; i++) k[i] = k[i] + bk[i];
        for (int i = 0; i < kd; i++) v[i] = v[i] + bv[i];
    }
    if (c->qk_norm == 1) {
        for (int h = 0; h < H; h++) rmsnorm(q + h * hd, q + h * hd, vec(m, l, "attn_q_norm"), hd, c->eps);
        for (int h = 0; h < Hkv; h++) rmsnorm(k + h * hd, k + h * hd, vec(m, l, "attn_k_norm"), hd, c->eps);
    } else if (c->qk_norm == 2) {
        rmsnorm(q, q, vec(m, l, "attn_q_norm"), qd, c->eps);
        rmsnorm(k, k, vec(m, l, "attn_k_norm"), kd, c->eps);
    }
    if (c->rope_dim / 2) {
        for (int h = 0; h < H; h++) rope(q + h * hd, m, pos);
        for (int h = 0; h < Hkv; h++) rope(k + h * hd, m, pos);
    }
    memcpy(K + (size_t)slot * kd, k, sizeof(float) * kd);
    memcpy(Vc + (size_t)slot * kd, v, sizeof(float) * kd);
    dump(m, "q", l, q, qd, 4);
    gqa_ctx ctx = {c, q, K, Vc, o, rows, nr, kd};
    par_heads(H, m->nthreads, gqa_head, &ctx, (size_t)nr + hd + (size_t)(nr + HO_ATTN_CHUNK - 1) / HO_ATTN_CHUNK);
    dump(m, "att", l, o, qd, 4);
    lin(m, l, "attn_o", o, out);
    free(q); free(k); free(v); free(o);
}

typedef struct {
    ho_model *m;
    const tens *kvb;
    size_t kvb_rb;
    float *q, *o;
    const float *Cc, *Kp;
    const int *rows;
    int nr, pos;
} mla_ctx;

/* head h of the absorbed MLA (model.c:650-737); scratch: ql, ol, wrow [C] then sc [nr] */
static void mla_head(void *p, int h, float *scr) {
    const mla_ctx *a = (const mla_ctx *)p;
    const cfg *c = &a->m->c;
    const int nope = c->nope, rd = c->rope_qk, vd = c->v_head, C = c->kv_lora, qh = nope + rd;
    float *ql = scr, *ol = scr + C, *wrow = scr + 2 * C, *sc = scr + 3 * C;
    float *qn = a->q + h * qh, *qpe = qn + nope;
    if (c->rope_dim / 2) rope(qpe, a->m, a->pos);
    for (int i = 0; i < C; i++) ql[i] = 0.0f;
    for (int n = 0; n < nope; n++) {
        dequant_row(a->kvb->dtype, a->kvb->data + (size_t)(h * (nope + vd) + n) * a->kvb_rb, wrow, C);
        for (int i = 0; i < C; i++) ql[i] = ql[i] + qn[n] * wrow[i];
    }
    for (int i = 0; i < a->nr; i++)
        sc[i] = c->attn_scale * (ho_dot16(ql, a->Cc + (size_t)a->rows[i] * C, C) +
                                 ho_dot16(qpe, a->Kp + (size_t)a->rows[i] * rd, rd));
    softmax(sc, a->nr);
    value_sum(sc, a->rows, a->nr, a->Cc, (size_t)C, C, ol);
    matvec(a->kvb->dtype, a->kvb->data, C, ol, 1, a->o + h * vd, vd, h * (nope + vd) + nope, h * (nope + vd) + nope + vd, 1);
}

static void attn_mla(ho_model *m, int l, const float *x, int pos, int slot, const int *rows, int nr, float *out) {
    const cfg *c = &m->c;
    const int H = c->n_heads, nope = c->nope, rd = c->rope_qk, vd = c->v_head, C = c->kv_lora, qh = nope + rd;
    const tens *kvb = find_tensor(m, l, "attn_kv_b");
    const size_t kvb_rb = ho_row_bytes(kvb->dtype, C);
    float *q = malloc(sizeof(float) * (size_t)H * qh), *kva = malloc(sizeof(float) * (size_t)(C + rd));
    float *o = malloc(sizeof(float) * (size_t)H * vd);
    float *Cc = m->kv + (size_t)l * m->per_layer, *Kp = Cc + (size_t)m->cap * C;
    if (c->q_lora) {
        float *qa = malloc(sizeof(float) * c->q_lora);
        lin(m, l, "attn_q_a", x, qa);
        rmsnorm(qa, qa, vec(m, l, "attn_q_a_norm"), c->q_lora, c->eps);
        lin(m, l, "attn_q_b", qa, q);
        free(qa);
    } else {
        lin(m, l, "attn_q", x, q);
    }
    lin(m, l, "attn_kv_a", x, kva);
    rmsnorm(Cc + (size_t)slot * C, kva, vec(m, l, "attn_kv_a_norm"), C, c->eps);
    memcpy(Kp + (size_t)slot * rd, kva + C, sizeof(float) * rd);
    if (c->rope_dim / 2) rope(Kp + (size_t)slot * rd, m, pos);
    mla_ctx ctx = {m, kvb, kvb_rb, q, o, Cc, Kp, rows, nr, pos};
    par_heads(H, m->nthreads, mla_head, &ctx, (size_t)3 * C + (size_t)nr);
    lin(m, l, "attn_o", o, out);
    free(q); free(kva); free(o);
}

static void ffn(ho_model *m, int l, const char *g, const char *u, const char *d, const float *x, float *out) {
    const tens *tg = find_tensor(m, l, g);
    const int64_t F = tg->shape[0];
    float *a = malloc(sizeof(float) * F), *b = malloc(sizeof(float) * F);
    lin(m, l, g, x, a);
    lin(m, l, u, x, b);
    for (int64_t i = 0; i < F; i++) a[i] = (a[i] / (1.0f + ho_expf(-a[i]))) * b[i];
    lin(m, l, d, a, out);
    free(a);
    free(b);
}

static uint64_t slab_layout(int dt, int64_t D, int64_t F, uint64_t *og, uint64_t *ou, uint64_t *od) {
    const uint64_t rd = ho_row_bytes(dt, D), rf = ho_row_bytes(dt, F);
    *og = 0;
    *ou = ((uint64_t)F * rd + 63) / 64 * 64;
    *od = (*ou + (uint64_t)F * rd + 63) / 64 * 64;
    return (*od + (uint64_t)D * rf + 4095) / 4096 * 4096;
}

static void expert(ho_model *m, int l, int e, const float *x, float *out) {
    const cfg *c = &m->c;
    const expent *ent = &m->ex[(size_t)l * c->n_experts + e];
    const int D = c->d_model, F = c->expert_ffn, dt = (int)ent->dtype;
    uint64_t og, ou, od;
    const uint8_t *slab = m->map + ent->off;
    float *a = malloc(sizeof(float) * F), *b = malloc(sizeof(float) * F);
    slab_layout(dt, D, F, &og, &ou, &od);
    matvec(dt, slab + og, D, x, 1, a, F, 0, F, m->nthreads);
    matvec(dt, slab + ou, D, x, 1, b, F, 0, F, m->nthreads);
    for (int i = 0; i < F; i++) a[i] = (a[i] / (1.0f + ho_expf(-a[i]))) * b[i];
    matvec(dt, slab + od, F, a, 1, out, D, 0, D, m->nthreads);
    free(a);
    free(b);
}

/* a ranks before b: larger first, NaN last, ties to the lower index (model.c:220-226). */
static int ranks_before(float va, int ia, float vb, int ib) {
    const int na = va != va, nb = vb != vb;
    if (na || nb) return na == nb ? ia < ib : nb;
    if (va != vb) return va > vb;
    return ia < ib;
}

/* NUMERICS §5.3 routing: ids[0..K) and weights w[0..K). */
static void route(ho_model *m, int l, const float *x, int *ids, float *w) {
    const cfg *c = &m->c;
    const int E = c->n_experts, K = c->top_k;
    float *score = malloc(sizeof(float) * E), *sel = malloc(sizeof(float) * E);
    uint8_t *taken = calloc((size_t)E, 1);
    lin(m, l, "moe_router", x, score);
    dump(m, "router", l, score, E, 4);
    if (c->score_fn == 0) softmax(score, E);
    else for (int e = 0; e < E; e++) score[e] = sigmoidf_(score[e]);
    if (m->replay) {
        /* route replay (model.c:1004-1012): the experts of the trace row of this token's
         * position, weights from the router's scores */
        const uint16_t *row = m->replay + (size_t)(m->cur_pos % m->replay_rows) * (size_t)(c->n_moe * K) +
                              (size_t)m->moe_ord[l] * K;
        for (int j = 0; j < K; j++) ids[j] = row[j];
        goto weights;
    }
    const float *bias = c->score_bias ? vec(m, l, "moe_router_bias") : NULL;
    for (int e = 0; e < E; e++) sel[e] = bias ? score[e] + bias[e] : score[e];
    if (c->n_group > 1) {
        const int ng = c->n_group, gs = E / ng;
        float *gsc = malloc(sizeof(float) * ng);
        uint8_t *keep = calloc((size_t)ng, 1);
        for (int g = 0; g < ng; g++) {
            const float *v = sel + (size_t)g * gs;
            int i1 = 0, i2 = -1;
            for (int i = 1; i < gs; i++) {
                if (ranks_before(v[i], i, v[i1], i1)) { i2 = i1; i1 = i; }
                else if (i2 < 0 || ranks_before(v[i], i, v[i2], i2)) i2 = i;
            }
            gsc[g] = i2 >= 0 ? v[i1] + v[i2] : v[i1];
        }
        for (int r = 0; r < c->topk_group; r++) {
            int best = -1;
            for (int g = 0; g < ng; g++)
                if (!keep[g] && (best < 0 || ranks_before(gsc[g], g, gsc[best], best))) best = g;
            keep[best] = 1;
        }
        for (int g = 0; g < ng; g++)
            if (!keep[g]) for (int i = 0; i < gs; i++) sel[(size_t)g * gs + i] = 0.0f;
        free(gsc);
        free(keep);
    }
    for (int j = 0; j < K; j++) {
        int best = -1;
        for (int e = 0; e < E; e++)
            if (!taken[e] && (best < 0 || ranks_before(sel[e], e, sel[best], best))) best = e;
        ids[j] = best;
        taken[best] = 1;
    }
    if (m->cur_margin) {
        /* the smallest gap between consecutive selection scores among the top K + 1, relative
         * to the larger one for softmax scoring, absolute for sigmoid scoring */
        const int n = K + 1 < E ? K + 1 : E;
        float prev = sel[ids[0]], g = 1e30f;
        for (int j = 1; j < n; j++) {
            float v;
            if (j < K) {
                v = sel[ids[j]];
            } else {
                int best = -1;
                for (int e = 0; e < E; e++)
                    if (!taken[e] && (best < 0 || ranks_before(sel[e], e, sel[best], best))) best = e;
                v = sel[best];
            }
            const double gap = (double)prev - (double)v;
            const double r = c->score_fn == 0 ? gap / (prev > 1e-30f ? prev : 1e-30f) : gap;
            if (r < g) g = (float)r;
            prev = v;
        }
        *m->cur_margin = g;
    }
weights:
    for (int j = 0; j < K; j++) w[j] = score[ids[j]];
    if (c->norm_topk) {
        float s = 0.0f;
        for (int j = 0; j < K; j++) s = s + w[j];
        const float den = s + 1e-20f;
        for (int j = 0; j < K; j++) w[j] = w[j] / den;
    }
    for (int j = 0; j < K; j++) w[j] = w[j] * c->routed_scale;
    free(score);
    free(sel);
    free(taken);
}

static void moe(ho_model *m, int l, const float *x, float *out, int32_t *route_out) {
    const cfg *c = &m->c;
    const int K = c->top_k, D = c->d_model;
    int *ids = malloc(sizeof(int) * K);
    float *w = malloc(sizeof(float) * K), *y = malloc(sizeof(float) * D);
    route(m, l, x, ids, w);
    dump(m, "ids", l, ids, K, 4);
    if (route_out) for (int j = 0; j < K; j++) route_out[j] = ids[j];
    for (int i = 0; i < D; i++) out[i] = 0.0f;
    for (int j = 0; j < K; j++) {
        expert(m, l, ids[j], x, y);
        for (int i = 0; i < D; i++) out[i] = out[i] + w[j] * y[i];
    }
    if (c->shared_ffn) {
        ffn(m, l, "shexp_gate", "shexp_up", "shexp_down", x, y);
        if (c->shared_gate) {
            const float g = sigmoidf_(ho_dot16(vec(m, l, "shexp_gate_inp"), x, D));
            for (int i = 0; i < D; i++) y[i] = y[i] * g;
        }
        for (int i = 0; i < D; i++) out[i] = out[i] + y[i];
    }
    free(ids);
    free(w);
    free(y);
}

static void forward_token(ho_model *m, int tok, int pos, int slot, const int *rows, int nr, float *logits, int32_t *routes,
                          float *margins) {
    m->cur_pos = pos;
    const cfg *c = &m->c;
    const int D = c->d_model;
    const tens *emb = find_tensor(m, -1, "tok_embd"), *head = c->tie ? emb : find_tensor(m, -1, "lm_head");
    float *h = malloc(sizeof(float) * D), *x = malloc(sizeof(float) * D), *a = malloc(sizeof(float) * D);
    dequant_row(emb->dtype, emb->data + (size_t)tok * ho_row_bytes(emb->dtype, D), h, D);
    for (int i = 0; i < D; i++) h[i] = c->emb_scale * h[i];
    for (int l = 0; l < c->n_layers; l++) {
        rmsnorm(x, h, vec(m, l, "attn_norm"), D, c->eps);
        if (c->attn_kind == 1) attn_mla(m, l, x, pos, slot, rows, nr, a);
        else attn_gqa(m, l, x, pos, slot, rows, nr, a);
        for (int i = 0; i < D; i++) h[i] = h[i] + c->resid_scale * a[i];
        rmsnorm(x, h, vec(m, l, "ffn_norm"), D, c->eps);
        dump(m, "h_mid", l, h, D, 4);
        dump(m, "x_ffn", l, x, D, 4);
        m->cur_margin = margins && c->layer_kind[l] ? margins + m->moe_ord[l] : NULL;
        if (c->layer_kind[l]) moe(m, l, x, a, routes ? routes + (size_t)m->moe_ord[l] * c->top_k : NULL);
        else ffn(m, l, "ffn_gate", "ffn_up", "ffn_down", x, a);
        m->cur_margin = NULL;
        for (int i = 0; i < D; i++) h[i] = h[i] + c->resid_scale * a[i];
        dump(m, "h", l, h, D, 4);
    }
    if (logits) {
        rmsnorm(x, h, vec(m, -1, "out_norm"), D, c->eps);
        matvec(head->dtype, head->data, D, x, 1, logits, c->vocab, 0, c->vocab, m->nthreads);
        for (int i = 0; i < c->vocab; i++) logits[i] = c->logit_scale * logits[i];
    }
    free(h);
    free(x);
    free(a);
}

void ho_set_margins(ho_model *m, float *buf) { m->margins = buf; }

int ho_eval(ho_model *m, const int32_t *tokens, int n, float *logits, int32_t *routes) {
    const cfg *c = &m->c;
    if (n < 0 || !tokens) return -1;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c->vocab) return -2;
    if ((int64_t)m->pos + n > m->cap) return -3;
    int *rows = malloc(sizeof(int) * (size_t)(m->pos + n));
    for (int i = 0; i < m->pos + n; i++) rows[i] = i;
    for (int i = 0; i < n; i++) {
        const int p = m->pos + i;
        forward_token(m, tokens[i], p, p, rows, p + 1, logits ? logits + (size_t)i * c->vocab : NULL,
                      routes ? routes + (size_t)i * c->n_moe * c->top_k : NULL,
                      m->margins ? m->margins + (size_t)i * c->n_moe : NULL);
    }
    m->margins = NULL;
    m->pos += n;
    free(rows);
    return 0;
}

int ho_eval_tree(ho_model *m, const int32_t *tokens, const int32_t *parent, int n, float *logits, int32_t *routes) {
    const cfg *c = &m->c;
    const int pos0 = m->pos;
    if (n < 0 || !tokens || !parent) return -1;
    for (int i = 0; i < n; i++) {
        if (tokens[i] < 0 || tokens[i] >= c->vocab) return -2;
        if ((i == 0 && parent[i] != -1) || (i > 0 && (parent[i] < 0 || parent[i] >= i))) return -1;
    }
    if ((int64_t)pos0 + n > m->cap) return -3;
    int *depth = malloc(sizeof(int) * (size_t)(n ? n : 1));
    int *rows = malloc(sizeof(int) * (size_t)(pos0 + n + 1));
    for (int i = 0; i < n; i++) depth[i] = i == 0 ? 0 : depth[parent[i]] + 1;
    for (int i = 0; i < n; i++) {
        const int d = depth[i];
        for (int r = 0; r < pos0; r++) rows[r] = r;
        for (int v = i, j = d; v >= 0; v = parent[v], j--) rows[pos0 + j] = pos0 + v;
        forward_token(m, tokens[i], pos0 + d, pos0 + i, rows, pos0 + d + 1,
                      logits ? logits + (size_t)i * c->vocab : NULL,
                      routes ? routes + (size_t)i * c->n_moe * c->top_k : NULL,
                      m->margins ? m->margins + (size_t)i * c->n_moe : NULL);
    }
    m->margins = NULL;
    free(depth);
    free(rows);
    return 0;
}

int ho_commit_path(ho_model *m, const int32_t *path, int n) {
    const cfg *c = &m->c;
    if (n < 0 || (int64_t)m->pos + n > m->cap) return -3;
    for (int j = 0; j < n; j++) {
        if (path[j] < j) return -1;
        if (path[j] == j) continue;
        for (int l = 0; l < c->n_layers; l++) {
            float *base = m->kv + (size_t)l * m->per_layer;
            if (c->attn_kind == 1) {
                const int C = c->kv_lora, r = c->rope_qk;
                memmove(base + (size_t)(m->pos + j) * C, base + (size_t)(m->pos + path[j]) * C, sizeof(float) * C);
                float *kp = base + (size_t)m->cap * C;
                memmove(kp + (size_t)(m->pos + j) * r, kp + (size_t)(m->pos + path[j]) * r, sizeof(float) * r);
            } else {
                const int kd = c->n_kv_heads * c->head_dim;
                float *V = base + (size_t)m->cap * kd;
                memmove(base + (size_t)(m->pos + j) * kd, base + (size_t)(m->pos + path[j]) * kd, sizeof(float) * kd);
                memmove(V + (size_t)(m->pos + j) * kd, V + (size_t)(m->pos + path[j]) * kd, sizeof(float) * kd);
            }
        }
    }
    m->pos += n;
    return 0;
}

/* KV snapshot of positions [0, n), every layer in turn: GQA K [Hkv][n][hd] then
 * V [Hkv][n][hd]; MLA latent c [n][C] then rotated k_pe [n][rope]. The same layout as
 * the reference engine's per-layer cache arrays restricted to n positions (model.c
 * keeps [Hkv][cap][hd] per K and V). Test infrastructure: lets a check start from a
 * context another implementation computed. */
int64_t ho_kv_row_floats(const ho_model *m) {
    const cfg *c = &m->c;
    return c->attn_kind == 1 ? (int64_t)c->kv_lora + c->rope_qk : 2 * (int64_t)c->n_kv_heads * c->head_dim;
}

static int kv_copy(ho_model *m, int n, float *ext, int to_ext) {
    const cfg *c = &m->c;
    if (n < 0 || n > m->cap || !ext) return -1;
    const int64_t W = ho_kv_row_floats(m);
    for (int l = 0; l < c->n_layers; l++) {
        float *base = m->kv + (size_t)l * m->per_layer, *e = ext + (size_t)l * (size_t)n * (size_t)W;
        if (c->attn_kind == 1) {
            const int C = c->kv_lora, r = c->rope_qk;
            float *kp = base + (size_t)m->cap * C;
            if (to_ext) {
                memcpy(e, base, sizeof(float) * (size_t)n * C);
                memcpy(e + (size_t)n * C, kp, sizeof(float) * (size_t)n * r);
            } else {
                memcpy(base, e, sizeof(float) * (size_t)n * C);
                memcpy(kp, e + (size_t)n * C, sizeof(float) * (size_t)n * r);
            }
            continue;
        }
        const int Hkv = c->n_kv_heads, hd = c->head_dim, kd = Hkv * hd;
        for (int kvi = 0; kvi < 2; kvi++) {
            float *cache = base + (size_t)kvi * m->cap * kd;
            for (int g = 0; g < Hkv; g++)
                for (int r = 0; r < n; r++) {
                    float *in = cache + (size_t)r * kd + (size_t)g * hd;
                    float *ex = e + (((size_t)kvi * Hkv + g) * n + r) * hd;
                    if (to_ext) memcpy(ex, in, sizeof(float) * hd);
                    else memcpy(in, ex, sizeof(float) * hd);
                }
        }
    }
    return 0;
}

int ho_kv_export(const ho_model *m, int n, float *dst) {
    if (n > m->pos) return -1;
    return kv_copy((ho_model *)m, n, dst, 1);
}

int ho_kv_import(ho_model *m, int n, const float *src) {
    const int rc = kv_copy(m, n, (float *)src, 0);
    if (rc == 0) m->pos = n;
    return rc;
}

/* ------------------------------------------------------------ acceptance (generate.py) */

/* numpy's pairwise summation of one contiguous run: 8 accumulators over blocks of at
 * most 128, halves split at multiples of 8. */
static double np_pairwise(const double *a, int64_t n) {
    if (n < 8) {
        double r = 0.0;
        for (int64_t i = 0; i < n; i++) r = r + a[i];
        return r;
    }
    if (n <= 128) {
        double r[8], res;
        int64_t i;
        for (int j = 0; j < 8; j++) r[j] = a[j];
        for (i = 8; i < n - (n % 8); i += 8)
            for (int j = 0; j < 8; j++) r[j] = r[j] + a[i + j];
        res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < n; i++) res = res + a[i];
        return res;
    }
    int64_t n2 = n / 2;
    n2 -= n2 % 8;
    return np_pairwise(a, n2) + np_pairwise(a + n2, n - n2);
}

/* numpy float64 add.reduce over a contiguous array: the reduction runs over buffers of
 * 8192 elements (numpy's default buffer size), each summed pairwise and added in order
 * to the accumulator, which starts at the identity 0.0. */
double ho_np_sum(const double *a, int64_t n) {
    double s = 0.0;
    for (int64_t i = 0; i < n; i += 8192) s = s + np_pairwise(a + i, n - i < 8192 ? n - i : 8192);
    return s;
}
#define np_sum ho_np_sum

static int bad_logits(const float *x, int V) {
    int all_neg_inf = 1;
    for (int i = 0; i < V; i++) {
        if (x[i] != x[i] || (x[i] == 1.0f / 0.0f)) return 1;
        if (x[i] != -1.0f / 0.0f) all_neg_inf = 0;
    }
    return all_neg_inf;
}

int ho_argmax(const float *x, int V) {
    if (V < 1 || bad_logits(x, V)) return -1;
    int best = 0;
    for (int i = 1; i < V; i++)
        if (x[i] > x[best]) best = i;
    return best;
}

/* descending by value, ascending index on ties (np.argsort(-p, kind="stable")) */
static const double *g_sort_key;
static int cmp_desc(const void *a, const void *b) {
    const int i = *(const int *)a, j = *(const int *)b;
    const double x = g_sort_key[i], y = g_sort_key[j];
    if (x != y) return x > y ? -1 : 1;
    return i < j ? -1 : (i > j);
}

static int cmp_dbl(const void *a, const void *b) {
    const double x = *(const double *)a, y = *(const double *)b;
    return x < y ? -1 : (x > y);
}

/* Sampler._penalised (generate.py:68-79) once the row has passed the logits check:
 * the row as float64, and each distinct id in [0, V) of the context (s->context plus
 * extra) divided by the penalty where positive, multiplied by it otherwise. */
static void penalised(const float *logits, int V, const ho_sampler *s, const int32_t *extra, int n_extra, double *x) {
    for (int i = 0; i < V; i++) x[i] = (double)logits[i];
    const double rp = s->repetition_penalty;
    if (rp == 1.0 || (s->n_context <= 0 && n_extra <= 0)) return;
    uint8_t *mark = calloc((size_t)V, 1);
    for (int j = 0; j < s->n_context; j++)
        if (s->context[j] >= 0 && s->context[j] < V) mark[s->context[j]] = 1;
    for (int j = 0; j < n_extra; j++)
        if (extra[j] >= 0 && extra[j] < V) mark[extra[j]] = 1;
    for (int i = 0; i < V; i++)
        if (mark[i]) x[i] = x[i] > 0.0 ? x[i] / rp : x[i] * rp;
    free(mark);
}

/* Sampler.probs (generate.py:84-111) with the penalty context s->context + extra. */
static int probs_core(const float *logits, int V, const ho_sampler *sp, const int32_t *extra, int n_extra, double *p) {
    if (V < 1 || bad_logits(logits, V)) return -1;
    penalised(logits, V, sp, extra, n_extra, p);
    const double T = sp->temperature;
    if (T == 0.0) {
        int best = 0;
        for (int i = 1; i < V; i++)
            if (p[i] > p[best]) best = i;
        for (int i = 0; i < V; i++) p[i] = 0.0;
        p[best] = 1.0;
        return 0;
    }
    double mx = p[0];
    for (int i = 1; i < V; i++) mx = p[i] > mx ? p[i] : mx;
    for (int i = 0; i < V; i++) p[i] = (p[i] - mx) / T;
    if (sp->top_k > 0 && sp->top_k < V) {
        double *tmp = malloc(sizeof(double) * V);
        memcpy(tmp, p, sizeof(double) * V);
        qsort(tmp, (size_t)V, sizeof(double), cmp_dbl);
        const double kth = tmp[V - sp->top_k];
        for (int i = 0; i < V; i++)
            if (p[i] < kth) p[i] = -1.0 / 0.0;
        free(tmp);
    }
    for (int i = 0; i < V; i++) p[i] = ho_exp_port_d(p[i]);
    double s = np_sum(p, V);
    for (int i = 0; i < V; i++) p[i] = p[i] / s;
    if (sp->top_p < 1.0) {
        int *order = malloc(sizeof(int) * V);
        for (int i = 0; i < V; i++) order[i] = i;
        g_sort_key = p;
        qsort(order, (size_t)V, sizeof(int), cmp_desc);
        double c = 0.0;
        uint8_t *drop = calloc((size_t)V, 1);
        for (int j = 0; j < V; j++) {
            const double ps = p[order[j]];
            c = c + ps;
            const double before = c - ps;
            if (before >= sp->top_p) drop[order[j]] = 1;
        }
        for (int i = 0; i < V; i++)
            if (drop[i]) p[i] = 0.0;
        s = np_sum(p, V);
        for (int i = 0; i < V; i++) p[i] = p[i] / s;
        free(order);
        free(drop);
    }
    if (sp->min_p > 0.0) {
        double mp = p[0];
        for (int i = 1; i < V; i++) mp = p[i] > mp ? p[i] : mp;
        const double thr = sp->min_p * mp;
        for (int i = 0; i < V; i++)
            if (p[i] < thr) p[i] = 0.0;
        s = np_sum(p, V);
        for (int i = 0; i < V; i++) p[i] = p[i] / s;
    }
    return 0;
}

int ho_probs(const float *logits, int V, double T, int top_k, double top_p, double min_p, double *p) {
    const ho_sampler s = {T, top_k, top_p, min_p, 1.0, NULL, 0};
    return probs_core(logits, V, &s, NULL, 0, p);
}

int ho_probs_s(const float *logits, int V, const ho_sampler *s, const int32_t *extra, int n_extra, double *p) {
    return probs_core(logits, V, s, extra, n_extra, p);
}

/* first i with c[i] > u (np.searchsorted side="right"), clamped, stepped back over
 * zero mass (generate.py:113-121) */
static int draw_scaled(const double *w, int V, double u) {
    double c = 0.0, last = 0.0;
    for (int i = 0; i < V; i++) last = last + w[i];
    const double target = u * last;
    int idx = V;
    for (int i = 0; i < V; i++) {
        c = c + w[i];
        if (c > target) { idx = i; break; }
    }
    if (idx > V - 1) idx = V - 1;
    while (w[idx] <= 0.0 && idx > 0) idx--;
    return idx;
}

int ho_draw(const double *p, int V, double u) { return draw_scaled(p, V, u); }

int ho_accept_general(const double *p, const double *q, int V, int d, double u0, double u1, int *tok) {
    const double ratio = p[d] / q[d];
    if (u0 < ratio) { *tok = d; return 1; }
    double *r = malloc(sizeof(double) * V);
    for (int i = 0; i < V; i++) { const double v = p[i] - q[i]; r[i] = v > 0.0 ? v : 0.0; }
    const double s = np_sum(r, V);
    if (s <= 0.0) { free(r); *tok = d; return 1; }
    *tok = draw_scaled(r, V, u1);
    free(r);
    return 0;
}

int ho_accept_point_mass(const double *p, int V, int d, double u0, double u1, int *tok) {
    if (u0 < p[d]) { *tok = d; return 1; }
    double *r = malloc(sizeof(double) * V);
    memcpy(r, p, sizeof(double) * V);
    r[d] = 0.0;
    const double s = np_sum(r, V);
    if (s <= 0.0) { free(r); *tok = d; return 1; }
    *tok = draw_scaled(r, V, u1);
    free(r);
    return 0;
}

/* Tree acceptance; see the header. The residual after a rejected child is kept
 * unnormalised (r) with its float64 sum s, so that for one child per node every step
 * is exactly generate.py's accept_point_mass; a following sibling is accepted with
 * probability (r[x] / s) / q[x]. The penalty context of node v is sp->context plus the
 * tokens of the path nodes 1..v (generate.py:380: full[:len(seq) + i]). */
static int accept_tree_core(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent, int mode,
                            const ho_sampler *sp, const double *q, const double *u, int32_t *path, int *n_path,
                            int *final_tok) {
    int v = 0, np_ = 0, rc = 0;
    double *p = malloc(sizeof(double) * V), *r = malloc(sizeof(double) * V), *qq = malloc(sizeof(double) * V);
    int32_t *extra = malloc(sizeof(int32_t) * (n > 0 ? n : 1));
    path[np_++] = 0;
    for (;;) {
        const float *row = rows + (size_t)v * V;
        int next = -1;
        for (int j = 1; j < np_; j++) extra[j - 1] = tokens[path[j]];
        if (mode == 0) {
            if (V < 1 || bad_logits(row, V)) { rc = -1; break; }
            penalised(row, V, sp, extra, np_ - 1, p);
            int t = 0;
            for (int i = 1; i < V; i++)
                if (p[i] > p[t]) t = i;
            for (int c = v + 1; c < n; c++)
                if (parent[c] == v && tokens[c] == t) { next = c; break; }
            if (next < 0) { *final_tok = t; break; }
        } else {
            if (probs_core(row, V, sp, extra, np_ - 1, p) != 0) { rc = -1; break; }
            double s = -1.0;   /* < 0: p itself is the current distribution */
            int done = 0;
            for (int c = v + 1; c < n && !done; c++) {
                if (parent[c] != v) continue;
                const int x = tokens[c];
                const double *qc = NULL;
                if (mode == 1) {
                    for (int i = 0; i < V; i++) qq[i] = 0.0;
                    qq[x] = 1.0;
                    qc = qq;
                } else {
                    qc = q + (size_t)v * V;
                }
                const double px = s < 0.0 ? p[x] : r[x] / s;
                const double ratio = px / qc[x];
                if (u[2 * c] < ratio) { next = c; done = 1; break; }
                /* residual max(0, p_cur - q) */
                for (int i = 0; i < V; i++) {
                    const double pc = s < 0.0 ? p[i] : r[i] / s;
                    const double d = pc - qc[i];
                    qq[i] = d > 0.0 ? d : 0.0;   /* qq no longer needed for this child */
                }
                const double ns = np_sum(qq, V);
                if (ns <= 0.0) { next = c; done = 1; break; }
                memcpy(r, qq, sizeof(double) * V);
                s = ns;
            }
            if (next < 0) {
                *final_tok = draw_scaled(s < 0.0 ? p : r, V, u[2 * v + 1]);
                break;
            }
        }
        path[np_++] = next;
        v = next;
    }
    *n_path = np_;
    free(p); free(r); free(qq); free(extra);
    return rc;
}

int ho_accept_tree(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                   int mode, double T, int top_k, double top_p, double min_p,
                   const double *q, const double *u, int32_t *path, int *n_path, int *final_tok) {
    const ho_sampler s = {T, top_k, top_p, min_p, 1.0, NULL, 0};
    return accept_tree_core(rows, n, V, tokens, parent, mode, &s, q, u, path, n_path, final_tok);
}

int ho_accept_tree_s(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                     const ho_sampler *s, const double *q, const double *u, int32_t *path, int *n_path,
                     int *final_tok) {
    return accept_tree_core(rows, n, V, tokens, parent, q ? 2 : 1, s, q, u, path, n_path, final_tok);
}

int ho_accept_chain(const float *rows, int k, int V, const int32_t *drafts, int mode,
                    double T, int top_k, double top_p, double min_p,
                    const double *q, const double *u, int *n_acc, int *final_tok) {
    const int n = k + 1;
    int32_t *tok = malloc(sizeof(int32_t) * n), *par = malloc(sizeof(int32_t) * n), *path = malloc(sizeof(int32_t) * n);
    int np_ = 0, rc;
    tok[0] = 0;
    par[0] = -1;
    for (int i = 1; i < n; i++) { tok[i] = drafts[i - 1]; par[i] = i - 1; }
    rc = ho_accept_tree(rows, n, V, tok, par, mode, T, top_k, top_p, min_p, q, u, path, &np_, final_tok);
    *n_acc = np_ - 1;
    free(tok); free(par); free(path);
    return rc;
}
