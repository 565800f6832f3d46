/*
 * hx_device.h — device data layouts and canonical arithmetic shared by the HIP
 * kernels of the MI355X verify engine (gfx950).
 *
 * Numerics follow the reference's docs/NUMERICS.md exactly: int8 x int8 block sums
 * are exact int32 (here from v_mfma_i32_16x16x64_i8, one 64-block per K step), the
 * f32 fold over blocks is acc = acc + (float)isum * (dw * dx) in block order with no
 * FMA (all sources are built with -ffp-contract=off and the fold uses explicit
 * round-to-nearest intrinsics), dot16/sum16 use 16 lanes then the 8/4/2/1 tree, and
 * NaN outputs are stored as 0x7fc00000. The only libm-dependent step, expf, is
 * exp_glibc_f, the platform libm's expf restated bit for bit (so results equal the
 * reference engine's on its glibc platform); RoPE cos/sin come from the host (libm), as
 * in the reference (engine/src/model.c:386-397). exp_port_d (double) serves the
 * float64 sampler.
 *
 * HBM layouts
 *   QMat (Q8/Q4 matrix, rows x cols, nb = cols/64 blocks, nbp = nb rounded up to even):
 *     w: 1 KiB tiles. Q8: tile (rt, g) = 16 rows x block g; Q4: tile (rt, gp) = 16 rows
 *        x blocks 2gp, 2gp+1. Lane l of a wave reads the 16 bytes at l*16 of a tile:
 *        row rt*16 + l%16, k-group kg = l/16. Q8: bytes b of lane l = element
 *        kperm(kg, b) of block g. Q4: bytes 0-7 = bytes 8kg..8kg+7 of block 2gp (their
 *        low nibbles are elements 8kg.., high nibbles 32+8kg..), bytes 8-15 the same of
 *        block 2gp+1. Rows are padded to a multiple of 16 with zero weights.
 *     d: binary16 scales, [nbp][rows_pad] (scale of row r, block g at g*rows_pad + r).
 *   Act (activation blocks of T vectors, NUMERICS §2): q int8 [T][nbp][64] in kperm
 *     order, d f32 [T][nbp], s int32 [T][nbp] (sum of the 64 q).
 *   kperm(kg, b) = b < 8 ? 8kg + b : 32 + 8kg + (b - 8): the k order of one MFMA step;
 *     weights and activations use the same order, so the int32 sum is the block's.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace hxd {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t CANON_NAN = 0x7fc00000u;

struct QMat {
    const uint8_t *w;
    const uint16_t *d;
    int dtype;        /* 3 = Q8, 4 = Q4 */
    int rows, rows_pad, nb, nbp;
};

struct Act {
    int8_t *q;
    float *d;
    int32_t *s;
    int nbp;
};

/* ---- read-ahead (device) ---- */

/* One byte of every 128-byte line of p[0, n) that falls to this thread: lines
 * part * blockDim.x + threadIdx.x + k * nparts * blockDim.x. Extra workgroups of a
 * latency-bound kernel use it to bring the weights of a later product into the
 * memory-side cache; the empty asm keeps each load, four of them in flight at once. */
__device__ __forceinline__ void read_lines_ahead(const uint8_t *p, size_t n, int part, int nparts) {
    const size_t step = (size_t)nparts * blockDim.x * 128;
    size_t o = ((size_t)part * blockDim.x + threadIdx.x) * 128;
    for (; o + 3 * step < n; o += 4 * step) {
        const unsigned x0 = p[o], x1 = p[o + step], x2 = p[o + 2 * step], x3 = p[o + 3 * step];
        asm volatile("" ::"v"(x0), "v"(x1), "v"(x2), "v"(x3));
    }
    for (; o < n; o += step) {
        const unsigned x = p[o];
        asm volatile("" ::"v"(x));
    }
}

/* bytes of a tile-repacked matrix: its weights and its scale rows */
__device__ __host__ __forceinline__ size_t qmat_w_bytes(const QMat &m) {
    return (size_t)(m.rows_pad / 16) * m.nbp * 1024 / (m.dtype == 4 ? 2 : 1);
}
__device__ __host__ __forceinline__ size_t qmat_d_bytes(const QMat &m) {
    return sizeof(uint16_t) * (size_t)m.nbp * m.rows_pad;
}

/* ---- canonical scalar helpers (device) ---- */

__device__ __forceinline__ float fadd(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float fmul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float fsub(float a, float b) { return __fsub_rn(a, b); }
__device__ __forceinline__ float fdiv(float a, float b) { return __fdiv_rn(a, b); }
__device__ __forceinline__ double dadd(double a, double b) { return __dadd_rn(a, b); }
__device__ __forceinline__ double dmul(double a, double b) { return __dmul_rn(a, b); }
__device__ __forceinline__ double dsub(double a, double b) { return __dsub_rn(a, b); }

__device__ __forceinline__ float canon(float v) { return v != v ? __uint_as_float(CANON_NAN) : v; }

/* IEEE square root (round to nearest) of a positive finite float, whatever the
 * compiler's sqrt lowering: the hardware estimate y (within one ulp) is corrected by
 * comparing s with the squares of the midpoints to its neighbours, computed exactly in
 * double (a 25-bit midpoint squares to at most 50 bits; s is never exactly such a
 * square). NUMERICS §4 needs the correctly rounded sqrtf of the reference. */
__device__ inline float sqrt_rn(float s) {
    if (!(s > 0.0f) || s == __builtin_huge_valf()) return __builtin_sqrtf(s);
    float y = __builtin_amdgcn_sqrtf(s);
    const double sd = (double)s;
    for (int it = 0; it < 2; it++) {
        const float yl = __uint_as_float(__float_as_uint(y) - 1u), yh = __uint_as_float(__float_as_uint(y) + 1u);
        const double mlo = ((double)yl + (double)y) * 0.5, mhi = ((double)y + (double)yh) * 0.5;
        if (sd < mlo * mlo) y = yl;
        else if (sd > mhi * mhi) y = yh;
        else break;
    }
    return y;
}

/* binary16 -> binary32 (exact) */
__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 x;
    __builtin_memcpy(&x, &h, 2);
    return (float)x;
}

/* ---- memory helpers (device) ---- */

/* s_waitcnt with vmcnt = n and the other counters unconstrained (gfx9 encoding) */
#define HX_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

/* LDS-direct load: lane l copies SZ (4 or 16) bytes from its src to dst + l * SZ, with
 * no register in between; counted by vmcnt like any other load */
template <int SZ>
__device__ __forceinline__ void lds_direct(const void *src, void *dst) {
    static_assert(SZ == 4 || SZ == 16, "LDS-direct loads of 4 or 16 bytes");
    if constexpr (SZ == 16)
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                         (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
    else
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                         (__attribute__((address_space(3))) void *)dst, 4, 0, 0);
}

/* 16-byte load from global memory (explicit address space: a global_load, never flat) */
template <typename V>
__device__ __forceinline__ V gload(const void *p) {
    return *(const __attribute__((address_space(1))) V *)p;
}

/* exp in IEEE double from basic operations (Cody & Waite 1980 reduction with a
 * 32-bit ln2 head, degree-13 Taylor series on |r| <= ln2/2, exact power-of-two
 * scaling); the CPU restatement's ho_exp_port_d is the same function.
 * Written without branches (NaN, overflow and underflow are selected at the end, the
 * arithmetic runs on 0 for them), so that independent calls interleave. */
__device__ inline double exp_port_d(double x) {
    const double inv_ln2 = 1.44269504088896338700e+00;
    const double ln2_hi = 6.93147180369123816490e-01;
    const double ln2_lo = 1.90821492927058770002e-10;
    const double shifter = 6755399441055744.0;
    const bool nan = x != x, hi = x > 709.79, lo = x < -745.2;
    const double xs = nan || hi || lo ? 0.0 : x;
    const double t = dmul(xs, inv_ln2);
    const double nd = dsub(dadd(t, shifter), shifter);
    const int n = (int)nd;   /* |n| <= 1076 for the inputs that reach here */
    const double r = dsub(dsub(xs, dmul(nd, ln2_hi)), dmul(nd, ln2_lo));
    double p = 1.0 / 6227020800.0;
    p = dadd(dmul(p, r), 1.0 / 479001600.0);
    p = dadd(dmul(p, r), 1.0 / 39916800.0);
    p = dadd(dmul(p, r), 1.0 / 3628800.0);
    p = dadd(dmul(p, r), 1.0 / 362880.0);
    p = dadd(dmul(p, r), 1.0 / 40320.0);
    p = dadd(dmul(p, r), 1.0 / 5040.0);
    p = dadd(dmul(p, r), 1.0 / 720.0);
    p = dadd(dmul(p, r), 1.0 / 120.0);
    p = dadd(dmul(p, r), 1.0 / 24.0);
    p = dadd(dmul(p, r), 1.0 / 6.0);
    p = dadd(dmul(p, r), 0.5);
    p = dadd(dmul(p, r), 1.0);
    p = dadd(dmul(p, r), 1.0);
    /* p * 2^n with one rounding: ldexp is exact for normal results and rounds subnormal
     * ones once, as the two-step product by 2^n1 * 2^n2 (n1, n2 normal) does */
    double y = __builtin_amdgcn_ldexp(p, n);
    y = lo ? 0.0 : y;
    y = hi ? __longlong_as_double(0x7ff0000000000000ll) : y;
    return nan ? x : y;
}

/* glibc's expf (sysdeps/ieee754/flt-32/e_expf.c, glibc 2.28+; the algorithm of the
 * optimized-routines library) as its x86-64 FMA build evaluates it, the platform expf
 * the reference engine calls: x = (k + r) ln2 / 32 with k and r from the exact product
 * x * 32/ln2 (fma), 2^(k/32) from a 32-entry table of 2^(i/32) (correctly rounded
 * doubles, stored minus i << 47), 2^(r/32) by a cubic in double (three fmas), one
 * rounding to float at the end. The CPU restatement ho_exp_glibc_f is the same function
 * and equals the libm expf on all 2^32 inputs. */
__constant__ static const unsigned long long HX_EXP2F_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

/* the glibc expf; written without branches (the special inputs are selected at the end,
 * the arithmetic runs on them too with a masked table index), so calls interleave.
 * tab(i) returns table entry i: from HX_EXP2F_TAB, from a copy in LDS (exp_table_to_lds:
 * a per-lane gather from LDS costs far less than one through the vector memory path) or
 * from the wave's registers (exp_glibc_f_wave). */
template <typename Fetch>
__device__ __forceinline__ float exp_glibc_core(float x, Fetch tab) {
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32.0;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double shift = 0x1.8p+52;
    const unsigned ux = __float_as_uint(x), abstop = (ux >> 20) & 0x7ffu;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_32, xd, shift);
    const unsigned long long ki = (unsigned long long)__double_as_longlong(kd);
    kd = dsub(kd, shift);
    const double r = __builtin_fma(inv_ln2_32, xd, -kd);
    const double s = __longlong_as_double((long long)(tab((int)(ki & 31)) + (ki << 47)));
    const double z = __builtin_fma(c0, r, c1), r2 = dmul(r, r);
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    float res = __double2float_rn(dmul(y, s));
    if (abstop >= 0x42bu) {                             /* |x| >= 88, inf or NaN */
        res = x > 0x1.62e42ep6f ? __builtin_huge_valf() : res;   /* overflow */
        res = x < -0x1.9fe368p6f ? 0.0f : res;                   /* underflow, -inf */
        res = abstop >= 0x7f8u && ux != 0xff800000u ? x + x : res;   /* NaN, +inf */
    }
    return res;
}

__device__ inline float exp_glibc_f(float x, const unsigned long long *tab) {
    return exp_glibc_core(x, [&](int i) { return tab[i]; });
}

__device__ __forceinline__ float exp_glibc_f(float x) { return exp_glibc_f(x, HX_EXP2F_TAB); }

/* the table entry a lane holds for exp_glibc_f_wave: entry lane % 32, loaded once (early:
 * nothing waits for it until the first exp) */
__device__ __forceinline__ unsigned long long exp_table_lane() { return HX_EXP2F_TAB[threadIdx.x & 31]; }

/* exp_glibc_f with the table in the registers of the wave (ev = exp_table_lane()), read by
 * ds_bpermute (no LDS memory, no barrier). Every lane of the wave must be active. */
__device__ inline float exp_glibc_f_wave(float x, unsigned long long ev) {
    return exp_glibc_core(x, [&](int i) {
        const unsigned lo = (unsigned)__builtin_amdgcn_ds_bpermute(i << 2, (int)(unsigned)ev);
        const unsigned hi = (unsigned)__builtin_amdgcn_ds_bpermute(i << 2, (int)(unsigned)(ev >> 32));
        return ((unsigned long long)hi << 32) | lo;
    });
}

/* copies the exp table into an LDS array of 32 entries (threads 0..31 of the block; the
 * caller synchronizes before use) */
__device__ __forceinline__ void exp_table_to_lds(unsigned long long *lds) {
    if (threadIdx.x < 32) lds[threadIdx.x] = HX_EXP2F_TAB[threadIdx.x];
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* DPP helpers (gfx9 row_shr / row_bcast controls). A row is 16 lanes. */
template <int CTRL, int ROWMASK>
__device__ __forceinline__ unsigned dpp_u32(unsigned old, unsigned v) {
    return (unsigned)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWMASK, 0xF, false);
}

/* maximum of a 64-bit key over the wave, in every lane: row_shr 1, 2, 4, 8 give lane 15 of
 * each row its row's maximum, row_bcast 15 / 31 carry rows 0 and 2 into rows 1 and 3 and
 * rows 0-1 into 2-3, lane 63 ends with the total, which is read back to all lanes. Lanes
 * whose source is outside the row keep their own key. VALU steps only (no LDS). */
__device__ inline unsigned long long wave_max_u64(unsigned long long k) {
    unsigned lo = (unsigned)k, hi = (unsigned)(k >> 32);
#define HX_MAX_STEP(CTRL, RM)                                                                  \
    {                                                                                          \
        const unsigned olo = dpp_u32<CTRL, RM>(lo, lo), ohi = dpp_u32<CTRL, RM>(hi, hi);       \
        const unsigned long long o = ((unsigned long long)ohi << 32) | olo;                    \
        const unsigned long long c = ((unsigned long long)hi << 32) | lo;                      \
        if (o > c) { lo = olo; hi = ohi; }                                                     \
    }
    HX_MAX_STEP(0x111, 0xF)
    HX_MAX_STEP(0x112, 0xF)
    HX_MAX_STEP(0x114, 0xF)
    HX_MAX_STEP(0x118, 0xF)
    HX_MAX_STEP(0x142, 0xA)
    HX_MAX_STEP(0x143, 0xC)
#undef HX_MAX_STEP
    lo = (unsigned)__builtin_amdgcn_readlane((int)lo, 63);
    hi = (unsigned)__builtin_amdgcn_readlane((int)hi, 63);
    return ((unsigned long long)hi << 32) | lo;
}

/* maximum of a non-negative float (NaN-free) and sum of an int over the wave, in every
 * lane, by the same DPP steps (both exact whatever the order) */
/* maximum of an unsigned value over the wave, in every lane (the same DPP steps) */
__device__ inline unsigned wave_max_u32(unsigned v) {
#define HX_UMAX_STEP(CTRL, RM)                                                                 \
    {                                                                                          \
        const unsigned o = dpp_u32<CTRL, RM>(v, v);                                            \
        v = o > v ? o : v;                                                                     \
    }
    HX_UMAX_STEP(0x111, 0xF)
    HX_UMAX_STEP(0x112, 0xF)
    HX_UMAX_STEP(0x114, 0xF)
    HX_UMAX_STEP(0x118, 0xF)
    HX_UMAX_STEP(0x142, 0xA)
    HX_UMAX_STEP(0x143, 0xC)
#undef HX_UMAX_STEP
    return (unsigned)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ inline float wave_max_f32(float x) {
    unsigned v = __float_as_uint(x);
#define HX_FMAX_STEP(CTRL, RM) v = __float_as_uint(fmaxf(__uint_as_float(v), __uint_as_float(dpp_u32<CTRL, RM>(v, v))));
    HX_FMAX_STEP(0x111, 0xF)
    HX_FMAX_STEP(0x112, 0xF)
    HX_FMAX_STEP(0x114, 0xF)
    HX_FMAX_STEP(0x118, 0xF)
    HX_FMAX_STEP(0x142, 0xA)
    HX_FMAX_STEP(0x143, 0xC)
#undef HX_FMAX_STEP
    return __uint_as_float((unsigned)__builtin_amdgcn_readlane((int)v, 63));
}

__device__ inline int wave_sum_i32(int v) {
    v += (int)dpp_u32<0x111, 0xF>(0u, (unsigned)v);
    v += (int)dpp_u32<0x112, 0xF>(0u, (unsigned)v);
    v += (int)dpp_u32<0x114, 0xF>(0u, (unsigned)v);
    v += (int)dpp_u32<0x118, 0xF>(0u, (unsigned)v);
    v += (int)dpp_u32<0x142, 0xA>(0u, (unsigned)v);
    v += (int)dpp_u32<0x143, 0xC>(0u, (unsigned)v);
    return __builtin_amdgcn_readlane(v, 63);
}

/* inclusive prefix sum of an int over the wave (lane order), by the same DPP steps; lanes
 * whose source is outside the row (or whose row is not selected) add 0 */
__device__ inline int wave_scan_incl(int v) {
    v += (int)dpp_u32<0x111, 0xF>(0u, (unsigned)v);
    v += (int)dpp_u32<0x112, 0xF>(0u, (unsigned)v);
    v += (int)dpp_u32<0x114, 0xF>(0u, (unsigned)v);
    v += (int)dpp_u32<0x118, 0xF>(0u, (unsigned)v);
    v += (int)dpp_u32<0x142, 0xA>(0u, (unsigned)v);
    v += (int)dpp_u32<0x143, 0xC>(0u, (unsigned)v);
    return v;
}

/* 16-lane canonical tree (NUMERICS §1) of the partials held by lanes 0..15 of a
 * 16-lane segment: returns the total in lane 0 of the segment. */
__device__ __forceinline__ float tree16(float L) {
    /* L[j] += L[j + s] for s = 8, 4, 2, 1 by DPP row shifts (lanes whose source lies past
     * the 16-lane row read 0; none of them feeds lane 0) */
    L = fadd(L, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(L), 0x108, 0xF, 0xF, true)));
    L = fadd(L, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(L), 0x104, 0xF, 0xF, true)));
    L = fadd(L, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(L), 0x102, 0xF, 0xF, true)));
    L = fadd(L, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(L), 0x101, 0xF, 0xF, true)));
    return L;
}

/* element i of a FORMAT.md row of dtype dt (embedding lookup) */
__device__ __forceinline__ float deq_elem(const uint8_t *row, int dt, int i) {
    switch (dt) {
    case 0: return ((const float *)row)[i];
    case 1: return h2f(((const uint16_t *)row)[i]);
    case 2: return __uint_as_float((uint32_t)((const uint16_t *)row)[i] << 16);
    case 3: {
        const uint8_t *b = row + (size_t)(i >> 6) * 66;
        return fmul(h2f((uint16_t)(b[0] | (b[1] << 8))), (float)(int8_t)b[2 + (i & 63)]);
    }
    default: {
        const uint8_t *b = row + (size_t)(i >> 6) * 34;
        const int w = i & 63, byte = b[2 + (w & 31)];
        const int q = (w < 32 ? (byte & 15) : (byte >> 4)) - 8;
        return fmul(h2f((uint16_t)(b[0] | (b[1] << 8))), (float)q);
    }
    }
}

/* position of element e (0..63) of a block in kperm order */
__device__ __forceinline__ int kperm_pos(int e) {
    return e < 32 ? (e >> 3) * 16 + (e & 7) : ((e - 32) >> 3) * 16 + 8 + ((e - 32) & 7);
}

/* NUMERICS §2 for the 64 values held one per lane by a full wave: this lane's q, the
 * block's d and sum (the same on every lane). Every lane must call it. */
__device__ inline void quant_block_vals(float x, int &q, float &d, int &sum) {
    float ax = fabsf(x);
    ax = ax == ax ? ax : 0.0f;                    /* NaN never wins the max */
    const float amax = wave_max_f32(ax);
    d = fdiv(amax, 127.0f);
    const float id = d != 0.0f ? fdiv(1.0f, d) : 0.0f;
    float v = fmul(x, id);
    if (v != v) v = 0.0f;
    v = v > 127.0f ? 127.0f : v;
    v = v < -127.0f ? -127.0f : v;
    q = (int)__builtin_rintf(v);
    sum = wave_sum_i32(q);
}

/* NUMERICS §2 for the 64 values held one per lane by a full wave: writes q (kperm
 * order), d and the sum of block g of token row tok. Every lane must call it. */
__device__ inline void quant_block_wave(float x, Act a, int tok, int g) {
    const int lane = threadIdx.x & 63;
    int q, sum;
    float d;
    quant_block_vals(x, q, d, sum);
    const size_t base = (size_t)tok * a.nbp + g;
    a.q[base * 64 + kperm_pos(lane)] = (int8_t)q;
    if (lane == 0) {
        a.d[base] = d;
        a.s[base] = sum;
    }
}

} // namespace hxd
