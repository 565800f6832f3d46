/*
 * quant_host.cpp — weight encodings (FORMAT.md §6) and the authoritative weight
 * quantizers behind hearth_quantize / hearth_dequantize / hearth_row_bytes.
 *
 * These are container-writing utilities (the converter path), not part of the
 * verify step; they run on the host like the reference's (engine/src/quant.c:97-307,
 * docs/NUMERICS.md §6) and produce byte-identical files: the reference's pinned
 * quantizer hashes (engine/tests/test_quant.c:55-62) are checked against this code.
 * Compiled with -ffp-contract=off: every float step is a single IEEE operation.
 */
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "hx_host.h"

namespace hx {

namespace {
inline float bits_f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t f_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float nan_to_zero(float v) { return v == v ? v : 0.0f; }
/* round half to even for |v| < 2^22 */
inline float round_even(float v) { return (v + 12582912.0f) - 12582912.0f; }

#pragma pack(push, 1)
struct BlockQ8 { uint16_t d; int8_t q[64]; };
struct BlockQ4 { uint16_t d; uint8_t qs[32]; };
#pragma pack(pop)
static_assert(sizeof(BlockQ8) == 66, "Q8 block is 66 bytes");
static_assert(sizeof(BlockQ4) == 34, "Q4 block is 34 bytes");

/* scale stored as binary16; overflow saturates to +-65504 (reference quant.c:67-72) */
uint16_t scale_to_f16(float d) {
    uint16_t h = f32_to_f16(d);
    if ((h & 0x7c00u) == 0x7c00u) h = (uint16_t)((h & 0x8000u) | 0x7bffu);
    return h;
}

void quant_q8(const float *x, BlockQ8 *out, int64_t nb) {
    for (int64_t b = 0; b < nb; b++, x += QK) {
        float amax = 0.0f;
        for (int i = 0; i < QK; i++) amax = std::fabs(nan_to_zero(x[i])) > amax ? std::fabs(nan_to_zero(x[i])) : amax;
        out[b].d = scale_to_f16(amax / 127.0f);
        const float d = f16_to_f32(out[b].d);
        for (int i = 0; i < QK; i++) {
            float v = d != 0.0f ? nan_to_zero(x[i]) / d : 0.0f;
            v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
            out[b].q[i] = (int8_t)round_even(v);
        }
    }
}

/* Candidate divisors of the Q4 scale search (NUMERICS §6; quant.c:139-142): map the
 * largest-magnitude element to about -8 (with clipping variants) or to about +7. */
constexpr float kQ4Div[20] = {-8.0f, -7.75f, -8.25f, -7.5f, -8.5f, -7.25f, -8.75f, -7.0f, -9.0f, -9.25f,
                              -9.5f, -9.75f, -10.0f, -10.5f, -11.0f, -12.0f, 7.0f, 7.5f, 7.75f, 8.0f};

inline float q4_code(float x, float inv_d) {
    float v = x * inv_d;
    v = v < -8.0f ? -8.0f : v;
    v = v > 7.0f ? 7.0f : v;
    return round_even(v);
}

/* Squared error of scale h on block x, err = sum x^2 - 2 d sum(xq) + d^2 sum(q^2) in
 * double, x*q exact, sum(xq) in four fixed lanes; also returns sum(xq), sum(q^2). */
double q4_score(const float *x, const double *xd, double sx2, uint16_t h, double &sxq, double &sqq) {
    const float d = f16_to_f32(h), inv = d != 0.0f ? 1.0f / d : 0.0f;
    const double dd = d;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    int32_t qq = 0;
    for (int i = 0; i < QK; i += 4)
        for (int j = 0; j < 4; j++) {
            const int q = (int)q4_code(x[i + j], inv);
            acc[j] = acc[j] + xd[i + j] * q;
            qq += q * q;
        }
    sxq = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    sqq = (double)qq;
    return (sx2 - (2.0 * dd) * sxq) + (dd * dd) * (double)qq;
}

void quant_q4(const float *src, BlockQ4 *out, int64_t nb) {
    for (int64_t b = 0; b < nb; b++, src += QK) {
        float x[QK], xm = 0.0f, amax = 0.0f;
        double xd[QK], sx2 = 0.0;
        for (int i = 0; i < QK; i++) {
            x[i] = nan_to_zero(src[i]);
            if (std::fabs(x[i]) > amax) { amax = std::fabs(x[i]); xm = x[i]; }
            xd[i] = x[i];
            sx2 = sx2 + xd[i] * xd[i];
        }
        uint16_t best = 0;
        if (amax > 0.0f) {
            uint16_t tried[20];
            int n_tried = 0;
            double best_err = 0.0, best_sxq = 0.0, best_sqq = 0.0;
            for (int k = 0; k < 20; k++) {
                const uint16_t h = scale_to_f16(xm / kQ4Div[k]);
                bool seen = false;
                for (int j = 0; j < n_tried; j++) seen = seen || tried[j] == h;
                if (seen) continue;
                tried[n_tried++] = h;
                double sxq, sqq;
                const double err = q4_score(x, xd, sx2, h, sxq, sqq);
                if (k == 0 || err < best_err) { best = h; best_err = err; best_sxq = sxq; best_sqq = sqq; }
            }
            for (int it = 0; it < 3 && best_sqq > 0.0; it++) {   /* least-squares refits */
                const uint16_t h = scale_to_f16((float)(best_sxq / best_sqq));
                if (h == best) break;
                double sxq, sqq;
                const double err = q4_score(x, xd, sx2, h, sxq, sqq);
                if (!(err < best_err)) break;
                best = h; best_err = err; best_sxq = sxq; best_sqq = sqq;
            }
        }
        out[b].d = best;
        const float d = f16_to_f32(best), inv = d != 0.0f ? 1.0f / d : 0.0f;
        int q[QK];
        for (int i = 0; i < QK; i++) q[i] = (int)q4_code(x[i], inv);
        for (int j = 0; j < 32; j++) out[b].qs[j] = (uint8_t)((q[j] + 8) | ((q[j + 32] + 8) << 4));
    }
}
} // namespace

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31u) return bits_f(sign | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0u));
    if (e) return bits_f(sign | ((e + 112u) << 23) | (m << 13));
    if (!m) return bits_f(sign);
    return bits_f(sign | f_bits((float)m * 5.9604644775390625e-8f));   /* m * 2^-24, exact */
}

uint16_t f32_to_f16(float f) {
    const uint32_t x = f_bits(f), sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) {
        uint32_t r = ax - 0x38000000u;
        r = r + 0x0fffu + ((r >> 13) & 1u);
        return (uint16_t)(sign | (r >> 13));
    }
    if (ax <= 0x33000000u) return (uint16_t)sign;
    const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, sh = 126u - e;
    uint32_t q = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

uint16_t f32_to_bf16(float f) {
    uint32_t x = f_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x = x + 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float bf16_to_f32(uint16_t h) { return bits_f((uint32_t)h << 16); }

bool dtype_is_quant(int dt) { return dt == HEARTH_Q8 || dt == HEARTH_Q4; }

const char *dtype_name(int dt) {
    static const char *names[] = {"f32", "f16", "bf16", "q8", "q4", "i32", "u8"};
    return dt >= 0 && dt <= 6 ? names[dt] : "invalid";
}

size_t row_bytes(int dtype, int64_t n) {
    if (n <= 0 || n > ((int64_t)1 << 40)) return 0;
    switch (dtype) {
    case HEARTH_F32: case HEARTH_I32: return (size_t)n * 4;
    case HEARTH_F16: case HEARTH_BF16: return (size_t)n * 2;
    case HEARTH_U8: return (size_t)n;
    case HEARTH_Q8: return n % QK ? 0 : (size_t)(n / QK) * 66;
    case HEARTH_Q4: return n % QK ? 0 : (size_t)(n / QK) * 34;
    default: return 0;
    }
}

void quantize_row(int dtype, const float *src, uint8_t *dst, int64_t n) {
    switch (dtype) {
    case HEARTH_F32: std::memcpy(dst, src, (size_t)n * 4); break;
    case HEARTH_F16: for (int64_t i = 0; i < n; i++) ((uint16_t *)dst)[i] = f32_to_f16(src[i]); break;
    case HEARTH_BF16: for (int64_t i = 0; i < n; i++) ((uint16_t *)dst)[i] = f32_to_bf16(src[i]); break;
    case HEARTH_Q8: if (n % QK == 0) quant_q8(src, (BlockQ8 *)dst, n / QK); break;
    case HEARTH_Q4: if (n % QK == 0) quant_q4(src, (BlockQ4 *)dst, n / QK); break;
    default: break;
    }
}

void dequantize_row(int dtype, const uint8_t *src, float *dst, int64_t n) {
    switch (dtype) {
    case HEARTH_F32: std::memcpy(dst, src, (size_t)n * 4); break;
    case HEARTH_F16: for (int64_t i = 0; i < n; i++) dst[i] = f16_to_f32(((const uint16_t *)src)[i]); break;
    case HEARTH_BF16: for (int64_t i = 0; i < n; i++) dst[i] = bf16_to_f32(((const uint16_t *)src)[i]); break;
    case HEARTH_Q8: {
        const BlockQ8 *b = (const BlockQ8 *)src;
        for (int64_t k = 0; k < n / QK; k++) {
            const float d = f16_to_f32(b[k].d);
            for (int i = 0; i < QK; i++) dst[k * QK + i] = d * (float)b[k].q[i];
        }
        break;
    }
    case HEARTH_Q4: {
        const BlockQ4 *b = (const BlockQ4 *)src;
        for (int64_t k = 0; k < n / QK; k++) {
            const float d = f16_to_f32(b[k].d);
            for (int j = 0; j < 32; j++) {
                dst[k * QK + j] = d * (float)((int)(b[k].qs[j] & 15) - 8);
                dst[k * QK + j + 32] = d * (float)((int)(b[k].qs[j] >> 4) - 8);
            }
        }
        break;
    }
    case HEARTH_I32: for (int64_t i = 0; i < n; i++) dst[i] = (float)((const int32_t *)src)[i]; break;
    case HEARTH_U8: for (int64_t i = 0; i < n; i++) dst[i] = (float)src[i]; break;
    default: break;
    }
}

} // namespace hx

using namespace hx;

extern "C" {

HEARTH_API size_t hearth_row_bytes(int dtype, int64_t n_cols) { return row_bytes(dtype, n_cols); }

/* reference quant.c:526-561: rows split over up to n_threads threads (0 = cores),
 * at least ~64K elements each; the result does not depend on the split. */
HEARTH_API int hearth_quantize(int dtype, const float *src, int64_t n_rows, int64_t n_cols, void *dst, int n_threads) {
    const size_t rb = row_bytes(dtype, n_cols);
    if (dtype < HEARTH_F32 || dtype > HEARTH_Q4 || rb == 0 || n_rows < 0) return -1;
    if (n_rows == 0) return 0;
    if (!src || !dst) return -1;
    int64_t nt = n_threads > 0 ? n_threads : (int64_t)std::thread::hardware_concurrency();
    if (nt < 1) nt = 1;
    if (nt > 256) nt = 256;
    if (nt > n_rows) nt = n_rows;
    const int64_t by_work = (n_rows * n_cols + 65535) / 65536;
    if (nt > by_work) nt = by_work < 1 ? 1 : by_work;
    auto run = [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; r++)
            quantize_row(dtype, src + (size_t)r * (size_t)n_cols, (uint8_t *)dst + (size_t)r * rb, n_cols);
    };
    std::vector<std::thread> th;
    for (int64_t t = 1; t < nt; t++) th.emplace_back(run, n_rows * t / nt, n_rows * (t + 1) / nt);
    run(0, n_rows / nt);
    for (auto &x : th) x.join();
    return 0;
}

HEARTH_API int hearth_dequantize(int dtype, const void *src, int64_t n_rows, int64_t n_cols, float *dst) {
    const size_t rb = row_bytes(dtype, n_cols);
    if (dtype < HEARTH_F32 || dtype > HEARTH_U8 || rb == 0 || n_rows < 0) return -1;
    if (n_rows == 0) return 0;
    if (!src || !dst) return -1;
    for (int64_t r = 0; r < n_rows; r++)
        dequantize_row(dtype, (const uint8_t *)src + (size_t)r * rb, dst + (size_t)r * (size_t)n_cols, n_cols);
    return 0;
}

} // extern "C"
