/*
 * k_mla.hip — the parts of multi-head latent attention (DeepSeek-V2/V3, Kimi-K2) that
 * GQA does not have, in the reference's absorbed form (engine/src/model.c:632-787):
 *
 *   c_t   = rmsnorm(kv_a(x)[0:C])                      (cached per slot, [cap][C])
 *   k_pe  = RoPE(kv_a(x)[C:C+r]); q_pe = RoPE(q[h][nope:])  (k_pe cached, [cap][r])
 *   ql[h][c] = sum_n q_nope[h][n] * W_UK[h][n][c]      (n ascending from 0.0f)
 *   s_v   = scale * (dot16(ql[h], c_v) + dot16(q_pe[h], k_pe_v))
 *   o_lat = sum_v p_v c_v                              (the GQA value sum, one group)
 *   o_h   = W_UV[h] . o_lat[h]                         (canonical Q8/Q4 matvec)
 *
 * The latent scores, the softmax and the value sum run through the GQA attention
 * kernels with one KV group of width C shared by all heads (the latent cache is read
 * once per step for every head); W_UV per head runs through the grouped projection
 * kernel with one slot per head. This file holds the rest: the post step, the
 * absorption, the RoPE score term and the gather of the per-head outputs.
 */
#include "hx_device.h"
#include "hx_launch.h"

using namespace hxd;

namespace {

/* rope_apply (model.c:400-408): pairs (j, j + half) (NEOX) or (2j, 2j + 1) (GPT-J) */
__device__ __forceinline__ void rope_wave(float *x, const float *cs, int half, int style, int lane) {
    for (int p = lane; p < half; p += 64) {
        const int ia = style == 1 ? 2 * p : p, ib = style == 1 ? 2 * p + 1 : p + half;
        const float av = x[ia], bv = x[ib], c = cs[2 * p], s = cs[2 * p + 1];
        x[ia] = fadd(fmul(av, c), -fmul(bv, s));
        x[ib] = fadd(fmul(bv, c), fmul(av, s));
    }
}

/* mla_post_range (model.c:631-648): one wave per (token, item); item 0 writes the
 * latent c (rmsnorm) and the rotated k_pe into the caches at slot pos0 + t, item
 * 1 + h rotates q_pe of head h in place. */
__global__ __launch_bounds__(256) void k_mla_post(MlaArgs a) {
    __shared__ float buf[4][MLA_RMAX];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + wave;
    if (item >= a.T * (1 + a.H)) return;
    const int t = item / (1 + a.H), j = item % (1 + a.H);
    const size_t slot = (size_t)(*a.pos + t);
    float *x = buf[wave];
    float *dst;
    if (j == 0) {
        const float *kv = a.kva + (size_t)t * (a.C + a.rdim);
        float L = 0.0f;
        if (lane < 16)
            for (int e = lane; e < a.C; e += 16) L = fadd(L, fmul(kv[e], kv[e]));
        L = tree16(L);
        L = __shfl(L, 0, 64);
        const float r = fdiv(1.0f, sqrt_rn(fadd(fdiv(L, (float)a.C), a.eps)));
        float *cc = a.cc + slot * a.C;
        for (int e = lane; e < a.C; e += 64) cc[e] = fmul(fmul(kv[e], r), a.kv_norm[e]);
        for (int e = lane; e < a.rdim; e += 64) x[e] = kv[a.C + e];
        dst = a.kp + slot * a.rdim;
    } else {
        dst = a.q + ((size_t)t * a.H + (j - 1)) * a.qh + a.nope;
        for (int e = lane; e < a.rdim; e += 64) x[e] = dst[e];
    }
    wave_sync();
    rope_wave(x, a.rope + (size_t)t * a.rope_dim, a.rope_dim / 2, a.rope_style, lane);
    wave_sync();
    for (int e = lane; e < a.rdim; e += 64) dst[e] = x[e];
}

/* bytes of one 64-column segment of a FORMAT.md row: a Q8 / Q4 block, or 64 floats */
__device__ __forceinline__ int seg_bytes(int dt) { return dt == 3 ? 66 : dt == 4 ? 34 : dt == 0 ? 256 : 128; }

/* mla_qlat (model.c:650-671): ql[t][h][c] = sum_n q[t][h][n] * W_UK[h][n][c], n ascending
 * from 0.0f, with the weight element dequantized as the reference does (d * q). One
 * workgroup per (head, 64 columns): the nope rows' segments of those columns are staged
 * in LDS once (coalesced 2-byte loads), then tiles of QL_TT tokens' q_nope; wave w sums
 * the tokens w, w + 4, ... of a tile, lane l column c0 + l. */
constexpr int QL_TT = 32;
__global__ __launch_bounds__(256) void k_mla_qlat(MlaArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t ql_lds[];
    const int dt = a.wuk_dtype, seg = seg_bytes(dt), stride = (seg + 3) & ~3;
    const int ncb = a.C / 64;
    const int h = (int)blockIdx.x / ncb, cb = (int)blockIdx.x % ncb;
    const int nope = a.nope, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float *qn = (float *)(ql_lds + (size_t)nope * stride);   /* [QL_TT][nope] */
    const size_t row0 = (size_t)h * (a.nope + a.vd);
    const size_t segoff = dt >= 3 ? (size_t)cb * seg : (size_t)cb * 64 * (dt == 0 ? 4 : 2);
    {
        const int hw = seg >> 1;   /* 2-byte words per segment */
        for (int i = tid; i < nope * hw; i += 256) {
            const int n = i / hw, w = i % hw;
            const uint16_t *src = (const uint16_t *)(a.wuk + (row0 + n) * a.wuk_rb + segoff);
            ((uint16_t *)(ql_lds + (size_t)n * stride))[w] = src[w];
        }
    }
    for (int t0 = 0; t0 < a.T; t0 += QL_TT) {
        const int tn = a.T - t0 < QL_TT ? a.T - t0 : QL_TT;
        __syncthreads();
        for (int i = tid; i < tn * nope; i += 256) {
            const int tt = i / nope, n = i % nope;
            qn[tt * nope + n] = a.q[((size_t)(t0 + tt) * a.H + h) * a.qh + n];
        }
        __syncthreads();
        float acc[QL_TT / 4];
#pragma unroll
        for (int j = 0; j < QL_TT / 4; j++) acc[j] = 0.0f;
        for (int n = 0; n < nope; n++) {
            const float w = deq_elem(ql_lds + (size_t)n * stride, dt, lane);
#pragma unroll
            for (int j = 0; j < QL_TT / 4; j++)
                if (wave + 4 * j < tn) acc[j] = fadd(acc[j], fmul(qn[(wave + 4 * j) * nope + n], w));
        }
#pragma unroll
        for (int j = 0; j < QL_TT / 4; j++)
            if (wave + 4 * j < tn)
                a.qlat[((size_t)(t0 + wave + 4 * j) * a.H + h) * a.C + cb * 64 + lane] = acc[j];
    }
}

/* mla_softmax's score (model.c:690-703): s = scale * (s_lat + dot16(q_pe, k_pe_v)),
 * s_lat already in S from the latent scores. One workgroup per (token, 256 rows, 16
 * heads), one thread per row: the 16 heads' q_pe are staged in LDS, the row's 16 s_lat
 * are loaded up front (independent loads), then the 16 sums. */
constexpr int PE_HG = 16;
__global__ __launch_bounds__(256) void k_mla_pe(MlaArgs a) {
    __shared__ float qpe[PE_HG * MLA_RMAX];
    const int ng = (a.H + PE_HG - 1) / PE_HG;
    int b = (int)blockIdx.x;
    const int hg = b % ng;
    b /= ng;
    const int t = b % a.T, chunk = b / a.T;
    const int pos0 = *a.g.pos, nr = pos0 + a.g.depth[t] + 1;
    if (chunk * 256 >= nr) return;   /* uniform */
    const int r = a.rdim, h0 = hg * PE_HG, nh = a.H - h0 < PE_HG ? a.H - h0 : PE_HG;
    for (int i = threadIdx.x; i < nh * r; i += 256) {
        const int hh = i / r, e = i % r;
        qpe[hh * MLA_RMAX + e] = a.q[((size_t)t * a.H + h0 + hh) * a.qh + a.nope + e];
    }
    __syncthreads();
    const int v = chunk * 256 + (int)threadIdx.x;
    if (v >= nr) return;
    const int slot = v < pos0 ? v : pos0 + a.g.anc[(size_t)t * a.g.anc_ld + (v - pos0)];
    const float *kr = a.kp + (size_t)slot * r;
    float k[MLA_RMAX];
#pragma unroll
    for (int e = 0; e < MLA_RMAX; e++) k[e] = e < r ? kr[e] : 0.0f;
    float *s = a.S + ((size_t)t * a.H + h0) * a.ldS + v;
    float sl[PE_HG];
#pragma unroll
    for (int hh = 0; hh < PE_HG; hh++) sl[hh] = hh < nh ? s[(size_t)hh * a.ldS] : 0.0f;
#pragma unroll
    for (int hh = 0; hh < PE_HG; hh++) {
        const float *qh = qpe + hh * MLA_RMAX;
        float L[16];
#pragma unroll
        for (int j = 0; j < 16; j++) L[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < MLA_RMAX; e++)
            if (e < r) L[e & 15] = fadd(L[e & 15], fmul(qh[e], k[e]));
#pragma unroll
        for (int st = 8; st >= 1; st >>= 1)
#pragma unroll
            for (int j = 0; j < st; j++) L[j] = fadd(L[j], L[j + st]);
        if (hh < nh) s[(size_t)hh * a.ldS] = fmul(a.scale, fadd(sl[hh], L[0]));
    }
}

/* att[t][h * vd + j] = Yv[h][t][j] and NUMERICS §2 of att rows; one wave per (token,
 * block) */
__global__ void k_mla_gather(MlaArgs a) {
    const int nbp = a.aatt.nbp, nb = (a.H * a.vd) / 64;
    const int wave = (int)((blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6);
    if (wave >= a.T * nbp) return;   /* uniform per wave */
    const int t = wave / nbp, b = wave % nbp, lane = threadIdx.x & 63, i = b * 64 + lane;
    float x = 0.0f;
    if (b < nb) {
        const int h = i / a.vd, j = i % a.vd;
        x = a.Yv[((size_t)h * a.T + t) * a.vd + j];
        a.att[(size_t)t * a.H * a.vd + i] = x;
    }
    quant_block_wave(x, a.aatt, t, b);
}

} // namespace

namespace hxl {

void mla_post(const MlaArgs &a, hipStream_t st) {
    const int items = a.T * (1 + a.H);
    k_mla_post<<<(items + 3) / 4, 256, 0, st>>>(a);
}

void mla_qlat(const MlaArgs &a, hipStream_t st) {
    /* C is a multiple of 128 (checked at open); LDS: nope segments + a token tile */
    const int dt = a.wuk_dtype, seg = dt == 3 ? 66 : dt == 4 ? 34 : dt == 0 ? 256 : 128;
    const size_t lds = (size_t)a.nope * ((seg + 3) & ~3) + sizeof(float) * (size_t)QL_TT * a.nope;
    k_mla_qlat<<<a.H * (a.C / 64), 256, lds, st>>>(a);
}

void mla_pe_scores(const MlaArgs &a, hipStream_t st) {
    const int max_nr = a.g.nr_max;
    const int nchunks = (max_nr + 255) / 256;
    k_mla_pe<<<a.T * nchunks * ((a.H + PE_HG - 1) / PE_HG), 256, 0, st>>>(a);
}

void mla_gather(const MlaArgs &a, hipStream_t st) {
    const int64_t waves = (int64_t)a.T * a.aatt.nbp;
    if (waves) k_mla_gather<<<(int)((waves + 3) / 4), 256, 0, st>>>(a);
}

} // namespace hxl
