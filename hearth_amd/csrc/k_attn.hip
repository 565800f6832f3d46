/*
 * k_attn.hip — GQA attention over the F32 KV cache with a causal or tree-ancestor
 * mask, in the reference's canonical order (docs/NUMERICS.md §5.1; engine/src/model.c
 * gqa_scores/gqa_softmax/gqa_values 519-589, value_sum 552-575):
 *   s_v = scale * dot16(q_h, k_v)           (16 lanes, then the 8/4/2/1 tree)
 *   p   = softmax(s)                         (max, exp, sum16, divide)
 *   o_h[d] = sum_v p_v * v_v[d]              (sequential in v from 0.0f)
 * v runs over the token's rows in order: the context slots 0..pos0-1, then its
 * ancestors' slots from the root to itself (for a chain: slots 0..pos0+t). A tree
 * node therefore computes exactly what the chain root->node computes.
 *
 * The value sum is one dependent f32 add chain per (token, head, d) of length
 * pos0 + depth + 1; it is the step's latency floor, so the value kernel keeps one
 * chain per lane and one summing wave per SIMD, fed from transposed V tiles that
 * eight loader waves keep three tiles ahead.
 *
 * Launch shapes are XCD-aware: workgroup IDs are dealt round-robin to the 8 XCDs,
 * so the KV-group index (and value d-chunk) is the fastest-varying part of the ID and
 * the workgroups of one XCD read the same group's K or V rows from that XCD's L2.
 */
#include <algorithm>
#include <type_traits>

#include "hx_device.h"
#include "hx_launch.h"

using namespace hxd;

namespace {

constexpr int SC_ROWS = 256;   /* rows per scores workgroup (one per thread) */
constexpr int KC = 16;         /* K floats per staged chunk (head_dim % 16 == 0) */
constexpr int MAX_ANC = 4096;  /* ancestors of one token (max_batch) */

__device__ __forceinline__ int row_slot(const TokGeom &g, int pos0, int t, int v) {
    return v < pos0 ? v : pos0 + g.anc[(size_t)t * g.anc_ld + (v - pos0)];
}

/* Scores of NH heads of KV group g for 256 rows v of token t: one thread per row, 16
 * partial sums per head (element c goes to partial c % 16), then the 8/4/2/1 tree.
 * K rows and the q chunk go through a double-buffered LDS stage, one barrier per
 * 16-float chunk; the next chunk's loads are in flight while the current one is used. */
template <int NH>
__global__ __launch_bounds__(256) void k_attn_scores(AttnArgs a) {
    __shared__ float kt[2][SC_ROWS][KC + 1];
    __shared__ float4 qs[2][NH][KC / 4];
    __shared__ int slot_s[SC_ROWS];
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd;
    int b = blockIdx.x;
    const int g = b % Hkv;
    b /= Hkv;
    const int t = b % a.T, c = b / a.T;
    const int pos0 = *a.g.pos, nr = pos0 + a.g.depth[t] + 1;
    const int v0 = c * SC_ROWS;
    if (v0 >= nr) return;   /* uniform */
    const int tid = threadIdx.x;
    const int nrows = nr - v0 < SC_ROWS ? nr - v0 : SC_ROWS;
    slot_s[tid] = row_slot(a.g, pos0, t, v0 + (tid < nrows ? tid : nrows - 1));
    __syncthreads();
    /* staging: float4 k = tid + 256u of the chunk: row k / 4, floats 4 (k % 4) .. + 3 */
    const float *src[4];
#pragma unroll
    for (int u = 0; u < 4; u++)
        src[u] = a.kc + ((size_t)g * a.cap + slot_s[(tid >> 2) + 64 * u]) * hd + (tid & 3) * 4;
    const float *qb = a.q + ((size_t)t * a.H + (size_t)g * grp) * hd;
    const bool qlane = tid < NH * 4;
    const float *qsrc = qb + (size_t)(qlane ? tid >> 2 : 0) * hd + (tid & 3) * 4;
    const int nchunk = hd / KC, niter = (grp / NH) * nchunk;
    float4 kr[4], qr = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto gload = [&](int it) {
        const int c0 = (it % nchunk) * KC, h0 = (it / nchunk) * NH;
#pragma unroll
        for (int u = 0; u < 4; u++) kr[u] = *(const float4 *)(src[u] + c0);
        if (qlane) qr = *(const float4 *)(qsrc + (size_t)h0 * hd + c0);
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            float *d = &kt[buf][(tid >> 2) + 64 * u][(tid & 3) * 4];
            d[0] = kr[u].x;
            d[1] = kr[u].y;
            d[2] = kr[u].z;
            d[3] = kr[u].w;
        }
        if (qlane) qs[buf][tid >> 2][tid & 3] = qr;
    };
    float L[NH][16];
#pragma unroll
    for (int hh = 0; hh < NH; hh++)
#pragma unroll
        for (int j = 0; j < 16; j++) L[hh][j] = 0.0f;
    gload(0);
    lstore(0);
    __syncthreads();
    float *Sb = a.S + ((size_t)t * a.H + (size_t)g * grp) * a.ldS + v0 + tid;
    for (int it = 0; it < niter; it++) {
        const int buf = it & 1;
        if (it + 1 < niter) gload(it + 1);
        float kv[16];
#pragma unroll
        for (int j = 0; j < 16; j++) kv[j] = kt[buf][tid][j];
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            float q[16];
#pragma unroll
            for (int j4 = 0; j4 < 4; j4++) {
                const float4 x = qs[buf][hh][j4];
                q[4 * j4] = x.x;
                q[4 * j4 + 1] = x.y;
                q[4 * j4 + 2] = x.z;
                q[4 * j4 + 3] = x.w;
            }
#pragma unroll
            for (int j = 0; j < 16; j++) L[hh][j] = fadd(L[hh][j], fmul(q[j], kv[j]));
        }
        if (it % nchunk == nchunk - 1) {
            const int h0 = (it / nchunk) * NH;
#pragma unroll
            for (int hh = 0; hh < NH; hh++) {
#pragma unroll
                for (int s = 8; s >= 1; s >>= 1)
#pragma unroll
                    for (int j = 0; j < s; j++) L[hh][j] = fadd(L[hh][j], L[hh][j + s]);
                if (tid < nrows) Sb[(size_t)(h0 + hh) * a.ldS] = fmul(a.scale, canon(L[hh][0]));
#pragma unroll
                for (int j = 0; j < 16; j++) L[hh][j] = 0.0f;
            }
        }
        if (it + 1 < niter) lstore(buf ^ 1);
        __syncthreads();
    }
}

/* The same scores with the 16 dot16 partials on 16 lanes instead of 16 registers
 * (head_dim a multiple of 64): thread (row, j) accumulates partial j of its row, the
 * elements j, j + 16, ... in order, for 8 heads at a time; the 8/4/2/1 tree then runs
 * across the 16 lanes of the row with DPP row shifts (lane j adds lane j + s, exactly
 * the canonical pairing). 8 accumulators per thread instead of 128 let eight waves per
 * SIMD hide the load latency. A row's K elements j + 16 i are loaded straight from the
 * cache (16 lanes read 64 contiguous bytes); q of the 8 heads is staged transposed in
 * LDS (qT[h][j][i] = q[h][16 i + j]), read four i at a time. Each lane's row of qT is
 * padded by 16 bytes, so the 16 lanes of a read hit 16 different bank groups (unpadded,
 * a head_dim of 512 put all 16 on the same banks). NP 16-row passes per workgroup keep
 * NP * HI = 32 K values in registers per thread. */
template <int HI> constexpr int s16_np() { return HI <= 8 ? 4 : HI <= 16 ? 2 : 1; }

/* bias, qk-norm and RoPE of one K or q head held by the 16 lanes of a row, lane j
 * holding elements j + 16 i (k_qkv_post's operations in its order): the squares summed
 * per lane in i order, the 8/4/2/1 tree across the row (DPP, lane j adds lane j + s),
 * r = 1 / sqrt(sum / hd + eps), x * r * w; NEOX RoPE pairs (p, p + hd / 2) sit in
 * registers i and i + HI / 2 of the same lane. Every lane of the wave calls it. */
template <int HI>
__device__ __forceinline__ void post_row(float (&x)[HI], const float *bias, const float *w, const float *cs, int qk_norm,
                                         float eps, int j) {
    if (bias) {
#pragma unroll
        for (int i = 0; i < HI; i++) x[i] = fadd(x[i], bias[j + 16 * i]);
    }
    if (qk_norm == 1) {
        float L = 0.0f;
#pragma unroll
        for (int i = 0; i < HI; i++) L = fadd(L, fmul(x[i], x[i]));
        L = tree16(L);
        L = __shfl(L, 0, 16);
        const float r = fdiv(1.0f, sqrt_rn(fadd(fdiv(L, (float)(16 * HI)), eps)));
#pragma unroll
        for (int i = 0; i < HI; i++) x[i] = fmul(fmul(x[i], r), w[j + 16 * i]);
    }
#pragma unroll
    for (int i = 0; i < HI / 2; i++) {
        const int pp = j + 16 * i;
        const float av = x[i], bv = x[i + HI / 2], c = cs[2 * pp], sn = cs[2 * pp + 1];
        x[i] = fadd(fmul(av, c), -fmul(bv, sn));
        x[i + HI / 2] = fadd(fmul(bv, c), fmul(av, sn));
    }
}

template <int HI, bool POST>
__global__ __launch_bounds__(256, (HI <= 8 ? 5 : 1)) void k_attn_scores16(AttnArgs a) {
    constexpr int S16_NP = s16_np<HI>(), S16_RB = 16 * S16_NP, QS = HI / 4 + 1;
    __shared__ float4 qT[8][16][QS];
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd;
    int b = blockIdx.x, g, t, c;
    if (a.g.live) {
        /* with padding tokens the token is the slowest index: the live tokens' workgroups
         * dispatch first and the padding ones (which exit at once) after them */
        const int per_t = (int)gridDim.x / a.T;
        t = b / per_t;
        b -= t * per_t;
        g = b % Hkv;
        c = b / Hkv;
        if (t >= *a.g.live) return;   /* padding token (uniform) */
    } else {
        g = b % Hkv;
        b /= Hkv;
        t = b % a.T;
        c = b / a.T;
    }
    const int pos0 = *a.g.pos, nr = pos0 + a.g.depth[t] + 1;
    const int v0 = c * S16_RB;
    if (v0 >= nr) return;   /* uniform */
    const int tid = threadIdx.x, j = tid & 15, rl = tid >> 4;
    const size_t kvd = (size_t)Hkv * hd;
    if (POST && c == 0 && tid < 64) {
        /* token t's K row of group g (processed) and V row (+ bias) into slot pos0 + t */
        float x[HI];
        const float *kr = a.rk + (size_t)t * kvd + (size_t)g * hd + j;
#pragma unroll
        for (int i = 0; i < HI; i++) x[i] = kr[16 * i];
        post_row<HI>(x, a.bk ? a.bk + (size_t)g * hd : nullptr, a.kn, a.rope + (size_t)t * hd, a.qk_norm, a.eps, j);
        const size_t slot = (size_t)g * a.cap + pos0 + t;
        if (tid < 16) {
#pragma unroll
            for (int i = 0; i < HI; i++) ((float *)a.kc)[slot * hd + j + 16 * i] = x[i];
        }
        const float *vs = a.rv + (size_t)t * kvd + (size_t)g * hd;
        for (int e = tid; e < hd; e += 64)
            ((float *)a.vc)[slot * hd + e] = a.bv ? fadd(vs[e], a.bv[(size_t)g * hd + e]) : vs[e];
    }
    float kv[S16_NP][HI];
    int vrow[S16_NP];
    bool isnew[S16_NP];
#pragma unroll
    for (int pass = 0; pass < S16_NP; pass++) {
        const int v = v0 + pass * 16 + rl;
        vrow[pass] = v;
        const int slot = row_slot(a.g, pos0, t, v < nr ? v : nr - 1);
        /* with the post-step, rows of this step's tokens come from the raw projection */
        isnew[pass] = POST && slot >= pos0;
        const float *kr = isnew[pass] ? a.rk + (size_t)(slot - pos0) * kvd + (size_t)g * hd + j
                                      : a.kc + ((size_t)g * a.cap + slot) * hd + j;
#pragma unroll
        for (int i = 0; i < HI; i++) kv[pass][i] = kr[16 * i];
    }
    if (POST) {
#pragma unroll
        for (int pass = 0; pass < S16_NP; pass++) {
            if (__ballot(isnew[pass]) == 0ull) continue;   /* uniform */
            const int slot = row_slot(a.g, pos0, t, vrow[pass] < nr ? vrow[pass] : nr - 1);
            const int tok = isnew[pass] ? slot - pos0 : 0;
            float x[HI];
#pragma unroll
            for (int i = 0; i < HI; i++) x[i] = kv[pass][i];
            post_row<HI>(x, a.bk ? a.bk + (size_t)g * hd : nullptr, a.kn, a.rope + (size_t)tok * hd, a.qk_norm, a.eps, j);
            if (isnew[pass]) {
#pragma unroll
                for (int i = 0; i < HI; i++) kv[pass][i] = x[i];
            }
        }
    }
    for (int h0 = 0; h0 < grp; h0 += 8) {
        __syncthreads();
        const float *qb = a.q + ((size_t)t * a.H + (size_t)g * grp + h0) * hd;
        float *qf = (float *)qT;
        if (POST) {
            /* a head per 16 lanes of the first two waves: raw q (+ bias), qk-norm and
             * RoPE in registers, then into the transposed stage */
            if (tid < 128) {
                const int hh = tid >> 4;
                const bool in = h0 + hh < grp;
                const int hq = in ? hh : 0;
                float x[HI];
#pragma unroll
                for (int i = 0; i < HI; i++) x[i] = qb[(size_t)hq * hd + j + 16 * i];
                post_row<HI>(x, a.bq ? a.bq + ((size_t)g * grp + h0 + hq) * hd : nullptr, a.qn, a.rope + (size_t)t * hd,
                             a.qk_norm, a.eps, j);
#pragma unroll
                for (int i = 0; i < HI; i++) qf[(hh * 16 + j) * (4 * QS) + i] = in ? x[i] : 0.0f;
                if (c == 0 && in && a.qout) {
                    float *qo = a.qout + ((size_t)t * a.H + (size_t)g * grp + h0 + hh) * hd + j;
#pragma unroll
                    for (int i = 0; i < HI; i++) qo[16 * i] = x[i];
                }
            }
        } else {
            for (int x = tid; x < 8 * hd; x += 256) {
                const int hh = x / hd, e = x % hd;
                qf[(hh * 16 + (e & 15)) * (4 * QS) + (e >> 4)] = h0 + hh < grp ? qb[(size_t)hh * hd + e] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int pass = 0; pass < S16_NP; pass++) {
            float acc[8];
#pragma unroll
            for (int hh = 0; hh < 8; hh++) acc[hh] = 0.0f;
#pragma unroll
            for (int i4 = 0; i4 < HI / 4; i4++) {
#pragma unroll
                for (int hh = 0; hh < 8; hh++) {
                    const float4 q4 = qT[hh][j][i4];
                    acc[hh] = fadd(acc[hh], fmul(q4.x, kv[pass][4 * i4]));
                    acc[hh] = fadd(acc[hh], fmul(q4.y, kv[pass][4 * i4 + 1]));
                    acc[hh] = fadd(acc[hh], fmul(q4.z, kv[pass][4 * i4 + 2]));
                    acc[hh] = fadd(acc[hh], fmul(q4.w, kv[pass][4 * i4 + 3]));
                }
            }
#pragma unroll
            for (int hh = 0; hh < 8; hh++) {
                /* row_shl:s (DPP control 0x100 + s): lane j reads lane j + s of its row */
#define HX_DPP_ADD(cc) acc[hh] = fadd(acc[hh], __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc[hh]), cc, 0xF, 0xF, true)))
                HX_DPP_ADD(0x108);
                HX_DPP_ADD(0x104);
                HX_DPP_ADD(0x102);
                HX_DPP_ADD(0x101);
#undef HX_DPP_ADD
            }
            const int v = vrow[pass];
            if (j == 0 && v < nr) {
                float *Sb = a.S + ((size_t)t * a.H + (size_t)g * grp + h0) * a.ldS + v;
#pragma unroll
                for (int hh = 0; hh < 8; hh++)
                    if (h0 + hh < grp) Sb[(size_t)hh * a.ldS] = fmul(a.scale, canon(acc[hh]));
            }
        }
    }
}

/* The same scores for a chain of at most ST_TMAX tokens at a large head_dim (the MLA
 * latent, 512), where every token reads row v from slot v: one workgroup per 64 rows and
 * block of up to ST_HB heads, for every token. Thread (row, j) loads its row's K elements
 * j + 16 i once and runs through all (token, 8-head) blocks of q, staged transposed in
 * LDS two at a time (one barrier per block), so the K rows are read once per block of
 * heads instead of once per token (more, smaller head blocks keep more workgroups in
 * flight: the K rows come from L2 after the first). Each score is the same sequence of operations as in
 * k_attn_scores16. (At head_dim 128 the per-token kernel is faster: it has nine times
 * the workgroups to hide its latencies with; measured 16.8 against 24.6 µs.) */
constexpr int ST_HB = 8;   /* 8 heads a workgroup: 24.99 ms per DeepSeek-V3 step against 25.84 with 16 and 27.02 with 32 */
constexpr int ST_TMAX = 64;

template <int HI>
__global__ __launch_bounds__(1024) void k_attn_scores16t(AttnArgs a, int nhb, int hbsz) {
    constexpr int QS = HI / 4 + 1;
    __shared__ float4 qT[2][8][16][QS];
    __shared__ int nr_s[ST_TMAX];
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd, T = a.T;
    int b = blockIdx.x;
    const int hb = b % nhb;
    b /= nhb;
    const int g = b % Hkv, c = b / Hkv;
    const int pos0 = *a.g.pos, nrmax = pos0 + T;
    const int v0 = c * 64;
    if (v0 >= nrmax) return;   /* uniform: past every token's rows */
    const int tid = threadIdx.x, j = tid & 15, v = v0 + (tid >> 4);
    if (tid < T) nr_s[tid] = pos0 + a.g.depth[tid] + 1;
    float kv[HI];
    {
        const float *kr = a.kc + ((size_t)g * a.cap + (v < nrmax ? v : nrmax - 1)) * hd + j;
#pragma unroll
        for (int i = 0; i < HI; i++) kv[i] = kr[16 * i];
    }
    const int h_lo = hb * hbsz, h_hi = min(grp, h_lo + hbsz), nh8 = (h_hi - h_lo + 7) / 8, nblk = T * nh8;
    auto stage = [&](int blk, int buf) {
        const int t = blk / nh8, h0 = h_lo + (blk % nh8) * 8;
        const float *qb = a.q + ((size_t)t * a.H + (size_t)g * grp + h0) * hd;
        float *qf = (float *)qT[buf];
        for (int x = tid; x < 8 * hd; x += 1024) {
            const int hh = x / hd, e = x % hd;
            qf[(hh * 16 + (e & 15)) * (4 * QS) + (e >> 4)] = h0 + hh < h_hi ? qb[(size_t)hh * hd + e] : 0.0f;
        }
    };
    stage(0, 0);
    for (int blk = 0; blk < nblk; blk++) {
        __syncthreads();   /* block blk staged; block blk - 1's buffer free */
        if (blk + 1 < nblk) stage(blk + 1, (blk + 1) & 1);
        const int t = blk / nh8, h0 = h_lo + (blk % nh8) * 8, buf = blk & 1;
        float acc[8];
#pragma unroll
        for (int hh = 0; hh < 8; hh++) acc[hh] = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < HI / 4; i4++) {
#pragma unroll
            for (int hh = 0; hh < 8; hh++) {
                const float4 q4 = qT[buf][hh][j][i4];
                acc[hh] = fadd(acc[hh], fmul(q4.x, kv[4 * i4]));
                acc[hh] = fadd(acc[hh], fmul(q4.y, kv[4 * i4 + 1]));
                acc[hh] = fadd(acc[hh], fmul(q4.z, kv[4 * i4 + 2]));
                acc[hh] = fadd(acc[hh], fmul(q4.w, kv[4 * i4 + 3]));
            }
        }
#pragma unroll
        for (int hh = 0; hh < 8; hh++) {
#define HX_DPP_ADD(cc) acc[hh] = fadd(acc[hh], __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc[hh]), cc, 0xF, 0xF, true)))
            HX_DPP_ADD(0x108);
            HX_DPP_ADD(0x104);
            HX_DPP_ADD(0x102);
            HX_DPP_ADD(0x101);
#undef HX_DPP_ADD
        }
        if (j == 0 && v < nr_s[t]) {
            float *Sb = a.S + ((size_t)t * a.H + (size_t)g * grp + h0) * a.ldS + v;
#pragma unroll
            for (int hh = 0; hh < 8; hh++)
                if (h0 + hh < h_hi) Sb[(size_t)hh * a.ldS] = fmul(a.scale, canon(acc[hh]));
        }
    }
}

__device__ __forceinline__ float sum16_lds(const float *es, int n, int lane16, float L) {
    /* lane lane16 of 16: continues the sequential sum L with es[lane16], es[lane16 + 16],
     * ..., the next 16 operands read while the current 16 are added */
    int i = lane16;
    float cur[16], nxt[16];
    const int full = n >= 16 * 16 ? (n - lane16) / 256 : 0;   /* groups of 16 in range */
    if (full > 0) {
#pragma unroll
        for (int u = 0; u < 16; u++) cur[u] = es[i + 16 * u];
        for (int gi = 0; gi < full; gi++) {
            const int inx = gi + 1 < full ? i + 256 : i;
#pragma unroll
            for (int u = 0; u < 16; u++) nxt[u] = es[inx + 16 * u];
#pragma unroll
            for (int u = 0; u < 16; u++) L = fadd(L, cur[u]);
#pragma unroll
            for (int u = 0; u < 16; u++) cur[u] = nxt[u];
            i += 256;
        }
    }
    for (; i < n; i += 16) L = fadd(L, es[i]);
    return L;
}

/* softmax over one (token, head) row of scores, in place (quant.c:634-642): running
 * max from s[0] (a NaN s[0] stays the max, later NaNs are skipped), e = exp(s - max),
 * sum16 of e, p = e / sum. Up to 8192 scores stay in registers (16 per thread); their
 * exps are computed four at a time (exp_glibc_f has no branches, so the four
 * double-precision evaluations interleave). Longer rows are processed in chunks of 8192
 * re-read from the row. */
constexpr int SM_T = 512;
constexpr int SM_PER = 16;
constexpr int SM_CH = SM_T * SM_PER;

__global__ __launch_bounds__(SM_T) void k_attn_softmax(AttnArgs a) {
    __shared__ float es[SM_CH];
    __shared__ float red[SM_T / 64];
    __shared__ float sum_sh;
    __shared__ unsigned long long etab[32];
    exp_table_to_lds(etab);
    const int t = blockIdx.x / a.H, h = blockIdx.x % a.H, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (a.g.live && t >= *a.g.live) return;   /* padding token (uniform) */
    const int pos0 = *a.g.pos, nr = pos0 + a.g.depth[t] + 1;
    float *s = a.S + ((size_t)t * a.H + h) * a.ldS;
    const bool inreg = nr <= SM_CH;
    const int wlo = __builtin_amdgcn_readfirstlane(tid >> 6) * 64;   /* first thread of the wave */
    float x[SM_PER];
    float m = -__builtin_huge_valf();
    if (inreg) {
#pragma unroll
        for (int u = 0; u < SM_PER; u++) {
            const int i = tid + SM_T * u;
            x[u] = i < nr ? s[i] : -__builtin_huge_valf();
        }
#pragma unroll
        for (int u = 0; u < SM_PER; u++)
            if (x[u] == x[u]) m = fmaxf(m, x[u]);
    } else {
        for (int i = tid; i < nr; i += SM_T) {
            const float v = s[i];
            if (v == v) m = fmaxf(m, v);
        }
    }
    m = wave_max_f32(m);   /* a maximum: any reduction order gives the same value */
    if (lane == 0) red[wave] = m;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < SM_T / 64; w++) m = fmaxf(m, red[w]);
    const float s0 = s[0];
    if (s0 != s0) m = s0;
    float L = 0.0f;   /* lane tid < 16: partial of the elements i = tid (mod 16) */
    for (int c0 = 0; c0 < nr; c0 += SM_CH) {
        const int n = nr - c0 < SM_CH ? nr - c0 : SM_CH;
        if (c0) __syncthreads();
        if (inreg) {
            /* entries past the row hold -inf; their exps are never stored or used */
#pragma unroll
            for (int u0 = 0; u0 < SM_PER; u0 += 4) {
                /* entry u of this wave holds a score iff wlo + SM_T u < n (wave-uniform):
                 * whole groups of four where all four hold scores, then one at a time */
                if (wlo + SM_T * (u0 + 3) < n) {
                    float e[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) e[k] = exp_glibc_f(fadd(x[u0 + k], -m), etab);
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        x[u0 + k] = e[k];
                        const int i = tid + SM_T * (u0 + k);
                        if (i < n) es[i] = e[k];
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        if (wlo + SM_T * (u0 + k) < n) {
                            const float e1 = exp_glibc_f(fadd(x[u0 + k], -m), etab);
                            x[u0 + k] = e1;
                            const int i = tid + SM_T * (u0 + k);
                            if (i < n) es[i] = e1;
                        }
                    }
                }
            }
        } else {
            for (int i = tid; i < n; i += SM_T) es[i] = exp_glibc_f(fadd(s[c0 + i], -m), etab);
        }
        __syncthreads();
        /* SM_CH is a multiple of 16, so element c0 + i keeps lane (c0 + i) % 16 = i % 16 */
        if (tid < 16) L = sum16_lds(es, n, tid, L);
        if (!inreg) {
            __syncthreads();
            for (int i = tid; i < n; i += SM_T) s[c0 + i] = es[i];
        }
    }
    if (tid < 16) {
        L = tree16(L);
        if (tid == 0) sum_sh = L;
    }
    __syncthreads();
    const float sum = sum_sh;
    if (inreg) {
#pragma unroll
        for (int u = 0; u < SM_PER; u++) {
            if (wlo + SM_T * u < nr) {
                const int i = tid + SM_T * u;
                if (i < nr) s[i] = fdiv(x[u], sum);
            }
        }
    } else {
        for (int i = tid; i < nr; i += SM_T) s[i] = fdiv(s[i], sum);
    }
}

/* The same softmax with one wave per (token, head) row, for many rows of at most
 * SMW_PER * 64 scores (a tree's or a prefill's): the row's scores and exps stay in the
 * lane's registers, the exps also go to the wave's own LDS slice for the 16 sequential
 * partial sums, and nothing waits on the workgroup: the same operations in the same
 * order as k_attn_softmax, so the same bits. */
constexpr int SMW_WAVES = 4;
constexpr int SMW_PER = 48;
constexpr int SMW_MAX = SMW_PER * 64;
constexpr int SMW_ROWS = 1024;   /* rows from which a wave per row beats a workgroup per row */

__global__ __launch_bounds__(64 * SMW_WAVES) void k_attn_softmax_w(AttnArgs a) {
    __shared__ float es_all[SMW_WAVES][SMW_MAX];
    __shared__ unsigned long long etab[32];
    exp_table_to_lds(etab);
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * SMW_WAVES + wave;
    if (row >= a.T * a.H) return;   /* uniform per wave; no barrier follows */
    const int t = row / a.H, h = row % a.H;
    if (a.g.live && t >= *a.g.live) return;   /* padding token */
    const int pos0 = *a.g.pos, nr = pos0 + a.g.depth[t] + 1;
    float *s = a.S + ((size_t)t * a.H + h) * a.ldS;
    float *es = es_all[wave];
    float x[SMW_PER];
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int u = 0; u < SMW_PER; u++) {
        const int i = lane + 64 * u;
        x[u] = i < nr ? s[i] : -__builtin_huge_valf();
    }
#pragma unroll
    for (int u = 0; u < SMW_PER; u++)
        if (x[u] == x[u]) m = fmaxf(m, x[u]);
    m = wave_max_f32(m);   /* a maximum: any reduction order gives the same value */
    const float s0 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x[0])));
    if (s0 != s0) m = s0;
#pragma unroll
    for (int u = 0; u < SMW_PER; u++) {
        if (64 * u < nr) {   /* uniform */
            const int i = lane + 64 * u;
            const float e = exp_glibc_f(fadd(x[u], -m), etab);
            x[u] = e;
            if (i < nr) es[i] = e;
        }
    }
    wave_sync();
    float L = 0.0f;   /* lane < 16: partial of the elements i = lane (mod 16) */
    if (lane < 16) L = sum16_lds(es, nr, lane, L);
    L = tree16(L);
    const float sum = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(L)));
#pragma unroll
    for (int u = 0; u < SMW_PER; u++) {
        const int i = lane + 64 * u;
        if (64 * u < nr && i < nr) s[i] = fdiv(x[u], sum);
    }
}

/* o[t][h][d] = sum_v p_v * V_v[d], v in order. A workgroup sums up to four heads of
 * one token t in one KV group g, for one 64-wide d chunk: one summing wave per head
 * (lane = column d, one dependent add chain per lane), and eight loader waves.
 *
 * The chain's floor is the add latency (about 8 cycles a row); what a summing wave
 * issues besides the add must fit beside it. So each lane reads its column four rows
 * at a time (one 16-byte LDS read): the loaders store V tiles transposed, as 4-row
 * blocks of [64 columns][4 rows] (+ 4 floats of padding, which puts the 64 lanes of
 * every transposed store in 64 different banks). The p row of the head is read one
 * value per lane per 16 rows and each row's p reaches all lanes by a DPP row broadcast
 * folded into the product (v_mul_f32 with row_newbcast), so p costs no instruction.
 *
 * Loaders: 16-byte buffer loads of V rows into registers, three tiles in flight, then
 * transposed 4-byte stores into one of two V slots; p goes straight from memory into a
 * 4-slot LDS ring (LDS-direct). For a chain geometry row v of every token is cache
 * slot v, so a tile's rows need no lookup, and the buffer's range check turns rows
 * past the cache into zeros; a tree maps each row through the token's ancestor table
 * (clamped to the token's rows). Rows past the token's chain are loaded but never
 * summed. Tiles are published by a barrier after each loader's own stores landed
 * (lgkmcnt(0)); loads in flight stay in flight across it. */
constexpr int TV_ROWS = 128;            /* rows per tile */
constexpr int TV_BQ = 260;              /* floats per 4-row block: [64 columns][4 rows] + 4 */
constexpr int TV_PS = 4;                /* p ring slots */
constexpr int TV_THREADS = 768;         /* 4 summing + 8 loader waves */
constexpr int TV_SUM = 4, TV_LOAD = 8;  /* summing waves (one head each), loader waves */
/* the staging map below: loader wave lw owns tile rows 16 lw .. 16 lw + 15 (lane % 16)
 * and p half lw % 2 of head lw / 2; lane / 16 picks 4 of each 16 columns */
static_assert(TV_THREADS == 64 * (TV_SUM + TV_LOAD), "k_attn_values: 4 summing + 8 loader waves");
static_assert(TV_ROWS == 16 * TV_LOAD, "k_attn_values: each loader wave stages 16 rows of a tile");
static_assert(TV_LOAD == 2 * TV_SUM && TV_ROWS == 2 * 64, "k_attn_values: two 64-row p halves per summed head");
static_assert(TV_BQ == 4 * 64 + 4, "k_attn_values: a 4-row block holds 64 columns");

typedef unsigned int tv_u4 __attribute__((ext_vector_type(4)));

/* x of lane J of this lane's 16-lane row (DPP row_newbcast) */
template <int J>
__device__ __forceinline__ float tv_bc(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + J, 0xF, 0xF, false));
}

/* 16 rows of the chain: P holds p of row j in lane j of each 16-lane row, V[k] rows
 * 4k..4k+3 of this lane's column */
__device__ __forceinline__ void tv_sum16(float &acc, float P, const float4 (&V)[4]) {
    const float q0 = fmul(tv_bc<0>(P), V[0].x), q1 = fmul(tv_bc<1>(P), V[0].y);
    const float q2 = fmul(tv_bc<2>(P), V[0].z), q3 = fmul(tv_bc<3>(P), V[0].w);
    const float q4 = fmul(tv_bc<4>(P), V[1].x), q5 = fmul(tv_bc<5>(P), V[1].y);
    const float q6 = fmul(tv_bc<6>(P), V[1].z), q7 = fmul(tv_bc<7>(P), V[1].w);
    const float q8 = fmul(tv_bc<8>(P), V[2].x), q9 = fmul(tv_bc<9>(P), V[2].y);
    const float q10 = fmul(tv_bc<10>(P), V[2].z), q11 = fmul(tv_bc<11>(P), V[2].w);
    const float q12 = fmul(tv_bc<12>(P), V[3].x), q13 = fmul(tv_bc<13>(P), V[3].y);
    const float q14 = fmul(tv_bc<14>(P), V[3].z), q15 = fmul(tv_bc<15>(P), V[3].w);
    acc = fadd(acc, q0); acc = fadd(acc, q1); acc = fadd(acc, q2); acc = fadd(acc, q3);
    acc = fadd(acc, q4); acc = fadd(acc, q5); acc = fadd(acc, q6); acc = fadd(acc, q7);
    acc = fadd(acc, q8); acc = fadd(acc, q9); acc = fadd(acc, q10); acc = fadd(acc, q11);
    acc = fadd(acc, q12); acc = fadd(acc, q13); acc = fadd(acc, q14); acc = fadd(acc, q15);
}

/* The extra workgroups of k_attn_values read the ranges pf_p[r][0, pf_n[r]) (the weights
 * of the products after the attention, so that those find them in the memory-side cache
 * instead of HBM). The value kernel is a chain of latencies on a part of the compute
 * units; these reads run beside it on the others. */
__device__ void values_read_ahead(const AttnArgs &a, int wg) {
    for (int r = 0; r < AF_NR; r++)
        if (a.pf_p[r]) read_lines_ahead(a.pf_p[r], a.pf_n[r], wg, a.pf_wgs);
}

__global__ __launch_bounds__(TV_THREADS) void k_attn_values(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) float vt[2][(TV_ROWS / 4) * TV_BQ];
    __shared__ __attribute__((aligned(16))) float pt[TV_PS][4][TV_ROWS];
    __shared__ int anc_s[MAX_ANC];
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd;
    const int nd = (hd + 63) / 64, qpt = (grp + TV_SUM - 1) / TV_SUM;
    const int nmain = a.T * qpt * Hkv * nd;
    if ((int)blockIdx.x >= nmain) {   /* a read-ahead workgroup (uniform) */
        values_read_ahead(a, blockIdx.x - nmain);
        return;
    }
    int b = blockIdx.x;
    const int dc = b % nd;
    b /= nd;
    const int g = b % Hkv;
    b /= Hkv;
    const int hq = b % qpt, t = b / qpt;
    if (a.g.live && t >= *a.g.live) return;   /* padding token (uniform) */
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int pos0 = *a.g.pos, dep = a.g.depth[t];
    const int nr = pos0 + dep + 1;
    const int ntiles = (nr + TV_ROWS - 1) / TV_ROWS;
    const bool chain = a.g.chain != 0;
    if (!chain) {
        for (int jj = tid; jj <= dep; jj += TV_THREADS) anc_s[jj] = pos0 + a.g.anc[(size_t)t * a.g.anc_ld + jj];
        __syncthreads();
    }
    if (wave >= TV_SUM) {
        /* loader wave lw: rows 16 lw + lane % 16 of each tile, columns 16 cb + 4 (lane / 16)
         * .. + 3 for cb = 0..3, and half lw % 2 of head lw / 2's p row */
        const int lw = wave - TV_SUM, r = lane & 15, cg = lane >> 4, half = lw & 1;
        const __amdgpu_buffer_rsrc_t vrs =
            __builtin_amdgcn_make_buffer_rsrc((void *)(a.vc + (size_t)g * a.cap * hd), 0, a.cap * hd * 4, 0x00020000);
        int coff[4];
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
            const int col = dc * 64 + 16 * cb + 4 * cg;
            coff[cb] = (col < hd ? col : 0) * 4;
        }
        const int phh = hq * TV_SUM + (lw >> 1);
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(a.S + ((size_t)t * a.H + (size_t)g * grp + (phh < grp ? phh : 0)) * a.ldS), 0, a.ldS * 4, 0x00020000);
        const int hd4 = hd * 4, roff = r * hd4;
        /* word of (row 16 lw + r, column 16 cb + 4 cg + e): bank 16 lw + r + 16 cg + 4 e mod 64 */
        const int wbase = (4 * lw + (r >> 2)) * TV_BQ + 16 * cg + (r & 3);
        auto store = [&](int slot, const tv_u4 (&R)[4]) {
            float *w = &vt[slot][wbase];
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                w[64 * cb + 0] = __uint_as_float(R[cb].x);
                w[64 * cb + 4] = __uint_as_float(R[cb].y);
                w[64 * cb + 8] = __uint_as_float(R[cb].z);
                w[64 * cb + 12] = __uint_as_float(R[cb].w);
            }
        };
        auto run = [&](auto chain_tag) {
            constexpr bool CHAIN = decltype(chain_tag)::value;
            auto load = [&](int i, tv_u4 (&R)[4]) {
                const int vb = i * TV_ROWS;
                if constexpr (CHAIN) {
                    const int vo = roff + (vb + 16 * lw) * hd4;
#pragma unroll
                    for (int cb = 0; cb < 4; cb++) R[cb] = __builtin_amdgcn_raw_buffer_load_b128(vrs, vo + coff[cb], 0, 0);
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(prs, (__attribute__((address_space(3))) void *)&pt[i % TV_PS][lw >> 1][64 * half],
                                                             4, (vb + 64 * half + lane) * 4, 0, 0, 0);
                } else {
                    int v = vb + 16 * lw + r;
                    v = v < nr ? v : nr - 1;
                    const int an = anc_s[v > pos0 ? v - pos0 : 0];
                    const int srow = v < pos0 ? v : an;
#pragma unroll
                    for (int cb = 0; cb < 4; cb++) R[cb] = __builtin_amdgcn_raw_buffer_load_b128(vrs, srow * hd4 + coff[cb], 0, 0);
                    int vp = vb + 64 * half + lane;
                    vp = vp < nr ? vp : nr - 1;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(prs, (__attribute__((address_space(3))) void *)&pt[i % TV_PS][lw >> 1][64 * half],
                                                             4, vp * 4, 0, 0, 0);
                }
            };
            tv_u4 R0[4], R1[4], R2[4];
            load(0, R0);
            load(1, R1);
            load(2, R2);
            HX_WAIT_VMCNT(10);
            store(0, R0);
            /* step i: tile i is published; tile i + 3 is loaded into the registers tile i came
             * from; tile i + 1 is stored into the slot tile i - 1 was summed from. The loop
             * has no exit inside its body, so the compiler keeps the exact load counts. */
#define TV_STEP(i_, RL, RW)                                                                 \
            __builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) only */                       \
            __builtin_amdgcn_s_barrier();                                                   \
            load((i_) + 3, RL);                                                             \
            HX_WAIT_VMCNT(10);                                                              \
            store(((i_) + 1) & 1, RW);
            int i = 0;
            for (; i + 3 <= ntiles; i += 3) {
                TV_STEP(i, R0, R1)
                TV_STEP(i + 1, R1, R2)
                TV_STEP(i + 2, R2, R0)
            }
            /* the last one or two steps load nothing (their tiles would lie past the
             * rows): the loads of the tiles still to publish are waited for in full. A
             * step's load count is not a bound here, because the compiler drops register
             * loads whose values are never used, so a count-based wait could let the
             * LDS-direct p rows of the tile being published still be in flight */
#define TV_LAST(i_, RW)                                                                     \
            __builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) only */                       \
            __builtin_amdgcn_s_barrier();                                                   \
            HX_WAIT_VMCNT(0);                                                               \
            store(((i_) + 1) & 1, RW);
            if (i < ntiles) {
                TV_LAST(i, R1)
                if (i + 1 < ntiles) {
                    TV_LAST(i + 1, R2)
                }
            }
#undef TV_LAST
#undef TV_STEP
        };
        if (chain) run(std::true_type{});
        else run(std::false_type{});
        HX_WAIT_VMCNT(0);              /* no LDS write may land after the workgroup ends */
    } else {
        const int hh = hq * TV_SUM + wave;
        const bool live = hh < grp;
        const int h = g * grp + (live ? hh : 0);
        float acc = 0.0f;
        for (int i = 0; i < ntiles; i++) {
            __syncthreads();
            const int slot = i & 1, nv = nr - i * TV_ROWS;
            const float4 *vw = (const float4 *)&vt[slot][lane * 4];
            if (nv >= TV_ROWS) {
                const float *pw1 = &pt[i % TV_PS][wave][lane & 15];
                float4 VA[4], VB[4];
                float PA, PB;
                /* one group of 16 rows is read while the previous one is summed; the
                 * scheduling barriers keep the compiler from sinking the reads */
#define TV_RD(V_, P_, g_) \
                _Pragma("unroll") for (int j = 0; j < 4; j++) V_[j] = vw[((g_) * 4 + j) * (TV_BQ / 4)]; P_ = pw1[(g_) * 16];
#define TV_SB __builtin_amdgcn_sched_barrier(0);
                TV_RD(VA, PA, 0)
                TV_RD(VB, PB, 1) TV_SB tv_sum16(acc, PA, VA); TV_SB
                TV_RD(VA, PA, 2) TV_SB tv_sum16(acc, PB, VB); TV_SB
                TV_RD(VB, PB, 3) TV_SB tv_sum16(acc, PA, VA); TV_SB
                TV_RD(VA, PA, 4) TV_SB tv_sum16(acc, PB, VB); TV_SB
                TV_RD(VB, PB, 5) TV_SB tv_sum16(acc, PA, VA); TV_SB
                TV_RD(VA, PA, 6) TV_SB tv_sum16(acc, PB, VB); TV_SB
                TV_RD(VB, PB, 7) TV_SB tv_sum16(acc, PA, VA); TV_SB
                tv_sum16(acc, PB, VB);
#undef TV_SB
#undef TV_RD
            } else {
                const float *pv = &pt[i % TV_PS][wave][0];
                for (int rr = 0; rr < nv; rr++) acc = fadd(acc, fmul(pv[rr], vt[slot][(rr >> 2) * TV_BQ + lane * 4 + (rr & 3)]));
            }
        }
        const int d = dc * 64 + lane;
        if (live && d < hd) a.out[(size_t)t * a.H * hd + (size_t)h * hd + d] = acc;
        if (a.qo_on && live) quant_block_wave(acc, a.qo, a.qo_hm ? h * a.T + t : t, a.qo_hm ? dc : h * (hd >> 6) + dc);
    }
}


constexpr long long TV_WIDE = 2048;     /* summing waves (one head each) from which the wide shapes pay */

/* The same sums when there are many chains (a tree's tokens, MLA's 128 heads): NS
 * summing waves of R heads each (NS * R heads of one KV group per workgroup, R
 * independent chains per lane sharing each V read), NL loader waves, ROWS rows per tile
 * (16 per loader wave). Each staged V tile then serves more chains, and several summing
 * waves share each SIMD (the single-chain kernel above keeps one per SIMD, where the
 * latency of its one chain is the floor). p of the workgroup's heads: load k of loader
 * lw takes 64 consecutive rows of one head (element f = (k NL + lw) 64 + lane of the
 * [head][row] tile). */
template <int NS, int NL, int R, int ROWS>
__global__ __launch_bounds__(64 * (NS + NL)) void k_attn_values_w(AttnArgs a) {
    constexpr int NT = 64 * (NS + NL), NH = NS * R, PL = NH * ROWS / (NL * 64), NG = ROWS / 16;
    constexpr int WV = 2 * (4 + PL);   /* loads of two tiles: the loads still in flight when a tile is stored */
    static_assert(ROWS == 16 * NL, "k_attn_values: each loader wave stages 16 rows of a tile");
    static_assert(ROWS % 64 == 0 && (NH * ROWS) % (NL * 64) == 0, "k_attn_values: p in loads of 64 rows of one head");
    static_assert(NG % 2 == 0 && WV < 64, "k_attn_values: groups of 16 rows in pairs; vmcnt fits");
    __shared__ __attribute__((aligned(16))) float vt[2][(ROWS / 4) * TV_BQ];
    __shared__ __attribute__((aligned(16))) float pt[TV_PS][NH][ROWS];
    __shared__ int anc_s[MAX_ANC];
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd;
    const int nd = (hd + 63) / 64, qpt = (grp + NH - 1) / NH;
    int b = blockIdx.x;
    const int dc = b % nd;
    b /= nd;
    const int g = b % Hkv;
    b /= Hkv;
    const int hq = b % qpt, t = b / qpt;
    if (a.g.live && t >= *a.g.live) return;   /* padding token (uniform) */
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int pos0 = *a.g.pos, dep = a.g.depth[t];
    const int nr = pos0 + dep + 1;
    const int ntiles = (nr + ROWS - 1) / ROWS;
    const bool chain = a.g.chain != 0;
    if (!chain) {
        for (int jj = tid; jj <= dep; jj += NT) anc_s[jj] = pos0 + a.g.anc[(size_t)t * a.g.anc_ld + jj];
        __syncthreads();
    }
    if (wave >= NS) {
        /* loader wave lw: rows 16 lw + lane % 16 of each tile, columns 16 cb + 4 (lane / 16)
         * .. + 3 for cb = 0..3, and PL 64-row pieces of the heads' p rows */
        const int lw = wave - NS, r = lane & 15, cg = lane >> 4;
        const __amdgpu_buffer_rsrc_t vrs =
            __builtin_amdgcn_make_buffer_rsrc((void *)(a.vc + (size_t)g * a.cap * hd), 0, a.cap * hd * 4, 0x00020000);
        int coff[4];
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
            const int col = dc * 64 + 16 * cb + 4 * cg;
            coff[cb] = (col < hd ? col : 0) * 4;
        }
        /* p piece k: 64 rows from row pro(k) of local head phl(k), from S by an LDS-direct load */
        const float *srow0 = a.S + ((size_t)t * a.H + (size_t)g * grp) * a.ldS;
        auto pload = [&](int k, int slot, auto voff) {
            const int f0 = (k * NL + lw) * 64, phl = f0 / ROWS, pro = f0 % ROWS, phh = hq * NH + phl;
            const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(srow0 + (size_t)(phh < grp ? phh : 0) * a.ldS), 0, a.ldS * 4, 0x00020000);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(prs, (__attribute__((address_space(3))) void *)&pt[slot][phl][pro], 4,
                                                     voff(pro) * 4, 0, 0, 0);
        };
        const int hd4 = hd * 4, roff = r * hd4;
        /* word of (row 16 lw + r, column 16 cb + 4 cg + e): bank 16 lw + r + 16 cg + 4 e mod 64 */
        const int wbase = (4 * lw + (r >> 2)) * TV_BQ + 16 * cg + (r & 3);
        auto store = [&](int slot, const tv_u4 (&Rg)[4]) {
            float *w = &vt[slot][wbase];
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                w[64 * cb + 0] = __uint_as_float(Rg[cb].x);
                w[64 * cb + 4] = __uint_as_float(Rg[cb].y);
                w[64 * cb + 8] = __uint_as_float(Rg[cb].z);
                w[64 * cb + 12] = __uint_as_float(Rg[cb].w);
            }
        };
        auto run = [&](auto chain_tag) {
            constexpr bool CHAIN = decltype(chain_tag)::value;
            auto load = [&](int i, tv_u4 (&Rg)[4]) {
                const int vb = i * ROWS;
                if constexpr (CHAIN) {
                    const int vo = roff + (vb + 16 * lw) * hd4;
#pragma unroll
                    for (int cb = 0; cb < 4; cb++) Rg[cb] = __builtin_amdgcn_raw_buffer_load_b128(vrs, vo + coff[cb], 0, 0);
#pragma unroll
                    for (int k = 0; k < PL; k++) pload(k, i % TV_PS, [&](int pro) { return vb + pro + lane; });
                } else {
                    int v = vb + 16 * lw + r;
                    v = v < nr ? v : nr - 1;
                    const int an = anc_s[v > pos0 ? v - pos0 : 0];
                    const int srow = v < pos0 ? v : an;
#pragma unroll
                    for (int cb = 0; cb < 4; cb++) Rg[cb] = __builtin_amdgcn_raw_buffer_load_b128(vrs, srow * hd4 + coff[cb], 0, 0);
#pragma unroll
                    for (int k = 0; k < PL; k++)
                        pload(k, i % TV_PS, [&](int pro) {
                            const int vp = vb + pro + lane;
                            return vp < nr ? vp : nr - 1;
                        });
                }
            };
            tv_u4 R0[4], R1[4], R2[4];
            load(0, R0);
            load(1, R1);
            load(2, R2);
            HX_WAIT_VMCNT(WV);
            store(0, R0);
            /* step i: tile i is published; tile i + 3 is loaded into the registers tile i came
             * from; tile i + 1 is stored into the slot tile i - 1 was summed from. The loop
             * has no exit inside its body, so the compiler keeps the exact load counts. */
#define TV_STEP(i_, RL, RW)                                                                 \
            __builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) only */                       \
            __builtin_amdgcn_s_barrier();                                                   \
            load((i_) + 3, RL);                                                             \
            HX_WAIT_VMCNT(WV);                                                              \
            store(((i_) + 1) & 1, RW);
            int i = 0;
            for (; i + 3 <= ntiles; i += 3) {
                TV_STEP(i, R0, R1)
                TV_STEP(i + 1, R1, R2)
                TV_STEP(i + 2, R2, R0)
            }
            /* the last one or two steps load nothing (their tiles would lie past the
             * rows): the loads of the tiles still to publish are waited for in full. A
             * step's load count is not a bound here, because the compiler drops register
             * loads whose values are never used, so a count-based wait could let the
             * LDS-direct p rows of the tile being published still be in flight */
#define TV_LAST(i_, RW)                                                                     \
            __builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) only */                       \
            __builtin_amdgcn_s_barrier();                                                   \
            HX_WAIT_VMCNT(0);                                                               \
            store(((i_) + 1) & 1, RW);
            if (i < ntiles) {
                TV_LAST(i, R1)
                if (i + 1 < ntiles) {
                    TV_LAST(i + 1, R2)
                }
            }
#undef TV_LAST
#undef TV_STEP
        };
        if (chain) run(std::true_type{});
        else run(std::false_type{});
        HX_WAIT_VMCNT(0);              /* no LDS write may land after the workgroup ends */
    } else {
        bool live[R];
        int h[R];
        float acc[R];
#pragma unroll
        for (int rr = 0; rr < R; rr++) {
            const int hh = hq * NH + wave * R + rr;
            live[rr] = hh < grp;
            h[rr] = g * grp + (live[rr] ? hh : 0);
            acc[rr] = 0.0f;
        }
        for (int i = 0; i < ntiles; i++) {
            __syncthreads();
            const int slot = i & 1, nv = nr - i * ROWS;
            const float4 *vw = (const float4 *)&vt[slot][lane * 4];
            if (nv >= ROWS) {
                const float *pw = &pt[i % TV_PS][wave * R][lane & 15];
                /* group by group of 16 rows: the R chains of a lane and the other summing
                 * waves of the SIMD cover the latency of the reads */
                for (int gr = 0; gr < NG; gr++) {
                    float4 V[4];
                    float P[R];
#pragma unroll
                    for (int j = 0; j < 4; j++) V[j] = vw[(gr * 4 + j) * (TV_BQ / 4)];
#pragma unroll
                    for (int rr = 0; rr < R; rr++) P[rr] = pw[rr * ROWS + gr * 16];
#pragma unroll
                    for (int rr = 0; rr < R; rr++) tv_sum16(acc[rr], P[rr], V);
                }
            } else {
                const float *pv = &pt[i % TV_PS][wave * R][0];
                for (int rw = 0; rw < nv; rw++) {
                    const float vv = vt[slot][(rw >> 2) * TV_BQ + lane * 4 + (rw & 3)];
#pragma unroll
                    for (int rr = 0; rr < R; rr++) acc[rr] = fadd(acc[rr], fmul(pv[rr * ROWS + rw], vv));
                }
            }
        }
        const int d = dc * 64 + lane;
#pragma unroll
        for (int rr = 0; rr < R; rr++) {
            if (live[rr] && d < hd) a.out[(size_t)t * a.H * hd + (size_t)h[rr] * hd + d] = acc[rr];
            if (a.qo_on && live[rr])
                quant_block_wave(acc[rr], a.qo, a.qo_hm ? h[rr] * a.T + t : t, a.qo_hm ? dc : h[rr] * (hd >> 6) + dc);
        }
    }
}

/* ---- chunked attention ------------------------------------------------------------
 * The engine's default order for GQA layers (a documented tolerance against the
 * reference's order above, not bit-exact to it): the token's row list in chunks of 64
 * rows (chunk c = logical rows 64c .. 64c+63), per chunk and head
 *   s_i = scale * dotf(q, k_i)        dotf: fmaf over d = 0 .. hd-1 in order from 0.0f
 *   m_c = max s_i (NaN if one is NaN), e_i = exp(s_i - m_c)
 *   l_c = pairwise sum of the 64 positions (e_i, 0 past the token's rows), over the lanes
 *         (ac_pairwise64)
 *   o_c[d] = fmaf(e_i, v_i[d], o) over the chunk's rows in order from 0.0f
 * and then, over the chunks in order, M = max m_c, w_c = exp(m_c - M),
 * L = fmaf(l_c, w_c, L), O[d] = fmaf(o_c[d], w_c, O), out = O / L. Each step depends on
 * the token's row list only (batch == sequential, tree node == chain root -> node).
 *
 * k_attn_chunk: one workgroup per (chunk, KV group, block of tokens), 8 waves. The
 * chunk's 64 K rows, its V rows (transposed in 4-row blocks) and the block's queries go
 * to LDS by LDS-direct loads, V last, so that the scores run while V lands. An item is
 * RW heads of one token: scores with one key per lane (queries read as LDS broadcasts),
 * the item's e kept in LDS, then the value sums with one column per lane. A tree node's
 * own rows (logical rows past pos0, at its ancestors' slots) are read from the cache
 * directly. k_attn_combine: one wave per (token, head, 64 columns) folds the chunks. */
constexpr int AC_CH = 64;          /* rows per chunk */
constexpr int AC_WAVES = 8;
constexpr int AC_IPW = 4;          /* items per wave */
constexpr int AC_QMAX = 12288;     /* floats of staged queries */

__device__ __forceinline__ float ac_nanmax(float a, float b) { return a != a || b != b ? a + b : fmaxf(a, b); }

/* the pairwise tree over the 64 lanes ((x0 + x1) + (x2 + x3)) + ..., in every lane: pairs
 * and quads by quad_perm, 8 and 16 lanes by the half-row and row mirrors (every lane of a
 * quad, then of a half-row, already holds the same partial), then the four row sums */
__device__ __forceinline__ float ac_pairwise64(float x) {
#define HX_PW_STEP(CTRL) x = fadd(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false)));
    HX_PW_STEP(0xB1)    /* quad_perm [1, 0, 3, 2] */
    HX_PW_STEP(0x4E)    /* quad_perm [2, 3, 0, 1] */
    HX_PW_STEP(0x141)   /* row_half_mirror */
    HX_PW_STEP(0x140)   /* row_mirror */
#undef HX_PW_STEP
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
    return fadd(fadd(r0, r1), fadd(r2, r3));
}

template <int HD, int RW>
__global__ __launch_bounds__(64 * AC_WAVES) void k_attn_chunk(AttnArgs a, int ntb, int nblk, int ncg) {
    constexpr int ND = HD / 64, KLD = HD + 4, VQ = 4 * HD + 4;
    constexpr int NKW = AC_CH * ND / AC_WAVES;   /* K loads per wave (64 dwords each) */
    constexpr int NVW = AC_CH * ND / AC_WAVES;   /* V loads per wave */
    static_assert(HD % 64 == 0 && (AC_CH * ND) % AC_WAVES == 0 && NKW + NVW < 48, "k_attn_chunk: staging map");
    __shared__ __attribute__((aligned(16))) float ks[AC_CH * KLD];
    __shared__ __attribute__((aligned(16))) float vq[(AC_CH / 4) * VQ];
    __shared__ __attribute__((aligned(16))) float qs[AC_QMAX];
    __shared__ __attribute__((aligned(16))) float es[AC_WAVES][AC_IPW][RW][AC_CH];
    __shared__ unsigned long long etab[32];
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd;
    int b = blockIdx.x;
    const int tb = b % nblk;
    b /= nblk;
    const int g = b % Hkv;
    const int c = ncg - 1 - b / Hkv;             /* the last (partial) chunk first */
    const int r0 = c * AC_CH;
    const int t0 = tb * ntb, nt = min(ntb, a.T - t0);
    if (nt <= 0) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    /* lane i holds the depth of token t0 + i (ntb <= 64), read once */
    const int pos0 = *a.g.pos;
    const int dep_l = lane < nt ? a.g.depth[t0 + lane] : 0;
    const int dmax = (int)wave_max_u32((unsigned)dep_l);
    if (pos0 + dmax + 1 <= r0) return;           /* no token of the block reaches the chunk */
    /* rows of the chunk that every token reads from the slot of the same index */
    const int kshared = min(max((a.g.chain ? pos0 + a.T : pos0) - r0, 0), AC_CH);
    const float *kbase = a.kc + (size_t)g * a.cap * hd, *vbase = a.vc + (size_t)g * a.cap * hd;
    exp_table_to_lds(etab);
    {
        const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc((void *)a.q, 0, a.T * a.H * hd * 4, 0x00020000);
        const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void *)kbase, 0, a.cap * hd * 4, 0x00020000);
        const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void *)vbase, 0, a.cap * hd * 4, 0x00020000);
        /* K: load f = k * 8 + wave is row f / ND, columns 64 (f % ND) .. + 63 */
#pragma unroll
        for (int k = 0; k < NKW; k++) {
            const int f = k * AC_WAVES + wave, j = f / ND, cb = f % ND;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (__attribute__((address_space(3))) void *)&ks[j * KLD + 64 * cb], 4,
                                                     ((r0 + j) * hd + 64 * cb + lane) * 4, 0, 0, 0);
        }
        /* queries of the block: a token's grp heads are grp * hd contiguous floats; load u
         * of token tl is its floats 64 u .. 64 u + 63 */
        const int qrow = grp * ND;
        for (int tl = 0; tl < nt; tl++)
            for (int u = wave; u < qrow; u += AC_WAVES)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    qrs, (__attribute__((address_space(3))) void *)&qs[tl * grp * HD + 64 * u], 4,
                    (((t0 + tl) * a.H + g * grp) * hd + 64 * u + lane) * 4, 0, 0, 0);
        /* V, transposed: load f is rows 4 qb .. 4 qb + 3 of columns 16 u .. 16 u + 15;
         * lane l takes row 4 qb + l % 4 of column 16 u + l / 4, so the 64 dwords land in
         * order in block qb: [column][4 rows] */
#pragma unroll
        for (int k = 0; k < NVW; k++) {
            const int f = k * AC_WAVES + wave, qb = f / (HD / 16), u = f % (HD / 16);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                vrs, (__attribute__((address_space(3))) void *)&vq[qb * VQ + 64 * u], 4,
                ((r0 + 4 * qb + (lane & 3)) * hd + 16 * u + (lane >> 2)) * 4, 0, 0, 0);
        }
        HX_WAIT_VMCNT(NVW);                      /* this wave's K and query loads landed */
        __builtin_amdgcn_s_waitcnt(0xC07F);      /* and its exp table stores */
        __builtin_amdgcn_s_barrier();            /* ... and every other wave's */
    }
    static_assert(AC_WAVES * AC_IPW <= 64, "k_attn_chunk: a block's tokens fit one wave's lanes");
    const int ipt = grp / RW, nitems = nt * ipt;
    const float scale = a.scale;
    /* scores, e, m, l of this wave's items */
#pragma unroll 1
    for (int k = 0; k < AC_IPW; k++) {
        const int it = wave + k * AC_WAVES;
        if (it >= nitems) break;
        const int tl = it / ipt, hb = it % ipt, t = t0 + tl;
        const int nk = min(pos0 + __builtin_amdgcn_readlane(dep_l, tl) + 1 - r0, AC_CH);
        if (nk <= 0) continue;
        const bool valid = lane < nk;
        float acc[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) acc[r] = 0.0f;
        const float4 *qv4 = (const float4 *)&qs[(tl * grp + hb * RW) * HD];
        if (valid && lane < kshared) {
            const float4 *kv4 = (const float4 *)&ks[lane * KLD];
#pragma unroll
            for (int d4 = 0; d4 < HD / 4; d4++) {
                const float4 kv = kv4[d4];
#pragma unroll
                for (int r = 0; r < RW; r++) {
                    const float4 qv = qv4[r * (HD / 4) + d4];
                    acc[r] = __builtin_fmaf(qv.x, kv.x, acc[r]);
                    acc[r] = __builtin_fmaf(qv.y, kv.y, acc[r]);
                    acc[r] = __builtin_fmaf(qv.z, kv.z, acc[r]);
                    acc[r] = __builtin_fmaf(qv.w, kv.w, acc[r]);
                }
            }
        } else if (valid) {
            /* a tree node's own rows: logical row r0 + lane >= pos0 at its ancestor's slot */
            const int slot = pos0 + a.g.anc[(size_t)t * a.g.anc_ld + (r0 + lane - pos0)];
            const float4 *kv4 = (const float4 *)(kbase + (size_t)slot * hd);
#pragma unroll 2
            for (int d4 = 0; d4 < HD / 4; d4++) {
                const float4 kv = kv4[d4];
#pragma unroll
                for (int r = 0; r < RW; r++) {
                    const float4 qv = qv4[r * (HD / 4) + d4];
                    acc[r] = __builtin_fmaf(qv.x, kv.x, acc[r]);
                    acc[r] = __builtin_fmaf(qv.y, kv.y, acc[r]);
                    acc[r] = __builtin_fmaf(qv.z, kv.z, acc[r]);
                    acc[r] = __builtin_fmaf(qv.w, kv.w, acc[r]);
                }
            }
        }
        const size_t row0 = (size_t)t * a.H + g * grp + hb * RW;
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const float sv = valid ? fmul(scale, acc[r]) : -__builtin_huge_valf();
            const bool anynan = __builtin_amdgcn_ballot_w64(sv != sv) != 0;
            const float m = anynan ? __builtin_nanf("") : wave_max_f32(sv);
            const float e = valid ? exp_glibc_f(fsub(sv, m), etab) : 0.0f;
            const float l = ac_pairwise64(e);
            es[wave][k][r][lane] = e;
            if (lane == 0) {
                a.pm[(row0 + r) * a.nc_ld + c] = m;
                a.pl[(row0 + r) * a.nc_ld + c] = l;
            }
        }
    }
    HX_WAIT_VMCNT(0);                            /* this wave's V loads landed */
    __builtin_amdgcn_s_waitcnt(0xC07F);          /* and its e stores */
    __builtin_amdgcn_s_barrier();
    /* value sums of this wave's items: lane = column */
#pragma unroll 1
    for (int k = 0; k < AC_IPW; k++) {
        const int it = wave + k * AC_WAVES;
        if (it >= nitems) break;
        const int tl = it / ipt, hb = it % ipt, t = t0 + tl;
        const int nk = min(pos0 + __builtin_amdgcn_readlane(dep_l, tl) + 1 - r0, AC_CH);
        if (nk <= 0) continue;
        const int jl = min(nk, kshared);
        const size_t row0 = (size_t)t * a.H + g * grp + hb * RW;
#pragma unroll 1
        for (int cb = 0; cb < ND; cb++) {
            const int d = 64 * cb + lane;
            float acc[RW];
#pragma unroll
            for (int r = 0; r < RW; r++) acc[r] = 0.0f;
            int j = 0;
            if (jl == AC_CH) {
                /* a whole chunk in LDS (all but the last one or two): straight-line code */
#pragma unroll
                for (int q = 0; q < AC_CH / 4; q++) {
                    const float4 vv = *(const float4 *)&vq[q * VQ + 4 * d];
#pragma unroll
                    for (int r = 0; r < RW; r++) {
                        const float4 ev = *(const float4 *)&es[wave][k][r][4 * q];
                        acc[r] = __builtin_fmaf(ev.x, vv.x, acc[r]);
                        acc[r] = __builtin_fmaf(ev.y, vv.y, acc[r]);
                        acc[r] = __builtin_fmaf(ev.z, vv.z, acc[r]);
                        acc[r] = __builtin_fmaf(ev.w, vv.w, acc[r]);
                    }
                }
                j = AC_CH;
            }
#pragma unroll 4
            for (; j + 4 <= jl; j += 4) {
                const float4 vv = *(const float4 *)&vq[(j >> 2) * VQ + 4 * d];
#pragma unroll
                for (int r = 0; r < RW; r++) {
                    const float4 ev = *(const float4 *)&es[wave][k][r][j];
                    acc[r] = __builtin_fmaf(ev.x, vv.x, acc[r]);
                    acc[r] = __builtin_fmaf(ev.y, vv.y, acc[r]);
                    acc[r] = __builtin_fmaf(ev.z, vv.z, acc[r]);
                    acc[r] = __builtin_fmaf(ev.w, vv.w, acc[r]);
                }
            }
            for (; j < jl; j++) {
                const float vv = vq[(j >> 2) * VQ + 4 * d + (j & 3)];
#pragma unroll
                for (int r = 0; r < RW; r++) acc[r] = __builtin_fmaf(es[wave][k][r][j], vv, acc[r]);
            }
            for (; j < nk; j++) {
                const int slot = pos0 + a.g.anc[(size_t)t * a.g.anc_ld + (r0 + j - pos0)];
                const float vv = vbase[(size_t)slot * hd + d];
#pragma unroll
                for (int r = 0; r < RW; r++) acc[r] = __builtin_fmaf(es[wave][k][r][j], vv, acc[r]);
            }
#pragma unroll
            for (int r = 0; r < RW; r++) a.po[((row0 + r) * a.nc_ld + c) * HD + d] = acc[r];
        }
    }
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a) {
    constexpr int ND = HD / 64;
    __shared__ unsigned long long etab[32];
    exp_table_to_lds(etab);
    __syncthreads();
    const int idx = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (idx >= a.T * a.H * ND) return;
    const int cb = idx % ND, row = idx / ND, t = row / a.H, h = row % a.H;
    const int nr = *a.g.pos + a.g.depth[t] + 1, nc = (nr + AC_CH - 1) / AC_CH;
    const float *pm = a.pm + (size_t)row * a.nc_ld, *pl = a.pl + (size_t)row * a.nc_ld;
    const float *po = a.po + (size_t)row * a.nc_ld * HD + 64 * cb + lane;
    /* M over the chunks, lane c % 64 holding chunk c (a maximum: any order) */
    float mx = -__builtin_huge_valf();
    bool nan = false;
    for (int c = lane; c < nc; c += 64) {
        const float v = pm[c];
        nan |= v != v;
        mx = fmaxf(mx, v);
    }
    const bool anynan = __builtin_amdgcn_ballot_w64(nan) != 0;
    const float M = anynan ? __builtin_nanf("") : wave_max_f32(mx);
    /* 64 chunks at a time: lane j computes w and holds l of chunk c0 + j; the folds over
     * the chunks in order take them by readlane */
    float L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += 64) {
        const int c = c0 + lane, n = min(64, nc - c0);
        const float w = c < nc ? exp_glibc_f(fsub(pm[c], M), etab) : 0.0f;
        const float l = c < nc ? pl[c] : 0.0f;
        const float *pc = po + (size_t)c0 * HD;
        int j = 0;
        for (; j + 4 <= n; j += 4) {
            float ov[4];
#pragma unroll
            for (int u = 0; u < 4; u++) ov[u] = pc[(size_t)(j + u) * HD];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j + u));
                L = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), j + u)), wj, L);
                O = __builtin_fmaf(ov[u], wj, O);
            }
        }
        for (; j < n; j++) {
            const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
            L = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), j)), wj, L);
            O = __builtin_fmaf(pc[(size_t)j * HD], wj, O);
        }
    }
    const float out = fdiv(O, L);
    a.out[(size_t)t * a.H * HD + (size_t)h * HD + 64 * cb + lane] = out;
    if (a.qo_on) quant_block_wave(out, a.qo, a.qo_hm ? h * a.T + t : t, a.qo_hm ? cb : h * ND + cb);
}

} // namespace

namespace hxl {

/* a.post (the fused QKV post-step) is set only for head_dim a multiple of 64 up to 256,
 * which takes the k_attn_scores16 launch below */
void attention_scores(const AttnArgs &a, hipStream_t st) {
    const int max_nr = a.g.nr_max;
    if (a.g.chain && a.T <= ST_TMAX && a.hd == 512) {
        const int nhb = (a.H / a.Hkv + ST_HB - 1) / ST_HB, grid = ((max_nr + 63) / 64) * a.Hkv * nhb;
        if (grid >= 128) {
            k_attn_scores16t<32><<<grid, 1024, 0, st>>>(a, nhb, ST_HB);
            return;
        }
    }
    if (a.hd % 64 == 0 && a.hd <= 512) {
#define HX_S16(HI_)                                                                         \
        {                                                                                   \
            constexpr int rb = 16 * s16_np<HI_>();                                          \
            const int grid = ((max_nr + rb - 1) / rb) * a.T * a.Hkv;                       \
            if (a.post) k_attn_scores16<HI_, (HI_ <= 16)><<<grid, 256, 0, st>>>(a);         \
            else k_attn_scores16<HI_, false><<<grid, 256, 0, st>>>(a);                      \
            return;                                                                         \
        }
        switch (a.hd / 16) {
        case 4: HX_S16(4)
        case 8: HX_S16(8)
        case 12: HX_S16(12)
        case 16: HX_S16(16)
        case 20: HX_S16(20)
        case 24: HX_S16(24)
        case 28: HX_S16(28)
        default: HX_S16(32)
        }
#undef HX_S16
    }
    const int nchunks = (max_nr + SC_ROWS - 1) / SC_ROWS;
    const int grp = a.H / a.Hkv, nsc = nchunks * a.T * a.Hkv;
    if (grp % 8 == 0) k_attn_scores<8><<<nsc, SC_ROWS, 0, st>>>(a);
    else if (grp % 4 == 0) k_attn_scores<4><<<nsc, SC_ROWS, 0, st>>>(a);
    else if (grp % 2 == 0) k_attn_scores<2><<<nsc, SC_ROWS, 0, st>>>(a);
    else k_attn_scores<1><<<nsc, SC_ROWS, 0, st>>>(a);
}

void attention_finish(const AttnArgs &a, hipStream_t st) {
    const int grp = a.H / a.Hkv, nd = (a.hd + 63) / 64;
    if (a.g.nr_max <= SMW_MAX && a.T * a.H >= SMW_ROWS)
        k_attn_softmax_w<<<(a.T * a.H + SMW_WAVES - 1) / SMW_WAVES, 64 * SMW_WAVES, 0, st>>>(a);
    else
        k_attn_softmax<<<a.T * a.H, SM_T, 0, st>>>(a);
    const bool wide = (long long)a.T * a.H * nd >= TV_WIDE;
#define HX_TV(NS_, NL_, R_, ROWS_)                                                                     \
    {                                                                                                  \
        const int qpt = (grp + NS_ * R_ - 1) / (NS_ * R_);                                             \
        k_attn_values_w<NS_, NL_, R_, ROWS_><<<a.T * qpt * a.Hkv * nd, 64 * (NS_ + NL_), 0, st>>>(a);  \
        return;                                                                                        \
    }
    /* groups of 8 or more heads: one head per summing wave, 8 of them (the tree's 85
     * tokens: 16.91 ms per step against 17.04 with two heads per wave on 4 waves, 17.97
     * with 8 loader waves and 128-row tiles, 19.91 with four heads per wave; MLA's 128
     * heads: 27.08 against 27.50 with two heads per wave on 8 waves, 28.4 with 12) */
    if (wide && grp >= 8) HX_TV(8, 4, 1, 64)
#undef HX_TV
    const int qpt = (grp + TV_SUM - 1) / TV_SUM;
    k_attn_values<<<a.T * qpt * a.Hkv * nd + a.pf_wgs, TV_THREADS, 0, st>>>(a);
}

/* the items of a block (grp / rw per token) must fit the block's waves: k_attn_chunk
 * processes items wave + k AC_WAVES, k < AC_IPW, only */
bool attention_chunked_ok(int hd, int grp) {
    const int rw = grp % 4 == 0 ? 4 : grp % 2 == 0 ? 2 : 1;
    return (hd == 64 || hd == 128) && grp >= 1 && grp * hd <= AC_QMAX && grp <= 32 * 4 && grp / rw <= AC_WAVES * AC_IPW;
}

void attention_chunked(const AttnArgs &a, hipStream_t st) {
    const int grp = a.H / a.Hkv, rw = grp % 4 == 0 ? 4 : grp % 2 == 0 ? 2 : 1, ipt = grp / rw;
    const int ntb_max = std::max(1, std::min(AC_WAVES * AC_IPW / ipt, AC_QMAX / (grp * a.hd)));
    const int nblk = (a.T + ntb_max - 1) / ntb_max, ntb = (a.T + nblk - 1) / nblk;
    const int ncg = (a.g.nr_max + AC_CH - 1) / AC_CH;
    const int grid = ncg * a.Hkv * nblk, nc_rows = a.T * a.H * (a.hd / 64);
#define HX_AC(HD_, RW_) k_attn_chunk<HD_, RW_><<<grid, 64 * AC_WAVES, 0, st>>>(a, ntb, nblk, ncg)
    if (a.hd == 128) {
        if (rw == 4) HX_AC(128, 4); else if (rw == 2) HX_AC(128, 2); else HX_AC(128, 1);
        k_attn_combine<128><<<(nc_rows + 3) / 4, 256, 0, st>>>(a);
    } else {
        if (rw == 4) HX_AC(64, 4); else if (rw == 2) HX_AC(64, 2); else HX_AC(64, 1);
        k_attn_combine<64><<<(nc_rows + 3) / 4, 256, 0, st>>>(a);
    }
#undef HX_AC
}

void attention(const AttnArgs &a, hipStream_t st) {
    attention_scores(a, st);
    attention_finish(a, st);
}

} // namespace hxl
