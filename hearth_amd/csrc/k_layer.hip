/*
 * k_layer.hip — per-layer elementwise work, routing and greedy acceptance on gfx950.
 *
 * Reference semantics (engine/src/model.c): embedding 1178-1182, residual adds
 * 1194-1198, rmsnorm quant.c:626-632, MoE combine moe_sum_range 904-923, routing
 * route_select/route_weights 793-843 with ranks_before 220-226, union/bucketing
 * 1020-1037, GQA post-processing gqa_post_range 484-517, SwiGLU quant.c:644-649;
 * greedy acceptance python/hearth/generate.py:365-392 (argmax: first index wins).
 */
#include "hx_device.h"
#include "hx_launch.h"
#include "hx_loop.h"

using namespace hxd;

namespace {

/* ------------------------------------------------------------ residual + rmsnorm + quant */

/* Residual update of token t's hidden row h (mode 0: h = embedding * emb_scale; 1:
 * h += rs * add; 2: h += rs * (sum_j w_j * Y[pair_j] (+ add)), j in rank order,
 * model.c:904-923; 3: h unchanged; 4: v = h (+ rs * gated add) into the norm only,
 * h unchanged -- the next-layer prediction input, model.c:1052-1058), then rmsnorm
 * (quant.c:626-632: ms = sum16(v^2)/D, r = 1/sqrt(ms + eps), x = (v * r) * w) and
 * NUMERICS §2 of x. */
__device__ __forceinline__ float norm_input(const NormArgs &a, const float *h, const float *wk, const int *pk, int t,
                                            int i) {
    const int D = a.D, K = a.K;
    if (a.mode == 0) {
        const uint8_t *row = a.emb + (size_t)a.tokens[t] * a.emb_rb;
        return fmul(a.es, deq_elem(row, a.emb_dtype, i));
    }
    if (a.mode == 1) return fadd(h[i], fmul(a.rs, a.add[(size_t)t * D + i]));
    if (a.mode == 3) return h[i];
    if (a.mode == 4) {
        float v = h[i];
        if (a.add) {
            float sv = a.add[(size_t)t * D + i];
            if (a.add_gate) sv = fmul(sv, fdiv(1.0f, fadd(1.0f, exp_glibc_f(-a.add_gate[t]))));
            v = fadd(v, fmul(a.rs, sv));
        }
        return v;
    }
    float out = 0.0f;
    for (int j0 = 0; j0 < K; j0 += 8) {
        float yv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u < K ? j0 + u : K - 1;
            yv[u] = a.Y[(size_t)pk[j] * D + i];
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (j0 + u < K) out = fadd(out, fmul(wk[j0 + u], yv[u]));
    }
    if (a.add) {
        float sv = a.add[(size_t)t * D + i];
        if (a.add_gate) sv = fmul(sv, fdiv(1.0f, fadd(1.0f, exp_glibc_f(-a.add_gate[t]))));
        out = fadd(out, sv);
    }
    return fadd(h[i], fmul(a.rs, out));
}

/* One workgroup per token; thread tid holds elements tid + nth u (u < EPT) in registers
 * from the residual step to the quantization, which is also the block layout of the
 * quantization (element g * 64 + lane is lane `lane` of wave g mod nw), so only the
 * squares go through LDS. They are stored transposed (square of element 16 k + j at
 * sq[j][k], rows padded by norm_sq_stride), so each of the 16 lanes of the sum16 reads
 * its own elements four at a time; entries past D hold +0 (adding +0 to a sum of
 * squares leaves it unchanged). Every load of the residual step (norm weights included)
 * is issued before the first of them is used: the mode is a template argument, indices
 * past the row are clamped to its last element (their values are replaced by 0), and
 * the trip count nu is uniform. */
constexpr int NM_PER = 8;   /* most elements per thread (rows up to 8192 wide) */

/* elements per lane of the sum16, rounded up to whole batches of 32 (8 reads of 16 bytes) */
__host__ __device__ __forceinline__ int norm_kp(int D) { return ((D + 15) / 16 + 31) & ~31; }

/* words per transposed row: norm_kp plus 4, so that the row length in 16-byte units is
 * odd (the 16 rows start in 16 different bank groups) */
__host__ __device__ __forceinline__ int norm_sq_stride(int D) { return norm_kp(D) + 4; }

/* the elements one row of the norm covers: the 16 lanes' padded squares and the
 * quantized blocks (padded blocks quantize zeros) */
__host__ __device__ __forceinline__ int norm_cover(int D, int nbp) {
    const int n = 16 * norm_kp(D);
    return n > nbp * 64 ? n : nbp * 64;
}

template <int MODE, int EPT>
__global__ __launch_bounds__(1024) void k_norm(NormArgs a) {
    extern __shared__ float sq[];
    __shared__ float r_sh;
    const int t = blockIdx.x, D = a.D, tid = threadIdx.x, nth = blockDim.x, K = a.K;
    const int kp = norm_kp(D), sqs = norm_sq_stride(D), nsq = 16 * kp;
    const int nu = (norm_cover(D, a.a.nbp) + nth - 1) / nth;   /* <= EPT, uniform */
    float *h = a.h + (size_t)t * D;
    const float *ad = a.add ? a.add + (size_t)t * D : nullptr;
    float wv[EPT], vv[EPT], hv[EPT], av[EPT];
#pragma unroll
    for (int u = 0; u < EPT; u++) {
        if (u < nu) {
            const int i = tid + nth * u, ic = i < D ? i : D - 1;
            wv[u] = a.norm_w[ic];
            if (MODE != 0) hv[u] = h[ic];
            if (MODE == 1 || ((MODE == 2 || MODE == 4) && ad)) av[u] = ad[ic];
        }
    }
    if (a.live && t >= *a.live) return;   /* padding token (uniform), after the row's loads are issued */
    float gs = 1.0f;   /* sigmoid of the shared expert's gate logit (modes 2, 4) */
    if ((MODE == 2 || MODE == 4) && a.add_gate) gs = fdiv(1.0f, fadd(1.0f, exp_glibc_f(-a.add_gate[t])));
    if (MODE == 0) {
        const uint8_t *row = a.emb + (size_t)a.tokens[t] * a.emb_rb;
#pragma unroll
        for (int u = 0; u < EPT; u++) {
            const int i = tid + nth * u, ic = i < D ? i : D - 1;
            if (u < nu) vv[u] = fmul(a.es, deq_elem(row, a.emb_dtype, ic));
        }
    } else if (MODE == 1) {
#pragma unroll
        for (int u = 0; u < EPT; u++)
            if (u < nu) vv[u] = fadd(hv[u], fmul(a.rs, av[u]));
    } else if (MODE == 3) {
#pragma unroll
        for (int u = 0; u < EPT; u++)
            if (u < nu) vv[u] = hv[u];
    } else if (MODE == 4) {
#pragma unroll
        for (int u = 0; u < EPT; u++) {
            if (u < nu) {
                vv[u] = hv[u];
                if (ad) {
                    const float sv = a.add_gate ? fmul(av[u], gs) : av[u];
                    vv[u] = fadd(vv[u], fmul(a.rs, sv));
                }
            }
        }
    } else {
        /* model.c:904-923: out = sum_j w_j * Y[pair_j] in rank order (+ gated shared add);
         * the token's pairs and weights are the same for every thread (scalar loads) */
        constexpr int JC = EPT <= 2 ? 8 : 4;   /* pairs loaded at once */
        const int *pt = a.pair_of + (size_t)t * K;
        const float *wt = a.wts + (size_t)t * K;
        float out[EPT];
#pragma unroll
        for (int u = 0; u < EPT; u++) out[u] = 0.0f;
        for (int j0 = 0; j0 < K; j0 += JC) {
            float yv[EPT][JC], wj[JC];
            int pj[JC];
            if (K % JC == 0) {
                /* one scalar load each of JC pair indices and weights (the rows of pair_of
                 * and wts start at multiples of JC words: K % JC == 0) */
                typedef int vji __attribute__((ext_vector_type(JC)));
                typedef float vjf __attribute__((ext_vector_type(JC)));
                const vji pv = *(const vji *)__builtin_assume_aligned(pt + j0, 4 * JC);
                const vjf wvv = *(const vjf *)__builtin_assume_aligned(wt + j0, 4 * JC);
#pragma unroll
                for (int jj = 0; jj < JC; jj++) {
                    pj[jj] = pv[jj];
                    wj[jj] = wvv[jj];
                }
            } else {
#pragma unroll
                for (int jj = 0; jj < JC; jj++) {
                    const int j = j0 + jj < K ? j0 + jj : K - 1;
                    pj[jj] = pt[j];
                    wj[jj] = wt[j];
                }
            }
#pragma unroll
            for (int jj = 0; jj < JC; jj++) {
                const float *yr = a.Y + (size_t)pj[jj] * D;
#pragma unroll
                for (int u = 0; u < EPT; u++) {
                    const int i = tid + nth * u;
                    if (u < nu) yv[u][jj] = yr[i < D ? i : D - 1];
                }
            }
#pragma unroll
            for (int u = 0; u < EPT; u++)
#pragma unroll
                for (int jj = 0; jj < JC; jj++)
                    if (u < nu && j0 + jj < K) out[u] = fadd(out[u], fmul(wj[jj], yv[u][jj]));
        }
#pragma unroll
        for (int u = 0; u < EPT; u++) {
            if (u < nu) {
                float o = out[u];
                if (ad) o = fadd(o, a.add_gate ? fmul(av[u], gs) : av[u]);
                vv[u] = fadd(hv[u], fmul(a.rs, o));
            }
        }
    }
#pragma unroll
    for (int u = 0; u < EPT; u++) {
        if (u < nu) {
            const int i = tid + nth * u;
            if (i >= D) vv[u] = 0.0f;
            if (i < D && MODE != 3 && MODE != 4) h[i] = vv[u];
            if (i < nsq) sq[(i & 15) * sqs + (i >> 4)] = fmul(vv[u], vv[u]);
        }
    }
    __syncthreads();
    if (tid < 16) {
        /* lane tid: the sequential sum of the squares of elements tid, tid + 16, ...,
         * eight 16-byte reads in flight while the previous eight are added */
        const float4 *row = (const float4 *)&sq[tid * sqs];
        const int n4 = kp / 4;   /* a multiple of 8 */
        float L = 0.0f;
        float4 cur[8], nxt[8];
#pragma unroll
        for (int u = 0; u < 8; u++) cur[u] = row[u];
        for (int c0 = 0; c0 < n4; c0 += 8) {
            const int cn = c0 + 8 < n4 ? c0 + 8 : c0;   /* the last batch reads itself again */
#pragma unroll
            for (int u = 0; u < 8; u++) nxt[u] = row[cn + u];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                L = fadd(L, cur[u].x);
                L = fadd(L, cur[u].y);
                L = fadd(L, cur[u].z);
                L = fadd(L, cur[u].w);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) cur[u] = nxt[u];
        }
        L = tree16(L);
        if (tid == 0) {
            const float ms = fdiv(L, (float)D);
            r_sh = fdiv(1.0f, sqrt_rn(fadd(ms, a.eps)));
        }
    }
    __syncthreads();
    const float r = r_sh;
    const int wave = tid >> 6, nw = nth >> 6;
#pragma unroll
    for (int u = 0; u < EPT; u++) {
        const int g = wave + nw * u;   /* the block of element tid + nth u (wave-uniform) */
        if (u < nu && g < a.a.nbp) {
            const int i = tid + nth * u;
            const float xv = i < D ? fmul(fmul(vv[u], r), wv[u]) : 0.0f;
            if (a.x && i < D) a.x[(size_t)t * D + i] = xv;
            quant_block_wave(xv, a.a, t, g);
        }
    }
}

/* The same for rows wider than NM_PER * 1024: the row goes through LDS. */
__global__ __launch_bounds__(1024) void k_norm_wide(NormArgs a) {
    extern __shared__ float hs[];
    __shared__ float wk[64];
    __shared__ int pk[64];
    __shared__ float r_sh;
    const int t = blockIdx.x, D = a.D, tid = threadIdx.x, nth = blockDim.x, K = a.K;
    if (a.live && t >= *a.live) return;   /* padding token (uniform) */
    float *h = a.h + (size_t)t * D;
    if (a.mode == 2) {
        if (tid < K) {
            wk[tid] = a.wts[(size_t)t * K + tid];
            pk[tid] = a.pair_of[(size_t)t * K + tid];
        }
        __syncthreads();
    }
    for (int i = tid; i < D; i += nth) {
        const float v = norm_input(a, h, wk, pk, t, i);
        if (a.mode != 4 && a.mode != 3) h[i] = v;
        hs[i] = v;
        hs[D + i] = fmul(v, v);
    }
    __syncthreads();
    if (tid < 16) {
        float L = 0.0f;
        for (int i = tid; i < D; i += 16) L = fadd(L, hs[D + i]);
        L = tree16(L);
        if (tid == 0) {
            const float ms = fdiv(L, (float)D);
            r_sh = fdiv(1.0f, sqrt_rn(fadd(ms, a.eps)));
        }
    }
    __syncthreads();
    const float r = r_sh;
    const int wave = tid >> 6, lane = tid & 63, nw = nth >> 6;
    for (int g = wave; g < a.a.nbp; g += nw) {
        const int i = g * 64 + lane;
        const float xv = i < D ? fmul(fmul(hs[i], r), a.norm_w[i]) : 0.0f;
        if (a.x && i < D) a.x[(size_t)t * D + i] = xv;
        quant_block_wave(xv, a.a, t, g);
    }
}

/* mid = silu(g) * u (written back into g, as the reference does in place) then
 * NUMERICS §2 (dense FFN / shared expert); one wave per (token, block). */
__global__ void k_swiglu_quant(float *__restrict__ g, const float *__restrict__ u, int T, int F, Act a) {
    const int wave = (int)((blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6);
    if (wave >= T * a.nbp) return;
    const int t = wave / a.nbp, b = wave % a.nbp, lane = threadIdx.x & 63, i = b * 64 + lane;
    float v = 0.0f;
    if (i < F) {
        const float gv = g[(size_t)t * F + i];
        v = fmul(fdiv(gv, fadd(1.0f, exp_glibc_f(-gv))), u[(size_t)t * F + i]);
        g[(size_t)t * F + i] = v;
    }
    quant_block_wave(v, a, t, b);
}

/* y = canon(s * y) on T rows of n values (logit_scale after a float lm_head) */
__global__ void k_scale_rows(float *y, int ldy, int T, int n, float s) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)T * n) return;
    float *p = y + (size_t)(i / n) * ldy + (i % n);
    *p = canon(fmul(s, *p));
}

/* ------------------------------------------------------------ routing */

/* a ranks before b: larger value first, NaN last, ties to the lower index */
__device__ __forceinline__ bool ranks_before(float va, int ia, float vb, int ib) {
    const bool na = va != va, nb = vb != vb;
    if (na || nb) return na == nb ? ia < ib : nb;
    if (va != vb) return va > vb;
    return ia < ib;
}

/* wave-wide best (value, index) over candidates; idx < 0 marks "none" */
__device__ __forceinline__ void wave_best(float &v, int &idx) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        const bool take = oi >= 0 && (idx < 0 || ranks_before(ov, oi, v, idx));
        v = take ? ov : v;
        idx = take ? oi : idx;
    }
}

constexpr int ROUTE_EMAX = 1024;

/* the router-logits row token t is routed from: padding tokens (t >= *live) take
 * token 0's, so they add no expert to the batch */
__device__ __forceinline__ int route_row(const RouteArgs &a, int t) { return a.live && t >= *a.live ? 0 : t; }

/* expert j of token t under route replay */
__device__ __forceinline__ int replay_id(const RouteArgs &a, int t, int j) {
    const long long pos = (long long)a.pos0 + a.depth[t];
    return a.replay[(size_t)(pos % a.replay_rows) * (size_t)(a.n_moe * a.K) + (size_t)a.moe_ord * a.K + j];
}

/* One wave per token: scores, selection values, group limit, top-K, weights. */
__global__ __launch_bounds__(64) void k_route_tokens(RouteArgs a) {
    __shared__ float score[ROUTE_EMAX], sel[ROUTE_EMAX];
    __shared__ unsigned char taken[ROUTE_EMAX], gkeep[64];
    __shared__ float gsc[64];
    const int t = blockIdx.x, lane = threadIdx.x, E = a.E, K = a.K;
    const float *lg = a.logits + (size_t)route_row(a, t) * E;
    if (a.score_fn == 0) {
        /* softmax (quant.c:634-642): m = running max from x[0] (a NaN x[0] makes m NaN) */
        float m = -__builtin_huge_valf();
        for (int e = lane; e < E; e += 64) {
            const float x = lg[e];
            score[e] = x;
            if (x == x) m = fmaxf(m, x);
        }
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        if (lg[0] != lg[0]) m = lg[0];
        wave_sync();
        for (int e = lane; e < E; e += 64) score[e] = exp_glibc_f(fadd(score[e], -m));
        wave_sync();
        float L = 0.0f;
        if (lane < 16)
            for (int e = lane; e < E; e += 16) L = fadd(L, score[e]);
        L = tree16(L);
        const float s = __shfl(L, 0, 64);
        wave_sync();
        for (int e = lane; e < E; e += 64) score[e] = fdiv(score[e], s);
    } else {
        for (int e = lane; e < E; e += 64) score[e] = fdiv(1.0f, fadd(1.0f, exp_glibc_f(-lg[e])));
    }
    wave_sync();
    for (int e = lane; e < E; e += 64) {
        sel[e] = a.bias ? fadd(score[e], a.bias[e]) : score[e];
        taken[e] = 0;
    }
    wave_sync();
    int my_id = -1;
    if (a.replay) {   /* uniform */
        if (lane < K) my_id = replay_id(a, t, lane);
        goto weights;
    }
    if (a.n_group > 1) {
        const int ng = a.n_group, gs = E / ng;
        for (int g = 0; g < ng; g++) {
            float v1 = 0.0f, v2 = 0.0f;
            int i1 = -1, i2 = -1;
            for (int i = lane; i < gs; i += 64)
                if (i1 < 0 || ranks_before(sel[g * gs + i], i, v1, i1)) { v1 = sel[g * gs + i]; i1 = i; }
            wave_best(v1, i1);
            for (int i = lane; i < gs; i += 64)
                if (i != i1 && (i2 < 0 || ranks_before(sel[g * gs + i], i, v2, i2))) { v2 = sel[g * gs + i]; i2 = i; }
            wave_best(v2, i2);
            if (lane == 0) { gsc[g] = i2 >= 0 ? fadd(v1, v2) : v1; gkeep[g] = 0; }
        }
        wave_sync();
        for (int r = 0; r < a.topk_group; r++) {
            float v = 0.0f;
            int bi = -1;
            for (int g = lane; g < ng; g += 64)
                if (!gkeep[g] && (bi < 0 || ranks_before(gsc[g], g, v, bi))) { v = gsc[g]; bi = g; }
            wave_best(v, bi);
            if (lane == 0) gkeep[bi] = 1;
            wave_sync();
        }
        for (int e = lane; e < E; e += 64)
            if (!gkeep[e / gs]) sel[e] = 0.0f;
        wave_sync();
    }
    for (int j = 0; j < K; j++) {
        float v = 0.0f;
        int bi = -1;
        for (int e = lane; e < E; e += 64)
            if (!taken[e] && (bi < 0 || ranks_before(sel[e], e, v, bi))) { v = sel[e]; bi = e; }
        wave_best(v, bi);
        if (lane == 0) taken[bi] = 1;
        if (lane == j) my_id = bi;
        wave_sync();
    }
weights:
    /* weights: w_j = score[id_j]; norm_topk: w_j / (sum_j w_j + 1e-20f), sum in rank order */
    float w = lane < K ? score[my_id] : 0.0f;
    if (a.norm_topk) {
        float s = 0.0f;
        for (int j = 0; j < K; j++) {
            const int idj = __shfl(my_id, j, 64);
            s = fadd(s, score[idj]);
        }
        const float den = fadd(s, 1e-20f);
        w = fdiv(w, den);
    }
    w = fmul(w, a.routed_scale);
    if (lane < K) {
        a.ids[(size_t)t * K + lane] = my_id;
        a.wts[(size_t)t * K + lane] = w;
        if (a.route_out) a.route_out[((size_t)t * a.n_moe + a.moe_ord) * K + lane] = my_id;
    }
}

/* Selection key of (value v, expert e): a larger key ranks first, and the order is
 * ranks_before's: larger value first (-0 equals +0), NaN after every number, ties to
 * the lower index. */
__device__ __forceinline__ uint32_t order_key(float v) {
    /* a larger value has a larger key (-0 equals +0); NaN has key 0, below every number */
    if (v != v) return 0u;
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ unsigned long long rank_key(float v, int e) {
    return ((unsigned long long)order_key(v) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}

/* Ungrouped routing (n_group <= 1), one workgroup per token: scores, selection values,
 * then each expert's rank = the number of experts that rank before it; the K experts of
 * rank < K are the reference's K rounds of best-remaining (route_select, model.c:793-843)
 * in the same order. Weights as in k_route_tokens. */
__global__ __launch_bounds__(256) void k_route_rank(RouteArgs a) {
    __shared__ float score[ROUTE_EMAX];
    __shared__ unsigned long long key[ROUTE_EMAX];
    __shared__ int chosen[64];
    __shared__ float red[4];
    __shared__ float sum_sh;
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, E = a.E, K = a.K;
    const float *lg = a.logits + (size_t)route_row(a, t) * E;
    if (a.score_fn == 0) {
        /* softmax (quant.c:634-642): m = running max from x[0] (a NaN x[0] makes m NaN) */
        float m = -__builtin_huge_valf();
        for (int e = tid; e < E; e += 256) {
            const float x = lg[e];
            score[e] = x;
            if (x == x) m = fmaxf(m, x);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        if (lane == 0) red[wave] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        if (score[0] != score[0]) m = score[0];
        for (int e = tid; e < E; e += 256) score[e] = exp_glibc_f(fadd(score[e], -m));
        __syncthreads();
        if (tid < 16) {
            float L = 0.0f;
            for (int e = tid; e < E; e += 16) L = fadd(L, score[e]);
            L = tree16(L);
            if (tid == 0) sum_sh = L;
        }
        __syncthreads();
        const float sum = sum_sh;
        for (int e = tid; e < E; e += 256) score[e] = fdiv(score[e], sum);
    } else {
        for (int e = tid; e < E; e += 256) score[e] = fdiv(1.0f, fadd(1.0f, exp_glibc_f(-lg[e])));
    }
    __syncthreads();
    if (a.replay) {   /* uniform */
        if (tid < K) chosen[tid] = replay_id(a, t, tid);
    } else {
        for (int e = tid; e < E; e += 256) key[e] = rank_key(a.bias ? fadd(score[e], a.bias[e]) : score[e], e);
        __syncthreads();
        for (int e = tid; e < E; e += 256) {
            const unsigned long long ke = key[e];
            int rank = 0;
            int o = 0;
            for (; o + 4 <= E; o += 4) {
                const unsigned long long k0 = key[o], k1 = key[o + 1], k2 = key[o + 2], k3 = key[o + 3];
                rank += (k0 > ke) + (k1 > ke) + (k2 > ke) + (k3 > ke);
            }
            for (; o < E; o++) rank += key[o] > ke;
            if (rank < K) chosen[rank] = e;
        }
    }
    __syncthreads();
    /* weights: w_j = score[id_j]; norm_topk: w_j / (sum_j w_j + 1e-20f), sum in rank order */
    if (tid < K) {
        const int id = chosen[tid];
        float w = score[id];
        if (a.norm_topk) {
            float s = 0.0f;
            for (int j = 0; j < K; j++) s = fadd(s, score[chosen[j]]);
            w = fdiv(w, fadd(s, 1e-20f));
        }
        w = fmul(w, a.routed_scale);
        a.ids[(size_t)t * K + tid] = id;
        a.wts[(size_t)t * K + tid] = w;
        if (a.route_out) a.route_out[((size_t)t * a.n_moe + a.moe_ord) * K + tid] = id;
    }
}

/* Union of the chosen experts in ascending id, pairs grouped by expert with tokens
 * ascending (model.c:1020-1037), by the nth threads of one workgroup. ids: the T*K
 * chosen experts (LDS or global); cnt/base: LDS scratch of E ints. Writes the pair
 * lists, the active-slot lists and the slot descriptors (unused slots get n = 0). */
/* u64 words of the per-expert token masks (ceil(T / 64) words per expert) */
constexpr int BK_MASKW = 2048;

__device__ void bucket_pairs(const RouteArgs &a, const int *ids, int *cnt, int *base, unsigned long long *tm, int tid,
                             int nth) {
    const int E = a.E, P = a.T * a.K, nw = (a.T + 63) >> 6;
    /* pairs of padding tokens (t >= *live, which routed from token 0's logits) are not
     * bucketed: each reads token 0's pair of the same rank, which is its expert's first */
    const int PL = (a.live ? *a.live : a.T) * a.K;
    const bool masks = nw * E <= BK_MASKW;
    for (int e = tid; e < E; e += nth) cnt[e] = 0;
    if (masks)
        for (int i = tid; i < nw * E; i += nth) tm[i] = 0ull;
    __syncthreads();
    for (int p = tid; p < PL; p += nth) {
        const int e = ids[p];
        atomicAdd(&cnt[e], 1);
        if (masks) {
            const int t = p / a.K;
            atomicOr(&tm[e * nw + (t >> 6)], 1ull << (t & 63));
        }
    }
    __syncthreads();
    __shared__ int nu_sh;
    if (tid < 64) {
        /* exclusive scan of cnt over experts by one wave, 64 experts per round */
        int run = 0, nu_run = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + tid;
            const int c = e < E ? cnt[e] : 0, act = c > 0;
            const int inc = wave_scan_incl(c), ninc = wave_scan_incl(act);
            const int pos = run + inc - c, slot = nu_run + ninc - act;
            if (e < E) {
                base[e] = pos;
                if (act) {
                    a.ulist[slot] = e;
                    a.u_p0[slot] = pos;
                    a.u_n[slot] = c;
                    SlotDesc d;
                    d.w = a.table[e];
                    d.p0 = pos;
                    d.n = c;
                    d.e = e;
                    d.pad = 0;
                    a.desc[slot] = d;
                }
            }
            run += __shfl(inc, 63, 64);
            nu_run += __shfl(ninc, 63, 64);
        }
        if (tid == 0) {
            nu_sh = nu_run;
            *a.n_active = nu_run;
            if (a.stats) {
                a.stats[0] += (unsigned long long)PL;
                a.stats[1] += (unsigned long long)nu_run;
            }
        }
    }
    __syncthreads();
    for (int u = nu_sh + tid; u < a.n_slots; u += nth) a.desc[u].n = 0;
    /* pair p goes after the earlier pairs of its expert (tokens ascending within an
     * expert, model.c:1030-1035): its rank = how many pairs q < p have the same id.
     * A token's K experts are distinct (route_select picks distinct experts; replayed
     * rows are checked), so with the token masks that is the number of tokens below
     * p's token that chose the expert */
    for (int p = tid; p < P; p += nth) {
        const int e = ids[p];
        if (p >= PL) {
            a.pair_of[p] = base[e];
            continue;
        }
        if (masks) {
            const int t = p / a.K, w0 = t >> 6;
            const unsigned long long *m = tm + (size_t)e * nw;
            int r = 0;
            for (int w = 0; w < w0; w++) r += __popcll(m[w]);
            r += __popcll(m[w0] & ((1ull << (t & 63)) - 1ull));
            const int pos = base[e] + r;
            a.pair_tok[pos] = t;
            a.pair_of[p] = pos;
            continue;
        }
        int r = 0, q = 0;
        for (; q + 8 <= p; q += 8) {
            int v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = ids[q + u];
#pragma unroll
            for (int u = 0; u < 8; u++) r += v[u] == e ? 1 : 0;
        }
        for (; q < p; q++) r += ids[q] == e ? 1 : 0;
        const int pos = base[e] + r;
        a.pair_tok[pos] = p / a.K;
        a.pair_of[p] = pos;
    }
}

constexpr int BUCKET_PMAX = 8192;

/* bucketing of a routed batch by one workgroup (the pair list staged in LDS when it fits) */
__global__ __launch_bounds__(1024) void k_route_bucket(RouteArgs a) {
    __shared__ int cnt[ROUTE_EMAX], base[ROUTE_EMAX];
    __shared__ int pid[BUCKET_PMAX];
    __shared__ unsigned long long tmk[BK_MASKW];
    const int tid = threadIdx.x, nth = blockDim.x, P = a.T * a.K;
    const bool in_lds = P <= BUCKET_PMAX;
    if (in_lds)
        for (int p = tid; p < P; p += nth) pid[p] = a.ids[p];
    __syncthreads();
    bucket_pairs(a, in_lds ? pid : a.ids, cnt, base, tmk, tid, nth);
}

/* Ungrouped routing of up to 16 tokens (E <= 256, K <= 64) and their bucketing in one
 * workgroup. Wave t routes token t: scores and weights as k_route_rank; the K experts by
 * K rounds of a wave maximum of the 32-bit order keys of the selection values, the winner
 * being the lowest expert index that holds the maximum (ballots in index order), which is
 * ranks_before's order. Each choice sets the token's bit in its expert's token mask, so
 * the bucketing needs no counting pass: an expert's pair count is the popcount of its
 * mask, and a pair's place among its expert's pairs (tokens ascending, model.c:1030-1035)
 * the popcount of the mask bits below its token (a token's K experts are distinct:
 * route_select picks distinct experts, and replayed routes were recorded from it). The
 * expert table is staged into LDS while the logits load, and all threads write the slot
 * descriptors at the end. */
constexpr int RS_TMAX = 16, RS_EMAX = 256;
constexpr int RS_TW = (int)(sizeof(ExpertW) / 4), RS_DW = (int)(sizeof(SlotDesc) / 4);
static_assert(sizeof(ExpertW) % 4 == 0 && sizeof(SlotDesc) == sizeof(ExpertW) + 16, "slot descriptor words");
static_assert(__builtin_offsetof(SlotDesc, p0) == sizeof(ExpertW) && __builtin_offsetof(SlotDesc, n) == sizeof(ExpertW) + 4 &&
                  __builtin_offsetof(SlotDesc, e) == sizeof(ExpertW) + 8,
              "slot descriptor fields after the matrices: p0, n, e, pad");

/* routing of token t by one wave (lane e % 64 holds expert e, NU experts per lane):
 * scores into sc, then the K experts, their weights (also into wk), and the token's
 * bits in tmask */
template <int NU>
__device__ __forceinline__ void route_token_small(const RouteArgs &a, int t, const float (&lgv)[RS_EMAX / 64],
                                                  const float (&bv)[RS_EMAX / 64], int live, float *sc, int *pid,
                                                  uint32_t *tmask, float *wk) {
    const int lane = threadIdx.x & 63, E = a.E, K = a.K;
    float x[NU];
    bool ok[NU];
#pragma unroll
    for (int u = 0; u < NU; u++) {
        ok[u] = lane + 64 * u < E;
        x[u] = lgv[u];
    }
    if (a.score_fn == 0) {
        /* softmax (quant.c:634-642): m = running max from x[0] (a NaN x[0] makes m NaN) */
        float m = -__builtin_huge_valf();
#pragma unroll
        for (int u = 0; u < NU; u++)
            if (ok[u] && x[u] == x[u]) m = fmaxf(m, x[u]);
        m = wave_max_f32(m);   /* a maximum: any reduction order gives the same value */
        const float x0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x[0]), 0));
        if (x0 != x0) m = x0;
        float ev[NU];
#pragma unroll
        for (int u = 0; u < NU; u++) ev[u] = exp_glibc_f(fadd(x[u], -m));
#pragma unroll
        for (int u = 0; u < NU; u++)
            if (ok[u]) sc[lane + 64 * u] = ev[u];
        wave_sync();
        float L = 0.0f;
        if (lane < 16)
            for (int e = lane; e < E; e += 16) L = fadd(L, sc[e]);
        L = tree16(L);
        const float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(L), 0));
#pragma unroll
        for (int u = 0; u < NU; u++) {
            x[u] = fdiv(ev[u], sum);
            if (ok[u]) sc[lane + 64 * u] = x[u];
        }
    } else {
#pragma unroll
        for (int u = 0; u < NU; u++) {
            x[u] = fdiv(1.0f, fadd(1.0f, exp_glibc_f(-x[u])));
            if (ok[u]) sc[lane + 64 * u] = x[u];
        }
    }
    wave_sync();
    int my_id = 0;
    if (a.replay) {   /* uniform */
        if (lane < K) my_id = replay_id(a, t, lane);
    } else {
        /* top-K: K rounds of the wave maximum of the order keys of the still unchosen
         * experts; the lowest expert index holding it wins */
        uint32_t kk[NU];
        bool live[NU];
#pragma unroll
        for (int u = 0; u < NU; u++) {
            const int e = lane + 64 * u;
            kk[u] = order_key(a.bias && ok[u] ? fadd(x[u], bv[u]) : x[u]);
            live[u] = ok[u];
        }
        for (int j = 0; j < K; j++) {
            uint32_t m = 0u;
#pragma unroll
            for (int u = 0; u < NU; u++) m = live[u] && kk[u] > m ? kk[u] : m;
            m = wave_max_u32(m);
            int e = 0;
#pragma unroll
            for (int u = NU - 1; u >= 0; u--) {
                const unsigned long long b = __ballot(live[u] && kk[u] == m);
                e = b ? 64 * u + __builtin_ctzll(b) : e;   /* the lowest u with a hit is taken last */
            }
#pragma unroll
            for (int u = 0; u < NU; u++)
                if (lane + 64 * u == e) live[u] = false;
            my_id = lane == j ? e : my_id;
        }
    }
    float w = lane < K ? sc[my_id] : 0.0f;
    if (a.norm_topk) {
        /* sum of the K weights in rank order (route_weights, model.c:830-838) */
        float s = 0.0f;
        for (int j = 0; j < K; j++) s = fadd(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j)));
        w = fdiv(w, fadd(s, 1e-20f));
    }
    if (lane < K) {
        w = fmul(w, a.routed_scale);
        a.ids[(size_t)t * K + lane] = my_id;
        a.wts[(size_t)t * K + lane] = w;
        pid[t * K + lane] = my_id;
        wk[t * K + lane] = w;
        if (t < live) atomicOr(&tmask[my_id], 1u << t);   /* padding tokens add no pair */
        if (a.route_out) a.route_out[((size_t)t * a.n_moe + a.moe_ord) * K + lane] = my_id;
    }
}

/* LDS of the small routing: scores, chosen experts, token masks, scan results and the
 * staged expert table */
struct RouteSmem {
    float score[RS_TMAX][RS_EMAX];
    int pid[RS_TMAX * 64];
    float wk[RS_TMAX * 64];
    uint32_t tmask[RS_EMAX];
    int base[RS_EMAX], slot_e[RS_EMAX];
    uint32_t tab[RS_EMAX * RS_TW];
    int nu;
};

/* the expert table into LDS (all loads of a round issued before its stores) and the
 * token masks cleared; the caller's barrier publishes both */
__device__ __forceinline__ void route_small_stage(const RouteArgs &a, RouteSmem &rs, int tid, int nth) {
    const uint32_t *tw = (const uint32_t *)a.table;
    const int nw = a.E * RS_TW;
    for (int w0 = 0; w0 < nw; w0 += 4 * nth) {
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int w = w0 + tid + k * nth;
            v[k] = w < nw ? tw[w] : 0u;
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int w = w0 + tid + k * nth;
            if (w < nw) rs.tab[w] = v[k];
        }
    }
    for (int e = tid; e < a.E; e += nth) rs.tmask[e] = 0u;
}

/* logits of token t and the selection bias, expert lane + 64 u, into registers: every
 * load issued at once */
__device__ __forceinline__ void route_small_logits(const RouteArgs &a, const float *logits, int t, float (&lgv)[RS_EMAX / 64],
                                                   float (&bv)[RS_EMAX / 64]) {
    const int lane = threadIdx.x & 63;
    const float *lg = logits + (size_t)t * a.E;
#pragma unroll
    for (int u = 0; u < RS_EMAX / 64; u++) {
        const int e = lane + 64 * u;
        lgv[u] = e < a.E ? lg[e] : 0.0f;
        bv[u] = e < a.E && a.bias ? a.bias[e] : 0.0f;
    }
}

/* token t's routing by the calling wave */
__device__ __forceinline__ void route_small_token(const RouteArgs &a, RouteSmem &rs, int t, const float (&lgv)[RS_EMAX / 64],
                                                  const float (&bv)[RS_EMAX / 64], int live) {
    switch ((a.E + 63) / 64) {
    case 1: route_token_small<1>(a, t, lgv, bv, live, rs.score[t], rs.pid, rs.tmask, rs.wk); break;
    case 2: route_token_small<2>(a, t, lgv, bv, live, rs.score[t], rs.pid, rs.tmask, rs.wk); break;
    case 3: route_token_small<3>(a, t, lgv, bv, live, rs.score[t], rs.pid, rs.tmask, rs.wk); break;
    default: route_token_small<4>(a, t, lgv, bv, live, rs.score[t], rs.pid, rs.tmask, rs.wk); break;
    }
}

/* bucketing after every token is routed: scan of the pair counts, pair places, slot
 * descriptors (all threads of the workgroup call it) */
__device__ __forceinline__ void route_small_bucket(const RouteArgs &a, RouteSmem &rs, int tid, int nth, int live) {
    const int E = a.E, K = a.K, P = a.T * K, wave = tid >> 6, lane = tid & 63;
    __syncthreads();
    /* padding tokens take token 0's experts and weights, rank by rank (no pairs of their
     * own: their bits are not in the token masks) */
    for (int p = live * K + tid; p < P; p += nth) {
        const int tt = p / K, r = p - tt * K, e = rs.pid[r];
        rs.pid[p] = e;
        a.ids[p] = e;
        a.wts[p] = rs.wk[r];
        if (a.route_out) a.route_out[((size_t)tt * a.n_moe + a.moe_ord) * K + r] = e;
    }
    if (wave == 0) {
        /* exclusive scan of the pair counts over experts, 64 experts per round */
        int run = 0, nu_run = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const int c = e < E ? __popc(rs.tmask[e]) : 0, act = c > 0;
            const int inc = wave_scan_incl(c), ninc = wave_scan_incl(act);
            const int pos = run + inc - c, slot = nu_run + ninc - act;
            if (e < E) {
                rs.base[e] = pos;
                if (act) {
                    a.ulist[slot] = e;
                    a.u_p0[slot] = pos;
                    a.u_n[slot] = c;
                    rs.slot_e[slot] = e;
                }
            }
            run += __builtin_amdgcn_readlane(inc, 63);
            nu_run += __builtin_amdgcn_readlane(ninc, 63);
        }
        if (lane == 0) {
            rs.nu = nu_run;
            *a.n_active = nu_run;
            if (a.stats) {   /* counters only: no return value, nothing waits for them */
                atomicAdd(&a.stats[0], (unsigned long long)run);
                atomicAdd(&a.stats[1], (unsigned long long)nu_run);
            }
        }
    }
    __syncthreads();
    const int nu = rs.nu;
    for (int p = tid; p < P; p += nth) {
        const int e = rs.pid[p], tt = p / K;
        if (tt >= live) {   /* a padding token reads token 0's pair of the same rank (same expert) */
            a.pair_of[p] = rs.base[e];
            continue;
        }
        const int pos = rs.base[e] + __popc(rs.tmask[e] & ((1u << tt) - 1u));
        a.pair_tok[pos] = tt;
        a.pair_of[p] = pos;
    }
    /* slot descriptors: the active slots in full, one word per thread, then n = 0 in the
     * rest, one slot per thread */
    uint32_t *dw = (uint32_t *)a.desc;
    for (int w = tid; w < nu * RS_DW; w += nth) {
        const int slot = w / RS_DW, k = w % RS_DW, e = rs.slot_e[slot];
        uint32_t v = 0u;
        if (k < RS_TW) v = rs.tab[e * RS_TW + k];
        else if (k == RS_TW) v = (uint32_t)rs.base[e];
        else if (k == RS_TW + 1) v = (uint32_t)__popc(rs.tmask[e]);
        else if (k == RS_TW + 2) v = (uint32_t)e;
        dw[w] = v;
    }
    for (int slot = nu + tid; slot < a.n_slots; slot += nth) dw[(size_t)slot * RS_DW + RS_TW + 1] = 0u;
}

__global__ __launch_bounds__(1024) void k_route_small(RouteArgs a) {
    __shared__ RouteSmem rs;
    const int tid = threadIdx.x, nth = blockDim.x, t = tid >> 6;
    /* the padding bound is read with the logits (route_row would make the logit loads
     * wait for it): padding tokens route nothing and take token 0's experts and weights */
    const int live = a.live ? *a.live : a.T;
    float lgv[RS_EMAX / 64], bv[RS_EMAX / 64];
    if (t < a.T) route_small_logits(a, a.logits, t, lgv, bv);
    route_small_stage(a, rs, tid, nth);
    __syncthreads();
    if (t < live) route_small_token(a, rs, t, lgv, bv, live);   /* padding tokens: after the barrier in the bucketing */
    route_small_bucket(a, rs, tid, nth, live);
}

/* ------------------------------------------------------------ GQA post-processing */

/* One wave per (token, head slot): slots [0, H) are query heads, [H, H + Hkv) key heads
 * (which also append the value head). Bias, qk-norm (per head), RoPE from the host
 * table, then the K/V cache at slot pos0 + t. */
__global__ __launch_bounds__(256) void k_qkv_post(QkvArgs a, const float *__restrict__ rfull) {
    __shared__ float buf[4][512];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nslot = a.H + a.Hkv, hd = a.hd;
    const int item = blockIdx.x * 4 + wave;
    if (item >= a.T * nslot) return;
    const int t = item / nslot, j = item % nslot;
    if (a.live && t >= *a.live) return;   /* padding token: its K/V slot is never read */
    const bool isq = j < a.H;
    const int g = isq ? j : j - a.H;
    const int qd = a.H * hd, kd = a.Hkv * hd;
    const float *src = isq ? a.q + (size_t)t * qd + (size_t)g * hd : a.k + (size_t)t * kd + (size_t)g * hd;
    const float *bias = isq ? (a.bq ? a.bq + (size_t)g * hd : nullptr) : (a.bk ? a.bk + (size_t)g * hd : nullptr);
    float *x = buf[wave];
    for (int e = lane; e < hd; e += 64) x[e] = bias ? fadd(src[e], bias[e]) : src[e];
    wave_sync();
    if (a.qk_norm == 1) {
        float L = 0.0f;
        if (lane < 16)
            for (int e = lane; e < hd; e += 16) L = fadd(L, fmul(x[e], x[e]));
        L = tree16(L);
        L = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(L), 0));
        const float r = fdiv(1.0f, sqrt_rn(fadd(fdiv(L, (float)hd), a.eps)));
        const float *w = isq ? a.qn : a.kn;
        wave_sync();
        for (int e = lane; e < hd; e += 64) x[e] = fmul(fmul(x[e], r), w[e]);
    } else if (a.qk_norm == 2) {
        const float r = rfull[(size_t)t * 2 + (isq ? 0 : 1)];
        const float *w = (isq ? a.qn : a.kn) + (size_t)g * hd;
        for (int e = lane; e < hd; e += 64) x[e] = fmul(fmul(x[e], r), w[e]);
    }
    wave_sync();
    const int half = a.rope_dim / 2;
    const float *cs = a.rope + (size_t)t * a.rope_dim;
    for (int p = lane; p < half; p += 64) {
        const int ia = a.rope_style == 1 ? 2 * p : p, ib = a.rope_style == 1 ? 2 * p + 1 : p + half;
        const float av = x[ia], bv = x[ib], c = cs[2 * p], s = cs[2 * p + 1];
        x[ia] = fadd(fmul(av, c), -fmul(bv, s));
        x[ib] = fadd(fmul(bv, c), fmul(av, s));
    }
    wave_sync();
    const size_t slot = (size_t)(*a.pos + t);
    if (isq) {
        for (int e = lane; e < hd; e += 64) a.qout[(size_t)t * qd + (size_t)g * hd + e] = x[e];
    } else {
        float *kc = a.kc + ((size_t)g * a.cap + slot) * hd, *vc = a.vc + ((size_t)g * a.cap + slot) * hd;
        const float *vs = a.v + (size_t)t * kd + (size_t)g * hd;
        for (int e = lane; e < hd; e += 64) {
            kc[e] = x[e];
            vc[e] = a.bv ? fadd(vs[e], a.bv[(size_t)g * hd + e]) : vs[e];
        }
    }
}

/* Full-width qk-norm (qk_norm = 2): r = 1/sqrt(dot16(x,x)/n + eps) of q (+bias) and
 * k (+bias) per token; one wave per (token, q|k). */
__global__ void k_fullnorm_r(QkvArgs a, float *rfull) {
    const int wave = (int)((blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6), lane = threadIdx.x & 63;
    if (wave >= a.T * 2) return;
    const int t = wave / 2, isk = wave % 2;
    const int n = (isk ? a.Hkv : a.H) * a.hd;
    const float *src = isk ? a.k + (size_t)t * n : a.q + (size_t)t * n;
    const float *b = isk ? a.bk : a.bq;
    float L = 0.0f;
    if (lane < 16)
        for (int e = lane; e < n; e += 16) {
            const float v = b ? fadd(src[e], b[e]) : src[e];
            L = fadd(L, fmul(v, v));
        }
    L = tree16(L);
    if (lane == 0) rfull[(size_t)t * 2 + isk] = fdiv(1.0f, sqrt_rn(fadd(fdiv(L, (float)n), a.eps)));
}

/* ------------------------------------------------------------ KV compaction */

/* Moves K/V of slot pos0 + path[j] to pos0 + j, j ascending (sources are >= their
 * destinations and increase with j, so one thread per element in order is safe). */
__global__ void k_kv_move(float *cache, size_t layer_stride, int L, int Hkv, int cap, int hd, int pos0,
                          const int *__restrict__ path, int n) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_layer = (int64_t)2 * Hkv * hd;
    if (idx >= per_layer * L) return;
    const int l = (int)(idx / per_layer), r = (int)(idx % per_layer);
    const int kvh = r / hd, e = r % hd;   /* kvh in [0, 2*Hkv): K heads then V heads */
    float *base = cache + (size_t)l * layer_stride + (size_t)kvh * cap * hd + e;
    for (int j = 0; j < n; j++) {
        const int src = path[j];
        if (src != j) base[(size_t)(pos0 + j) * hd] = base[(size_t)(pos0 + src) * hd];
    }
}

/* The same for a [cap][width] array at offset off of every layer (MLA caches). */
__global__ void k_kv_move_rows(float *cache, size_t layer_stride, int L, size_t off, int width, int pos0,
                               const int *__restrict__ path, int n) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)width * L) return;
    const int l = (int)(idx / width), e = (int)(idx % width);
    float *base = cache + (size_t)l * layer_stride + off + e;
    for (int j = 0; j < n; j++) {
        const int src = path[j];
        if (src != j) base[(size_t)(pos0 + j) * width] = base[(size_t)(pos0 + src) * width];
    }
}

/* Slot descriptors' matrices after the expert cache made the layer's experts resident
 * (the bucketing wrote them from the table before the cache updated it). */
__global__ void k_desc_refresh(SlotDesc *desc, const ExpertW *table, const int *ulist, const int *n_active,
                               int n_slots) {
    const int u = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (u < n_slots && u < *n_active) desc[u].w = table[ulist[u]];
}

/* ------------------------------------------------------------ greedy acceptance */

/* Greedy argmax of the verify rows, first index on ties, -1 for rows with a NaN or +inf
 * or only -inf (generate.py:69-82). Each row is cut into ACCEPT_PARTS slices, one
 * workgroup each, 8 loads in flight per thread; the walk merges the slices in order. */
__global__ __launch_bounds__(256) void k_argmax_part(AcceptArgs a) {
    __shared__ float bv[256];
    __shared__ int bi[256], bf[256];
    const int row = blockIdx.x / ACCEPT_PARTS, part = blockIdx.x % ACCEPT_PARTS, tid = threadIdx.x;
    const int len = (a.V + ACCEPT_PARTS - 1) / ACCEPT_PARTS, lo = part * len;
    const int hi = lo + len < a.V ? lo + len : a.V;
    const float *x = a.rows + (size_t)row * a.V;
    float v = 0.0f;
    int idx = -1, flags = 0;
    for (int i0 = lo + tid; i0 < hi; i0 += 256 * 8) {
        float xv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + 256 * u;
            xv[u] = x[i < hi ? i : lo];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + 256 * u;
            if (i < hi) {
                const float xi = xv[u];
                if (xi != xi || xi == __builtin_huge_valf()) flags |= 1;
                if (xi != -__builtin_huge_valf()) flags |= 2;
                if (idx < 0 || xi > v) { v = xi; idx = i; }
            }
        }
    }
    bv[tid] = v; bi[tid] = idx; bf[tid] = flags;
    __syncthreads();
    for (int s = 128; s >= 1; s >>= 1) {
        if (tid < s) {
            const float ov = bv[tid + s];
            const int oi = bi[tid + s];
            if (oi >= 0 && (bi[tid] < 0 || ov > bv[tid] || (ov == bv[tid] && oi < bi[tid]))) { bv[tid] = ov; bi[tid] = oi; }
            bf[tid] |= bf[tid + s];
        }
        __syncthreads();
    }
    if (tid == 0) {
        const size_t o = (size_t)row * ACCEPT_PARTS + part;
        a.part_v[o] = bv[0];
        a.part_i[o] = bi[0];
        a.part_f[o] = bf[0];
    }
}

/* argmax of row v from its slices (slices in index order: equal maxima keep the earlier) */
__device__ int row_argmax(const AcceptArgs &a, int v) {
    float best = 0.0f;
    int bi = -1, fl = 0;
    for (int p = 0; p < ACCEPT_PARTS; p++) {
        const size_t o = (size_t)v * ACCEPT_PARTS + p;
        const int pi = a.part_i[o];
        fl |= a.part_f[o];
        if (pi >= 0 && (bi < 0 || a.part_v[o] > best)) { best = a.part_v[o]; bi = pi; }
    }
    return ((fl & 1) || !(fl & 2)) ? -1 : bi;
}

/* rows whose argmax the walk's workgroup merges from the slices up front, in parallel
 * (the walk then reads them from LDS); rows past it are merged when the walk reaches them */
constexpr int AW_ROWS = 1024;

/* the walk by thread 0, every row's argmax merged first by the whole workgroup */
__device__ void accept_walk(const AcceptArgs &a) {
    __shared__ int am_s[AW_ROWS];
    const int nw = a.n < AW_ROWS ? a.n : AW_ROWS;
    for (int v = threadIdx.x; v < nw; v += blockDim.x) am_s[v] = row_argmax(a, v);
    __syncthreads();
    if (threadIdx.x != 0) return;
    int v = 0, np = 0, status = 0, fin = -1;
    a.path[np++] = 0;
    for (;;) {
        const int t = v < nw ? am_s[v] : row_argmax(a, v);
        a.amax[v] = t;
        if (t < 0) { status = -1; break; }
        int next = -1;
        for (int c = v + 1; c < a.n; c++)
            if (a.parent[c] == v && a.tokens[c] == t) { next = c; break; }
        if (next < 0) { fin = t; break; }
        a.path[np++] = next;
        v = next;
    }
    a.result[0] = np;
    a.result[1] = fin;
    a.result[2] = status;
}

__global__ __launch_bounds__(256) void k_accept_walk(AcceptArgs a) { accept_walk(a); }

/* the device loop's greedy step: the walk, the commit in the same thread (it reads the
 * result the walk just wrote), then the next step's draft by the whole workgroup: one
 * launch instead of three */
__global__ __launch_bounds__(1024) void k_accept_walk_commit(AcceptArgs a, LoopArgs la) {
    accept_walk(a);
    if (threadIdx.x == 0) loop_commit_thread(la);
    __syncthreads();
    draft_body(la);
}

} // namespace

namespace hxl {

void route(const RouteArgs &a, hipStream_t st) {
    if (a.n_group <= 1 && a.T <= RS_TMAX && a.E <= RS_EMAX && a.K <= 64) {
        k_route_small<<<1, 1024, 0, st>>>(a);
        return;
    }
    if (a.n_group > 1) k_route_tokens<<<a.T, 64, 0, st>>>(a);
    else k_route_rank<<<a.T, 256, 0, st>>>(a);
    k_route_bucket<<<1, 1024, 0, st>>>(a);
}

void norm(const NormArgs &a, hipStream_t st) {
    const int n = norm_cover(a.D, a.a.nbp);
    if (n <= NM_PER * 1024) {
        const int nth = n < 1024 ? n : 1024;   /* a multiple of 64 */
        const int ept = (n + nth - 1) / nth;
        const size_t lds = (size_t)16 * norm_sq_stride(a.D) * sizeof(float);
#define HX_NORM(M_)                                                              \
        if (ept <= 2) k_norm<M_, 2><<<a.T, nth, lds, st>>>(a);                   \
        else if (ept <= 4) k_norm<M_, 4><<<a.T, nth, lds, st>>>(a);              \
        else k_norm<M_, 8><<<a.T, nth, lds, st>>>(a);                            \
        return;
        switch (a.mode) {
        case 0: HX_NORM(0)
        case 1: HX_NORM(1)
        case 2: HX_NORM(2)
        case 3: HX_NORM(3)
        default: HX_NORM(4)
        }
#undef HX_NORM
    }
    k_norm_wide<<<a.T, 1024, (size_t)a.D * 2 * sizeof(float), st>>>(a);
}

void swiglu_quant(float *g, const float *u, int T, int F, const Act &a, hipStream_t st) {
    const int64_t waves = (int64_t)T * a.nbp;
    if (waves) k_swiglu_quant<<<(int)((waves + 3) / 4), 256, 0, st>>>(g, u, T, F, a);
}

void scale_rows(float *y, int ldy, int T, int n, float s, hipStream_t st) {
    const int64_t m = (int64_t)T * n;
    if (m) k_scale_rows<<<(int)((m + 255) / 256), 256, 0, st>>>(y, ldy, T, n, s);
}

void qkv_post(const QkvArgs &a, hipStream_t st) {
    if (a.qk_norm == 2) k_fullnorm_r<<<(a.T * 2 + 3) / 4, 256, 0, st>>>(a, a.rfull);
    const int items = a.T * (a.H + a.Hkv);
    k_qkv_post<<<(items + 3) / 4, 256, 0, st>>>(a, a.rfull);
}

void kv_move(float *cache, size_t layer_stride, int L, int Hkv, int cap, int hd, int pos0, const int *path, int n,
             hipStream_t st) {
    const int64_t threads = (int64_t)L * 2 * Hkv * hd;
    if (threads && n > 0) k_kv_move<<<(int)((threads + 255) / 256), 256, 0, st>>>(cache, layer_stride, L, Hkv, cap, hd, pos0, path, n);
}

void kv_move_rows(float *cache, size_t layer_stride, int L, size_t off, int width, int pos0, const int *path, int n,
                  hipStream_t st) {
    const int64_t threads = (int64_t)L * width;
    if (threads && n > 0)
        k_kv_move_rows<<<(int)((threads + 255) / 256), 256, 0, st>>>(cache, layer_stride, L, off, width, pos0, path, n);
}

void desc_refresh(SlotDesc *desc, const ExpertW *table, const int *ulist, const int *n_active, int n_slots,
                  hipStream_t st) {
    if (n_slots > 0) k_desc_refresh<<<(n_slots + 255) / 256, 256, 0, st>>>(desc, table, ulist, n_active, n_slots);
}

void accept_greedy(const AcceptArgs &a, hipStream_t st) {
    k_argmax_part<<<a.n * ACCEPT_PARTS, 256, 0, st>>>(a);
    k_accept_walk<<<1, 256, 0, st>>>(a);
}

void accept_greedy_commit(const AcceptArgs &a, const LoopArgs &la, hipStream_t st) {
    k_argmax_part<<<a.n * ACCEPT_PARTS, 256, 0, st>>>(a);
    k_accept_walk_commit<<<1, 1024, 0, st>>>(a, la);
}

} // namespace hxl
