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
 * Launch shapes are XCD-aware: workgroup IDs are dealt round-robin to the 8 XCDs,
 * so the KV-group index is the fastest-varying part of the ID and every workgroup of
 * one XCD reads the same group's K or V rows from that XCD's L2.
 */
#include "hx_device.h"
#include "hx_launch.h"

using namespace hxd;

namespace {

constexpr int SC_ROWS = 256;   /* rows per scores workgroup (one per thread) */
constexpr int VT = 64;         /* rows per value tile */

__device__ __forceinline__ int row_slot(const TokGeom &g, int t, int v) {
    return v < g.pos0 ? v : g.pos0 + g.anc[(size_t)t * g.anc_ld + (v - g.pos0)];
}

/* One thread per row v; the heads of the KV group in passes of four. */
__global__ __launch_bounds__(256) void k_attn_scores(AttnArgs a) {
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd;
    int b = blockIdx.x;
    const int g = b % Hkv;
    b /= Hkv;
    const int t = b % a.T, c = b / a.T;
    const int nr = a.g.pos0 + a.g.depth[t] + 1;
    const int v = c * SC_ROWS + threadIdx.x;
    if (c * SC_ROWS >= nr || v >= nr) return;
    const float *krow = a.kc + ((size_t)g * a.cap + row_slot(a.g, t, v)) * hd;
    const float *qb = a.q + ((size_t)t * a.H + (size_t)g * grp) * hd;
    float *Sb = a.S + ((size_t)t * a.H + (size_t)g * grp) * a.ldS + v;
    for (int h0 = 0; h0 < grp; h0 += 4) {
        const int nh = grp - h0 < 4 ? grp - h0 : 4;
        float L[4][16];
#pragma unroll
        for (int hh = 0; hh < 4; hh++)
#pragma unroll
            for (int j = 0; j < 16; j++) L[hh][j] = 0.0f;
        for (int c16 = 0; c16 < hd; c16 += 16) {
            float kv[16];
#pragma unroll
            for (int j = 0; j < 16; j++) kv[j] = c16 + j < hd ? krow[c16 + j] : 0.0f;
#pragma unroll
            for (int hh = 0; hh < 4; hh++) {
                if (hh >= nh) break;
                const float *qh = qb + (size_t)(h0 + hh) * hd + c16;
#pragma unroll
                for (int j = 0; j < 16; j++)
                    if (c16 + j < hd) L[hh][j] = fadd(L[hh][j], fmul(qh[j], kv[j]));
            }
        }
#pragma unroll
        for (int hh = 0; hh < 4; hh++) {
            if (hh >= nh) break;
#pragma unroll
            for (int s = 8; s >= 1; s >>= 1)
#pragma unroll
                for (int j = 0; j < s; j++) L[hh][j] = fadd(L[hh][j], L[hh][j + s]);
            Sb[(size_t)(h0 + hh) * a.ldS] = fmul(a.scale, canon(L[hh][0]));
        }
    }
}

/* softmax over one (token, head) row of scores, in place (quant.c:634-642) */
__global__ __launch_bounds__(256) void k_attn_softmax(AttnArgs a) {
    __shared__ float red[256];
    __shared__ float sum_sh;
    const int t = blockIdx.x / a.H, h = blockIdx.x % a.H, tid = threadIdx.x;
    const int nr = a.g.pos0 + a.g.depth[t] + 1;
    float *s = a.S + ((size_t)t * a.H + h) * a.ldS;
    float m = -__builtin_huge_valf();
    for (int i = tid; i < nr; i += 256) {
        const float x = s[i];
        if (x == x) m = fmaxf(m, x);
    }
    red[tid] = m;
    __syncthreads();
    for (int k = 128; k >= 1; k >>= 1) {
        if (tid < k) red[tid] = fmaxf(red[tid], red[tid + k]);
        __syncthreads();
    }
    m = s[0] != s[0] ? s[0] : red[0];   /* the reference's running max starts at s[0] */
    for (int i = tid; i < nr; i += 256) s[i] = exp_port_f(fadd(s[i], -m));
    __syncthreads();
    if (tid < 16) {
        float L = 0.0f;
        for (int i = tid; i < nr; i += 16) L = fadd(L, s[i]);
#pragma unroll
        for (int k = 8; k >= 1; k >>= 1) L = fadd(L, __shfl_down(L, k, 16));
        if (tid == 0) sum_sh = L;
    }
    __syncthreads();
    const float sum = sum_sh;
    for (int i = tid; i < nr; i += 256) s[i] = fdiv(s[i], sum);
}

/* o[t][h][d] = sum_v p_v * V_v[d], v in order: one wave per head (four heads of one
 * KV group per workgroup), one lane per d; V rows staged through LDS tiles shared by
 * the four waves. */
__global__ __launch_bounds__(256) void k_attn_values(AttnArgs a) {
    __shared__ float vt[VT][64];
    __shared__ float pt[4][VT];
    __shared__ int slots[VT];
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd;
    const int nq = (grp + 3) / 4, nd = (hd + 63) / 64;
    int b = blockIdx.x;
    const int dc = b % nd;
    b /= nd;
    const int g = b % Hkv;
    b /= Hkv;
    const int hq = b % nq, t = b / nq;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, tid = threadIdx.x;
    const int hin = hq * 4 + wave;                    /* head within the group */
    const bool head_live = hin < grp;
    const int h = g * grp + (head_live ? hin : 0);
    const int d = dc * 64 + lane;
    const int nr = a.g.pos0 + a.g.depth[t] + 1;
    const float *p = a.S + ((size_t)t * a.H + h) * a.ldS;
    const float *vbase = a.vc + (size_t)g * a.cap * hd;
    float acc = 0.0f;
    for (int v0 = 0; v0 < nr; v0 += VT) {
        const int nv = nr - v0 < VT ? nr - v0 : VT;
        if (tid < nv) slots[tid] = row_slot(a.g, t, v0 + tid);
        if (lane < nv) pt[wave][lane] = head_live ? p[v0 + lane] : 0.0f;
        __syncthreads();
        for (int k = tid; k < nv * 64; k += 256) {
            const int r = k >> 6, col = k & 63, dd = dc * 64 + col;
            vt[r][col] = dd < hd ? vbase[(size_t)slots[r] * hd + dd] : 0.0f;
        }
        __syncthreads();
        if (nv == VT) {
#pragma unroll 16
            for (int i = 0; i < VT; i++) acc = fadd(acc, fmul(pt[wave][i], vt[i][lane]));
        } else {
            for (int i = 0; i < nv; i++) acc = fadd(acc, fmul(pt[wave][i], vt[i][lane]));
        }
        __syncthreads();
    }
    if (head_live && d < hd) a.out[(size_t)t * a.H * hd + (size_t)h * hd + d] = acc;
}

} // namespace

namespace hxl {

void attention(const AttnArgs &a, hipStream_t st) {
    const int max_nr = a.g.pos0 + a.T;   /* depth[t] <= t */
    const int nchunks = (max_nr + SC_ROWS - 1) / SC_ROWS;
    k_attn_scores<<<nchunks * a.T * a.Hkv, SC_ROWS, 0, st>>>(a);
    k_attn_softmax<<<a.T * a.H, 256, 0, st>>>(a);
    const int grp = a.H / a.Hkv, nq = (grp + 3) / 4, nd = (a.hd + 63) / 64;
    k_attn_values<<<a.T * nq * a.Hkv * nd, 256, 0, st>>>(a);
}

} // namespace hxl
