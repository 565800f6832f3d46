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
 * chain per lane, one summing wave per SIMD, and V tiles streamed three tiles ahead
 * into an LDS ring shared by the four summing waves (heads) of a workgroup.
 *
 * Launch shapes are XCD-aware: workgroup IDs are dealt round-robin to the 8 XCDs,
 * so the KV-group index (and value d-chunk) is the fastest-varying part of the ID and
 * the workgroups of one XCD read the same group's K or V rows from that XCD's L2.
 */
#include "hx_device.h"
#include "hx_launch.h"

using namespace hxd;

namespace {

constexpr int SC_ROWS = 256;   /* rows per scores workgroup (one per thread) */
constexpr int KC = 16;         /* K floats per staged chunk (head_dim % 16 == 0) */
constexpr int MAX_ANC = 4096;  /* ancestors of one token (max_batch) */

__device__ __forceinline__ int row_slot(const TokGeom &g, int t, int v) {
    return v < g.pos0 ? v : g.pos0 + g.anc[(size_t)t * g.anc_ld + (v - g.pos0)];
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
    const int nr = a.g.pos0 + a.g.depth[t] + 1;
    const int v0 = c * SC_ROWS;
    if (v0 >= nr) return;   /* uniform */
    const int tid = threadIdx.x;
    const int nrows = nr - v0 < SC_ROWS ? nr - v0 : SC_ROWS;
    slot_s[tid] = row_slot(a.g, t, v0 + (tid < nrows ? tid : nrows - 1));
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
 * LDS (qT[h][j][i] = q[h][16 i + j]), read four i at a time. */
constexpr int S16_NP = 2;              /* 16-row passes per workgroup */
constexpr int S16_RB = 16 * S16_NP;    /* rows per workgroup */

template <int HI>
__global__ __launch_bounds__(256) void k_attn_scores16(AttnArgs a) {
    __shared__ float4 qT[8][16][HI / 4];
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd;
    int b = blockIdx.x;
    const int g = b % Hkv;
    b /= Hkv;
    const int t = b % a.T, c = b / a.T;
    const int nr = a.g.pos0 + a.g.depth[t] + 1;
    const int v0 = c * S16_RB;
    if (v0 >= nr) return;   /* uniform */
    const int tid = threadIdx.x, j = tid & 15, rl = tid >> 4;
    float kv[S16_NP][HI];
    int vrow[S16_NP];
#pragma unroll
    for (int pass = 0; pass < S16_NP; pass++) {
        const int v = v0 + pass * 16 + rl;
        vrow[pass] = v;
        const float *kr = a.kc + ((size_t)g * a.cap + row_slot(a.g, t, v < nr ? v : nr - 1)) * hd + j;
#pragma unroll
        for (int i = 0; i < HI; i++) kv[pass][i] = kr[16 * i];
    }
    for (int h0 = 0; h0 < grp; h0 += 8) {
        __syncthreads();
        {
            const float *qb = a.q + ((size_t)t * a.H + (size_t)g * grp + h0) * hd;
            float *qf = (float *)qT;
            for (int x = tid; x < 8 * hd; x += 256) {
                const int hh = x / hd, e = x % hd;
                qf[(hh * 16 + (e & 15)) * HI + (e >> 4)] = h0 + hh < grp ? qb[(size_t)hh * hd + e] : 0.0f;
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

__device__ __forceinline__ float sum16_lds(const float *es, int n, int lane16, float L) {
    /* lane lane16 of 16: continues the sequential sum L with es[lane16], es[lane16 + 16],
     * ..., the next 8 operands read while the current 8 are added */
    int i = lane16;
    float cur[8], nxt[8];
    const int full = n >= 16 * 8 ? (n - lane16) / 128 : 0;   /* groups of 8 in range */
    if (full > 0) {
#pragma unroll
        for (int u = 0; u < 8; u++) cur[u] = es[i + 16 * u];
        for (int gi = 0; gi < full; gi++) {
            const int inx = gi + 1 < full ? i + 128 : i;
#pragma unroll
            for (int u = 0; u < 8; u++) nxt[u] = es[inx + 16 * u];
#pragma unroll
            for (int u = 0; u < 8; u++) L = fadd(L, cur[u]);
#pragma unroll
            for (int u = 0; u < 8; u++) cur[u] = nxt[u];
            i += 128;
        }
    }
    for (; i < n; i += 16) L = fadd(L, es[i]);
    return L;
}

/* softmax over one (token, head) row of scores, in place (quant.c:634-642): running
 * max from s[0] (a NaN s[0] stays the max, later NaNs are skipped), e = exp(s - max),
 * sum16 of e, p = e / sum. Up to 8192 scores stay in registers; longer rows are
 * processed in chunks of 8192 re-read from the row. */
constexpr int SM_PER = 32;
constexpr int SM_CH = 256 * SM_PER;

__global__ __launch_bounds__(256) void k_attn_softmax(AttnArgs a) {
    __shared__ float es[SM_CH];
    __shared__ float red[4];
    __shared__ float sum_sh;
    const int t = blockIdx.x / a.H, h = blockIdx.x % a.H, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nr = a.g.pos0 + a.g.depth[t] + 1;
    float *s = a.S + ((size_t)t * a.H + h) * a.ldS;
    const bool inreg = nr <= SM_CH;
    float x[SM_PER];
    float m = -__builtin_huge_valf();
    if (inreg) {
#pragma unroll
        for (int u = 0; u < SM_PER; u++) {
            const int i = tid + 256 * u;
            x[u] = i < nr ? s[i] : -__builtin_huge_valf();
        }
#pragma unroll
        for (int u = 0; u < SM_PER; u++)
            if (x[u] == x[u]) m = fmaxf(m, x[u]);
    } else {
        for (int i = tid; i < nr; i += 256) {
            const float v = s[i];
            if (v == v) m = fmaxf(m, v);
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s0 = s[0];
    if (s0 != s0) m = s0;
    float L = 0.0f;   /* lane tid < 16: partial of the elements i = tid (mod 16) */
    for (int c0 = 0; c0 < nr; c0 += SM_CH) {
        const int n = nr - c0 < SM_CH ? nr - c0 : SM_CH;
        if (c0) __syncthreads();
        if (inreg) {
#pragma unroll
            for (int u = 0; u < SM_PER; u++) {
                const int i = tid + 256 * u;
                if (i < n) {
                    x[u] = exp_port_f(fadd(x[u], -m));
                    es[i] = x[u];
                }
            }
        } else {
            for (int i = tid; i < n; i += 256) es[i] = exp_port_f(fadd(s[c0 + i], -m));
        }
        __syncthreads();
        /* SM_CH is a multiple of 16, so element c0 + i keeps lane (c0 + i) % 16 = i % 16 */
        if (tid < 16) L = sum16_lds(es, n, tid, L);
        if (!inreg) {
            __syncthreads();
            for (int i = tid; i < n; i += 256) s[c0 + i] = es[i];
        }
    }
    if (tid < 16) {
#pragma unroll
        for (int k = 8; k >= 1; k >>= 1) L = fadd(L, __shfl_down(L, k, 16));
        if (tid == 0) sum_sh = L;
    }
    __syncthreads();
    const float sum = sum_sh;
    if (inreg) {
#pragma unroll
        for (int u = 0; u < SM_PER; u++) {
            const int i = tid + 256 * u;
            if (i < nr) s[i] = fdiv(x[u], sum);
        }
    } else {
        for (int i = tid; i < nr; i += 256) s[i] = fdiv(s[i], sum);
    }
}

/* o[t][h][d] = sum_v p_v * V_v[d], v in order. A workgroup sums up to four heads of
 * one token t in one KV group g, for one 64-wide d chunk (one wave per head, lane = d),
 * and has four more waves that only move data: they issue LDS-direct loads
 * (global_load_lds: the bytes go from memory straight into LDS, no registers, a few
 * address instructions per KiB), so the summing waves keep their SIMD's VALU to the
 * product + dependent add of each row. Tiles of 128 rows and their p values cycle
 * through a 4-slot LDS ring: while tile i is summed, tiles i+1 and i+2 are in flight
 * and tile i+3 is issued into the slot of tile i-1. A loader wave waits (vmcnt) only
 * for the tile it is about to publish and then joins the barrier without a release
 * fence (a fence would wait for every load in flight). Products of 16 rows are formed
 * before their 16 adds, so no product waits in front of the chain. Loads are
 * unconditional: tile indexes are clamped to the last tile and rows to valid ones;
 * rows past the chain are never read back, columns past head_dim only feed discarded
 * lanes; every LDS write has landed before the workgroup ends. */
constexpr int VT2 = 128;              /* rows per tile */
constexpr int VNS = 4;                /* LDS ring slots: one summed, three in flight */
constexpr int VLPT = 10;              /* loads per loader wave per tile: 8 x 1 KiB of V, 2 x 64 p */
constexpr int VPS = VT2 + 4;          /* p row stride: the four heads' rows in different banks */

__global__ __launch_bounds__(512) void k_attn_values(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) float vt[VNS][VT2][64];
    __shared__ __attribute__((aligned(16))) float pt[VNS][4][VPS];
    __shared__ int anc_s[MAX_ANC];
    const int Hkv = a.Hkv, grp = a.H / Hkv, hd = a.hd;
    const int nd = (hd + 63) / 64, qpt = (grp + 3) / 4;
    int b = blockIdx.x;
    const int dc = b % nd;
    b /= nd;
    const int g = b % Hkv;
    b /= Hkv;
    const int hq = b % qpt, t = b / qpt;
    const int tid = threadIdx.x, wave = (tid >> 6) & 3, lane = tid & 63;
    const bool loader = tid >= 256;
    const int hh = hq * 4 + wave;
    const bool live = hh < grp;
    const int h = g * grp + (live ? hh : 0);
    const int pos0 = a.g.pos0, dep = a.g.depth[t];
    const int nr = pos0 + dep + 1;
    const int ntiles = (nr + VT2 - 1) / VT2, last = ntiles - 1;
    for (int jj = tid; jj <= dep; jj += 512) anc_s[jj] = pos0 + a.g.anc[(size_t)t * a.g.anc_ld + jj];
    __syncthreads();
    float acc = 0.0f;
    if (loader) {
        /* loader wave w: rows w*32 + 4k + lane/16 of each tile (k = 0..7), float4 column
         * lane%16; its head's p (two 64-entry dword loads per tile) */
        const int c4 = (lane & 15) * 4, rsub = lane >> 4;
        const float *vcol = a.vc + (size_t)g * a.cap * hd + (dc * 64 + c4 < hd ? dc * 64 + c4 : 0);
        const float *prow = a.S + ((size_t)t * a.H + h) * a.ldS;
        auto issue = [&](int i) {
            const int ti = i < last ? i : last, slot = i % VNS;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                int v = ti * VT2 + wave * 32 + 4 * k + rsub;
                v = v < nr ? v : nr - 1;
                const float *src = vcol + (size_t)(v < pos0 ? v : anc_s[v - pos0]) * hd;
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                                 (__attribute__((address_space(3))) void *)&vt[slot][wave * 32 + 4 * k][0],
                                                 16, 0, 0);
            }
#pragma unroll
            for (int c = 0; c < 2; c++) {
                int vp = ti * VT2 + c * 64 + lane;
                vp = vp < nr ? vp : nr - 1;
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(prow + vp),
                                                 (__attribute__((address_space(3))) void *)&pt[slot][wave][c * 64], 4,
                                                 0, 0);
            }
        };
        issue(0);
        issue(1);
        issue(2);
        for (int i = 0; i < ntiles; i++) {
            /* tile i landed (tiles i+1, i+2 may be in flight); a bare barrier, so that no
             * release fence waits for the loads still in flight */
            HX_WAIT_VMCNT(2 * VLPT);
            __builtin_amdgcn_s_barrier();
            issue(i + 3);              /* into the slot of tile i - 1, summed before this barrier */
        }
        HX_WAIT_VMCNT(0);              /* no LDS write may land after the loop */
    } else {
        /* summing wave w: heads hq * 4 + lane / 16, columns w * 16 + lane % 16 of the
         * chunk -- the 16 lanes of a head read 64 bytes of each V row and the four heads
         * share them (broadcast), a quarter of the LDS reads of one head per wave */
        const float *const pw0 = pt[0][lane >> 4], *const vw0 = &vt[0][0][wave * 16 + (lane & 15)];
        for (int i = 0; i < ntiles; i++) {
            __syncthreads();
            const int slot = i % VNS, nv = nr - i * VT2;
            const float *pw = pw0 + slot * (4 * VPS), *vw = vw0 + slot * (VT2 * 64);
            if (nv >= VT2) {
                float pA[16], vA[16], pB[16], vB[16];
#define HX_GRD(P_, V_, c_)                                                               \
                _Pragma("unroll") for (int j = 0; j < 16; j++) { P_[j] = pw[(c_) + j]; V_[j] = vw[((c_) + j) * 64]; }
#define HX_GSUM(P_, V_)                                                                  \
                {                                                                        \
                    float pr[16];                                                        \
                    _Pragma("unroll") for (int j = 0; j < 16; j++) pr[j] = fmul(P_[j], V_[j]); \
                    _Pragma("unroll") for (int j = 0; j < 16; j++) acc = fadd(acc, pr[j]); \
                }
                HX_GRD(pA, vA, 0)
                HX_GRD(pB, vB, 16) HX_GSUM(pA, vA)
                HX_GRD(pA, vA, 32) HX_GSUM(pB, vB)
                HX_GRD(pB, vB, 48) HX_GSUM(pA, vA)
                HX_GRD(pA, vA, 64) HX_GSUM(pB, vB)
                HX_GRD(pB, vB, 80) HX_GSUM(pA, vA)
                HX_GRD(pA, vA, 96) HX_GSUM(pB, vB)
                HX_GRD(pB, vB, 112) HX_GSUM(pA, vA)
                HX_GSUM(pB, vB)
#undef HX_GSUM
#undef HX_GRD
            } else {
                for (int r = 0; r < nv; r++) acc = fadd(acc, fmul(pw[r], vw[r * 64]));
            }
        }
    }
    /* every LDS-direct load has landed and every tile has been read: the sums go through
     * LDS so that wave w writes (and quantizes) the 64 columns of head hq * 4 + w */
    __syncthreads();
    float *ot = &vt[0][0][0];   /* [4 heads][64 columns] */
    if (!loader) ot[(lane >> 4) * 64 + wave * 16 + (lane & 15)] = acc;
    __syncthreads();
    if (!loader) {
        const float x = ot[wave * 64 + lane];
        const int d = dc * 64 + lane;
        if (live && d < hd) a.out[(size_t)t * a.H * hd + (size_t)h * hd + d] = x;
        if (a.qo_on && live) quant_block_wave(x, a.qo, a.qo_hm ? h * a.T + t : t, a.qo_hm ? dc : h * (hd >> 6) + dc);
    }
}

} // namespace

namespace hxl {

void attention_scores(const AttnArgs &a, hipStream_t st) {
    const int max_nr = a.g.pos0 + a.T;   /* depth[t] <= t */
    if (a.hd % 64 == 0 && a.hd <= 512) {
        const int grid = ((max_nr + S16_RB - 1) / S16_RB) * a.T * a.Hkv;
        switch (a.hd / 16) {
        case 4: k_attn_scores16<4><<<grid, 256, 0, st>>>(a); return;
        case 8: k_attn_scores16<8><<<grid, 256, 0, st>>>(a); return;
        case 12: k_attn_scores16<12><<<grid, 256, 0, st>>>(a); return;
        case 16: k_attn_scores16<16><<<grid, 256, 0, st>>>(a); return;
        case 20: k_attn_scores16<20><<<grid, 256, 0, st>>>(a); return;
        case 24: k_attn_scores16<24><<<grid, 256, 0, st>>>(a); return;
        case 28: k_attn_scores16<28><<<grid, 256, 0, st>>>(a); return;
        default: k_attn_scores16<32><<<grid, 256, 0, st>>>(a); return;
        }
    }
    const int nchunks = (max_nr + SC_ROWS - 1) / SC_ROWS;
    const int grp = a.H / a.Hkv, nsc = nchunks * a.T * a.Hkv;
    if (grp % 8 == 0) k_attn_scores<8><<<nsc, SC_ROWS, 0, st>>>(a);
    else if (grp % 4 == 0) k_attn_scores<4><<<nsc, SC_ROWS, 0, st>>>(a);
    else if (grp % 2 == 0) k_attn_scores<2><<<nsc, SC_ROWS, 0, st>>>(a);
    else k_attn_scores<1><<<nsc, SC_ROWS, 0, st>>>(a);
}

void attention_finish(const AttnArgs &a, hipStream_t st) {
    const int grp = a.H / a.Hkv;
    k_attn_softmax<<<a.T * a.H, 256, 0, st>>>(a);
    const int nd = (a.hd + 63) / 64, qpt = (grp + 3) / 4;
    k_attn_values<<<a.T * qpt * a.Hkv * nd, 512, 0, st>>>(a);
}

void attention(const AttnArgs &a, hipStream_t st) {
    attention_scores(a, st);
    attention_finish(a, st);
}

} // namespace hxl
