/*
 * k_gemm.hip — weight repacking, activation quantization and the matrix products of
 * the verify step on gfx950.
 *
 * Reference semantics: NUMERICS §2-3 (engine/src/quant.c:325-427). Every (token, row)
 * output is one lane's fold acc = acc + (float)isum_g * (dw_g * dx_g) over the blocks
 * g of its row in ascending order; isum_g is the exact int32 block sum from one
 * v_mfma_i32_16x16x64_i8 (K = one 64-block). Which other tokens share the MFMA tile
 * cannot change any output, so a batch equals T single-token calls bit for bit
 * (reference INV-DET-2, governance/INVARIANTS.md:12).
 */
#include "hx_device.h"
#include "hx_launch.h"
#include <hip/hip_ext.h>

using namespace hxd;

namespace {

constexpr uint32_t LO4 = 0x0F0F0F0Fu;

/* ------------------------------------------------------------ repacking */

/* FORMAT.md §6 Q8 rows (66-byte blocks) -> tiles + transposed scales. src holds rows
 * [r0, r0 + count) (pad rows beyond `rows` are not read); one thread per (row, block);
 * pad rows and the pad block get zeros. */
__global__ void k_repack_q8(const uint8_t *__restrict__ src, int r0, int count, int rows, int nb, QMat m, uint8_t *w,
                            uint16_t *d) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)count * m.nbp) return;
    const int r = r0 + (int)(idx / m.nbp), g = (int)(idx % m.nbp);
    const bool real = r < rows && g < nb;
    const uint8_t *blk = src + ((size_t)(r - r0) * nb + g) * 66;
    d[(size_t)g * m.rows_pad + r] = real ? (uint16_t)(blk[0] | (blk[1] << 8)) : (uint16_t)0;
    uint8_t *tile = w + ((size_t)(r >> 4) * m.nbp + g) * 1024;
    for (int kg = 0; kg < 4; kg++)
        for (int b = 0; b < 16; b++) {
            const int e = b < 8 ? 8 * kg + b : 32 + 8 * kg + (b - 8);
            tile[(size_t)((r & 15) + 16 * kg) * 16 + b] = real ? blk[2 + e] : (uint8_t)0;
        }
}

/* FORMAT.md §6 Q4 rows (34-byte blocks) -> tiles of block pairs + transposed scales. */
__global__ void k_repack_q4(const uint8_t *__restrict__ src, int r0, int count, int rows, int nb, QMat m, uint8_t *w,
                            uint16_t *d) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)count * m.nbp) return;
    const int r = r0 + (int)(idx / m.nbp), g = (int)(idx % m.nbp);
    const bool real = r < rows && g < nb;
    const uint8_t *blk = src + ((size_t)(r - r0) * nb + g) * 34;
    d[(size_t)g * m.rows_pad + r] = real ? (uint16_t)(blk[0] | (blk[1] << 8)) : (uint16_t)0;
    uint8_t *tile = w + ((size_t)(r >> 4) * (m.nbp / 2) + (g >> 1)) * 1024;
    for (int kg = 0; kg < 4; kg++)
        for (int b = 0; b < 8; b++)
            tile[(size_t)((r & 15) + 16 * kg) * 16 + (g & 1) * 8 + b] = real ? blk[2 + 8 * kg + b] : (uint8_t)0;
}

/* ------------------------------------------------------------ activation quantization */

/* NUMERICS §2 on rows of x (f32 [T][n], row stride ldx): one wave per (row, block). */
__global__ void k_quant_rows(const float *__restrict__ x, int64_t ldx, int T, int nb, Act a) {
    const int wave = (int)((blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6);
    if (wave >= T * a.nbp) return;   /* uniform per wave */
    const int t = wave / a.nbp, g = wave % a.nbp, lane = threadIdx.x & 63;
    const float v = g < nb ? x[(size_t)t * ldx + (size_t)g * 64 + lane] : 0.0f;
    quant_block_wave(v, a, t, g);
}

/* ------------------------------------------------------------ the MFMA fold */

__device__ __forceinline__ v4i load16(const uint8_t *p) { return *(const v4i *)p; }

__device__ __forceinline__ void unpack_q4(v4i raw, v4i &a0, v4i &a1) {
    a0.x = raw.x & LO4; a0.y = raw.y & LO4; a0.z = (raw.x >> 4) & LO4; a0.w = (raw.y >> 4) & LO4;
    a1.x = raw.z & LO4; a1.y = raw.w & LO4; a1.z = (raw.z >> 4) & LO4; a1.w = (raw.w >> 4) & LO4;
}

/* Folds blocks [0, nb) of row tile rt of m against NT*16 tokens starting at token
 * index t0 (token t's activation row is row_of(t); tokens >= n read row_of(n - 1) and
 * their results are discarded). acc[tt][i] holds (row rt*16 + 4*(lane/16) + i,
 * token t0 + tt*16 + lane%16).
 *
 * A wave walks K one block pair at a time; the loads of pair gp + 1 (weights, scales,
 * the tokens' activation blocks and their scales) are issued before pair gp is folded,
 * so each pair's loads wait behind the previous pair's MFMAs and folds instead of
 * stalling the wave. */
template <int NT>
struct FoldStage {
    v4i w0, w1;          /* Q8: the two blocks; Q4: w0 the packed pair */
    uint2 s0, s1;        /* the blocks' f16 scales of this lane's 4 rows */
    v4i b[2][NT];        /* activation blocks (16 bytes of each token's block) */
    float dx[2][NT];
    int sx[2][NT];       /* Q4: the activation block sums */
};

template <int NT>
__device__ __forceinline__ void fold_load(FoldStage<NT> &f, const QMat &m, int rt, const Act &a, int gp,
                                          const int (&arow)[NT], const uint16_t *dcol) {
    const int lane = threadIdx.x & 63, kg = lane >> 4, npair = m.nbp >> 1;
    if (m.dtype == 4) {
        f.w0 = load16(m.w + ((size_t)rt * npair + gp) * 1024 + lane * 16);
    } else {
        const uint8_t *base = m.w + ((size_t)rt * m.nbp + 2 * gp) * 1024 + lane * 16;
        f.w0 = load16(base);
        f.w1 = load16(base + 1024);
    }
    f.s0 = *(const uint2 *)(dcol + (size_t)(2 * gp) * m.rows_pad);
    f.s1 = *(const uint2 *)(dcol + (size_t)(2 * gp + 1) * m.rows_pad);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int g = 2 * gp + j < m.nb ? 2 * gp + j : m.nb - 1;   /* a pad block is never folded */
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
            const size_t ab = (size_t)arow[tt] * a.nbp + g;
            f.b[j][tt] = load16((const uint8_t *)(a.q + ab * 64 + kg * 16));
            f.dx[j][tt] = a.d[ab];
            if (m.dtype == 4) f.sx[j][tt] = a.s[ab];
        }
    }
}

template <int NT, typename RowOf>
__device__ __forceinline__ void fold_tile(const QMat &m, int rt, const Act &a, int t0, int n, RowOf row_of,
                                          float (&acc)[NT][4]) {
    const int lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
    int arow[NT];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        int t = t0 + tt * 16 + lr;
        t = t < n ? t : n - 1;
        arow[tt] = row_of(t);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[tt][i] = 0.0f;
    }
    const v4i zero = {0, 0, 0, 0};
    const int npair = m.nbp >> 1;
    const uint16_t *dcol = m.d + rt * 16 + 4 * kg;
    FoldStage<NT> cur, nxt;
    fold_load<NT>(cur, m, rt, a, 0, arow, dcol);
    for (int gp = 0; gp < npair; gp++) {
        if (gp + 1 < npair) fold_load<NT>(nxt, m, rt, a, gp + 1, arow, dcol);
        v4i w0 = cur.w0, w1 = cur.w1;
        if (m.dtype == 4) unpack_q4(cur.w0, w0, w1);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int g = 2 * gp + j;
            if (g >= m.nb) break;
            const uint2 sw = j ? cur.s1 : cur.s0;
            float dw[4];
            dw[0] = h2f((uint16_t)(sw.x & 0xffff));
            dw[1] = h2f((uint16_t)(sw.x >> 16));
            dw[2] = h2f((uint16_t)(sw.y & 0xffff));
            dw[3] = h2f((uint16_t)(sw.y >> 16));
            const v4i wa = j ? w1 : w0;
#pragma unroll
            for (int tt = 0; tt < NT; tt++) {
                v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, cur.b[j][tt], zero, 0, 0, 0);
                const float dx = cur.dx[j][tt];
                if (m.dtype == 4) {
                    const int off = 8 * cur.sx[j][tt];   /* sum(nib * q) - 8 sum(q) = sum((nib - 8) q) */
                    c.x -= off; c.y -= off; c.z -= off; c.w -= off;
                }
                acc[tt][0] = fadd(acc[tt][0], fmul((float)c.x, fmul(dw[0], dx)));
                acc[tt][1] = fadd(acc[tt][1], fmul((float)c.y, fmul(dw[1], dx)));
                acc[tt][2] = fadd(acc[tt][2], fmul((float)c.z, fmul(dw[2], dx)));
                acc[tt][3] = fadd(acc[tt][3], fmul((float)c.w, fmul(dw[3], dx)));
            }
        }
        cur = nxt;
    }
}

/* ------------------------------------------------------------ dense segmented GEMM */

/* One wave per (16-row tile, group of NT 16-token tiles). Workgroup b covers row tiles
 * of workgroup-row b % wgr and token group b / wgr; wgr is a multiple of 8, so every
 * token group of a row tile runs on the same XCD (IDs are dealt round-robin to the 8
 * XCDs) and re-reads its weights from that XCD's L2. */
template <int NT>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs args, int wgr) {
    const int rw = (int)blockIdx.x % wgr, tg = (int)blockIdx.x / wgr;
    int s = 0;
    while (s + 1 < args.nseg && rw >= args.seg[s + 1].wg0) s++;
    const GemmSeg &sg = args.seg[s];
    if (rw >= sg.wg0 + (sg.m.rows_pad / 16 + 3) / 4) return;   /* padding workgroup */
    const int rt = (rw - sg.wg0) * 4 + (int)(threadIdx.x >> 6);
    if (rt * 16 >= sg.m.rows_pad) return;
    const int t0 = args.t0 + tg * NT * 16;
    if (t0 >= args.T) return;
    float acc[NT][4];
    fold_tile<NT>(sg.m, rt, args.a, t0, args.T, [](int t) { return t; }, acc);
    const int lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        const int t = t0 + tt * 16 + lr;
        if (t >= args.T) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = rt * 16 + 4 * kg + i;
            if (row < sg.m.rows) {
                float y = canon(acc[tt][i]);
                if (sg.scale_on) y = canon(fmul(sg.scale, y));
                sg.Y[(size_t)t * sg.ldy + row] = y;
            }
        }
    }
}

/* ------------------------------------------------------------ split-K products (few tokens) */

/* With few tokens a product is bound by how many weight bytes are in flight, not by the
 * MFMA rate. The split-K kernels give each wave of a workgroup a contiguous range of
 * block pairs of one 16-row tile and issue all its loads at once; each wave writes the
 * NUMERICS §3 terms (float)isum_g * (dw_g * dx_g) of its blocks to LDS, and after one
 * barrier one thread per (row, token) folds the terms of blocks 0, 1, ... in order, so
 * the result is the one-lane fold bit for bit. */
constexpr int SK_MAXP = 4;      /* block pairs per wave */
constexpr int TK_WAVES_GATEUP = 8;   /* waves per workgroup of k_expert_tk: gate/up (token blocks staged once for 8 waves) */
constexpr int TK_WAVES_DOWN = 4;     /* and down (more, smaller workgroups over the shorter rows) */
constexpr size_t TK_LDS_MAX = 65536;
constexpr int TK_CHUNK_ROWS = 128;   /* rows of a slot kept on one XCD (two 128-byte scale lines) */
constexpr int SK_LDS = 65536;   /* bytes of terms per workgroup */
constexpr int SK_DUMMY = 1024;  /* LDS after the terms: stores of padding token columns */

/* Terms of pairs [p0, p1) of row tile rt of the NM matrices ms (same dtype DT and
 * blocks, one shared activation) for tokens t0 .. t0 + 15 (token t's activation row
 * is row_of(t); tokens >= n repeat row_of(n - 1)). Term (matrix mi, block g, token c,
 * row r) goes to P[mi * pstride + (g * ntok + c) * 16 + r] for c < ntok. */
template <int DT, int NM>
__device__ __forceinline__ void tile_terms_chunk(const QMat *ms, int rt, const Act &a, int arow, int ntok, int p0,
                                                 int p1, float *P, int pstride) {
    const int lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
    const int npair = ms[0].nbp >> 1, nb = ms[0].nb;
    v4i raw[NM][SK_MAXP][DT == 4 ? 1 : 2];
    uint2 sc[NM][SK_MAXP][2];
    v4i xq[SK_MAXP][2];
    float dx[SK_MAXP][2];
    int sx[SK_MAXP][2];
#pragma unroll
    for (int k = 0; k < SK_MAXP; k++) {
        const int gp = p0 + k < p1 ? p0 + k : p1 - 1;
#pragma unroll
        for (int mi = 0; mi < NM; mi++) {
            const QMat &m = ms[mi];
            if (DT == 4) {
                raw[mi][k][0] = load16(m.w + ((size_t)rt * npair + gp) * 1024 + lane * 16);
            } else {
                const uint8_t *base = m.w + ((size_t)rt * m.nbp + 2 * gp) * 1024 + lane * 16;
                raw[mi][k][0] = load16(base);
                raw[mi][k][DT == 4 ? 0 : 1] = load16(base + 1024);
            }
            const uint16_t *dcol = m.d + rt * 16 + 4 * kg;
            sc[mi][k][0] = *(const uint2 *)(dcol + (size_t)(2 * gp) * m.rows_pad);
            sc[mi][k][1] = *(const uint2 *)(dcol + (size_t)(2 * gp + 1) * m.rows_pad);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const size_t ab = (size_t)arow * a.nbp + 2 * gp + j;
            xq[k][j] = load16((const uint8_t *)(a.q + ab * 64 + kg * 16));
            dx[k][j] = a.d[ab];
            sx[k][j] = DT == 4 ? a.s[ab] : 0;
        }
    }
    /* all MFMAs first (each into its own registers), then the f32 terms: no term waits on
     * the MFMA just issued. Lanes of token columns >= ntok store to the dummy area. */
    const v4i zero = {0, 0, 0, 0};
    v4i cc[NM][SK_MAXP][2];
#pragma unroll
    for (int k = 0; k < SK_MAXP; k++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int mi = 0; mi < NM; mi++) {
                v4i wa;
                if (DT == 4) {
                    v4i w0, w1;
                    unpack_q4(raw[mi][k][0], w0, w1);
                    wa = j ? w1 : w0;
                } else {
                    wa = raw[mi][k][DT == 4 ? 0 : j];
                }
                cc[mi][k][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, xq[k][j], zero, 0, 0, 0);
            }
    float *dmy = P + (size_t)NM * nb * ntok * 16 + lane * 4;   /* after the NM matrices' terms */
#pragma unroll
    for (int k = 0; k < SK_MAXP; k++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int g = 2 * (p0 + k) + j;
            if (p0 + k >= p1 || g >= nb) continue;   /* uniform */
#pragma unroll
            for (int mi = 0; mi < NM; mi++) {
                v4i c = cc[mi][k][j];
                if (DT == 4) {
                    const int off = 8 * sx[k][j];   /* sum(nib * q) - 8 sum(q) = sum((nib - 8) q) */
                    c.x -= off; c.y -= off; c.z -= off; c.w -= off;
                }
                const uint2 sw = sc[mi][k][j];
                const float d = dx[k][j];
                float4 v;
                v.x = fmul((float)c.x, fmul(h2f((uint16_t)(sw.x & 0xffff)), d));
                v.y = fmul((float)c.y, fmul(h2f((uint16_t)(sw.x >> 16)), d));
                v.z = fmul((float)c.z, fmul(h2f((uint16_t)(sw.y & 0xffff)), d));
                v.w = fmul((float)c.w, fmul(h2f((uint16_t)(sw.y >> 16)), d));
                float *dst = lr < ntok ? P + (size_t)mi * pstride + ((size_t)g * ntok + lr) * 16 + 4 * kg : dmy;
                *(float4 *)dst = v;
            }
        }
    }
}

template <int DT, int NM, typename RowOf>
__device__ __forceinline__ void tile_terms(const QMat *ms, int rt, const Act &a, int t0, int n, int ntok,
                                           RowOf row_of, int p0, int p1, float *P, int pstride) {
    int t = t0 + (threadIdx.x & 15);
    t = t < n ? t : n - 1;
    const int arow = row_of(t);
    for (int pc = p0; pc < p1; pc += SK_MAXP)   /* uniform */
        tile_terms_chunk<DT, NM>(ms, rt, a, arow, ntok, pc, pc + SK_MAXP < p1 ? pc + SK_MAXP : p1, P, pstride);
}

/* sum of the terms P[(g * ntok) * 16 + tid] over blocks g = 0 .. nb-1, in order */
__device__ __forceinline__ float fold_terms(const float *P, int nb, int ntok, int tid) {
    float acc = 0.0f;
    const int st = ntok * 16;
    int g = 0;
    for (; g + 8 <= nb; g += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = P[(g + u) * st + tid];
#pragma unroll
        for (int u = 0; u < 8; u++) acc = fadd(acc, v[u]);
    }
    for (; g < nb; g++) acc = fadd(acc, P[g * st + tid]);
    return acc;
}

/* pair range of wave w of W over npair pairs */
__device__ __forceinline__ void wave_pairs(int npair, int W, int w, int &p0, int &p1) {
    const int ppw = (npair + W - 1) / W;
    p0 = w * ppw;
    p1 = p0 + ppw < npair ? p0 + ppw : npair;
}

/* Resident split-K: a wave's weights and scales of NM matrices for its block pairs
 * [p0, p1) (at most SK_MAXP) stay in registers while token tiles pass through them;
 * skm_load_x loads one tile's activation blocks (row arow of a for this lane's token),
 * skm_terms writes the tile's terms as tile_terms_chunk does. */
template <int DT, int NM>
struct SkmRegs {
    v4i raw[NM][SK_MAXP][DT == 4 ? 1 : 2];
    uint2 sc[NM][SK_MAXP][2];
    v4i xq[SK_MAXP][2];
    float dx[SK_MAXP][2];
    int sx[SK_MAXP][2];
};

template <int DT, int NM>
__device__ __forceinline__ void skm_load_w(SkmRegs<DT, NM> &r, const QMat *ms, int rt, int p0, int p1) {
    const int lane = threadIdx.x & 63, kg = lane >> 4;
    const int npair = ms[0].nbp >> 1;
#pragma unroll
    for (int k = 0; k < SK_MAXP; k++) {
        const int gp = p0 + k < p1 ? p0 + k : p1 - 1;
#pragma unroll
        for (int mi = 0; mi < NM; mi++) {
            const QMat &m = ms[mi];
            if (DT == 4) {
                r.raw[mi][k][0] = load16(m.w + ((size_t)rt * npair + gp) * 1024 + lane * 16);
            } else {
                const uint8_t *base = m.w + ((size_t)rt * m.nbp + 2 * gp) * 1024 + lane * 16;
                r.raw[mi][k][0] = load16(base);
                r.raw[mi][k][DT == 4 ? 0 : 1] = load16(base + 1024);
            }
            const uint16_t *dcol = m.d + rt * 16 + 4 * kg;
            r.sc[mi][k][0] = *(const uint2 *)(dcol + (size_t)(2 * gp) * m.rows_pad);
            r.sc[mi][k][1] = *(const uint2 *)(dcol + (size_t)(2 * gp + 1) * m.rows_pad);
        }
    }
}

template <int DT, int NM>
__device__ __forceinline__ void skm_load_x(SkmRegs<DT, NM> &r, const Act &a, int arow, int p0, int p1) {
    const int kg = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int k = 0; k < SK_MAXP; k++) {
        const int gp = p0 + k < p1 ? p0 + k : p1 - 1;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const size_t ab = (size_t)arow * a.nbp + 2 * gp + j;
            r.xq[k][j] = load16((const uint8_t *)(a.q + ab * 64 + kg * 16));
            r.dx[k][j] = a.d[ab];
            r.sx[k][j] = DT == 4 ? a.s[ab] : 0;
        }
    }
}

template <int DT, int NM>
__device__ __forceinline__ void skm_terms(const SkmRegs<DT, NM> &r, int nb, int ntok, int p0, int p1, float *P,
                                          int pstride) {
    const int lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
    const v4i zero = {0, 0, 0, 0};
    float *dmy = P + (size_t)NM * nb * ntok * 16 + lane * 4;   /* after the NM matrices' terms */
    /* one matrix at a time: its MFMAs first (each into its own registers), then its f32
     * terms, so no term waits on the MFMA just issued */
#pragma unroll
    for (int mi = 0; mi < NM; mi++) {
        v4i cc[SK_MAXP][2];
#pragma unroll
        for (int k = 0; k < SK_MAXP; k++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                v4i wa;
                if (DT == 4) {
                    v4i w0, w1;
                    unpack_q4(r.raw[mi][k][0], w0, w1);
                    wa = j ? w1 : w0;
                } else {
                    wa = r.raw[mi][k][DT == 4 ? 0 : j];
                }
                cc[k][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, r.xq[k][j], zero, 0, 0, 0);
            }
#pragma unroll
        for (int k = 0; k < SK_MAXP; k++) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int g = 2 * (p0 + k) + j;
                if (p0 + k >= p1 || g >= nb) continue;   /* uniform */
                v4i c = cc[k][j];
                if (DT == 4) {
                    const int off = 8 * r.sx[k][j];   /* sum(nib * q) - 8 sum(q) = sum((nib - 8) q) */
                    c.x -= off; c.y -= off; c.z -= off; c.w -= off;
                }
                const uint2 sw = r.sc[mi][k][j];
                const float d = r.dx[k][j];
                float4 v;
                v.x = fmul((float)c.x, fmul(h2f((uint16_t)(sw.x & 0xffff)), d));
                v.y = fmul((float)c.y, fmul(h2f((uint16_t)(sw.x >> 16)), d));
                v.z = fmul((float)c.z, fmul(h2f((uint16_t)(sw.y & 0xffff)), d));
                v.w = fmul((float)c.w, fmul(h2f((uint16_t)(sw.y >> 16)), d));
                float *dst = lr < ntok ? P + (size_t)mi * pstride + ((size_t)g * ntok + lr) * 16 + 4 * kg : dmy;
                *(float4 *)dst = v;
            }
        }
    }
}

/* dense product of few tokens: one workgroup per 16-row tile of a segment. */
template <int DT>
__global__ __launch_bounds__(512) void k_gemm_sk(GemmArgs args, int ntok) {
    extern __shared__ float P[];
    int s = 0;
    while (s + 1 < args.nseg && (int)blockIdx.x >= args.seg[s + 1].wg0) s++;
    const GemmSeg &sg = args.seg[s];
    const int rt = (int)blockIdx.x - sg.wg0;
    const int W = blockDim.x >> 6, wave = threadIdx.x >> 6, tid = threadIdx.x;
    int p0, p1;
    wave_pairs(sg.m.nbp >> 1, W, wave, p0, p1);
    /* padding tokens (t >= *live): no columns of their own (their activation loads repeat
     * the last live row's), no folds, no rows written. Bounding the columns only after
     * the loads (every padding row's activations loaded) cost 0.96 us a launch in a loop
     * with short drafts. */
    const int lv = args.live ? *args.live : args.T;
    const int T = lv < args.T ? lv : args.T;
    for (int t0 = args.t0; t0 < T; t0 += ntok) {
        tile_terms<DT, 1>(&sg.m, rt, args.a, t0, T, ntok, [](int t) { return t; }, p0, p1, P, 0);
        __syncthreads();
        const int nc = T - t0 < ntok ? T - t0 : ntok;
        for (int f = tid; f < nc * 16; f += blockDim.x) {
            const int c = f >> 4, row = rt * 16 + (f & 15), t = t0 + c;
            const float acc = fold_terms(P, sg.m.nb, ntok, f);
            if (row < sg.m.rows) {
                float y = canon(acc);
                if (sg.scale_on) y = canon(fmul(sg.scale, y));
                sg.Y[(size_t)t * sg.ldy + row] = y;
            }
        }
        __syncthreads();
    }
}

/* Dense product of more tokens than one tile (a tree's, a prefill chunk's) with each
 * weight byte read once: one workgroup per 16-row tile of a segment, as k_gemm_sk; each
 * wave keeps the weights and scales of its block pairs (at most SK_MAXP) in registers
 * and runs every token tile through them: the MFMAs, the terms into LDS, the next
 * tile's activation loads (in flight during the barrier and the fold), one thread per
 * (row, token) folding the terms in block order. The same terms and fold as k_gemm_sk,
 * so the same bits as every other product kernel. */
template <int DT>
__global__ __launch_bounds__(512) void k_gemm_skm(GemmArgs args, int ntok, int nwg, int nsplit) {
    extern __shared__ float P[];
    /* workgroup b takes row tile b % nwg and token tiles b / nwg, b / nwg + nsplit, ... */
    const int bid = (int)blockIdx.x % nwg, split = (int)blockIdx.x / nwg;
    int s = 0;
    while (s + 1 < args.nseg && bid >= args.seg[s + 1].wg0) s++;
    const GemmSeg &sg = args.seg[s];
    const QMat &m = sg.m;
    const int rt = bid - sg.wg0;
    const int tfirst = args.t0 + split * ntok, tstep = nsplit * ntok;
    const int W = blockDim.x >> 6, wave = threadIdx.x >> 6, tid = threadIdx.x, lr = tid & 15;
    int p0, p1;
    wave_pairs(m.nbp >> 1, W, wave, p0, p1);
    const bool has = p0 < p1;   /* uniform per wave */
    auto arow = [&](int t0) { const int t = t0 + lr; return t < args.T ? t : args.T - 1; };
    SkmRegs<DT, 1> r;
    if (has) {
        skm_load_w<DT, 1>(r, &m, rt, p0, p1);
        if (tfirst < args.T) skm_load_x<DT, 1>(r, args.a, arow(tfirst), p0, p1);
    }
    for (int t0 = tfirst; t0 < args.T; t0 += tstep) {
        if (has) {
            skm_terms<DT, 1>(r, m.nb, ntok, p0, p1, P, 0);
            if (t0 + tstep < args.T) skm_load_x<DT, 1>(r, args.a, arow(t0 + tstep), p0, p1);
        }
        __syncthreads();
        for (int f = tid; f < ntok * 16; f += blockDim.x) {
            const int c = f >> 4, row = rt * 16 + (f & 15), t = t0 + c;
            const float acc = fold_terms(P, m.nb, ntok, f);
            if (t < args.T && row < m.rows) {
                float y = canon(acc);
                if (sg.scale_on) y = canon(fmul(sg.scale, y));
                sg.Y[(size_t)t * sg.ldy + row] = y;
            }
        }
        __syncthreads();
    }
}

/* gate/up with resident weights: a slot's gate and up weights are read once and every
 * token tile of the slot runs through them (as k_gemm_skm); for waves of at most SK_MAXP
 * block pairs and 4 waves a workgroup, held to 256 VGPRs (two waves per SIMD: with
 * 272 the kernel ran one and was slower than reloading the weights per tile) */
template <int DT>
__global__ __launch_bounds__(256, 2) void k_expert_gateup_skm(MoeArgs a, int ntok) {
    extern __shared__ float P[];
    const int ntile = a.F / 16;
    const int u = (int)blockIdx.x / ntile, rt = (int)blockIdx.x % ntile;
    const SlotDesc &sd = a.desc[u];
    const int n = sd.n, p0 = sd.p0;
    if (n == 0) return;
    const ExpertW ew = sd.w;
    if (ew.gate.dtype != DT) return;   /* the launcher runs one instantiation per dtype */
    const QMat ms[2] = {ew.gate, ew.up};
    const int W = blockDim.x >> 6, wave = threadIdx.x >> 6, tid = threadIdx.x, lr = tid & 15;
    int q0, q1;
    wave_pairs(ew.gate.nbp >> 1, W, wave, q0, q1);
    const bool has = q0 < q1;
    const int nb = ew.gate.nb, pstride = nb * ntok * 16;
    const int *ptok = a.pair_tok + p0;
    auto arow = [&](int t0) { const int t = t0 + lr; return ptok[t < n ? t : n - 1]; };
    SkmRegs<DT, 2> r;
    if (has) {
        skm_load_w<DT, 2>(r, ms, rt, q0, q1);
        skm_load_x<DT, 2>(r, a.x, arow(0), q0, q1);
    }
    for (int t0 = 0; t0 < n; t0 += ntok) {
        if (has) {
            skm_terms<DT, 2>(r, nb, ntok, q0, q1, P, pstride);
            if (t0 + ntok < n) skm_load_x<DT, 2>(r, a.x, arow(t0 + ntok), q0, q1);
        }
        __syncthreads();
        for (int f = tid; f < ntok * 16; f += blockDim.x) {
            const int c = f >> 4, row = rt * 16 + (f & 15);
            const float gv = canon(fold_terms(P, nb, ntok, f));
            const float uv = canon(fold_terms(P + pstride, nb, ntok, f));
            if (t0 + c < n) {
                const float sg = fdiv(gv, fadd(1.0f, exp_glibc_f(-gv)));
                a.midf[(size_t)(p0 + t0 + c) * a.F + row] = fmul(sg, uv);
            }
        }
        __syncthreads();
    }
}

/* gate/up of one 16-row F tile of one active expert for its n tokens, then
 * mid = silu(g) * u (NUMERICS §4, quant.c:644-649) as f32 [pair][F]. */
template <int DT>
__global__ __launch_bounds__(512) void k_expert_gateup_sk(MoeArgs a, int ntok) {
    extern __shared__ float P[];
    const int ntile = a.F / 16;
    const int u = (int)blockIdx.x / ntile, rt = (int)blockIdx.x % ntile;
    const SlotDesc &sd = a.desc[u];
    const int n = sd.n, p0 = sd.p0;
    if (n == 0) return;
    const ExpertW ew = sd.w;
    if (ew.gate.dtype != DT) return;   /* the launcher runs one instantiation per dtype */
    const QMat ms[2] = {ew.gate, ew.up};
    const int W = blockDim.x >> 6, wave = threadIdx.x >> 6, tid = threadIdx.x;
    int q0, q1;
    wave_pairs(ew.gate.nbp >> 1, W, wave, q0, q1);
    const int pstride = ew.gate.nb * ntok * 16;
    const int *ptok = a.pair_tok + p0;
    for (int t0 = 0; t0 < n; t0 += ntok) {
        tile_terms<DT, 2>(ms, rt, a.x, t0, n, ntok, [ptok](int t) { return ptok[t]; }, q0, q1, P, pstride);
        __syncthreads();
        for (int f = tid; f < ntok * 16; f += blockDim.x) {
            const int c = f >> 4, row = rt * 16 + (f & 15);
            const float gv = canon(fold_terms(P, ew.gate.nb, ntok, f));
            const float uv = canon(fold_terms(P + pstride, ew.gate.nb, ntok, f));
            if (t0 + c < n) {
                const float sg = fdiv(gv, fadd(1.0f, exp_glibc_f(-gv)));
                a.midf[(size_t)(p0 + t0 + c) * a.F + row] = fmul(sg, uv);
            }
        }
        __syncthreads();
    }
}

/* Persistent gate/up for few tokens (every expert's tokens fit one token tile and a
 * wave's pair range fits SK_MAXP): workgroups loop over the items (active slot, 16-row
 * F tile); as soon as an item's MFMAs have consumed its operand registers, the next
 * item's loads are issued into them, and the barrier, the ordered fold and the SwiGLU
 * epilogue of the current item run while those bytes are in flight. */
template <int DT>
__device__ __forceinline__ void gu_issue(const SlotDesc &sd, int rt, const Act &a, const int *pair_tok, int q0,
                                         int q1, v4i (&rw)[2][SK_MAXP][DT == 4 ? 1 : 2], uint2 (&sc)[2][SK_MAXP][2],
                                         v4i (&xq)[SK_MAXP][2], float (&dx)[SK_MAXP][2], int (&sx)[SK_MAXP][2]) {
    const int lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
    const int n = sd.n;
    const int arow = pair_tok[sd.p0 + (lr < n ? lr : n - 1)];
    const int npair = sd.w.gate.nbp >> 1;
#pragma unroll
    for (int k = 0; k < SK_MAXP; k++) {
        const int gp = q0 + k < q1 ? q0 + k : q1 - 1;
#pragma unroll
        for (int mi = 0; mi < 2; mi++) {
            const QMat &m = mi ? sd.w.up : sd.w.gate;
            if (DT == 4) {
                rw[mi][k][0] = load16(m.w + ((size_t)rt * npair + gp) * 1024 + lane * 16);
            } else {
                const uint8_t *base = m.w + ((size_t)rt * m.nbp + 2 * gp) * 1024 + lane * 16;
                rw[mi][k][0] = load16(base);
                rw[mi][k][DT == 4 ? 0 : 1] = load16(base + 1024);
            }
            const uint16_t *dcol = m.d + rt * 16 + 4 * kg;
            sc[mi][k][0] = *(const uint2 *)(dcol + (size_t)(2 * gp) * m.rows_pad);
            sc[mi][k][1] = *(const uint2 *)(dcol + (size_t)(2 * gp + 1) * m.rows_pad);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const size_t ab = (size_t)arow * a.nbp + 2 * gp + j;
            xq[k][j] = load16((const uint8_t *)(a.q + ab * 64 + kg * 16));
            dx[k][j] = a.d[ab];
            sx[k][j] = DT == 4 ? a.s[ab] : 0;
        }
    }
}

template <int DT>
__device__ __forceinline__ void gu_terms(int nb, int ntok, int q0, int q1, const v4i (&rw)[2][SK_MAXP][DT == 4 ? 1 : 2],
                                         const uint2 (&sc)[2][SK_MAXP][2], const v4i (&xq)[SK_MAXP][2],
                                         const float (&dx)[SK_MAXP][2], const int (&sx)[SK_MAXP][2], float *P,
                                         int pstride) {
    const int lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
    const v4i zero = {0, 0, 0, 0};
    v4i cc[2][SK_MAXP][2];
#pragma unroll
    for (int k = 0; k < SK_MAXP; k++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                v4i wa;
                if (DT == 4) {
                    v4i w0, w1;
                    unpack_q4(rw[mi][k][0], w0, w1);
                    wa = j ? w1 : w0;
                } else {
                    wa = rw[mi][k][DT == 4 ? 0 : j];
                }
                cc[mi][k][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, xq[k][j], zero, 0, 0, 0);
            }
    float *dmy = P + (size_t)2 * nb * ntok * 16 + lane * 4;   /* after both matrices' terms */
#pragma unroll
    for (int k = 0; k < SK_MAXP; k++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int g = 2 * (q0 + k) + j;
            if (q0 + k >= q1 || g >= nb) continue;   /* uniform */
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                v4i c = cc[mi][k][j];
                if (DT == 4) {
                    const int off = 8 * sx[k][j];
                    c.x -= off; c.y -= off; c.z -= off; c.w -= off;
                }
                const uint2 sw = sc[mi][k][j];
                const float d = dx[k][j];
                float4 v;
                v.x = fmul((float)c.x, fmul(h2f((uint16_t)(sw.x & 0xffff)), d));
                v.y = fmul((float)c.y, fmul(h2f((uint16_t)(sw.x >> 16)), d));
                v.z = fmul((float)c.z, fmul(h2f((uint16_t)(sw.y & 0xffff)), d));
                v.w = fmul((float)c.w, fmul(h2f((uint16_t)(sw.y >> 16)), d));
                float *dst = lr < ntok ? P + (size_t)mi * pstride + ((size_t)g * ntok + lr) * 16 + 4 * kg : dmy;
                *(float4 *)dst = v;
            }
        }
    }
}

template <int DT>
__global__ __launch_bounds__(256) void k_expert_gateup_pp(MoeArgs a, int ntok) {
    extern __shared__ float P[];
    const int ntile = a.F / 16;
    const int n_items = *a.n_active * ntile;
    const int W = blockDim.x >> 6, wave = threadIdx.x >> 6, tid = threadIdx.x;
    int item = blockIdx.x;
    if (item >= n_items) return;   /* uniform */
    v4i rw[2][SK_MAXP][DT == 4 ? 1 : 2];
    uint2 sc[2][SK_MAXP][2];
    v4i xq[SK_MAXP][2];
    float dx[SK_MAXP][2];
    int sx[SK_MAXP][2];
    const SlotDesc *sd = &a.desc[item / ntile];
    int q0, q1;
    wave_pairs(sd->w.gate.nbp >> 1, W, wave, q0, q1);
    gu_issue<DT>(*sd, item % ntile, a.x, a.pair_tok, q0, q1, rw, sc, xq, dx, sx);
    while (item < n_items) {
        const int rt = item % ntile, p0 = sd->p0, n = sd->n, nb = sd->w.gate.nb;
        const int pstride = nb * ntok * 16;
        if (sd->w.gate.dtype == DT) gu_terms<DT>(nb, ntok, q0, q1, rw, sc, xq, dx, sx, P, pstride);
        const int next = item + (int)gridDim.x;
        const SlotDesc *nsd = &a.desc[(next < n_items ? next : item) / ntile];
        if (next < n_items) gu_issue<DT>(*nsd, next % ntile, a.x, a.pair_tok, q0, q1, rw, sc, xq, dx, sx);
        __syncthreads();
        if (sd->w.gate.dtype == DT) {
            for (int f = tid; f < ntok * 16; f += blockDim.x) {
                const int c = f >> 4, row = rt * 16 + (f & 15);
                const float gv = canon(fold_terms(P, nb, ntok, f));
                const float uv = canon(fold_terms(P + pstride, nb, ntok, f));
                if (c < n) {
                    const float sg = fdiv(gv, fadd(1.0f, exp_glibc_f(-gv)));
                    a.midf[(size_t)(p0 + c) * a.F + row] = fmul(sg, uv);
                }
            }
        }
        __syncthreads();
        item = next;
        sd = nsd;
    }
}

/* Expert products for experts of at most 16 tokens, K split over S waves per row tile:
 * gate and up with the SwiGLU epilogue (MODE TK_GATEUP), or the down projection of
 * quantized rows (TK_DOWN: the SwiGLU rows, MLA's W_UV).
 *
 * Workgroup = (token group g, active slot, rpw row tiles of 16 rows); S waves per row
 * tile. Wave (row tile r, part p) streams block pairs [p TK_NP, (p + 1) TK_NP) of the
 * tile's matrices into registers, every load issued at once. The slot's activation
 * blocks are staged once per workgroup in LDS by LDS-direct loads, [block][token][64 B]
 * (the Act block of each token, k-group kg at 16 kg).
 *
 * Tokens go in groups of four: for group g the B operand of column c is read from token
 * 4 g + c % 4, so the MFMA result holds each (row, token) pair four times and lane
 * (kg = l / 16, lr = l % 16) keeps register lr / 4: row 4 kg + lr / 4, token
 * 4 g + lr % 4 -- one useful term per lane, matrix and block, where the 16 token
 * columns of the plain layout would leave most lanes working on padding.
 *
 * Sums: part 0 folds its blocks from 0.0; part p > 0 keeps its terms in registers,
 * takes the running sums of part p - 1 through LDS after barrier p and adds its terms
 * in block order, so each sum is the sequential fold acc = acc + isum (dw dx) over
 * blocks 0 .. nb-1. The last part writes the result. */
template <int DT>
struct TkCfg {
    static constexpr int NP = DT == 4 ? 8 : 4;   /* block pairs per wave (registers) */
    static constexpr int NV = DT == 4 ? 1 : 2;   /* 16-byte loads per pair, matrix and lane */
};

/* register q of c */
__device__ __forceinline__ int pick4(const v4i &c, int q) {
    const int lo = (q & 1) ? c.y : c.x, hi = (q & 1) ? c.w : c.z;
    return (q & 2) ? hi : lo;
}

/* tile sets per XCD chunk: a workgroup of fewer than 64 rows shares the 128-byte scale
 * lines with its neighbours, so TK_CHUNK_ROWS rows stay on one XCD; from 64 rows on the
 * workgroups go round the XCDs one by one */
__host__ __device__ inline int tk_chunk(int rpw) {
    return 16 * rpw >= 64 ? 1 : TK_CHUNK_ROWS / (16 * rpw);
}

/* LDS bytes of one workgroup (qf: plus the SwiGLU rows [4 tokens][16 rpw] it quantizes) */
__host__ __device__ inline size_t tk_lds_bytes(int nbp, int nm, int np, int rpw, int S, bool qf = false) {
    const int nbp4 = (nbp + 3) & ~3;
    return (size_t)nbp * 1024 + (size_t)nbp4 * 128 + (size_t)rpw * S * nm * 2 * np * 32 + (size_t)rpw * nm * 64 * 4 +
           (qf ? (size_t)4 * 16 * rpw * 4 : 0);
}

/* TK_GATEUP_Q: gate/up whose workgroups cover whole 64-row blocks of the SwiGLU rows
 * (4 or 8 row tiles) and quantize them (NUMERICS §2) in the epilogue */
enum { TK_GATEUP = 0, TK_DOWN = 1, TK_GATEUP_Q = 2 };

/* s_waitcnt vmcnt(n) for an n known once loops are unrolled (0 <= n <= 31) */
__device__ __forceinline__ void wait_vmcnt_le(int n) {
    switch (n) {
#define HX_W(k) case k: HX_WAIT_VMCNT(k); break;
    HX_W(0) HX_W(1) HX_W(2) HX_W(3) HX_W(4) HX_W(5) HX_W(6) HX_W(7) HX_W(8) HX_W(9) HX_W(10) HX_W(11)
    HX_W(12) HX_W(13) HX_W(14) HX_W(15) HX_W(16) HX_W(17) HX_W(18) HX_W(19) HX_W(20) HX_W(21) HX_W(22)
    HX_W(23) HX_W(24) HX_W(25) HX_W(26) HX_W(27) HX_W(28) HX_W(29) HX_W(30) HX_W(31)
#undef HX_W
    default: HX_WAIT_VMCNT(0);
    }
}

template <int DT, int MODE>
__global__ __launch_bounds__(512) void k_expert_tk(MoeArgs a, int rpw, int S, int gmax, int n_slots) {
    constexpr bool DOWN = MODE == TK_DOWN, QF = MODE == TK_GATEUP_Q;
    extern __shared__ __attribute__((aligned(16))) uint8_t tk_lds[];
    /* the exp table of the SwiGLU epilogue, one entry per lane, loaded with the weights */
    const unsigned long long ev = DOWN ? 0ull : exp_table_lane();
    constexpr int NP = TkCfg<DT>::NP, NV = TkCfg<DT>::NV, NBK = 2 * NP, NM = DOWN ? 1 : 2;
    const int rows_out = DOWN ? a.D : a.F;
    const int ntile = (rows_out + 15) / 16, tpw = (ntile + rpw - 1) / rpw;
    /* workgroup i runs on XCD i % 8. Chunks of TK_CHUNK_ROWS rows of one slot are dealt
     * to the XCDs in turn and a chunk's workgroups follow each other on its XCD, so the
     * row tiles that share 128-byte lines of the scale rows meet in one L2 while every
     * XCD gets the same share of the bytes */
    const int ch = tk_chunk(rpw);   /* tile sets per chunk */
    const int cps = (tpw + ch - 1) / ch, per_chunk = ch * gmax;
    const int xcd = (int)blockIdx.x & 7, k = (int)blockIdx.x >> 3;
    const int c = xcd + 8 * (k / per_chunk), within = k % per_chunk;
    const int u = c / cps, tile = (c % cps) * ch + within / gmax, g = within % gmax;
    if (u >= n_slots || tile >= tpw) return;   /* uniform */
    int n, p0;
    QMat mat[NM];
    if (DOWN && a.head_slots) {
        n = a.T;
        p0 = u * a.T;
        mat[0] = a.table[u].down;
    } else {
        if (u >= *a.n_active) return;   /* uniform */
        const SlotDesc &sd = a.desc[u];
        n = sd.n;
        p0 = sd.p0;
        if (DOWN) {
            mat[0] = sd.w.down;
        } else {
            mat[0] = sd.w.gate;
            mat[NM - 1] = sd.w.up;
        }
    }
    if (mat[0].dtype != DT || 4 * g >= n) return;   /* uniform */
    const Act &x = DOWN ? a.mid : a.x;
    const int W = rpw * S;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int rtl = wave / S, part = wave % S;
    const int lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
    const int rt0 = tile * rpw + rtl;
    const bool live = rt0 < ntile;   /* uniform per wave */
    const int rt = live ? rt0 : ntile - 1;   /* a dead wave loads a live tile and discards it */
    const int nb = mat[0].nb, nbp = mat[0].nbp, npair = nbp >> 1, nbp4 = (nbp + 3) & ~3;
    const int g0 = part * NP, kb0 = 2 * g0;   /* first pair / block of this part */
    uint8_t *xs = tk_lds;                                   /* [nbp][16 tokens][64 B] */
    float *dxs = (float *)(xs + (size_t)nbp * 1024);        /* [nbp4][16 tokens] */
    int *sxs = (int *)(dxs + nbp4 * 16);                    /* [nbp4][16 tokens] */
    uint8_t *scl = (uint8_t *)(sxs + nbp4 * 16) + wave * NM * NBK * 32;   /* [NM][NBK][16 halves] */
    float *const relay0 = (float *)((uint8_t *)(sxs + nbp4 * 16) + W * NM * NBK * 32);   /* [rpw][NM][64] */
    float *relay = relay0 + rtl * NM * 64;
    /* issue order: the token rows, the weights (straight-line loads), then the
     * LDS-direct loads that need the token rows. The q loads cover token lane / 4,
     * k-group lane % 4 of a block; the d and s loads token lane % 16 of four blocks. */
    const int tq = (lane >> 2) < n ? (lane >> 2) : n - 1, tds = lr < n ? lr : n - 1;
    const int arow_q = !DOWN ? a.pair_tok[p0 + tq] : p0 + tq;
    const int arow_d = !DOWN ? a.pair_tok[p0 + tds] : p0 + tds;
    v4i w[NM][NP][NV];
    /* pairs [0, NA) go before the token rows, pairs [NA, NP) after them: the wait for the
     * token rows then leaves the later weights in flight, and each pair's MFMAs start as
     * soon as its own bytes are in (the compiler waits for each register as it is used) */
    constexpr int NA = NP / 4 > 0 ? NP / 4 : 1;
    auto load_pair = [&](int k, int dep) {
        const int gp = g0 + k < npair ? g0 + k : npair - 1;
#pragma unroll
        for (int mi = 0; mi < NM; mi++) {
            const QMat &m = mat[mi];
            if (DT == 4) {
                w[mi][k][0] = gload<v4i>(m.w + ((size_t)rt * npair + gp) * 1024 + lane * 16 + dep);
            } else {
                const uint8_t *base = m.w + ((size_t)rt * nbp + 2 * gp) * 1024 + lane * 16 + dep;
                w[mi][k][0] = gload<v4i>(base);
                w[mi][k][NV - 1] = gload<v4i>(base + 1024);
            }
        }
    };
#pragma unroll
    for (int k = 0; k < NA; k++) load_pair(k, 0);
    /* one loop for every LDS-direct load */
    {
        const int nxq = (nbp - wave + W - 1) / W, nit = nxq > NBK / 8 ? nxq : NBK / 8;
        int it = 0;
        do {   /* nit >= 1 */
            const int b = wave + it * W;
            if (b < nbp) lds_direct<16>(x.q + ((size_t)arow_q * x.nbp + b) * 64 + (lane & 3) * 16, xs + (size_t)b * 1024);
            if (4 * b < nbp4) {
                const int bb = 4 * b + kg < nbp ? 4 * b + kg : nbp - 1;
                lds_direct<4>(x.d + (size_t)arow_d * x.nbp + bb, dxs + 4 * b * 16);
                if (DT == 4) lds_direct<4>(x.s + (size_t)arow_d * x.nbp + bb, sxs + 4 * b * 16);
            }
            const int b0 = it * 8;
            if (b0 < NBK) {
                const int bg = kb0 + b0 + (lane >> 3), bs = bg < nbp ? bg : nbp - 1, h2 = (lane & 7) * 2;
#pragma unroll
                for (int mi = 0; mi < NM; mi++)
                    lds_direct<4>(mat[mi].d + (size_t)bs * mat[mi].rows_pad + rt * 16 + h2, scl + (mi * NBK + b0) * 32);
            }
        } while (++it < nit);
    }
    /* the later weights: their addresses depend on an empty volatile asm after the
     * LDS-direct loads, so no load of them can be issued before those */
    int dep = 0;
    asm volatile("" : "+v"(dep));
#pragma unroll
    for (int k = NA; k < NP; k++) load_pair(k, dep);
    HX_WAIT_VMCNT(NM * (NP - NA) * NV);   /* the token rows, scales and pairs [0, NA) */
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);    /* no weight use moves above the barrier */
    const int q = lr >> 2;                /* register of this lane's pair: row 4 kg + q */
    /* one group of 4 tokens: the MFMAs, the fold over the parts and the epilogue */
    auto group = [&](int g) {
        const int col = 4 * g + (lr & 3);     /* token of this lane's pair */
        const int colc = col < n ? col : n - 1;   /* its staged row (columns past n are discarded) */
        const v4i zero = {0, 0, 0, 0};
        const bool full = kb0 + NBK <= nb;    /* uniform */
        /* terms of local block kb (global kb0 + kb); the MFMA gives sum q x with q the
         * stored nibble (Q4), so isum = sum q x - 8 sx */
        auto terms = [&](const v4i (&wa)[NM], int kb, float (&t)[NM]) {
            const int blk = kb0 + kb;
            const v4i xq = *(const v4i *)(xs + ((size_t)blk * 16 + colc) * 64 + kg * 16);
            const float d = dxs[blk * 16 + colc];
            const int off = DT == 4 ? 8 * sxs[blk * 16 + colc] : 0;
#pragma unroll
            for (int mi = 0; mi < NM; mi++) {
                const v4i cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[mi], xq, zero, 0, 0, 0);
                const float dw = h2f(*((const uint16_t *)(scl + (size_t)(mi * NBK + kb) * 32) + 4 * kg + q));
                t[mi] = fmul((float)(pick4(cc, q) - off), fmul(dw, d));
            }
        };
        float acc[NM];
        float tm[NBK][NM];
        auto run_part = [&](bool fold) {
#pragma unroll
            for (int k = 0; k < NP; k++) {
                /* pair k's loads are in when at most the later pairs' are outstanding */
                if (k >= NA) wait_vmcnt_le(NM * NV * (NP - 1 - k));
                v4i wv[2][NM];
#pragma unroll
                for (int mi = 0; mi < NM; mi++) {
                    if (DT == 4) {
                        unpack_q4(w[mi][k][0], wv[0][mi], wv[1][mi]);
                    } else {
                        wv[0][mi] = w[mi][k][0];
                        wv[1][mi] = w[mi][k][NV - 1];
                    }
                }
#pragma unroll
                for (int j2 = 0; j2 < 2; j2++) {
                    const int kb = 2 * k + j2;
                    if (!full && kb0 + kb >= nb) break;   /* uniform */
                    float t[NM];
                    terms(wv[j2], kb, t);
#pragma unroll
                    for (int mi = 0; mi < NM; mi++) {
                        if (fold) acc[mi] = fadd(acc[mi], t[mi]);
                        else tm[kb][mi] = t[mi];
                    }
                }
            }
        };
        if (part == 0) {
#pragma unroll
            for (int mi = 0; mi < NM; mi++) acc[mi] = 0.0f;
            run_part(true);
        } else {
            run_part(false);
        }
        for (int stage = 1; stage < S; stage++) {
            if (part == stage - 1) {
#pragma unroll
                for (int mi = 0; mi < NM; mi++) relay[mi * 64 + lane] = acc[mi];
            }
            __syncthreads();
            if (part == stage) {
#pragma unroll
                for (int mi = 0; mi < NM; mi++) acc[mi] = relay[mi * 64 + lane];
#pragma unroll
                for (int kb = 0; kb < NBK; kb++) {
                    if (!full && kb0 + kb >= nb) break;   /* uniform */
#pragma unroll
                    for (int mi = 0; mi < NM; mi++) acc[mi] = fadd(acc[mi], tm[kb][mi]);
                }
            }
            __syncthreads();   /* the relay slot is read before the next stage writes it */
        }
        const int row = rt * 16 + 4 * kg + q;
        const bool out = part == S - 1 && live && col < n;
        if (DOWN) {
            if (out && row < mat[0].rows) a.Y[(size_t)(p0 + col) * a.D + row] = canon(acc[0]);
            return;
        }
        float mv = 0.0f;
        {
            /* every lane takes the exp (the table is read across the wave); the outputs keep it */
            const float gv = canon(acc[0]), uv = canon(acc[NM - 1]);
            const float sg = fdiv(gv, fadd(1.0f, exp_glibc_f_wave(-gv, ev)));
            if (out) {
                mv = fmul(sg, uv);
                if (!QF) a.midf[(size_t)(p0 + col) * a.F + row] = mv;
            }
        }
        if constexpr (QF) {
            /* the workgroup's rows [16 rpw tile, +16 rpw) are whole blocks of F: the last
             * parts put them in LDS by (token, row), then wave j quantizes block j / 4 of
             * token 4 g + j % 4 -- the values k_quant_rows would read from midf */
            const int nr = 16 * rpw;
            float *qb = relay0 + rpw * NM * 64;   /* [4 tokens][16 rpw], after the relay slots */
            if (part == S - 1) qb[(lr & 3) * nr + rtl * 16 + 4 * kg + q] = mv;
            __syncthreads();
            if (wave < rpw) {
                const int tt = wave & 3, bb = wave >> 2, tcol = 4 * g + tt;
                if (tcol < n) quant_block_wave(qb[tt * nr + bb * 64 + lane], a.mid, p0 + tcol, (tile * nr) / 64 + bb);
            }
        }
    };
    if (DOWN) {
        /* down runs every group of the slot from the same weight registers (the
         * stage loop's last barrier orders the relay slots between groups) */
        const int ng = (n + 3) >> 2;
        for (int gi = 0; gi < ng; gi++) group(gi);
    } else {
        group(g);
    }
}

/* launches k_expert_tk for experts of at most 16 tokens and one dtype; false when the
 * shape does not fit (the caller uses the general kernels) */
int launch_tk(const MoeArgs &a, int mode, int n_slots, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    const bool down = mode == TK_DOWN;
    const bool q4 = a.dtype_mask & (1 << 4), q8 = a.dtype_mask & (1 << 3);
    if (a.T > 16 || q4 == q8) return 0;
    const int K = down ? a.F : a.D, rows = down ? a.D : a.F;
    const int nb = (K + 63) / 64, nbp = (nb + 1) & ~1, npair = nbp / 2;
    const int NP = q4 ? TkCfg<4>::NP : TkCfg<3>::NP, NM = down ? 1 : 2;
    const int S = (npair + NP - 1) / NP;
    const int waves = down ? TK_WAVES_DOWN : TK_WAVES_GATEUP;
    const int rpw = S < waves ? waves / S : 1, W = rpw * S;
    /* gate/up workgroups of 4 or 8 row tiles cover whole blocks of the SwiGLU rows: they
     * quantize them too (F a multiple of 128, so the blocks need no padding block) */
    const bool qf = mode == TK_GATEUP && a.mid.q && a.F % 128 == 0 && (rpw == 4 || rpw == 8) && a.mid.nbp == a.F / 64;
    const size_t lds = tk_lds_bytes(nbp, NM, NP, rpw, S, qf);
    if (W > 8 || lds > TK_LDS_MAX) return 0;
    const int tpw = ((rows + 15) / 16 + rpw - 1) / rpw;
    /* gate/up: a workgroup per group of 4 tokens; down: one runs all of its slot's groups */
    const int gmax = down ? 1 : (a.T + 3) / 4;   /* tokens per slot <= T */
    const int ch = tk_chunk(rpw);
    const int chunks = n_slots * ((tpw + ch - 1) / ch);
    const dim3 grid(8 * ((chunks + 7) / 8) * ch * gmax), block(64 * W);
#define TK_LAUNCH(DT_, MODE_) \
    hipExtLaunchKernelGGL(k_expert_tk<DT_, MODE_>, grid, block, (uint32_t)lds, st, ev0, ev1, 0u, a, rpw, S, gmax, n_slots)
    if (mode == TK_GATEUP) {
        if (qf) { if (q4) TK_LAUNCH(4, TK_GATEUP_Q); else TK_LAUNCH(3, TK_GATEUP_Q); }
        else { if (q4) TK_LAUNCH(4, TK_GATEUP); else TK_LAUNCH(3, TK_GATEUP); }
    }
    if (mode == TK_DOWN) { if (q4) TK_LAUNCH(4, TK_DOWN); else TK_LAUNCH(3, TK_DOWN); }
#undef TK_LAUNCH
    return qf ? 2 : 1;
}

/* down projection of one 16-row D tile of one active expert for its n tokens. */
template <int DT>
__global__ __launch_bounds__(512) void k_expert_down_sk(MoeArgs a, int ntok) {
    extern __shared__ float P[];
    const int ntile = (a.D + 15) / 16;
    const int u = (int)blockIdx.x / ntile, rt = (int)blockIdx.x % ntile;
    int n, p0;
    QMat m;
    if (a.head_slots) {
        n = a.T;
        p0 = u * a.T;
        m = a.table[u].down;
    } else {
        const SlotDesc &sd = a.desc[u];
        n = sd.n;
        p0 = sd.p0;
        m = sd.w.down;
    }
    if (n == 0) return;
    if (m.dtype != DT) return;
    const int W = blockDim.x >> 6, wave = threadIdx.x >> 6, tid = threadIdx.x;
    int q0, q1;
    wave_pairs(m.nbp >> 1, W, wave, q0, q1);
    for (int t0 = 0; t0 < n; t0 += ntok) {
        tile_terms<DT, 1>(&m, rt, a.mid, t0, n, ntok, [p0](int t) { return p0 + t; }, q0, q1, P, 0);
        __syncthreads();
        for (int f = tid; f < ntok * 16; f += blockDim.x) {
            const int c = f >> 4, row = rt * 16 + (f & 15);
            const float acc = fold_terms(P, m.nb, ntok, f);
            if (t0 + c < n && row < m.rows) a.Y[(size_t)(p0 + t0 + c) * a.D + row] = canon(acc);
        }
        __syncthreads();
    }
}

/* ------------------------------------------------------------ grouped expert GEMMs */

/* ------------------------------------------------------------ float matrices (dot16) */

/* y = dot16(w_r, x_t) (NUMERICS §1/§3; quant.c:352-376): 16 lanes per (row, token),
 * lane j sums elements j, j+16, ... in order, then the 8/4/2/1 tree. Any shape. */
template <int WDT>
__global__ __launch_bounds__(256) void k_fgemv_any(const void *__restrict__ W, int rows, int cols,
                                                  const float *__restrict__ X, int ldx, int T, float *__restrict__ Y,
                                                  int ldy) {
    const int64_t pair = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4;
    const int j = threadIdx.x & 15;
    const bool live = pair < (int64_t)rows * T;
    const int r = live ? (int)(pair % rows) : 0, t = live ? (int)(pair / rows) : 0;
    float L = 0.0f;
    if (live) {
        const float *x = X + (size_t)t * ldx;
        for (int i = j; i < cols; i += 16) {
            float w;
            if (WDT == 0) w = ((const float *)W)[(size_t)r * cols + i];
            else if (WDT == 1) w = h2f(((const uint16_t *)W)[(size_t)r * cols + i]);
            else w = __uint_as_float((uint32_t)((const uint16_t *)W)[(size_t)r * cols + i] << 16);
            L = fadd(L, fmul(w, x[i]));
        }
    }
#pragma unroll
    for (int s = 8; s >= 1; s >>= 1) L = fadd(L, __shfl_down(L, s, 16));
    if (live && j == 0) Y[(size_t)t * ldy + r] = canon(L);
}

/* The same products for cols % 4 == 0 and ldx % 4 == 0: a workgroup computes 4 rows x 4
 * tokens; the rows of W and X go to LDS in chunks of 2048 columns, each thread issuing
 * all its loads of a chunk at once, and the 16 lanes of each (row, token) then run their
 * sums from LDS (chunk boundaries are multiples of 16, so lane j keeps its elements). */
constexpr int FG_R = 4, FG_T = 4, FG_CH = 2048;
constexpr int FG_PER = (FG_R + FG_T) * FG_CH / 4 / 256;   /* float4 loads per thread per chunk */

template <int WDT>
__device__ __forceinline__ float4 fg_w4(const void *W, size_t idx) {
    if (WDT == 0) return *(const float4 *)((const float *)W + idx);
    const uint2 u = *(const uint2 *)((const uint16_t *)W + idx);
    float4 v;
    if (WDT == 1) {
        v.x = h2f((uint16_t)(u.x & 0xffff)); v.y = h2f((uint16_t)(u.x >> 16));
        v.z = h2f((uint16_t)(u.y & 0xffff)); v.w = h2f((uint16_t)(u.y >> 16));
    } else {
        v.x = __uint_as_float(u.x << 16); v.y = __uint_as_float(u.x & 0xffff0000u);
        v.z = __uint_as_float(u.y << 16); v.w = __uint_as_float(u.y & 0xffff0000u);
    }
    return v;
}

template <int WDT>
__global__ __launch_bounds__(256) void k_fgemv(const void *__restrict__ W, int rows, int cols,
                                              const float *__restrict__ X, int ldx, int T, float *__restrict__ Y,
                                              int ldy) {
    __shared__ float buf[FG_R + FG_T][FG_CH];
    const int nrb = (rows + FG_R - 1) / FG_R;
    const int rb = (int)blockIdx.x % nrb, tb = (int)blockIdx.x / nrb;
    const int tid = threadIdx.x, pr = tid >> 4, j = tid & 15;
    const int rr = pr % FG_R, tt = pr / FG_R;
    const int r = rb * FG_R + rr, t = tb * FG_T + tt;
    float L = 0.0f;
    for (int c0 = 0; c0 < cols; c0 += FG_CH) {
        const int n = cols - c0 < FG_CH ? cols - c0 : FG_CH;
        if (c0) __syncthreads();
        float4 v[FG_PER];
        /* load u: row q = u / 2 of the stage (rows of W first, then rows of X), float4
         * column tid + 256 (u % 2); columns past the chunk read column 0 and are unused */
#pragma unroll
        for (int u = 0; u < FG_PER; u++) {
            const int q = u >> 1;
            int c4 = (tid + 256 * (u & 1)) * 4;
            c4 = c4 < n ? c4 : 0;
            if (q < FG_R) {
                const int rq = rb * FG_R + q < rows ? rb * FG_R + q : rows - 1;
                v[u] = fg_w4<WDT>(W, (size_t)rq * cols + c0 + c4);
            } else {
                const int tq = tb * FG_T + (q - FG_R) < T ? tb * FG_T + (q - FG_R) : T - 1;
                v[u] = *(const float4 *)(X + (size_t)tq * ldx + c0 + c4);
            }
        }
#pragma unroll
        for (int u = 0; u < FG_PER; u++)
            *(float4 *)&buf[u >> 1][(tid + 256 * (u & 1)) * 4] = v[u];
        __syncthreads();
        const float *wr = buf[rr], *xr = buf[FG_R + tt];
        int i = j;
        for (; i + 112 < n; i += 128) {
            float a[8], b[8];
#pragma unroll
            for (int u = 0; u < 8; u++) { a[u] = wr[i + 16 * u]; b[u] = xr[i + 16 * u]; }
#pragma unroll
            for (int u = 0; u < 8; u++) L = fadd(L, fmul(a[u], b[u]));
        }
        for (; i < n; i += 16) L = fadd(L, fmul(wr[i], xr[i]));
    }
#pragma unroll
    for (int s = 8; s >= 1; s >>= 1) L = fadd(L, __shfl_down(L, s, 16));
    if (r < rows && t < T && j == 0) Y[(size_t)t * ldy + r] = canon(L);
}

} // namespace

/* ------------------------------------------------------------ launchers */

namespace hxl {

void repack(const uint8_t *src_dev, int r0, int count, const QMat &m, hipStream_t st) {
    const int64_t n = (int64_t)count * m.nbp;
    if (!n) return;
    const int blocks = (int)((n + 255) / 256);
    if (m.dtype == 3) k_repack_q8<<<blocks, 256, 0, st>>>(src_dev, r0, count, m.rows, m.nb, m, (uint8_t *)m.w, (uint16_t *)m.d);
    else k_repack_q4<<<blocks, 256, 0, st>>>(src_dev, r0, count, m.rows, m.nb, m, (uint8_t *)m.w, (uint16_t *)m.d);
}

void quant_rows(const float *x, int64_t ldx, int T, int nb, const Act &a, hipStream_t st) {
    const int64_t waves = (int64_t)T * a.nbp;
    if (!waves) return;
    k_quant_rows<<<(int)((waves + 3) / 4), 256, 0, st>>>(x, ldx, T, nb, a);
}

/* compute units of the current device (cached per device) */
static int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    return cached[dev];
}

/* waves per split-K workgroup for npair block pairs */
static int sk_waves(int npair) {
    const int w = (npair + SK_MAXP - 1) / SK_MAXP;
    return w < 1 ? 1 : (w > 8 ? 8 : w);
}

/* tokens per split-K token tile: the terms of NM matrices of nb blocks fit SK_LDS */
static int sk_ntok(int T, int NM, int nb) {
    int n = T < 16 ? T : 16;
    const int fit = (SK_LDS - SK_DUMMY) / (NM * nb * 64);
    n = n < fit ? n : fit;
    return n < 1 ? 1 : n;
}

/* k_gemm_skm applies: every segment's block pairs fit its waves' registers (at most 8
 * waves of SK_MAXP pairs) and its terms the LDS */
static bool skm_ok(const GemmArgs &in) {
    for (int s = 0; s < in.nseg; s++) {
        const QMat &m = in.seg[s].m;
        if ((m.nbp >> 1) > 8 * SK_MAXP || (size_t)m.nb * 64 > (size_t)SK_LDS) return false;
    }
    return true;
}

/* dense product through the split-K kernels (k_gemm_sk, or k_gemm_skm when resident):
 * one launch per run of consecutive segments of one dtype */
static void gemm_sk(const GemmArgs &in, hipStream_t st, bool resident = false) {
    for (int s0 = 0; s0 < in.nseg;) {
        int s1 = s0 + 1;
        while (s1 < in.nseg && in.seg[s1].m.dtype == in.seg[s0].m.dtype && in.seg[s1].m.nb == in.seg[s0].m.nb) s1++;
        GemmArgs g = in;
        g.nseg = s1 - s0;
        int wg = 0;
        for (int s = 0; s < g.nseg; s++) {
            g.seg[s] = in.seg[s0 + s];
            g.seg[s].wg0 = wg;
            wg += g.seg[s].m.rows_pad / 16;
        }
        const QMat &m = g.seg[0].m;
        const int ntok = sk_ntok(in.T, 1, m.nb);
        const int threads = 64 * sk_waves(m.nbp / 2);
        const size_t lds = (size_t)m.nb * ntok * 64 + SK_DUMMY;
        if (wg && resident) {
            /* token tiles split over workgroups until the row tiles fill the CUs */
            const int ntile = (in.T + ntok - 1) / ntok;
            int nsplit = 1;
            while (nsplit < ntile && wg * (nsplit + 1) <= cu_count()) nsplit++;
            if (m.dtype == 4) k_gemm_skm<4><<<wg * nsplit, threads, lds, st>>>(g, ntok, wg, nsplit);
            else k_gemm_skm<3><<<wg * nsplit, threads, lds, st>>>(g, ntok, wg, nsplit);
        } else if (wg) {
            if (m.dtype == 4) k_gemm_sk<4><<<wg, threads, lds, st>>>(g, ntok);
            else k_gemm_sk<3><<<wg, threads, lds, st>>>(g, ntok);
        }
        s0 = s1;
    }
}

void gemm(const GemmArgs &in, hipStream_t st) {
    if (in.T <= 16 && in.t0 == 0) {
        bool ok = true;
        for (int s = 0; s < in.nseg; s++) ok = ok && (size_t)in.seg[s].m.nb * 64 <= (size_t)SK_LDS;
        if (ok) { gemm_sk(in, st); return; }
    }
    if (in.t0 == 0 && skm_ok(in)) { gemm_sk(in, st, true); return; }
    GemmArgs g = in;
    int wg = 0, tiles = 0;
    for (int s = 0; s < g.nseg; s++) {
        g.seg[s].wg0 = wg;
        wg += (g.seg[s].m.rows_pad / 16 + 3) / 4;
        tiles += g.seg[s].m.rows_pad / 16;
    }
    if (!wg || in.T <= 0) return;
    const int wgr = (wg + 7) & ~7;
    /* tokens tiles per wave: as many as keep about 8 waves per CU busy (each wave walks
     * all of K for its tiles, so more tiles per wave means fewer, longer waves) */
    const int ntile = (in.T + 15) / 16, want = 8 * cu_count();
    int nt = 8;
    while (nt > 1 && (long long)tiles * ((ntile + nt - 1) / nt) < want) nt >>= 1;
    if (nt > ntile) nt = ntile <= 1 ? 1 : ntile <= 2 ? 2 : ntile <= 4 ? 4 : 8;
    g.t0 = 0;
    const int grid = wgr * ((ntile + nt - 1) / nt);
    if (nt == 1) k_gemm<1><<<grid, 256, 0, st>>>(g, wgr);
    else if (nt == 2) k_gemm<2><<<grid, 256, 0, st>>>(g, wgr);
    else if (nt == 4) k_gemm<4><<<grid, 256, 0, st>>>(g, wgr);
    else k_gemm<8><<<grid, 256, 0, st>>>(g, wgr);
}

/* gate/up (split-K, one launch per expert dtype present); true when the launch also
 * quantized the SwiGLU rows into a.mid */
bool expert_gateup(const MoeArgs &a, int n_slots, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    if (n_slots <= 0) return false;
    const int nb = (a.D + 63) / 64, nbp = (nb + 1) & ~1;
    const int ntok = sk_ntok(a.T, 2, nb);
    const int threads = 64 * sk_waves(nbp / 2);
    const size_t lds = (size_t)2 * nb * ntok * 64 + SK_DUMMY;
    const int grid = n_slots * (a.F / 16);
    /* ev0/ev1 (optional) are recorded by the dispatch itself: ev0 at the start of the
     * first launch, ev1 at the end of the last */
    const bool q4 = a.dtype_mask & (1 << 4), q8 = a.dtype_mask & (1 << 3);
    /* at most 16 tokens per expert, one dtype: the split-K kernel (one term per lane) */
    if (const int r = launch_tk(a, TK_GATEUP, n_slots, st, ev0, ev1)) return r == 2;
    /* few tokens, one dtype, one pair chunk per wave: the persistent kernel (two
     * workgroups per CU on every CU) */
    const int npair = nbp / 2, W = threads / 64;
    if (a.T <= ntok && (q4 != q8) && (npair + W - 1) / W <= SK_MAXP && threads <= 256) {
        const int ncu = cu_count();
        const int pgrid = grid < 2 * ncu ? grid : 2 * ncu;
        if (q4) hipExtLaunchKernelGGL(k_expert_gateup_pp<4>, dim3(pgrid), dim3(threads), (uint32_t)lds, st, ev0, ev1, 0u, a, ntok);
        else hipExtLaunchKernelGGL(k_expert_gateup_pp<3>, dim3(pgrid), dim3(threads), (uint32_t)lds, st, ev0, ev1, 0u, a, ntok);
        return false;
    }
    if ((npair + W - 1) / W <= SK_MAXP && threads <= 256) {   /* the wave's pairs fit its registers */
        if (q4) hipExtLaunchKernelGGL(k_expert_gateup_skm<4>, dim3(grid), dim3(threads), (uint32_t)lds, st, ev0,
                                      q8 ? nullptr : ev1, 0u, a, ntok);
        if (q8) hipExtLaunchKernelGGL(k_expert_gateup_skm<3>, dim3(grid), dim3(threads), (uint32_t)lds, st,
                                      q4 ? nullptr : ev0, ev1, 0u, a, ntok);
        return false;
    }
    if (q4) hipExtLaunchKernelGGL(k_expert_gateup_sk<4>, dim3(grid), dim3(threads), (uint32_t)lds, st, ev0,
                                  q8 ? nullptr : ev1, 0u, a, ntok);
    if (q8) hipExtLaunchKernelGGL(k_expert_gateup_sk<3>, dim3(grid), dim3(threads), (uint32_t)lds, st,
                                  q4 ? nullptr : ev0, ev1, 0u, a, ntok);
    return false;
}

/* NUMERICS §2 of the SwiGLU rows of all T * top_k pairs (unless the gate/up launch did
 * it: mid_done), then the down projections */
void expert_down(const MoeArgs &a, int n_slots, hipStream_t st, bool mid_done) {
    if (n_slots <= 0) return;
    if (!mid_done) quant_rows(a.midf, a.F, a.P, a.F / 64, a.mid, st);
    expert_down_q(a, n_slots, st);
}

void expert_down_q(const MoeArgs &a, int n_slots, hipStream_t st) {
    if (n_slots <= 0) return;
    if (launch_tk(a, TK_DOWN, n_slots, st, nullptr, nullptr)) return;
    const int nb = (a.F + 63) / 64, nbp = (nb + 1) & ~1;
    const int ntok = sk_ntok(a.T, 1, nb);
    const int threads = 64 * sk_waves(nbp / 2);
    const size_t lds = (size_t)nb * ntok * 64 + SK_DUMMY;
    const int grid = n_slots * ((a.D + 15) / 16);
    if (a.dtype_mask & (1 << 4)) k_expert_down_sk<4><<<grid, threads, lds, st>>>(a, ntok);
    if (a.dtype_mask & (1 << 3)) k_expert_down_sk<3><<<grid, threads, lds, st>>>(a, ntok);
}

void fgemv(int dtype, const void *W, int rows, int cols, const float *X, int ldx, int T, float *Y, int ldy, hipStream_t st) {
    if (rows <= 0 || T <= 0) return;
    if (cols % 4 == 0 && ldx % 4 == 0) {
        const int grid = ((rows + FG_R - 1) / FG_R) * ((T + FG_T - 1) / FG_T);
        if (dtype == 0) k_fgemv<0><<<grid, 256, 0, st>>>(W, rows, cols, X, ldx, T, Y, ldy);
        else if (dtype == 1) k_fgemv<1><<<grid, 256, 0, st>>>(W, rows, cols, X, ldx, T, Y, ldy);
        else k_fgemv<2><<<grid, 256, 0, st>>>(W, rows, cols, X, ldx, T, Y, ldy);
        return;
    }
    const int64_t threads = (int64_t)rows * T * 16;
    const int blocks = (int)((threads + 255) / 256);
    if (dtype == 0) k_fgemv_any<0><<<blocks, 256, 0, st>>>(W, rows, cols, X, ldx, T, Y, ldy);
    else if (dtype == 1) k_fgemv_any<1><<<blocks, 256, 0, st>>>(W, rows, cols, X, ldx, T, Y, ldy);
    else k_fgemv_any<2><<<blocks, 256, 0, st>>>(W, rows, cols, X, ldx, T, Y, ldy);
}

} // namespace hxl
