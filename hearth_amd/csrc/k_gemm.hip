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
 * token t0 + tt*16 + lane%16). */
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
    for (int gp = 0; gp < npair; gp++) {
        v4i w0, w1;
        if (m.dtype == 4) {
            const v4i raw = load16(m.w + ((size_t)rt * npair + gp) * 1024 + lane * 16);
            unpack_q4(raw, w0, w1);
        } else {
            const uint8_t *base = m.w + ((size_t)rt * m.nbp + 2 * gp) * 1024 + lane * 16;
            w0 = load16(base);
            w1 = load16(base + 1024);
        }
        const uint2 s0 = *(const uint2 *)(dcol + (size_t)(2 * gp) * m.rows_pad);
        const uint2 s1 = *(const uint2 *)(dcol + (size_t)(2 * gp + 1) * m.rows_pad);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int g = 2 * gp + j;
            if (g >= m.nb) break;
            const uint2 sw = j ? s1 : s0;
            float dw[4];
            dw[0] = h2f((uint16_t)(sw.x & 0xffff));
            dw[1] = h2f((uint16_t)(sw.x >> 16));
            dw[2] = h2f((uint16_t)(sw.y & 0xffff));
            dw[3] = h2f((uint16_t)(sw.y >> 16));
            const v4i wa = j ? w1 : w0;
#pragma unroll
            for (int tt = 0; tt < NT; tt++) {
                const size_t ab = (size_t)arow[tt] * a.nbp + g;
                const v4i b = load16((const uint8_t *)(a.q + ab * 64 + kg * 16));
                v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, b, zero, 0, 0, 0);
                const float dx = a.d[ab];
                if (m.dtype == 4) {
                    const int off = 8 * a.s[ab];   /* sum(nib * q) - 8 sum(q) = sum((nib - 8) q) */
                    c.x -= off; c.y -= off; c.z -= off; c.w -= off;
                }
                acc[tt][0] = fadd(acc[tt][0], fmul((float)c.x, fmul(dw[0], dx)));
                acc[tt][1] = fadd(acc[tt][1], fmul((float)c.y, fmul(dw[1], dx)));
                acc[tt][2] = fadd(acc[tt][2], fmul((float)c.z, fmul(dw[2], dx)));
                acc[tt][3] = fadd(acc[tt][3], fmul((float)c.w, fmul(dw[3], dx)));
            }
        }
    }
}

/* ------------------------------------------------------------ dense segmented GEMM */

template <int NT>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs args) {
    int s = 0;
    while (s + 1 < args.nseg && (int)blockIdx.x >= args.seg[s + 1].wg0) s++;
    const GemmSeg &sg = args.seg[s];
    const int rt = ((int)blockIdx.x - sg.wg0) * 4 + (int)(threadIdx.x >> 6);
    if (rt * 16 >= sg.m.rows_pad) return;
    float acc[NT][4];
    fold_tile<NT>(sg.m, rt, args.a, args.t0, args.T, [](int t) { return t; }, acc);
    const int lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        const int t = args.t0 + tt * 16 + lr;
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

/* ------------------------------------------------------------ grouped expert GEMMs */

/* gate/up of one 64-row F block of one active expert for all its tokens, then
 * mid = silu(g) * u (NUMERICS §4, quant.c:644-649) and its NUMERICS §2 block. */
__global__ __launch_bounds__(256) void k_expert_gateup(MoeArgs a) {
    __shared__ float mid[16][64];
    const int nfb = a.F / 64;
    const int u = (int)blockIdx.x / nfb, fb = (int)blockIdx.x % nfb;
    if (u >= *a.n_active) return;
    const int e = a.ulist[u], p0 = a.u_p0[u], n = a.u_n[u];
    const ExpertW ew = a.table[e];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
    const int rt = fb * 4 + wave;
    const int *ptok = a.pair_tok + p0;
    for (int t0 = 0; t0 < n; t0 += 16) {
        float g[1][4], up[1][4];
        fold_tile<1>(ew.gate, rt, a.x, t0, n, [ptok](int t) { return ptok[t]; }, g);
        fold_tile<1>(ew.up, rt, a.x, t0, n, [ptok](int t) { return ptok[t]; }, up);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float gv = canon(g[0][i]), uv = canon(up[0][i]);
            const float sg = fdiv(gv, fadd(1.0f, exp_port_f(-gv)));
            mid[lr][wave * 16 + 4 * kg + i] = fmul(sg, uv);
        }
        __syncthreads();
        for (int tt = wave; tt < 16; tt += 4) {
            if (t0 + tt < n) quant_block_wave(mid[tt][lane], a.mid, p0 + t0 + tt, fb);
        }
        __syncthreads();
    }
}

/* down projection of one 64-row D block of one active expert for all its tokens. */
__global__ __launch_bounds__(256) void k_expert_down(MoeArgs a) {
    const int ndb = (a.D + 63) / 64;
    const int u = (int)blockIdx.x / ndb, db = (int)blockIdx.x % ndb;
    if (u >= *a.n_active) return;
    const int e = a.ulist[u], p0 = a.u_p0[u], n = a.u_n[u];
    const QMat m = a.table[e].down;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, kg = lane >> 4, lr = lane & 15;
    const int rt = db * 4 + wave;
    if (rt * 16 >= m.rows_pad) return;
    for (int t0 = 0; t0 < n; t0 += 16) {
        float acc[1][4];
        fold_tile<1>(m, rt, a.mid, t0, n, [p0](int t) { return p0 + t; }, acc);
        const int t = t0 + lr;
        if (t < n) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = rt * 16 + 4 * kg + i;
                if (row < m.rows) a.Y[(size_t)(p0 + t) * a.D + row] = canon(acc[0][i]);
            }
        }
    }
}

/* ------------------------------------------------------------ float matrices (dot16) */

/* y = dot16(w_r, x_t) (NUMERICS §1/§3; quant.c:352-376): 16 lanes per (row, token),
 * lane j sums elements j, j+16, ... in order, then the 8/4/2/1 tree. */
template <int WDT>
__global__ __launch_bounds__(256) void k_fgemv(const void *__restrict__ W, int rows, int cols, const float *__restrict__ X,
                                              int ldx, int T, float *__restrict__ Y, int ldy) {
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

void gemm(const GemmArgs &in, hipStream_t st) {
    GemmArgs g = in;
    int wg = 0;
    for (int s = 0; s < g.nseg; s++) {
        g.seg[s].wg0 = wg;
        wg += (g.seg[s].m.rows_pad / 16 + 3) / 4;
    }
    if (!wg) return;
    /* token passes of up to 128 tokens; each pass re-reads the weights */
    for (int t0 = 0; t0 < in.T; t0 += 128) {
        g.t0 = t0;
        const int nt = (in.T - t0 + 15) / 16;
        if (nt <= 1) k_gemm<1><<<wg, 256, 0, st>>>(g);
        else if (nt <= 2) k_gemm<2><<<wg, 256, 0, st>>>(g);
        else if (nt <= 4) k_gemm<4><<<wg, 256, 0, st>>>(g);
        else k_gemm<8><<<wg, 256, 0, st>>>(g);
    }
}

void expert_gateup(const MoeArgs &a, int n_slots, hipStream_t st) {
    if (n_slots > 0) k_expert_gateup<<<n_slots * (a.F / 64), 256, 0, st>>>(a);
}

void expert_down(const MoeArgs &a, int n_slots, hipStream_t st) {
    if (n_slots > 0) k_expert_down<<<n_slots * ((a.D + 63) / 64), 256, 0, st>>>(a);
}

void fgemv(int dtype, const void *W, int rows, int cols, const float *X, int ldx, int T, float *Y, int ldy, hipStream_t st) {
    const int64_t threads = (int64_t)rows * T * 16;
    if (!threads) return;
    const int blocks = (int)((threads + 255) / 256);
    if (dtype == 0) k_fgemv<0><<<blocks, 256, 0, st>>>(W, rows, cols, X, ldx, T, Y, ldy);
    else if (dtype == 1) k_fgemv<1><<<blocks, 256, 0, st>>>(W, rows, cols, X, ldx, T, Y, ldy);
    else k_fgemv<2><<<blocks, 256, 0, st>>>(W, rows, cols, X, ldx, T, Y, ldy);
}

} // namespace hxl
