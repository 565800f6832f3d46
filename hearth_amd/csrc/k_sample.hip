/*
 * k_sample.hip — sampled speculative acceptance on the device: the reference's
 * Sampler.probs / draw / accept_point_mass (python/hearth/generate.py:68-147) inside its
 * verify block (generate.py:365-392), generalised to a tree of drafts (recursive
 * rejection sampling over a node's children in index order) and to a draft
 * distribution q per node.
 *
 * Everything runs in float64 in the reference's operation order, so the result is the
 * CPU restatement's bit for bit:
 *   - probs: penalty on the context ids, (x - max) / T, top-k by the exact k-th value,
 *     exp (the portable double exp), division by numpy's sum, top-p over the stable
 *     descending order with a sequential cumulative sum, min-p;
 *   - numpy's sum: 0.0, then in order the pairwise sum of each 8192-element buffer
 *     (8 accumulators over leaves of at most 128, halves split at multiples of 8);
 *   - cumulative sums (top-p, the inverse-CDF draw) are one sequential float64 chain,
 *     run by one wave over the nonzero entries only (adding +0.0 changes nothing).
 *
 * Top-p does not sort the whole row. A histogram of the probabilities by exponent
 * (and one mantissa bit) picks the highest bins whose approximate mass exceeds top_p;
 * only their entries (tier 0, gathered in any order) take part in the running sum, and
 * they are not sorted whole either: by fine bins of their top bits from the top down,
 * a bin is added in bulk when no entry of it can take the running sum out of its binade,
 * to top_p or onto a rounding tie (then the sum over the bin is order-independent), and
 * otherwise gathered, sorted (descending p, index order on ties: the stable descending
 * argsort) and summed entry by entry (top_p_binned). Once the running sum c has reached
 * top_p * (1 + 2^-48), every later entry e of the descending order has
 * before_e = fl(c_e - p_e) >= c_{e-1} (1 - 3 * 2^-53) > top_p and is dropped, so the
 * entries below the chosen bins never need ordering. If tier 0 runs out before that
 * (the histogram is approximate), the rest of the row is sorted in the workgroup
 * (bitonic, in LDS up to 8192 entries, else in the row's global scratch) and the chain
 * continues -- the result never depends on the histogram.
 *
 * k_wide_scan, k_wide_exp, k_wide_norm, k_wide_cand: a workgroup per numpy reduction
 *                  buffer (8192 entries) of each verify row; the distribution up to top-p,
 *                  then the row's top-p candidates (tier 0);
 * k_sample_probs:  the same with one workgroup per row, for top-k (an exact k-th value
 *                  over the row) and for min-p without top-p;
 * k_tp_count, k_tp_scatter: a workgroup per 8192 candidates; tier 0 bucketed by fine bin;
 * k_sample_top_p:  one workgroup per row; the cumulative-sum chain over tier 0 by fine
 *                  bins, the rest of the row if needed (and, with min-p, the
 *                  renormalization and min-p);
 * k_wide_tsum, k_wide_tdiv: a workgroup per buffer; top-p's cut and renormalization;
 * k_sib, k_resid:  every child's rejection residual and its buffers' sums, a launch per
 *                  sibling rank, a workgroup per buffer of each child;
 * k_sample_walk:   one workgroup walks the tree from the root with the uniforms (reading
 *                  single entries of the residuals) and draws the final token.
 */
#include <climits>
#include <functional>
#include <vector>

#include "hx_launch.h"

namespace hxd {
namespace {

constexpr int SP_T = 1024;
constexpr int SP_WAVES = SP_T / 64;
constexpr int NP_BUF = 8192;                     /* numpy's reduction buffer (elements) */
constexpr int SORT_LDS = 8192;                   /* candidates sorted in LDS */
constexpr int HBINS = SAMPLE_HBINS;              /* p in (0, 1]: bits >> 51 < 2048 */
static_assert(HBINS == 2048 && SAMPLE_WB * NP_BUF == SAMPLE_VMAX, "histogram and buffer counts");
constexpr int SMEM = SORT_LDS * 12;              /* LDS reused by the stages of a row */
constexpr double INF = __builtin_huge_val();

__device__ __forceinline__ double ddiv(double a, double b) { return __ddiv_rn(a, b); }

/* ---------------------------------------------------------------- workgroup helpers */

/* every thread gets the maximum */
__device__ double wg_max(double v, double *red) {
    for (int off = 32; off >= 1; off >>= 1) v = fmax(v, __shfl_xor(v, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double m = red[0];
    for (int i = 1; i < SP_WAVES; i++) m = fmax(m, red[i]);
    __syncthreads();
    return m;
}

/* exclusive prefix sum over the workgroup in thread order; *total gets the sum */
__device__ int wg_scan_excl(int v, int *red, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int inc = v;
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(inc, off, 64);
        if (lane >= off) inc += y;
    }
    if (lane == 63) red[w] = inc;
    __syncthreads();
    int before = 0, tot = 0;
    for (int i = 0; i < SP_WAVES; i++) {
        if (i < w) before += red[i];
        tot += red[i];
    }
    __syncthreads();
    *total = tot;
    return before + inc - v;
}

/* value of lane t (t uniform) of a per-lane double */
__device__ __forceinline__ double lane_value(double x, int t) {
    const long long b = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_readlane((int)b, t), hi = __builtin_amdgcn_readlane((int)(b >> 32), t);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

/* ---------------------------------------------------------------- row passes */

/* A pass over a row of up to SAMPLE_VMAX entries runs on one workgroup, so it is bound by
 * the latency of its loads unless many are in flight: each thread issues the loads of
 * SP_U of its indices before it runs their bodies. row_pass visits i = threadIdx.x + k SP_T
 * (k ascending), range_pass a thread's contiguous [lo, hi) in order: the orders of the
 * plain loops they replace. */
constexpr int SP_U = 8;

struct KeyIdx {   /* a candidate: its p's bits and its index, loaded together */
    unsigned long long k;
    int i;
};

template <class Load, class Body>
__device__ __forceinline__ void row_pass(int n, Load load, Body body) {
    for (int i0 = threadIdx.x; i0 < n; i0 += SP_T * SP_U) {
        decltype(load(0)) x[SP_U];
#pragma unroll
        for (int k = 0; k < SP_U; k++) {
            const int i = i0 + k * SP_T;
            if (i < n) x[k] = load(i);
        }
#pragma unroll
        for (int k = 0; k < SP_U; k++) {
            const int i = i0 + k * SP_T;
            if (i < n) body(i, x[k]);
        }
    }
}

template <class Load, class Body>
__device__ __forceinline__ void range_pass(int lo, int hi, Load load, Body body) {
    for (int i0 = lo; i0 < hi; i0 += SP_U) {
        decltype(load(0)) x[SP_U];
#pragma unroll
        for (int k = 0; k < SP_U; k++)
            if (i0 + k < hi) x[k] = load(i0 + k);
#pragma unroll
        for (int k = 0; k < SP_U; k++)
            if (i0 + k < hi) body(i0 + k, x[k]);
    }
}

/* rounds of SP_T indices covering [0, n), SP_U rounds' loads issued at once, every lane
 * of the workgroup running every round (index i valid iff i < n), for passes whose
 * bodies use wave operations */
template <class Load, class Body>
__device__ __forceinline__ void row_pass_converged(int n, Load load, Body body) {
    const int nr = (n + SP_T - 1) / SP_T;
    for (int r0 = 0; r0 < nr; r0 += SP_U) {
        decltype(load(0)) x[SP_U];
#pragma unroll
        for (int k = 0; k < SP_U; k++) {
            const int i = (int)threadIdx.x + (r0 + k) * SP_T;
            x[k] = (r0 + k < nr && i < n) ? load(i) : decltype(load(0))(0);
        }
#pragma unroll
        for (int k = 0; k < SP_U; k++) {
            if (r0 + k >= nr) break;   /* uniform */
            const int i = (int)threadIdx.x + (r0 + k) * SP_T;
            body(i, i < n, x[k]);
        }
    }
}

/* ---------------------------------------------------------------- numpy's sum */

/* numpy's pairwise_sum on one leaf (n <= 128) */
__device__ double pw_leaf(const double *a, int n) {
    if (n < 8) {
        double r = 0.0;
        for (int i = 0; i < n; i++) r = dadd(r, a[i]);
        return r;
    }
    double r0 = a[0], r1 = a[1], r2 = a[2], r3 = a[3], r4 = a[4], r5 = a[5], r6 = a[6], r7 = a[7];
    const int lim = n - (n % 8);
    int i = 8;
    for (; i < lim; i += 8) {
        r0 = dadd(r0, a[i]);
        r1 = dadd(r1, a[i + 1]);
        r2 = dadd(r2, a[i + 2]);
        r3 = dadd(r3, a[i + 3]);
        r4 = dadd(r4, a[i + 4]);
        r5 = dadd(r5, a[i + 5]);
        r6 = dadd(r6, a[i + 6]);
        r7 = dadd(r7, a[i + 7]);
    }
    double res = dadd(dadd(dadd(r0, r1), dadd(r2, r3)), dadd(dadd(r4, r5), dadd(r6, r7)));
    for (; i < n; i++) res = dadd(res, a[i]);
    return res;
}

/* np.sum(a[0:V]) for float64: full 8192-element buffers are balanced trees of 64 leaves
 * of 128; the partial last buffer follows tail. Every thread gets the sum. */
__device__ double np_sum(const double *a, int V, const PwTail &tail, double *lv, double *bcast) {
    const int nfull = V / NP_BUF;
    const int tl = V - nfull * NP_BUF;
    const int nleaf = nfull * 64 + (tl ? tail.nleaf : 0);
    __syncthreads();                               /* a[] was written by other threads */
    /* leaves: eight lanes a leaf, lane k running pw_leaf's accumulator r_k (its loads all
     * in flight at once for a full leaf), the group combining ((r0 + r1) + (r2 + r3)) +
     * ((r4 + r5) + (r6 + r7)) by exchanges (the two lanes of a pair hold the same sum) and
     * lane 0 adding the leaf's last len % 8 entries; leaves below 8 entries go in order */
    for (int L8 = threadIdx.x; L8 < nleaf * 8; L8 += SP_T) {   /* a leaf's 8 lanes are active together */
        const int L = L8 >> 3, k = L8 & 7;
        int start, len;
        if (L < nfull * 64) {
            start = (L >> 6) * NP_BUF + (L & 63) * 128;
            len = 128;
        } else {
            const int t = L - nfull * 64;
            start = nfull * NP_BUF + tail.leaf_start[t];
            len = tail.leaf_len[t];
        }
        const double *x = a + start;
        if (len < 8) {
            if (k == 0) lv[L] = pw_leaf(x, len);
            continue;
        }
        const int lim = len - (len % 8);
        double r = x[k];
        if (lim == 128) {
            double y[15];
#pragma unroll
            for (int u = 0; u < 15; u++) y[u] = x[8 * (u + 1) + k];
#pragma unroll
            for (int u = 0; u < 15; u++) r = dadd(r, y[u]);
        } else {
            for (int i = 8; i < lim; i += 8) r = dadd(r, x[i + k]);
        }
        r = dadd(r, __shfl_xor(r, 1, 64));
        r = dadd(r, __shfl_xor(r, 2, 64));
        r = dadd(r, __shfl_xor(r, 4, 64));
        if (k == 0) {
            for (int i = lim; i < len; i++) r = dadd(r, x[i]);
            lv[L] = r;
        }
    }
    __syncthreads();
    for (int h = 1; h <= 7; h++) {
        const int per = h <= 6 ? (64 >> h) : 0;
        const int nf = nfull * per;
        const int nt = (tl && h <= tail.nlev) ? tail.lev_off[h] - tail.lev_off[h - 1] : 0;
        for (int o = threadIdx.x; o < nf + nt; o += SP_T) {
            if (o < nf) {
                const int s = (o / per) * 64 + (o % per) * (1 << h);
                lv[s] = dadd(lv[s], lv[s + (1 << (h - 1))]);
            } else {
                const int t = tail.lev_off[h - 1] + (o - nf), base = nfull * 64;
                lv[base + tail.op_a[t]] = dadd(lv[base + tail.op_a[t]], lv[base + tail.op_b[t]]);
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        double s = 0.0;
        for (int b = 0; b < nfull; b++) s = dadd(s, lv[b * 64]);
        if (tl) s = dadd(s, lv[nfull * 64]);
        *bcast = s;
    }
    __syncthreads();
    const double s = *bcast;
    __syncthreads();
    return s;
}

/* ---------------------------------------------------------------- top-k */

/* order-preserving key of a non-NaN double (ascending keys = ascending values) */
__device__ __forceinline__ unsigned long long okey(double x) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(x);
    return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}
__device__ __forceinline__ double okey_value(unsigned long long k) {
    const unsigned long long b = (k >> 63) ? (k & 0x7fffffffffffffffull) : ~k;
    return __longlong_as_double((long long)b);
}

/* value at ascending rank r (0-based) of x[0..V): radix select, 8 bits per pass */
__device__ double select_rank(const double *x, int V, int r, uint32_t *hist, int *sh) {
    unsigned long long prefix = 0, mask = 0;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += SP_T) hist[i] = 0;
        __syncthreads();
        row_pass(V, [&](int i) { return x[i]; }, [&](int, double xv) {
            const unsigned long long k = okey(xv);
            if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255], 1u);
        });
        __syncthreads();
        if (threadIdx.x < 64) {
            const int l = threadIdx.x;
            const uint32_t h0 = hist[4 * l], h1 = hist[4 * l + 1], h2 = hist[4 * l + 2], h3 = hist[4 * l + 3];
            const uint32_t tot = h0 + h1 + h2 + h3;
            uint32_t inc = tot;
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t y = __shfl_up(inc, off, 64);
                if (l >= off) inc += y;
            }
            const uint32_t exc = inc - tot, rr0 = (uint32_t)r;
            if (exc <= rr0 && rr0 < inc) {
                uint32_t rr = rr0 - exc;
                int d = 4 * l;
                if (rr >= h0) {
                    rr -= h0; d++;
                    if (rr >= h1) {
                        rr -= h1; d++;
                        if (rr >= h2) { rr -= h2; d++; }
                    }
                }
                sh[0] = d;
                sh[1] = (int)rr;
            }
        }
        __syncthreads();
        prefix |= (unsigned long long)sh[0] << shift;
        mask |= 255ull << shift;
        r = sh[1];
        __syncthreads();
    }
    return okey_value(prefix);
}

/* ---------------------------------------------------------------- sorting (top-p) */

/* descending probability, ascending index on ties (np.argsort(-p, kind="stable")) */
__device__ __forceinline__ bool before(unsigned long long ka, int ia, unsigned long long kb, int ib) {
    return ka > kb || (ka == kb && ia < ib);
}

/* one compare-exchange stage (k, j) of a bitonic network over key/idx[0..N); base is
 * the global index of element 0 (the direction of element i is ((base + i) & k) == 0) */
__device__ void bitonic_stage(unsigned long long *key, int *idx, int N, int k, int j, int base) {
    for (int t = threadIdx.x; t < N / 2; t += SP_T) {
        const int i = ((t & ~(j - 1)) << 1) | (t & (j - 1));
        const int p = i + j;
        const bool asc = ((base + i) & k) == 0;
        const unsigned long long ki = key[i], kp = key[p];
        const int ii = idx[i], ip = idx[p];
        if (asc ? before(kp, ip, ki, ii) : before(ki, ii, kp, ip)) {
            key[i] = kp; key[p] = ki;
            idx[i] = ip; idx[p] = ii;
        }
    }
}

/* stages k in [k0, k1] (j from min(k/2, jmax) down to 1) on an LDS block */
__device__ void bitonic_block(unsigned long long *key, int *idx, int N, int k0, int k1, int jmax, int base) {
    for (int k = k0; k <= k1; k <<= 1)
        for (int j = (k >> 1) < jmax ? (k >> 1) : jmax; j > 0; j >>= 1) {
            bitonic_stage(key, idx, N, k, j, base);
            __syncthreads();
        }
}

/* sorts gkey/gidx[0..N) (N a power of two > SORT_LDS, in global memory) with LDS blocks
 * for the strides below SORT_LDS */
__device__ void bitonic_global(unsigned long long *gkey, int *gidx, int N, unsigned long long *lkey, int *lidx) {
    const int nb = N / SORT_LDS;
    for (int k = 2; k <= N; k <<= 1) {
        if (k > SORT_LDS)
            for (int j = k >> 1; j >= SORT_LDS; j >>= 1) {
                bitonic_stage(gkey, gidx, N, k, j, 0);
                __syncthreads();
            }
        for (int b = 0; b < nb; b++) {
            for (int i = threadIdx.x; i < SORT_LDS; i += SP_T) {
                lkey[i] = gkey[b * SORT_LDS + i];
                lidx[i] = gidx[b * SORT_LDS + i];
            }
            __syncthreads();
            if (k <= SORT_LDS) bitonic_block(lkey, lidx, SORT_LDS, 2, SORT_LDS, SORT_LDS, b * SORT_LDS);
            else bitonic_block(lkey, lidx, SORT_LDS, k, k, SORT_LDS / 2, b * SORT_LDS);
            for (int i = threadIdx.x; i < SORT_LDS; i += SP_T) {
                gkey[b * SORT_LDS + i] = lkey[i];
                gidx[b * SORT_LDS + i] = lidx[i];
            }
            __syncthreads();
        }
        if (k <= SORT_LDS) k = SORT_LDS;   /* the block pass ran every stage up to SORT_LDS */
    }
}

/* ---------------------------------------------------------------- exact running sums */

/* The float64 running sum c_j = fl(c_{j-1} + x_j), j = 0..m-1, from c_{-1} = 0, of
 * finite x_j >= 0 (np.cumsum's chain), computed CE SP_T entries at a time by the whole
 * workgroup (thread t takes CE consecutive entries of a chunk; CE 1 where entries added
 * on their own are frequent, as in the sorted top-p bins near c's binade, since each
 * restarts the chunk; CE 8 for the draw's chain over the row in index order). While c stays
 * in one binade [2^e, 2^(e+1)) every partial sum is a multiple of u = 2^(e-52) and so is
 * every rounded sum, so fl(c + x) = c + RN_u(x): the integer prefix sums of RN_u(x_j) / u
 * give every c_j of a chunk at once. An entry whose sum would leave the binade, or whose
 * x / u is halfway between two integers (round-half-even then depends on the parity of
 * c / u), is added on its own and the chunk restarts after it. on_entry(j, c_j) is
 * called once per entry by one thread. The chain stops after the chunk in which
 * c_j >= stop_at first holds; *stop_j gets that j (m if never). Returns the last c
 * computed. */
struct ChainShared {
    long long wsum[SP_WAVES];
    int wtie[SP_WAVES], wdel[SP_WAVES];   /* per wave: a of its last tie (-1: none), its ties' adjustments */
    long long dfb[SP_T];                  /* per thread: the units before its first entry that leaves the binade */
    long long dend;                       /* the units after the block's last entry */
    double c, cnext;
    int first_bad, stop;
};

template <int CE_PER = 1, class GetX, class OnEntry>
__device__ double chain_exact(GetX get_x, int m, double stop_at, int *stop_j, OnEntry on_entry, ChainShared &cs) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    double c = 0.0;
    int j0 = 0, stop = m;
    bool in_order = true;   /* the next 64 entries one after the other (from c = 0, or after a round that gained little) */
    while (j0 < m && stop == m) {
        if (in_order) {
            /* wave 0 loads 64 entries at once and every lane runs the chain through them
             * (fl(0 + x) = x, so c = 0 needs no case of its own); lane k keeps c after
             * entry j0 + k. Where entries added on their own are frequent (c small, or
             * near the entries' own binade), this costs one dependent add an entry
             * instead of a round of the workgroup. */
            if (w == 0) {
                const int n = m - j0 < 64 ? m - j0 : 64;
                const double x = lane < n ? get_x(j0 + lane) : 0.0;
                double cc = c, mine = 0.0;
                for (int k = 0; k < n; k++) {
                    cc = dadd(cc, lane_value(x, k));
                    if (lane == k) mine = cc;
                }
                if (lane < n) on_entry(j0 + lane, mine);
                const unsigned long long hit = __ballot(lane < n && mine >= stop_at);
                if (lane == 0) {
                    cs.c = cc;
                    cs.stop = hit ? j0 + __builtin_ctzll(hit) : INT_MAX;
                }
            }
            __syncthreads();
            c = cs.c;
            if (cs.stop != INT_MAX) {
                stop = cs.stop;
                break;
            }
            j0 = j0 + 64 < m ? j0 + 64 : m;
            in_order = c == 0.0;
            __syncthreads();
            continue;
        }
        /* a block of SP_T CE_PER entries is loaded once; sub-rounds run the chain through
         * it from js, each in the binade of the current c, until it is used up */
        const int jb = j0, jend = j0 + SP_T * CE_PER < m ? j0 + SP_T * CE_PER : m;
        const int jt = jb + tid * CE_PER;   /* this thread's first entry */
        double xv[CE_PER];
#pragma unroll
        for (int k = 0; k < CE_PER; k++) xv[k] = jt + k < jend ? get_x(jt + k) : 0.0;
        int js = j0;
        while (js < jend && stop == m) {
            int e = ilogb(c);
            if (e < -1022) e = -1022;
            const double u = ldexp(1.0, e - 52);
            const long long base = (long long)(c / u);   /* exact: c is a multiple of u below 2^53 u */
            long long d[CE_PER];
            bool tie[CE_PER], huge[CE_PER];
            long long tsum = 0;
            bool has_tie = false;
#pragma unroll
            for (int k = 0; k < CE_PER; k++) {
                const int j = jt + k;
                d[k] = 0;
                tie[k] = huge[k] = false;
                if (j >= js && j < jend) {
                    const double q = ldexp(xv[k], 52 - e);   /* x / u: a power-of-two scaling, exact */
                    if (!(q < 0x1p53)) {
                        huge[k] = true;
                    } else {
                        const double f = floor(q), r = q - f;
                        d[k] = (long long)f + (r > 0.5 ? 1 : 0);
                        tie[k] = r == 0.5;   /* its d is the floor until its parity is known */
                        has_tie |= tie[k];
                    }
                }
                tsum += d[k];
            }
            long long inc = tsum;
            for (int off = 1; off < 64; off <<= 1) {
                const long long y = __shfl_up(inc, off, 64);
                if (lane >= off) inc += y;
            }
            if (lane == 63) cs.wsum[w] = inc;
            if (tid == 0) { cs.first_bad = INT_MAX; cs.stop = INT_MAX; }
            const bool any_tie = __syncthreads_or(has_tie);
            long long before = 0;
            for (int i = 0; i < w; i++) before += cs.wsum[i];
            const long long D0 = base + before + inc - tsum;   /* units before entry jt (ties at their floor) */
            /* A tie i rounds to even: with P_i the units before it at the floor of every
             * earlier tie and a_i = (P_i + floor_i) mod 2, it adds floor_i + (a_i xor
             * a_(i-1)) (a of the previous tie of the round, 0 for the first): the parity of
             * the adjustments so far is always a of the last tie. */
            int dl[CE_PER];
            long long Dx = 0;   /* adjustments before this thread's first entry */
#pragma unroll
            for (int k = 0; k < CE_PER; k++) dl[k] = 0;
            if (any_tie) {
                int a_last = 0;
                long long P = D0;
#pragma unroll
                for (int k = 0; k < CE_PER; k++) {
                    if (tie[k]) { dl[k] = (int)((P + d[k]) & 1); a_last = dl[k]; }   /* a_k for now */
                    P += d[k];
                }
                /* a of the last tie before this thread: in the wave, then the earlier waves */
                const unsigned long long tb = __ballot(has_tie);
                const unsigned long long before_me = tb & ((1ull << lane) - 1ull);
                const int src = before_me ? 63 - __builtin_clzll(before_me) : 0;
                const int got = __shfl(a_last, src, 64);
                int a_prev = before_me ? got : 0;
                const int wl = tb ? 63 - __builtin_clzll(tb) : 0;
                const int wa = __shfl(a_last, wl, 64);
                if (lane == 0) cs.wtie[w] = tb ? wa : -1;
                __syncthreads();
                if (!before_me)
                    for (int i = w - 1; i >= 0; i--)
                        if (cs.wtie[i] >= 0) { a_prev = cs.wtie[i]; break; }
                int dsum = 0;
#pragma unroll
                for (int k = 0; k < CE_PER; k++)
                    if (tie[k]) {
                        const int ak = dl[k];
                        dl[k] = ak ^ a_prev;
                        a_prev = ak;
                        dsum += dl[k];
                    }
                int di = dsum;
                for (int off = 1; off < 64; off <<= 1) {
                    const int y = __shfl_up(di, off, 64);
                    if (lane >= off) di += y;
                }
                if (lane == 63) cs.wdel[w] = di;
                __syncthreads();
                long long db = 0;
                for (int i = 0; i < w; i++) db += cs.wdel[i];
                Dx = db + di - dsum;
            }
            /* the sums of this thread's entries up to its first entry that leaves the binade
             * (or is huge), which it reports with the units before it; the sub-round ends at
             * the first such entry of the block */
            double cjv[CE_PER];
            {
                long long D = D0 + Dx;
                int myfb = INT_MAX;
#pragma unroll
                for (int k = 0; k < CE_PER; k++) {
                    cjv[k] = 0.0;
                    const int j = jt + k;
                    if (j < js || j >= jend || myfb != INT_MAX) continue;
                    if (huge[k] || D + d[k] + dl[k] >= (1ll << 53)) {
                        myfb = j;
                        continue;
                    }
                    D += d[k] + dl[k];
                    cjv[k] = (double)D * u;   /* an integer below 2^53 times a power of two: exact */
                    if (cjv[k] >= stop_at) atomicMin(&cs.stop, j);
                }
                if (myfb != INT_MAX) {
                    atomicMin(&cs.first_bad, myfb);
                    cs.dfb[tid] = D;
                } else if (jend - 1 >= jt && jend - 1 < jt + CE_PER) {
                    cs.dend = D;   /* the block's last entry is this thread's */
                }
            }
            __syncthreads();
            const int fb = cs.first_bad, fend = fb < jend ? fb : jend;
            if (fend > js) c = (double)(fb < jend ? cs.dfb[(fb - jb) / CE_PER] : cs.dend) * u;
#pragma unroll
            for (int k = 0; k < CE_PER; k++) {
                const int j = jt + k;
                if (j >= js && j < fend) on_entry(j, cjv[k]);
            }
            if (cs.stop < fend) {   /* a stop past fb came from sums that do not hold */
                stop = cs.stop;
                break;
            }
            if (fb < jend) {   /* entry fb on its own, from the value its thread holds */
                if (fb >= jt && fb < jt + CE_PER) {
                    double xf = 0.0;
#pragma unroll
                    for (int k = 0; k < CE_PER; k++)
                        if (jt + k == fb) xf = xv[k];
                    const double cf = dadd(c, xf);
                    cs.cnext = cf;
                    on_entry(fb, cf);
                }
                __syncthreads();
                c = cs.cnext;
                if (c >= stop_at) stop = fb;
                const bool little = fb - js < 64;
                js = fb + 1;
                if (little) {   /* entries added on their own are frequent here: go on in order */
                    in_order = true;
                    break;
                }
            } else {
                js = jend;
            }
            /* no barrier before the next sub-round (there is one after fb's entry, and the
             * loop ends otherwise): every thread read cs.first_bad, cs.stop, cs.wsum, cs.dfb
             * and cs.dend before that barrier, and cs.cnext is written again only after two
             * more */
        }
        j0 = js;
        __syncthreads();
    }
    *stop_j = stop;
    return c;
}

/* ---------------------------------------------------------------- per-row distribution */

struct RowShared {
    double red_d[SP_WAVES];
    int red_i[SP_WAVES];
    int red_f[SP_WAVES];
    double bd[4];
    int bi[8];
};

/* the approximate mass of bin b from its integer sum (histogram passes: the significands
 * less their low 12 bits, summed as integers in units of 2^(E - 1063) for exponent field
 * E, 2^-1062 for subnormals; below 2^41 each, so that SAMPLE_VMAX of them cannot wrap) */
__device__ __forceinline__ unsigned long long hist_units(double p) {
    const unsigned long long bits = (unsigned long long)__double_as_longlong(p);
    const unsigned long long sig = (bits & 0xFFFFFFFFFFFFFull) | ((bits >> 52) ? (1ull << 52) : 0ull);
    return sig >> 12;
}
__device__ __forceinline__ double hist_mass(unsigned long long units, int b) {
    const int ef = b >> 1;
    return ldexp((double)units, (ef ? ef - 1075 : -1074) + 12);
}

/* b*: the highest histogram bin whose suffix mass reaches top_p + 1e-9 (approximate
 * sums), -1 if none; hsum[HBINS] are the bins' integer sums */
__device__ int select_bstar(const unsigned long long *hsum, double top_p, RowShared &rs) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (tid == 0) rs.bi[2] = -1;
    __syncthreads();
    const int b1 = 2 * (SP_T - 1 - tid) + 1, b0 = b1 - 1;   /* thread 0 holds the top bins */
    const double m1 = hist_mass(hsum[b1], b1), m0 = hist_mass(hsum[b0], b0);
    double inc = dadd(m1, m0);
    for (int off = 1; off < 64; off <<= 1) {
        const double y = __shfl_up(inc, off, 64);
        if (lane >= off) inc = dadd(inc, y);
    }
    if (lane == 63) rs.red_d[wv] = inc;
    __syncthreads();
    double above = 0.0;
    for (int i = 0; i < wv; i++) above = dadd(above, rs.red_d[i]);
    const double excl = dadd(above, dsub(inc, dadd(m1, m0)));
    const double s1 = dadd(excl, m1), s0 = dadd(s1, m0);
    const double thr = top_p + 1e-9;
    if (s0 >= thr) atomicMax(&rs.bi[2], s1 >= thr ? b1 : b0);
    __syncthreads();
    const int r = rs.bi[2];
    __syncthreads();
    return r;
}

/* the Sampler.probs pipeline on row v; returns 0 or -1 (bad logits) */
__global__ __launch_bounds__(SP_T) void k_sample_probs(SampleArgs a) {
    __shared__ __align__(16) unsigned char smem[SMEM];
    __shared__ RowShared rs;
    const int v = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (a.live && v >= *a.live) return;   /* padding row (uniform) */
    const int V = a.V;
    const float *row = a.rows + (size_t)v * V;
    double *P = a.P + (size_t)v * V;
    double *lv = (double *)smem;
    if (tid == 0) {   /* no candidates unless top-p runs */
        a.seg_begin[v] = v * a.sort_n;
        a.seg_end[v] = v * a.sort_n;
    }
    for (int i = tid; i < HBINS; i += SP_T) {
        a.bcnt[(size_t)v * HBINS + i] = 0;
        a.brel[(size_t)v * HBINS + i] = 0;
    }

    /* Sampler._penalised: the ids of the context and of the path nodes 1..v */
    const bool pen = a.rp != 1.0;
    uint32_t *bits = (uint32_t *)smem;
    if (pen) {
        for (int i = tid; i < (V + 31) / 32; i += SP_T) bits[i] = 0;
        __syncthreads();
        const int n_ctx = a.n_ctx_dev ? *a.n_ctx_dev : a.n_ctx;
        for (int j = tid; j < n_ctx; j += SP_T) {
            const int t = a.ctx[j];
            if (t >= 0 && t < V) atomicOr(&bits[t >> 5], 1u << (t & 31));
        }
        if (tid == 0)
            for (int c = v; c > 0; c = a.parent[c]) {
                const int t = a.tokens[c];
                if (t >= 0 && t < V) atomicOr(&bits[t >> 5], 1u << (t & 31));
            }
        __syncthreads();
    }
    double best = -INF;
    int bidx = -1, flags = 0;
    row_pass(V, [&](int i) { return row[i]; }, [&](int i, float l) {
        if (l != l || l == __builtin_huge_valf()) flags |= 1;
        if (l != -__builtin_huge_valf()) flags |= 2;
        double x = (double)l;
        if (pen && ((bits[i >> 5] >> (i & 31)) & 1u)) x = x > 0.0 ? ddiv(x, a.rp) : dmul(x, a.rp);
        P[i] = x;
        if (bidx < 0 || x > best) { best = x; bidx = i; }
    });
    /* max and first argmax over the workgroup, flags */
    for (int off = 32; off >= 1; off >>= 1) {
        const double ob = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(bidx, off, 64);
        if (oi >= 0 && (bidx < 0 || ob > best || (ob == best && oi < bidx))) { best = ob; bidx = oi; }
        flags |= __shfl_xor(flags, off, 64);
    }
    if (lane == 0) { rs.red_d[wv] = best; rs.red_i[wv] = bidx; rs.red_f[wv] = flags; }
    __syncthreads();
    best = rs.red_d[0]; bidx = rs.red_i[0]; flags = rs.red_f[0];
    for (int i = 1; i < SP_WAVES; i++) {
        const double ob = rs.red_d[i];
        const int oi = rs.red_i[i];
        if (oi >= 0 && (bidx < 0 || ob > best || (ob == best && oi < bidx))) { best = ob; bidx = oi; }
        flags |= rs.red_f[i];
    }
    __syncthreads();
    if ((flags & 1) || !(flags & 2)) {
        if (tid == 0) a.row_rc[v] = -1;
        return;
    }
    if (a.temperature == 0.0) {
        for (int i = tid; i < V; i += SP_T) P[i] = i == bidx ? 1.0 : 0.0;
        if (tid == 0) a.row_rc[v] = 0;
        return;
    }
    const double mx = best, T = a.temperature;
    const bool use_k = a.top_k > 0 && a.top_k < V;
    double kth = -INF;
    if (use_k) {
        row_pass(V, [&](int i) { return P[i]; }, [&](int i, double x) { P[i] = ddiv(dsub(x, mx), T); });
        __syncthreads();
        kth = select_rank(P, V, V - a.top_k, (uint32_t *)smem, rs.bi);
        row_pass(V, [&](int i) { return P[i]; }, [&](int i, double x) { P[i] = x < kth ? 0.0 : exp_port_d(x); });
    } else {
        /* the same values as the scaling pass and the exp pass one after the other */
        row_pass(V, [&](int i) { return P[i]; }, [&](int i, double x) { P[i] = exp_port_d(ddiv(dsub(x, mx), T)); });
    }
    double s = np_sum(P, V, a.tail, lv, rs.bd);
    row_pass(V, [&](int i) { return P[i]; }, [&](int i, double x) { P[i] = ddiv(x, s); });

    if (a.top_p < 1.0) {
        const double top_p = a.top_p;
        /* the approximate mass of each bin (exponent and first significand bit) */
        unsigned long long *hsum = (unsigned long long *)smem;
        for (int i = tid; i < HBINS; i += SP_T) hsum[i] = 0ull;
        __syncthreads();
        row_pass(V, [&](int i) { return P[i]; }, [&](int, double p) {
            if (p > 0.0) atomicAdd(&hsum[(unsigned long long)__double_as_longlong(p) >> 51], hist_units(p));
        });
        __syncthreads();
        const int bstar = select_bstar(hsum, top_p, rs);
        /* tier 0 (bins >= b*; all nonzero entries when b* < 0), gathered a wave at a time (in
         * no particular order: every use of it is by bins, and the bins it sorts are
         * sorted by (p descending, index ascending), a total order) */
        const int blo = bstar < 0 ? 0 : bstar;
        unsigned long long *key = a.skey + (size_t)v * a.sort_n;
        int *idx = a.sidx + (size_t)v * a.sort_n;
        if (tid == 0) rs.bi[3] = 0;
        __syncthreads();
        row_pass_converged(V, [&](int i) { return P[i]; }, [&](int i, bool in, double p) {
            const bool cand = in && p > 0.0 && (int)((unsigned long long)__double_as_longlong(p) >> 51) >= blo;
            const unsigned long long bal = __ballot(cand);
            int base = 0;
            if (lane == 0 && bal) base = atomicAdd(&rs.bi[3], __popcll(bal));
            base = __shfl(base, 0, 64);
            if (cand) {
                const int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
                key[pos] = (unsigned long long)__double_as_longlong(p);
                idx[pos] = i;
            }
        });
        __syncthreads();
        const int m = rs.bi[3];
        if (tid == 0) {
            a.seg_end[v] = v * a.sort_n + m;
            a.bstar[v] = bstar;
        }
        return;   /* k_sample_top_p continues with the sorted candidates */
    }
    if (a.min_p > 0.0) {
        double mp = -INF;
        __syncthreads();
        row_pass(V, [&](int i) { return P[i]; }, [&](int, double x) { mp = fmax(mp, x); });
        mp = wg_max(mp, rs.red_d);
        const double thr = dmul(a.min_p, mp);
        row_pass(V, [&](int i) { return P[i]; }, [&](int i, double x) { if (x < thr) P[i] = 0.0; });
        s = np_sum(P, V, a.tail, lv, rs.bd);
        row_pass(V, [&](int i) { return P[i]; }, [&](int i, double x) { P[i] = ddiv(x, s); });
    }
    if (tid == 0) a.row_rc[v] = 0;
}

/* ---------------------------------------------------------------- the distribution, wide */

/* Sampler.probs without top-k, spread over the row: workgroup b of row v takes numpy's
 * reduction buffer b (entries [8192 b, 8192 b + 8192)), so that a row runs on
 * ceil(V / 8192) compute units and each buffer's pairwise sum is a workgroup's own.
 *   k_wide_scan:  the penalty, the logits as float64, the buffer's max and first argmax;
 *   k_wide_exp:   the row's max and first argmax from the buffers' (a total order:
 *                 value descending, index ascending), bad rows, temperature 0,
 *                 exp((x - max) / T), the buffer's pairwise sum;
 *   k_wide_norm:  numpy's sum (0.0, then the buffers' sums in order), the division, the
 *                 buffer's bin masses added into the row's histogram (integer sums);
 *   k_wide_cand:  b* from the row's histogram, the buffer's candidates of tier 0
 *                 appended to the row's (one global atomic per workgroup; any order).
 * Every value is computed by the operations of k_sample_probs in the same order, so the
 * distribution and the candidates (as a set) are the same. row_rc[v] is 1 while the row
 * goes on, -1 for bad logits, 0 once final. */
__device__ __forceinline__ void wide_range(int V, int &r0, int &len) {
    r0 = blockIdx.x * NP_BUF;
    len = V - r0 < NP_BUF ? V - r0 : NP_BUF;
}

__global__ __launch_bounds__(SP_T) void k_wide_scan(SampleArgs a) {
    __shared__ uint32_t bits[NP_BUF / 32];
    __shared__ RowShared rs;
    const int v = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (a.live && v >= *a.live) return;   /* padding row (uniform) */
    const int V = a.V;
    int r0, len;
    wide_range(V, r0, len);
    const float *row = a.rows + (size_t)v * V + r0;
    double *P = a.P + (size_t)v * V + r0;
    if (blockIdx.x == 0 && tid == 0) {   /* no candidates unless top-p runs */
        a.seg_begin[v] = v * a.sort_n;
        a.seg_end[v] = v * a.sort_n;
    }
    for (int i = blockIdx.x * SP_T + tid; i < HBINS; i += gridDim.x * SP_T) {
        a.whist[(size_t)v * HBINS + i] = 0ull;
        a.bcnt[(size_t)v * HBINS + i] = 0;
        a.brel[(size_t)v * HBINS + i] = 0;
    }
    /* Sampler._penalised: the ids of the context and of the path nodes 1..v in this buffer */
    const bool pen = a.rp != 1.0;
    if (pen) {
        for (int i = tid; i < NP_BUF / 32; i += SP_T) bits[i] = 0;
        __syncthreads();
        const int n_ctx = a.n_ctx_dev ? *a.n_ctx_dev : a.n_ctx;
        for (int j = tid; j < n_ctx; j += SP_T) {
            const int t = a.ctx[j];
            if (t >= r0 && t < r0 + len) atomicOr(&bits[(t - r0) >> 5], 1u << ((t - r0) & 31));
        }
        if (tid == 0)
            for (int c = v; c > 0; c = a.parent[c]) {
                const int t = a.tokens[c];
                if (t >= r0 && t < r0 + len) atomicOr(&bits[(t - r0) >> 5], 1u << ((t - r0) & 31));
            }
        __syncthreads();
    }
    double best = -INF;
    int bidx = -1, flags = 0;
    row_pass(len, [&](int i) { return row[i]; }, [&](int i, float l) {
        if (l != l || l == __builtin_huge_valf()) flags |= 1;
        if (l != -__builtin_huge_valf()) flags |= 2;
        double x = (double)l;
        if (pen && ((bits[i >> 5] >> (i & 31)) & 1u)) x = x > 0.0 ? ddiv(x, a.rp) : dmul(x, a.rp);
        P[i] = x;
        if (bidx < 0 || x > best) { best = x; bidx = r0 + i; }
    });
    for (int off = 32; off >= 1; off >>= 1) {
        const double ob = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(bidx, off, 64);
        if (oi >= 0 && (bidx < 0 || ob > best || (ob == best && oi < bidx))) { best = ob; bidx = oi; }
        flags |= __shfl_xor(flags, off, 64);
    }
    if (lane == 0) { rs.red_d[wv] = best; rs.red_i[wv] = bidx; rs.red_f[wv] = flags; }
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < SP_WAVES; i++) {
            const double ob = rs.red_d[i];
            const int oi = rs.red_i[i];
            if (oi >= 0 && (bidx < 0 || ob > best || (ob == best && oi < bidx))) { best = ob; bidx = oi; }
            flags |= rs.red_f[i];
        }
        const size_t o = (size_t)v * SAMPLE_WB + blockIdx.x;
        a.wmax[o] = best;
        a.widx[o] = bidx;
        a.wflag[o] = flags;
    }
}

__global__ __launch_bounds__(SP_T) void k_wide_exp(SampleArgs a) {
    __shared__ double lv[128];
    __shared__ double bc;
    const int v = blockIdx.y, tid = threadIdx.x;
    if (a.live && v >= *a.live) return;
    const int V = a.V;
    int r0, len;
    wide_range(V, r0, len);
    double *P = a.P + (size_t)v * V + r0;
    double best = -INF;
    int bidx = -1, flags = 0;
    for (int b = 0; b < (int)gridDim.x; b++) {
        const size_t o = (size_t)v * SAMPLE_WB + b;
        const double ob = a.wmax[o];
        const int oi = a.widx[o];
        if (oi >= 0 && (bidx < 0 || ob > best || (ob == best && oi < bidx))) { best = ob; bidx = oi; }
        flags |= a.wflag[o];
    }
    const bool lead = blockIdx.x == 0 && tid == 0;
    if ((flags & 1) || !(flags & 2)) {
        if (lead) a.row_rc[v] = -1;
        return;
    }
    if (a.temperature == 0.0) {
        for (int i = tid; i < len; i += SP_T) P[i] = r0 + i == bidx ? 1.0 : 0.0;
        if (lead) a.row_rc[v] = 0;
        return;
    }
    if (lead) a.row_rc[v] = 1;
    const double mx = best, T = a.temperature;
    row_pass(len, [&](int i) { return P[i]; }, [&](int i, double x) { P[i] = exp_port_d(ddiv(dsub(x, mx), T)); });
    /* the buffer's pairwise sum: a full buffer, or the row's partial last one */
    const double s = np_sum(P, len, a.tail, lv, &bc);
    if (tid == 0) a.wsum[(size_t)v * SAMPLE_WB + blockIdx.x] = s;
}

__global__ __launch_bounds__(SP_T) void k_wide_norm(SampleArgs a) {
    __shared__ unsigned long long hs[HBINS];
    const int v = blockIdx.y, tid = threadIdx.x;
    if (a.live && v >= *a.live) return;
    if (a.row_rc[v] != 1) return;   /* final already (uniform) */
    const int V = a.V;
    int r0, len;
    wide_range(V, r0, len);
    double *P = a.P + (size_t)v * V + r0;
    double s = 0.0;
    for (int b = 0; b < (int)gridDim.x; b++) s = dadd(s, a.wsum[(size_t)v * SAMPLE_WB + b]);
    const bool hist = a.top_p < 1.0;
    if (hist) {
        for (int i = tid; i < HBINS; i += SP_T) hs[i] = 0ull;
        __syncthreads();
    }
    row_pass(len, [&](int i) { return P[i]; }, [&](int i, double x) {
        const double p = ddiv(x, s);
        P[i] = p;
        if (hist && p > 0.0) atomicAdd(&hs[(unsigned long long)__double_as_longlong(p) >> 51], hist_units(p));
    });
    if (hist) {
        __syncthreads();
        unsigned long long *g = a.whist + (size_t)v * HBINS;
        for (int b = tid; b < HBINS; b += SP_T)
            if (hs[b]) atomicAdd(&g[b], hs[b]);
    }
}

__global__ __launch_bounds__(SP_T) void k_wide_cand(SampleArgs a) {
    __shared__ __align__(16) unsigned char stage[NP_BUF * 12];
    __shared__ RowShared rs;
    const int v = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    if (a.live && v >= *a.live) return;
    if (a.row_rc[v] != 1) return;   /* (uniform) */
    const int V = a.V;
    int r0, len;
    wide_range(V, r0, len);
    const double *P = a.P + (size_t)v * V + r0;
    const int bstar = select_bstar(a.whist + (size_t)v * HBINS, a.top_p, rs);
    if (blockIdx.x == 0 && tid == 0) a.bstar[v] = bstar;
    const int blo = bstar < 0 ? 0 : bstar;
    /* the buffer's tier 0, gathered a wave at a time into LDS, then appended to the row's */
    unsigned long long *lk = (unsigned long long *)stage;
    int *li = (int *)(stage + NP_BUF * 8);
    if (tid == 0) rs.bi[3] = 0;
    __syncthreads();
    row_pass_converged(len, [&](int i) { return P[i]; }, [&](int i, bool in, double p) {
        const bool cand = in && p > 0.0 && (int)((unsigned long long)__double_as_longlong(p) >> 51) >= blo;
        const unsigned long long bal = __ballot(cand);
        int base = 0;
        if (lane == 0 && bal) base = atomicAdd(&rs.bi[3], __popcll(bal));
        base = __shfl(base, 0, 64);
        if (cand) {
            const int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
            lk[pos] = (unsigned long long)__double_as_longlong(p);
            li[pos] = r0 + i;
        }
    });
    __syncthreads();
    const int cnt = rs.bi[3];
    if (tid == 0) rs.bi[4] = cnt ? atomicAdd(&a.seg_end[v], cnt) : 0;
    __syncthreads();
    const int at = rs.bi[4];   /* the place of the first in skey / sidx */
    for (int j = tid; j < cnt; j += SP_T) {
        a.skey[at + j] = lk[j];
        a.sidx[at + j] = li[j];
    }
}

/* ---------------------------------------------------------------- top-p over fine bins */

/* Tier 0 is summed without sorting it whole. The candidates (p bits and index, in any
 * order) fall into fine bins by their top bits: bin = (bits >> (51 - mb)) - (blo << mb),
 * a larger bin holding larger p, and the descending order is the bins from the top down,
 * each bin in its own order. The running sum c only needs that order inside a bin when
 * (a) c is 0 (the first entry sets c, the top bin), (b) the bin takes c out of its
 * binade [2^e, 2^(e+1)), (c) the bin takes c to top_p (from there the drop decisions
 * fl(c_j - p_j) >= top_p and the stop need each c_j), or (d) one of its p is halfway
 * between two multiples of u = 2^(e-52) (the tie goes to the even result, which depends
 * on c). Otherwise fl(c + p) = c + u RN(p / u) for each of its entries, whatever their
 * order, and every entry is kept (each c_j < top_p): the bin adds u times the sum of the
 * integers RN(p / u). The candidates are first bucketed by bin (a counting sort), so a
 * bin's entries are contiguous. A round walks the bins down from the current one in
 * chunks of whole bins of about TB_CHUNK entries: a prefix sum of RN(p / u) over the
 * chunk's entries in walk order finds the first bin that meets (b)-(d) (the bin of the
 * first entry whose running units reach top_p or leave the binade, or of a tie: the
 * units at a bin's last entry are those after the bin, whatever its order), adds the
 * bins above it in bulk (or the whole chunk, and goes on with the next), then sorts that
 * bin (p descending, index ascending: the stable descending argsort) and runs
 * chain_exact over it from c. Rounds continue down the bins until the chain stops
 * (c >= top_p (1 + 2^-48): the rest of the row is dropped) or tier 0 runs out (c carries
 * over to tier 1). Every p left is at most c (the top entry is summed first), so
 * p / u <= 2^53; the unsigned 64-bit prefix sums saturate at 2^60, past every test. */
constexpr int TB_NBIN = 2048;
static_assert(TB_NBIN == HBINS, "fine bins share the histogram's arrays");
constexpr int TB_PER = 8, TB_CHUNK = TB_PER * SP_T;
constexpr unsigned long long TB_FLAG = 1ull << 63, TB_SAT = 1ull << 60, TB_LIM = 1ull << 53;

struct TopPBins {
    int cnt[TB_NBIN];
    int off[TB_NBIN + 1];      /* bucket starts: bin b's entries are [off[b], off[b + 1]) */
    unsigned long long wpre[SP_WAVES];
    unsigned long long dpre;   /* units before the crossing bin (or after the chunk, when none) */
    int ib[4];                 /* [0] top bin, [2] crossing bin, [3] chunk's lowest bin */
};

__device__ __forceinline__ unsigned long long tb_sat_add(unsigned long long a, unsigned long long b) {
    const unsigned long long s = a + b;   /* a, b <= TB_SAT: no wrap */
    return s > TB_SAT ? TB_SAT : s;
}

/* the fine bins of tier 0 (bins >= blo of the histogram): bin = (bits >> sh) - bofs in
 * [0, nb), nb = (2048 - blo) 2^mb <= TB_NBIN */
__device__ __forceinline__ void fine_bins(int blo, int &mb, int &nb, int &sh, int &bofs) {
    mb = 0;
    while (mb < 7 && ((2048 - blo) << (mb + 1)) <= TB_NBIN) mb++;
    nb = (2048 - blo) << mb;
    sh = 51 - mb;
    bofs = blo << mb;
}

/* The candidates of tier 0 bucketed by fine bin (a counting sort), a workgroup per
 * TB_SLICE of a row's candidates: k_tp_count adds each slice's counts into the row's
 * bcnt; k_tp_scatter takes, per bin, its places after the bin's start with one global
 * atomic per slice and bin, and scatters the slice into skey2 / sidx2 (any order within a
 * bin: every use of a bin sums it or sorts it). */
constexpr int TB_SLICE = 8192;

__device__ __forceinline__ bool tp_slice(const SampleArgs &a, int v, int &j0, int &j1) {
    const int m = a.seg_end[v] - v * a.sort_n;
    j0 = blockIdx.x * TB_SLICE;
    j1 = m - j0 < TB_SLICE ? m : j0 + TB_SLICE;
    return j0 < m;
}

__device__ __forceinline__ void tp_count_slice(const SampleArgs &a, int v, int j0, int j1, int nb, int sh, int bofs,
                                               int *cnt) {
    for (int b = threadIdx.x; b < nb; b += SP_T) cnt[b] = 0;
    __syncthreads();
    const unsigned long long *key = a.skey + (size_t)v * a.sort_n + j0;
    row_pass(j1 - j0, [&](int j) { return key[j]; }, [&](int, unsigned long long k) {
        const int b = (int)(k >> sh) - bofs;   /* in [0, nb): 0 < p <= 1 in a bin >= blo */
        if (b >= 0 && b < nb) atomicAdd(&cnt[b], 1);
    });
    __syncthreads();
}

__global__ __launch_bounds__(SP_T) void k_tp_count(SampleArgs a) {
    __shared__ int cnt[TB_NBIN];
    const int v = blockIdx.y;
    if (a.live && v >= *a.live) return;   /* padding row (uniform) */
    int j0, j1;
    if (!tp_slice(a, v, j0, j1)) return;   /* (uniform) */
    const int bstar = a.bstar[v], blo = bstar < 0 ? 0 : bstar;
    int mb, nb, sh, bofs;
    fine_bins(blo, mb, nb, sh, bofs);
    tp_count_slice(a, v, j0, j1, nb, sh, bofs, cnt);
    int *g = a.bcnt + (size_t)v * HBINS;
    for (int b = threadIdx.x; b < nb; b += SP_T)
        if (cnt[b]) atomicAdd(&g[b], cnt[b]);
}

__global__ __launch_bounds__(SP_T) void k_tp_scatter(SampleArgs a) {
    __shared__ int cnt[TB_NBIN], cur[TB_NBIN];
    __shared__ int red[SP_WAVES];
    const int v = blockIdx.y, tid = threadIdx.x;
    if (a.live && v >= *a.live) return;
    int j0, j1;
    if (!tp_slice(a, v, j0, j1)) return;
    const int bstar = a.bstar[v], blo = bstar < 0 ? 0 : bstar;
    int mb, nb, sh, bofs;
    fine_bins(blo, mb, nb, sh, bofs);
    {
        /* bucket starts: the exclusive scan of the row's counts, bins ascending */
        const int *g = a.bcnt + (size_t)v * HBINS;
        const int b0 = 2 * tid, c0 = b0 < nb ? g[b0] : 0, c1 = b0 + 1 < nb ? g[b0 + 1] : 0;
        int total;
        const int o0 = wg_scan_excl(c0 + c1, red, &total);
        if (b0 < nb) cur[b0] = o0;
        if (b0 + 1 < nb) cur[b0 + 1] = o0 + c0;
    }
    tp_count_slice(a, v, j0, j1, nb, sh, bofs, cnt);
    int *rel = a.brel + (size_t)v * HBINS;
    for (int b = tid; b < nb; b += SP_T)
        if (cnt[b]) cur[b] += atomicAdd(&rel[b], cnt[b]);
    __syncthreads();
    const unsigned long long *key = a.skey + (size_t)v * a.sort_n + j0;
    const int *idx = a.sidx + (size_t)v * a.sort_n + j0;
    unsigned long long *bkey = a.skey2 + (size_t)v * a.sort_n;
    int *bidx = a.sidx2 + (size_t)v * a.sort_n;
    row_pass(j1 - j0, [&](int j) { return KeyIdx{key[j], idx[j]}; }, [&](int, KeyIdx e) {
        const int b = (int)(e.k >> sh) - bofs;
        if (b >= 0 && b < nb) {
            const int pos = atomicAdd(&cur[b], 1);
            bkey[pos] = e.k;
            bidx[pos] = e.i;
        }
    });
}

/* returns c after tier 0; stopped: the chain reached its stop (every later entry of the
 * row, below tier 0 included, is to be dropped; those of tier 0 are dropped here) */
__device__ double top_p_binned(const SampleArgs &a, int v, int blo, double top_p, double thr_hi, double *P,
                               unsigned char *smem, TopPBins &tb, ChainShared &cs, bool &stopped) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    /* the buckets (k_tp_scatter), in the second candidate arrays; the first ones hold the
     * sorts too large for LDS */
    const unsigned long long *bkey = a.skey2 + (size_t)v * a.sort_n;
    const int *bidx = a.sidx2 + (size_t)v * a.sort_n;
    int mb, nb, sh, bofs;
    fine_bins(blo, mb, nb, sh, bofs);
    if (tid == 0) tb.ib[0] = -1;
    {
        /* the bins' counts, their starts (bins ascending) and the top bin */
        const int *gcnt = a.bcnt + (size_t)v * HBINS;
        const int b0 = 2 * tid, c0 = b0 < nb ? gcnt[b0] : 0, c1 = b0 + 1 < nb ? gcnt[b0 + 1] : 0;
        int total;
        const int o0 = wg_scan_excl(c0 + c1, (int *)tb.wpre, &total);
        if (b0 < nb) { tb.cnt[b0] = c0; tb.off[b0] = o0; }
        if (b0 + 1 < nb) { tb.cnt[b0 + 1] = c1; tb.off[b0 + 1] = o0 + c0; }
        if (tid == 0) tb.off[nb] = total;
        if (c1 > 0) atomicMax(&tb.ib[0], b0 + 1);
        else if (c0 > 0) atomicMax(&tb.ib[0], b0);
        __syncthreads();
    }
    int cur = tb.ib[0];
    double c = 0.0;
    stopped = false;
    int stop_bin = -1;
    while (cur >= 0) {
        int bx = cur;   /* the bin summed entry by entry this round */
        if (c >= top_p) {
            /* every bin left is summed entry by entry: the next one that holds entries */
            while (bx >= 0 && tb.cnt[bx] == 0) bx--;
        } else if (c > 0.0) {
            int e = ilogb(c);
            if (e < -1022) e = -1022;
            const double u = ldexp(1.0, e - 52);
            unsigned long long D = (unsigned long long)(c / u);   /* exact: c is a multiple of u below 2^53 u */
            bx = -1;
            int top_b = cur;
            while (top_b >= 0) {
                /* the chunk [lo_b, top_b]: the lowest lo_b with at most TB_CHUNK entries in
                 * it, and at least the bin top_b (bucket starts ascend with the bin) */
                if (tid == 0) {
                    const int want = tb.off[top_b + 1] - TB_CHUNK;
                    int lo = 0, hi = top_b;   /* the smallest lo in [0, top_b] with off[lo] >= want */
                    while (lo < hi) {
                        const int mid = (lo + hi) >> 1;
                        if (tb.off[mid] >= want) hi = mid; else lo = mid + 1;
                    }
                    tb.ib[3] = lo;
                    tb.ib[2] = -1;
                }
                __syncthreads();
                const int lo_b = tb.ib[3];
                const int j0 = tb.off[lo_b], j1 = tb.off[top_b + 1];
                auto crosses = [&](unsigned long long after) {
                    return after >= TB_LIM || (double)after * u >= top_p;
                };
                /* the chunk's entries in the descending order of bins: walk position q is
                 * bucket entry j1 - 1 - q; thread t takes positions q0 + TB_PER t .. + TB_PER - 1
                 * of each block of TB_CHUNK (a chunk of one bin can hold more). The first
                 * position whose running units cross (or whose p is a tie) names the bin:
                 * the running units at a bin's last position are those after the bin. */
                const unsigned long long Dc = D;
                int bc = -1;
                for (int q0 = 0; q0 < j1 - j0 && bc < 0; q0 += TB_CHUNK) {
                    unsigned long long dk[TB_PER];
                    int bk[TB_PER];
                    bool tk[TB_PER];
                    unsigned long long tsum = 0ull;
#pragma unroll
                    for (int k = 0; k < TB_PER; k++) {
                        const int q = q0 + TB_PER * tid + k;
                        dk[k] = 0ull;
                        bk[k] = -1;
                        tk[k] = false;
                        if (q < j1 - j0) {
                            const unsigned long long key_q = bkey[j1 - 1 - q];
                            const double qv = ldexp(__longlong_as_double((long long)key_q), 52 - e);   /* p / u, exact */
                            const double f = floor(qv), r = qv - f;
                            bk[k] = (int)(key_q >> sh) - bofs;
                            tk[k] = r == 0.5;
                            dk[k] = (unsigned long long)f + (r > 0.5 ? 1ull : 0ull);
                        }
                        tsum = tb_sat_add(tsum, dk[k]);
                    }
                    unsigned long long inc = tsum;
                    for (int off = 1; off < 64; off <<= 1) {
                        const unsigned long long y = __shfl_up(inc, off, 64);
                        if (lane >= off) inc = tb_sat_add(inc, y);
                    }
                    if (lane == 63) tb.wpre[w] = inc;
                    __syncthreads();
                    unsigned long long excl = __shfl_up(inc, 1, 64);
                    excl = lane ? excl : 0ull;
                    for (int i = 0; i < w; i++) excl = tb_sat_add(excl, tb.wpre[i]);
                    excl = tb_sat_add(D, excl);   /* units before this thread's first position */
                    {
                        unsigned long long run = excl;
#pragma unroll
                        for (int k = 0; k < TB_PER; k++) {
                            if (bk[k] < 0) break;
                            run = tb_sat_add(run, dk[k]);
                            if (tk[k] || crosses(run)) {   /* bins descend along k: the first is the highest */
                                atomicMax(&tb.ib[2], bk[k]);
                                break;
                            }
                        }
                    }
                    __syncthreads();
                    bc = tb.ib[2];
                    if (bc >= 0) {
                        /* the units before bin bc's first position */
                        const int qs = j1 - tb.off[bc + 1] - q0;
                        if (qs < 0) {   /* a chunk of one bin, found in a later block */
                            if (tid == 0) tb.dpre = Dc;
                        } else if (qs >= TB_PER * tid && qs < TB_PER * (tid + 1)) {
                            unsigned long long run = excl;
#pragma unroll
                            for (int k = 0; k < TB_PER; k++)
                                if (k < qs - TB_PER * tid) run = tb_sat_add(run, dk[k]);
                            tb.dpre = run;
                        }
                    } else if (tid == SP_T - 1) {
                        unsigned long long run = excl;
#pragma unroll
                        for (int k = 0; k < TB_PER; k++) run = tb_sat_add(run, dk[k]);
                        tb.dpre = run;   /* the whole block */
                    }
                    __syncthreads();
                    D = tb.dpre;
                    __syncthreads();
                }
                if (bc >= 0) {
                    bx = bc;
                    break;
                }
                top_b = lo_b - 1;
            }
            c = (double)D * u;   /* below 2^53 u: exact */
        }
        if (bx < 0) break;   /* every bin left was added in bulk */
        const int n = tb.cnt[bx];
        if (n > 0) {
            int N = 1;
            while (N < n) N <<= 1;
            const bool in_lds = N <= SORT_LDS;
            unsigned long long *sk = in_lds ? (unsigned long long *)smem : a.skey + (size_t)v * a.sort_n;
            int *si = in_lds ? (int *)(smem + SORT_LDS * 8) : a.sidx + (size_t)v * a.sort_n;
            const int j0 = tb.off[bx];
            for (int j = tid; j < n; j += SP_T) {
                sk[j] = bkey[j0 + j];
                si[j] = bidx[j0 + j];
            }
            unsigned long long *ko = sk;   /* the sorted bin */
            int *io = si;
            if (n <= SP_T) {
                /* a small bin: each entry's place is the number of entries before it
                 * (the order is total: indices differ), counted by G neighbouring lanes
                 * over a G-th of the bin each, and written after the inputs */
                __syncthreads();
                int np2 = 1;
                while (np2 < n) np2 <<= 1;
                const int G = SP_T / np2 < 64 ? SP_T / np2 : 64;   /* a power of two */
                const int j = tid / G, part = tid % G;
                unsigned long long kj = 0ull;
                int ij = 0, r = 0;
                if (j < n) {
                    kj = sk[j];
                    ij = si[j];
#pragma unroll 4
                    for (int i = part; i < n; i += G) r += before(sk[i], si[i], kj, ij) ? 1 : 0;
                }
                for (int off = 1; off < G; off <<= 1) r += __shfl_xor(r, off, 64);
                if (j < n && part == 0) {
                    sk[SP_T + r] = kj;
                    si[SP_T + r] = ij;
                }
                ko = sk + SP_T;
                io = si + SP_T;
                __syncthreads();
            } else {
                for (int j = n + tid; j < N; j += SP_T) { sk[j] = 0ull; si[j] = INT_MAX; }
                __syncthreads();
                if (in_lds) bitonic_block(sk, si, N, 2, N, N, 0);
                else bitonic_global(sk, si, N, (unsigned long long *)smem, (int *)(smem + SORT_LDS * 8));
            }
            int stop;
            const double c_in = c;
            auto px = [&](int j) { return __longlong_as_double((long long)ko[j]); };
            auto drop = [&](int j, double cj) {
                if (dsub(cj, px(j)) >= top_p) P[io[j]] = 0.0;
            };
            if (c_in == 0.0) {
                c = chain_exact(px, n, thr_hi, &stop, drop, cs);
            } else {
                auto px1 = [&](int j) { return j == 0 ? c_in : px(j - 1); };
                auto drop1 = [&](int j, double cj) { if (j > 0) drop(j - 1, cj); };
                c = chain_exact(px1, n + 1, thr_hi, &stop, drop1, cs);
                stop = stop - 1;
            }
            for (int j = stop + 1 + tid; j < n; j += SP_T) P[io[j]] = 0.0;
            __syncthreads();
            if (stop < n) {
                stopped = true;
                stop_bin = bx;
                break;
            }
        }
        cur = bx - 1;
    }
    if (stopped) {
        /* the bins below the stop's: their entries are the buckets' first off[stop_bin] */
        const int j1 = tb.off[stop_bin];
        row_pass(j1, [&](int j) { return bidx[j]; }, [&](int, int i) { P[i] = 0.0; });
    }
    __syncthreads();
    return c;
}

/* the top-p tail of Sampler.probs on row v (after the candidates of tier 0 were gathered),
 * then min-p; row_rc[v] = 0 when done. Rows that finished in k_sample_probs have an
 * empty candidate segment and are left alone. */
__global__ __launch_bounds__(SP_T) void k_sample_top_p(SampleArgs a) {
    __shared__ __align__(16) unsigned char smem[SMEM];
    __shared__ RowShared rs;
    __shared__ ChainShared cs;
    __shared__ TopPBins tb;
    const int v = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (a.live && v >= *a.live) return;   /* padding row (uniform) */
    const int V = a.V;
    double *P = a.P + (size_t)v * V;
    double *lv = (double *)smem;
    if (a.seg_end[v] == v * a.sort_n) {   /* no top-p candidates: final (uniform) */
        if (tid == 0 && a.row_rc[v] == 1) a.row_rc[v] = 0;
        return;
    }
    double s;
    if (a.top_p < 1.0) {
        const double top_p = a.top_p, thr_hi = dmul(top_p, 1.0 + 0x1p-48);
        const int bstar = a.bstar[v];
        /* tier 0: bins >= b* (all nonzero entries when b* < 0), sorted by the radix sort;
         * tier 1: the rest, sorted here */
        double c = 0.0;
        bool done = false;
        int cut = 0;   /* entries of histogram bins below cut are dropped */
        for (int tier = 0; tier < 2 && !done; tier++) {
            const int blo = tier == 0 ? (bstar < 0 ? 0 : bstar) : 0;
            const int bhi = tier == 0 ? HBINS : bstar;
            if (blo >= bhi) break;
            int m;
            unsigned long long *key;
            int *idx;
            if (tier == 0) {
                m = a.seg_end[v] - v * a.sort_n;
                if (m == 0) continue;
                bool stopped;
                c = top_p_binned(a, v, blo, top_p, thr_hi, P, smem, tb, cs, stopped);
                if (stopped || c >= thr_hi) {
                    done = true;
                    cut = blo;
                    if (blo > 0 && !a.tail_wide)
                        row_pass(V, [&](int i) { return P[i]; }, [&](int i, double p) {
                            const int b = (int)((unsigned long long)__double_as_longlong(p) >> 51);
                            if (p > 0.0 && b < blo) P[i] = 0.0;
                        });
                }
                __syncthreads();
                continue;
            } else {
            /* count, then gather the tier's entries */
            int cnt = 0;
            row_pass(V, [&](int i) { return P[i]; }, [&](int, double p) {
                const int b = (int)((unsigned long long)__double_as_longlong(p) >> 51);
                cnt += (p > 0.0 && b >= blo && b < bhi) ? 1 : 0;
            });
            const int off0 = wg_scan_excl(cnt, rs.red_i, &m);
            (void)off0;
            if (m == 0) continue;
            int N = 1;
            while (N < m) N <<= 1;
            const bool in_lds = N <= SORT_LDS;
            key = in_lds ? (unsigned long long *)smem : a.skey + (size_t)v * a.sort_n;
            idx = in_lds ? (int *)(smem + SORT_LDS * 8) : a.sidx + (size_t)v * a.sort_n;
            if (tid == 0) rs.bi[3] = 0;
            __syncthreads();
            for (int i0 = 0; i0 < V; i0 += SP_T) {
                const int i = i0 + tid;
                const double p = i < V ? P[i] : 0.0;
                const int b = (int)((unsigned long long)__double_as_longlong(p) >> 51);
                const bool cand = i < V && p > 0.0 && b >= blo && b < bhi;
                const unsigned long long bal = __ballot(cand);
                int base = 0;
                if (lane == 0 && bal) base = atomicAdd(&rs.bi[3], __popcll(bal));
                base = __shfl(base, 0, 64);
                if (cand) {
                    const int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
                    key[pos] = (unsigned long long)__double_as_longlong(p);
                    idx[pos] = i;
                }
            }
            for (int j = m + tid; j < N; j += SP_T) { key[j] = 0ull; idx[j] = INT_MAX; }
            __syncthreads();
            if (in_lds) bitonic_block(key, idx, N, 2, N, N, 0);
            else bitonic_global(key, idx, N, (unsigned long long *)smem, (int *)(smem + SORT_LDS * 8));
            }
            if (m == 0) continue;
            /* the running sum over the entries in descending order, continuing from c;
             * entry j is dropped when fl(c_j - p_j) >= top_p; once c_j >= top_p (1 +
             * 2^-48), every later entry is dropped too (see above) */
            int stop;
            {
                const double c_in = c;
                auto px = [&](int j) { return __longlong_as_double((long long)key[j]); };
                auto drop = [&](int j, double cj) {
                    if (dsub(cj, px(j)) >= top_p) P[idx[j]] = 0.0;
                };
                if (c_in == 0.0) {
                    c = chain_exact(px, m, thr_hi, &stop, drop, cs);
                } else {
                    /* the chain continues from tier 0's end: prepend c as entry -1 */
                    auto px1 = [&](int j) { return j == 0 ? c_in : px(j - 1); };
                    auto drop1 = [&](int j, double cj) { if (j > 0) drop(j - 1, cj); };
                    c = chain_exact(px1, m + 1, thr_hi, &stop, drop1, cs);
                    stop = stop - 1;
                }
            }
            for (int j = stop + 1 + tid; j < m; j += SP_T) P[idx[j]] = 0.0;
            __syncthreads();
            if (stop < m || c >= thr_hi) {
                done = true;
                /* every entry below the tier is dropped */
                if (blo > 0)
                    row_pass(V, [&](int i) { return P[i]; }, [&](int i, double p) {
                        const int b = (int)((unsigned long long)__double_as_longlong(p) >> 51);
                        if (p > 0.0 && b < blo) P[i] = 0.0;
                    });
            }
            __syncthreads();
        }
        if (a.tail_wide) {   /* the cut and the renormalization: k_wide_tsum, k_wide_tdiv */
            if (tid == 0) a.tcut[v] = cut;
            return;
        }
        s = np_sum(P, V, a.tail, lv, rs.bd);
        row_pass(V, [&](int i) { return P[i]; }, [&](int i, double x) { P[i] = ddiv(x, s); });
    }
    if (a.min_p > 0.0) {
        double mp = -INF;
        __syncthreads();
        row_pass(V, [&](int i) { return P[i]; }, [&](int, double x) { mp = fmax(mp, x); });
        mp = wg_max(mp, rs.red_d);
        const double thr = dmul(a.min_p, mp);
        row_pass(V, [&](int i) { return P[i]; }, [&](int i, double x) { if (x < thr) P[i] = 0.0; });
        s = np_sum(P, V, a.tail, lv, rs.bd);
        row_pass(V, [&](int i) { return P[i]; }, [&](int i, double x) { P[i] = ddiv(x, s); });
    }
    if (tid == 0) a.row_rc[v] = 0;
}

/* top-p's renormalization spread like the distribution (rows whose top-p ran, without
 * min-p): k_wide_tsum drops the entries of histogram bins below the row's cut and takes
 * each buffer's pairwise sum, k_wide_tdiv divides by numpy's sum of the row */
__global__ __launch_bounds__(SP_T) void k_wide_tsum(SampleArgs a) {
    __shared__ double lv[128];
    __shared__ double bc;
    const int v = blockIdx.y, tid = threadIdx.x;
    if (a.live && v >= *a.live) return;
    if (a.seg_end[v] == v * a.sort_n) return;   /* no top-p candidates (uniform) */
    const int V = a.V;
    int r0, len;
    wide_range(V, r0, len);
    double *P = a.P + (size_t)v * V + r0;
    const int cut = a.tcut[v];
    if (cut > 0)
        row_pass(len, [&](int i) { return P[i]; }, [&](int i, double p) {
            const int b = (int)((unsigned long long)__double_as_longlong(p) >> 51);
            if (p > 0.0 && b < cut) P[i] = 0.0;
        });
    const double s = np_sum(P, len, a.tail, lv, &bc);
    if (tid == 0) a.wsum[(size_t)v * SAMPLE_WB + blockIdx.x] = s;
}

__global__ __launch_bounds__(SP_T) void k_wide_tdiv(SampleArgs a) {
    const int v = blockIdx.y;
    if (a.live && v >= *a.live) return;
    if (a.seg_end[v] == v * a.sort_n) return;
    const int V = a.V;
    int r0, len;
    wide_range(V, r0, len);
    double *P = a.P + (size_t)v * V + r0;
    double s = 0.0;
    for (int b = 0; b < (int)gridDim.x; b++) s = dadd(s, a.wsum[(size_t)v * SAMPLE_WB + b]);
    row_pass(len, [&](int i) { return P[i]; }, [&](int i, double x) { P[i] = ddiv(x, s); });
    if (blockIdx.x == 0 && threadIdx.x == 0) a.row_rc[v] = 0;
}

/* ---------------------------------------------------------------- the walk */

/* inverse-CDF draw from w[0..V) (unnormalised, nonnegative, not all zero) with
 * uniform u: np.cumsum order, first index whose running sum exceeds u * total. The chain
 * runs over w itself from its first nonzero entry (a zero adds +0.0, which changes no
 * running sum, so the sums at the nonzero entries are those of the nonzero entries
 * alone); the first sum above the target is at a nonzero entry, and when none is (u
 * close to 1) the last nonzero entry is drawn. */
/* ---------------------------------------------------------------- residuals, ahead of the walk */

/* The walk rejects the children of a node in index order; after child c of v is
 * rejected the next sibling is tried against r_c = max(d_prev - q_v, 0), d_prev being p_v
 * (first child) or the previous sibling's residual divided by its numpy sum, q_v the
 * point mass at c's token or v's draft distribution (generate.py:113-147 applied
 * recursively). None of this depends on the uniforms, so every child's residual is
 * computed before the walk, a launch per sibling rank (the ranks depend on each other
 * through the previous sibling's sum) and a workgroup per numpy buffer of each child:
 * the walk then reads one entry of a residual where it used to compute the whole row. */
__global__ void k_sib(SampleArgs a, int n) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    int prev = -1, rank = 0;
    if (c > 0) {
        const int v = a.parent[c];
        for (int j = 1; j < c; j++)
            if (a.parent[j] == v) { prev = j; rank++; }
    }
    a.sib_prev[c] = prev;
    a.sib_rank[c] = c > 0 ? rank : -1;
}

__global__ __launch_bounds__(SP_T) void k_resid(SampleArgs a, int rank) {
    __shared__ double lv[128];
    __shared__ double bc;
    const int c = blockIdx.y, tid = threadIdx.x;
    const int n = a.live ? *a.live : a.n;
    if (c >= n || a.sib_rank[c] != rank) return;   /* (uniform) */
    const int v = a.parent[c], prev = a.sib_prev[c];
    if (a.row_rc[v] != 0) return;   /* the walk stops at a bad row */
    const int V = a.V;
    int r0, len;
    wide_range(V, r0, len);
    double s = -1.0;   /* < 0: p_v itself */
    if (prev >= 0) {
        s = 0.0;
        for (int b = 0; b < (int)gridDim.x; b++) s = dadd(s, a.rsum[(size_t)prev * SAMPLE_WB + b]);
        if (s <= 0.0) return;   /* the walk accepts prev: c is never tried */
    }
    const double *src = (prev >= 0 ? a.R + (size_t)prev * V : a.P + (size_t)v * V) + r0;
    const double *qv = a.q ? a.q + (size_t)v * V + r0 : nullptr;
    const int x = a.tokens[c] - r0;
    double *dst = a.R + (size_t)c * V + r0;
    row_pass(len, [&](int i) { return make_double2(src[i], qv ? qv[i] : (i == x ? 1.0 : 0.0)); }, [&](int i, double2 pq) {
        const double pc = s < 0.0 ? pq.x : ddiv(pq.x, s);
        const double d = dsub(pc, pq.y);
        dst[i] = d > 0.0 ? d : 0.0;
    });
    const double bs = np_sum(dst, len, a.tail, lv, &bc);
    if (tid == 0) a.rsum[(size_t)c * SAMPLE_WB + blockIdx.x] = bs;
}

/* numpy's sum of residual c from its buffers' sums (0.0, then each in order) */
__device__ double resid_sum(const SampleArgs &a, int c) {
    const int nb = (a.V + NP_BUF - 1) / NP_BUF;
    double s = 0.0;
    for (int b = 0; b < nb; b++) s = dadd(s, a.rsum[(size_t)c * SAMPLE_WB + b]);
    return s;
}

__device__ int draw(const double *w, int V, double u, const SampleArgs &a, int *red, int *sh, ChainShared &cs) {
    const int tid = threadIdx.x, lane = tid & 63;
    (void)red;
    if (tid == 0) { sh[1] = INT_MAX; sh[2] = -1; }
    __syncthreads();
    {
        int lo = INT_MAX, hi = -1;
        row_pass(V, [&](int i) { return w[i]; }, [&](int i, double x) {
            if (x > 0.0) {
                lo = i < lo ? i : lo;
                hi = i > hi ? i : hi;
            }
        });
        for (int off = 32; off >= 1; off >>= 1) {
            const int ol = __shfl_xor(lo, off, 64), oh = __shfl_xor(hi, off, 64);
            lo = ol < lo ? ol : lo;
            hi = oh > hi ? oh : hi;
        }
        if (lane == 0) {
            if (lo != INT_MAX) atomicMin(&sh[1], lo);
            if (hi >= 0) atomicMax(&sh[2], hi);
        }
    }
    __syncthreads();
    const int j_first = sh[1], j_last = sh[2];
    if (j_last < 0) {   /* uniform: nothing to draw from */
        __syncthreads();
        return 0;
    }
    const int m = V - j_first, ng = (m + 7) / 8;
    int stop;
    /* the running sums are kept at the end of each group of 8 entries only (cc[g]): the
     * search finds the group, then runs the chain through it again */
    const double total = chain_exact<8>([&](int j) { return w[j_first + j]; }, m, INF, &stop,
                                        [&](int j, double cj) {
                                            if ((j & 7) == 7 || j == m - 1) a.cc[j >> 3] = cj;
                                        }, cs);
    if (tid == 0) sh[0] = INT_MAX;
    __syncthreads();
    const double target = dmul(u, total);
    {
        /* the first group whose last sum passes the target (the sums rise along the row);
         * a thread's first such group is its smallest */
        bool found = false;
        row_pass(ng, [&](int g) { return a.cc[g]; }, [&](int g, double cg) {
            if (!found && cg > target) { atomicMin(&sh[0], g); found = true; }
        });
    }
    __syncthreads();
    const int gb = sh[0];
    int jb = m;
    if (gb < ng) {   /* uniform */
        if (tid == 0) {
            /* the same adds from the sum before the group give the same sums */
            double c = gb > 0 ? a.cc[gb - 1] : 0.0;
            const int je = 8 * gb + 8 < m ? 8 * gb + 8 : m;
            int hit = je - 1;
            for (int j = 8 * gb; j < je; j++) {
                c = dadd(c, w[j_first + j]);
                if (c > target) { hit = j; break; }
            }
            sh[3] = hit;
        }
        __syncthreads();
        jb = sh[3];
    }
    const int r = jb < m ? j_first + jb : j_last;
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(SP_T) void k_sample_walk(SampleArgs a) {
    __shared__ int head[SAMPLE_NMAX], nxt[SAMPLE_NMAX];
    __shared__ int red[SP_WAVES];
    __shared__ int sh[4];
    __shared__ ChainShared cs;
    const int V = a.V, tid = threadIdx.x;
    const int n = a.live ? *a.live : a.n;   /* padding rows are not in the tree */
    for (int i = tid; i < n; i += SP_T) head[i] = -1;
    __syncthreads();
    if (tid == 0)
        for (int c = n - 1; c >= 1; c--) {
            const int pa = a.parent[c];
            nxt[c] = head[pa];
            head[pa] = c;
        }
    __syncthreads();
    int v = 0, np = 1, status = 0, fin = -1;
    if (tid == 0) a.path[0] = 0;
    for (;;) {
        if (a.row_rc[v] != 0) { status = -1; break; }
        const double *p = a.P + (size_t)v * V;
        const double *qv = a.q ? a.q + (size_t)v * V : nullptr;
        const double *r = nullptr;
        double s = -1.0;                       /* < 0: p itself is the current distribution */
        int next = -1;
        for (int c = head[v]; c >= 0; c = nxt[c]) {
            const int x = a.tokens[c];
            const double px = s < 0.0 ? p[x] : ddiv(r[x], s);
            const double ratio = ddiv(px, qv ? qv[x] : 1.0);
            if (a.u[2 * c] < ratio) { next = c; break; }
            /* the residual after c (k_resid) and its numpy sum */
            const double ns = resid_sum(a, c);
            if (ns <= 0.0) { next = c; break; }
            r = a.R + (size_t)c * V;
            s = ns;
        }
        if (next < 0) {
            fin = draw(s < 0.0 ? p : r, V, a.u[2 * v + 1], a, red, sh, cs);
            break;
        }
        if (tid == 0) a.path[np] = next;
        np++;
        v = next;
    }
    if (tid == 0) {
        a.result[0] = np;
        a.result[1] = fin;
        a.result[2] = status;
    }
}

} // namespace
} // namespace hxd

namespace hxl {

namespace {

int sort_len(int V) {
    int N = SORT_LDS;
    while (N < V) N <<= 1;
    return N;
}

/* numpy's pairwise tree of the last partial buffer (length V % 8192) */
void build_tail(int V, PwTail &t) {
    t = PwTail{};
    const int len = V % NP_BUF;
    t.len = len;
    if (len == 0) return;
    std::vector<std::pair<int, int>> ops[12];
    std::function<std::pair<int, int>(int, int)> rec = [&](int s, int n) -> std::pair<int, int> {
        if (n <= 128) {
            const int L = t.nleaf++;
            t.leaf_start[L] = (unsigned short)s;
            t.leaf_len[L] = (unsigned char)n;
            return {L, 0};
        }
        int n2 = n / 2;
        n2 -= n2 % 8;
        const auto A = rec(s, n2), B = rec(s + n2, n - n2);
        const int h = 1 + (A.second > B.second ? A.second : B.second);
        ops[h].push_back({A.first, B.first});
        return {A.first, h};
    };
    t.nlev = rec(0, len).second;
    int o = 0;
    t.lev_off[0] = 0;
    for (int h = 1; h <= t.nlev; h++) {
        for (const auto &op : ops[h]) {
            t.op_a[o] = (unsigned char)op.first;
            t.op_b[o] = (unsigned char)op.second;
            o++;
        }
        t.lev_off[h] = (unsigned char)o;
    }
}

template <class T> hipError_t grow(T *&p, size_t count) {
    if (p) (void)hipFree(p);
    p = nullptr;
    return hipMalloc((void **)&p, sizeof(T) * (count ? count : 1));
}

} // namespace

void SampleScratch::release() {
    void *ps[] = {P, q, u, cc, skey, skey2, sidx, sidx2, seg_begin, seg_end, bstar, row_rc, path,
                  result, ctx, tok, par, wmax, wsum, widx, wflag, whist, bcnt, brel, tcut, R, rsum, sib_prev, sib_rank};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    P = q = u = cc = wmax = wsum = R = rsum = nullptr;
    widx = wflag = bcnt = brel = tcut = sib_prev = sib_rank = nullptr;
    whist = nullptr;
    skey = skey2 = nullptr;
    sidx = sidx2 = seg_begin = seg_end = bstar = row_rc = path = result = ctx = tok = par = nullptr;
    n_cap = V = ctx_cap = sort_n = 0;
    has_q = false;
}

hipError_t SampleScratch::ensure(int n, int V_, bool need_q, int n_ctx) {
    hipError_t e = hipSuccess;
    if (V_ != V) {
        release();
        V = V_;
        sort_n = sort_len(V);
        if ((e = grow(cc, V)) ||
            (e = grow(result, 4)))
            return e;
    }
    if (n > n_cap) {
        const size_t rows = (size_t)n;
        if ((e = grow(P, rows * V)) || (e = grow(skey, rows * sort_n)) || (e = grow(sidx, rows * sort_n)) ||
            (e = grow(skey2, rows * sort_n)) || (e = grow(sidx2, rows * sort_n)) || (e = grow(seg_begin, rows)) ||
            (e = grow(seg_end, rows)) || (e = grow(bstar, rows)) || (e = grow(u, 2 * rows)) ||
            (e = grow(row_rc, rows)) || (e = grow(path, rows)) || (e = grow(tok, rows)) || (e = grow(par, rows)) ||
            (e = grow(wmax, rows * SAMPLE_WB)) || (e = grow(wsum, rows * SAMPLE_WB)) || (e = grow(widx, rows * SAMPLE_WB)) ||
            (e = grow(wflag, rows * SAMPLE_WB)) || (e = grow(whist, rows * SAMPLE_HBINS)) ||
            (e = grow(bcnt, rows * SAMPLE_HBINS)) || (e = grow(brel, rows * SAMPLE_HBINS)) || (e = grow(tcut, rows)) ||
            (e = grow(R, rows * V)) || (e = grow(rsum, rows * SAMPLE_WB)) || (e = grow(sib_prev, rows)) ||
            (e = grow(sib_rank, rows)))
            return e;
        if (has_q && (e = grow(q, rows * V))) return e;
        n_cap = n;
    }
    if (need_q && !has_q) {
        if ((e = grow(q, (size_t)n_cap * V))) return e;
        has_q = true;
    }
    if (n_ctx > ctx_cap) {
        if ((e = grow(ctx, (size_t)n_ctx))) return e;
        ctx_cap = n_ctx;
    }
    return hipSuccess;
}

namespace {

hipError_t make_args(SampleArgs &a, SampleScratch &m, const float *rows, int n, int V, const int *tok, const int *par,
                     const SamplerSpec &s, const double *q, const double *u, hipStream_t st, bool q_dev = false) {
    a = SampleArgs{};
    a.rows = rows; a.n = n; a.V = V; a.tokens = tok; a.parent = par;
    a.temperature = s.temperature; a.top_p = s.top_p; a.min_p = s.min_p; a.rp = s.rp; a.top_k = s.top_k;
    a.n_ctx = s.rp != 1.0 ? s.n_ctx : 0;
    a.ctx = m.ctx;
    a.q = q ? (q_dev ? q : m.q) : nullptr;   /* q_dev: the caller's device rows, read in place */
    a.u = m.u;
    a.P = m.P; a.skey = m.skey; a.sidx = m.sidx; a.skey2 = m.skey2; a.sidx2 = m.sidx2; a.sort_n = m.sort_n;
    a.seg_begin = m.seg_begin; a.seg_end = m.seg_end; a.bstar = m.bstar;
    a.cc = m.cc;
    a.row_rc = m.row_rc; a.path = m.path; a.result = m.result;
    a.wmax = m.wmax; a.wsum = m.wsum; a.widx = m.widx; a.wflag = m.wflag; a.whist = m.whist;
    a.bcnt = m.bcnt; a.brel = m.brel; a.tcut = m.tcut;
    a.R = m.R; a.rsum = m.rsum; a.sib_prev = m.sib_prev; a.sib_rank = m.sib_rank;
    build_tail(V, a.tail);
    hipError_t e = hipSuccess;
    if (q && !q_dev && (e = hipMemcpyAsync(m.q, q, sizeof(double) * (size_t)n * V, hipMemcpyHostToDevice, st)) != hipSuccess)
        return e;
    if (u && (e = hipMemcpyAsync(m.u, u, sizeof(double) * 2 * (size_t)n, hipMemcpyHostToDevice, st)) != hipSuccess) return e;
    if (a.n_ctx && (e = hipMemcpyAsync(m.ctx, s.ctx, sizeof(int) * (size_t)a.n_ctx, hipMemcpyHostToDevice, st)) != hipSuccess)
        return e;
    return hipSuccess;
}

/* Sampler.probs of n rows: the distribution and top-p candidates (a workgroup per numpy
 * buffer of each row; one per row with top-k, or min-p without top-p), then the top-p tail */
hipError_t probs(SampleScratch &, const SampleArgs &a0, int n, hipStream_t st) {
    SampleArgs a = a0;
    const bool wide = !(a.top_k > 0 && a.top_k < a.V) && !(a.top_p >= 1.0 && a.min_p > 0.0);
    a.tail_wide = wide && a.top_p < 1.0 && a.min_p == 0.0;
    const dim3 g((a.V + NP_BUF - 1) / NP_BUF, n), gs((a.V + TB_SLICE - 1) / TB_SLICE, n);
    if (wide) {
        k_wide_scan<<<g, SP_T, 0, st>>>(a);
        k_wide_exp<<<g, SP_T, 0, st>>>(a);
        k_wide_norm<<<g, SP_T, 0, st>>>(a);
        if (a.top_p < 1.0) k_wide_cand<<<g, SP_T, 0, st>>>(a);
    } else {
        k_sample_probs<<<n, SP_T, 0, st>>>(a);
    }
    if (a.top_p < 1.0) {
        k_tp_count<<<gs, SP_T, 0, st>>>(a);
        k_tp_scatter<<<gs, SP_T, 0, st>>>(a);
    }
    k_sample_top_p<<<n, SP_T, 0, st>>>(a);
    if (a.tail_wide) {
        k_wide_tsum<<<g, SP_T, 0, st>>>(a);
        k_wide_tdiv<<<g, SP_T, 0, st>>>(a);
    }
    return hipGetLastError();
}

} // namespace

/* the residuals of every child, ahead of the walk */
void residuals(const SampleArgs &a, int n, int max_sib, hipStream_t st) {
    if (n <= 1) return;
    if (max_sib < 0 || max_sib > n - 1) max_sib = n - 1;
    k_sib<<<(n + 255) / 256, 256, 0, st>>>(a, n);
    const dim3 g((a.V + NP_BUF - 1) / NP_BUF, n);
    for (int k = 0; k < max_sib; k++) k_resid<<<g, SP_T, 0, st>>>(a, k);
}

hipError_t accept_sample(SampleScratch &m, const float *rows, int n, int V, const int *tok, const int *par,
                         const SamplerSpec &s, const double *q, const double *u, hipStream_t st, bool q_dev,
                         int max_sib) {
    SampleArgs a;
    hipError_t e = make_args(a, m, rows, n, V, tok, par, s, q, u, st, q_dev);
    if (e != hipSuccess || (e = probs(m, a, n, st)) != hipSuccess) return e;
    residuals(a, n, max_sib, st);
    k_sample_walk<<<1, SP_T, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t accept_sample_dev(SampleScratch &m, const float *rows, int n, int V, const int *tok, const int *par,
                             const SamplerSpec &s, const int *ctx_dev, const int *n_ctx_dev, const int *live,
                             hipStream_t st) {
    SampleArgs a;
    SamplerSpec sp = s;
    sp.n_ctx = 0;   /* nothing to copy: the context is on the device */
    hipError_t e = make_args(a, m, rows, n, V, tok, par, sp, nullptr, nullptr, st);
    if (e != hipSuccess) return e;
    if (s.rp != 1.0) {
        a.ctx = ctx_dev;
        a.n_ctx_dev = n_ctx_dev;
    }
    a.live = live;
    if ((e = probs(m, a, n, st)) != hipSuccess) return e;
    residuals(a, n, 1, st);   /* the loop verifies a chain */
    k_sample_walk<<<1, SP_T, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t sample_probs(SampleScratch &m, const float *rows, int n, int V, const int *tok, const int *par,
                        const SamplerSpec &s, hipStream_t st) {
    SampleArgs a;
    const hipError_t e = make_args(a, m, rows, n, V, tok, par, s, nullptr, nullptr, st);
    return e != hipSuccess ? e : probs(m, a, n, st);
}

} // namespace hxl
