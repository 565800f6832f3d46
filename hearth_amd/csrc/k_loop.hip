/*
 * k_loop.hip — the speculative decoding loop on the device: the prompt-lookup
 * drafter (the reference's NgramIndex, python/hearth/generate.py:150-186) and the
 * commit of one verify step's tokens (the verify block, generate.py:365-392, and the
 * token loop of generate(), generate.py:292-400), so that a run of verify steps needs no
 * host round trip.
 *
 * One step is: k_loop_draft (the drafts, the forward's token ids and RoPE rows, and for a
 * sampled run the step's uniforms), the forward of T = k + 1 rows, the greedy or sampled
 * acceptance (accept_greedy, accept_sample_dev), k_loop_commit. T is
 * the same for every step of a run, so one captured graph serves them all. A step whose
 * draft is shorter than k fills the rows after it with the last token (a valid id for
 * the embedding) and gives those rows the comparison id -1, which no argmax equals, so
 * the greedy acceptance never walks into them (the sampled walk takes rows past the
 * draft as padding: LS_LIVE); the routing gives padding rows the experts of
 * row 0 (they load no expert of their own). Rows are causal, and every row's result is
 * independent of the batch it is computed in, so padding changes nothing in the rows
 * before it.
 *
 * Prompt lookup. The reference keeps, for every n-gram of length 1..max_n, the latest
 * start that is followed by at least one token, and proposes the tokens after the
 * latest earlier occurrence of the longest suffix that has one. Equivalently: for each
 * end e in [1, len - 1] (the n-gram hist[e - n, e) is followed by hist[e]), let m(e) be
 * the number of trailing tokens hist[e - m, e) that equal the sequence's last m tokens,
 * capped at max_n; the proposal follows the largest e among those with the largest
 * m(e) > 0, and is hist[e, min(e + k, len)). One workgroup scans every e and takes the
 * maximum of the key (m << 32) | e.
 */
#include "hx_launch.h"
#include "hx_loop.h"

namespace {

using namespace hxd;

__global__ __launch_bounds__(1024) void k_loop_draft(LoopArgs a) {
    __shared__ unsigned long long best_sh;
    const int tid = threadIdx.x;
    int *s = a.state;
    const int len = s[LS_LEN], ng = s[LS_NGRAM];
    /* draft length bound (generate.py advance: the token budget leaves room for the
     * step's own token); a finished run verifies its last token alone */
    int nmax = 0;
    if (s[LS_DONE] == LOOP_RUNNING) {
        const int left = s[LS_MAXNEW] - s[LS_NEW] - 1;
        nmax = a.T - 1 < left ? a.T - 1 : left;
    }
    /* RoPE rows of positions pos0 + i from the table (the engine checks that every step
     * of a run stays below the capacity; the clamp only keeps the read in the table);
     * first, so their loads overlap the lookup's */
    const int p = *a.pos;
    for (int idx = tid; idx < a.T * a.rope_dim; idx += blockDim.x) {
        const int i = idx / a.rope_dim, d = idx - i * a.rope_dim;
        const int r = p + i < a.cap ? p + i : a.cap - 1;
        a.rope[idx] = a.rtab[(size_t)r * a.rope_dim + d];
    }
    if (tid == 0) best_sh = 0ull;
    __syncthreads();
    if (nmax > 0 && ng > 0) {
        unsigned long long best = 0ull;
        const int *h = a.hist;
        for (int e = 1 + tid; e < len; e += blockDim.x) {
            int m = 0;
            while (m < ng && m < e && h[e - 1 - m] == h[len - 1 - m]) m++;
            const unsigned long long key = ((unsigned long long)m << 32) | (unsigned)e;
            if (m > 0 && key > best) best = key;
        }
        if (best) atomicMax(&best_sh, best);
    }
    __syncthreads();
    const unsigned long long best = best_sh;
    const int e0 = (int)(best & 0xffffffffull);
    const int nd = best ? (nmax < len - e0 ? nmax : len - e0) : 0;
    const int last = a.hist[len - 1];
    for (int i = tid; i < a.T; i += blockDim.x) {
        const int tk = i >= 1 && i <= nd ? a.hist[e0 + i - 1] : last;
        a.tokens[i] = tk;
        a.cmp[i] = i <= nd ? tk : -1;
    }
    if (tid == 0) {
        s[LS_ND] = nd;
        s[LS_LIVE] = nd + 1;
    }
    /* sampled runs: the step's uniforms from the run's stream r (from LS_UOFF on) in the
     * reference's order (generate.py:376-392: one per tried draft, then one for the draw
     * at the node where the walk ends), laid out for the sampled walk: u[2c] decides node
     * c, u[2v + 1] draws at node v -- so u[2c] = r[c - 1] (c = 1..nd), u[2v + 1] = r[v + 1]
     * (v < nd) and u[2 nd + 1] = r[nd]; a step uses at most nd + 1 of them */
    if (a.u) {
        const int o = s[LS_UOFF];
        auto r = [&](int i) { return a.ustream && o + i < a.ustream_n ? a.ustream[o + i] : 0.0; };
        for (int i = tid; i < 2 * a.T; i += blockDim.x) {
            const int c = i >> 1;
            double v = 0.0;
            if (!(i & 1)) {
                if (c >= 1 && c <= nd) v = r(c - 1);
            } else if (c <= nd) {
                v = r(c < nd ? c + 1 : nd);
            }
            a.u[i] = v;
        }
    }
}

__global__ void k_loop_commit(LoopArgs a) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    loop_commit_thread(a);
}

} // namespace

namespace hxl {

void loop_draft(const LoopArgs &a, hipStream_t st) { k_loop_draft<<<1, 1024, 0, st>>>(a); }

void loop_commit(const LoopArgs &a, hipStream_t st) { k_loop_commit<<<1, 64, 0, st>>>(a); }

} // namespace hxl
