/*
 * hx_loop.h — the device loop's commit of one verify step and the prompt-lookup draft
 * of the next, shared by k_loop_draft / k_loop_commit_draft (k_loop.hip) and the greedy
 * acceptance walk that commits and drafts in the same launch (k_layer.hip).
 */
#pragma once
#include "hx_launch.h"

namespace hxd {

/* The step's tokens in order: the accepted drafts, then the final token; each is
 * checked against the stop ids (a stop token ends the run and is not committed), then
 * committed, and the run ends when the token budget is spent (generate(), generate.py
 * 292-400). The engine position becomes pos0 + n_path (the accepted path's KV); a
 * finished run keeps at most the committed tokens' KV (generate()'s release rewinds to
 * them). */
__device__ inline void commit_step(const LoopArgs &a) {
    int *s = a.state;
    const int p = *a.pos;
    if (a.result[2] != 0) {   /* a row with a NaN or +inf, or only -inf: the step fails */
        s[LS_DONE] = LOOP_BAD;
        s[LS_KVPOS] = p;
        return;
    }
    const int np = a.result[0], fin = a.result[1], nacc = np - 1, nstop = s[LS_NSTOP];
    int len = s[LS_LEN], nw = s[LS_NEW], nout = s[LS_NOUT], done = LOOP_RUNNING, handled = 0;
    for (int j = 0; j <= nacc; j++) {
        const int tok = j < nacc ? a.tokens[1 + j] : fin;
        if (nout < a.out_cap) a.out[nout] = tok;
        nout++;
        handled++;
        bool stop = false;
        for (int q = 0; q < nstop; q++) stop = stop || a.stops[q] == tok;
        if (stop) {
            done = LOOP_STOP;
            s[LS_STOP] = tok;
            break;
        }
        if (len < a.hist_cap) a.hist[len] = tok;
        len++;
        nw++;
        if (nw >= s[LS_MAXNEW]) {
            done = LOOP_LENGTH;
            break;
        }
    }
    /* uniforms the sampled walk used: one per tried draft (accepted ones and the first
     * rejected one), one for the final draw */
    if (a.sampled) s[LS_UOFF] += nacc + 1 + (nacc < s[LS_ND] ? 1 : 0);
    const int step = s[LS_STEP];
    if (step < a.rec_cap) {
        a.rec[3 * step] = s[LS_ND];
        a.rec[3 * step + 1] = nacc;
        a.rec[3 * step + 2] = handled;
    }
    int kv = p + np;
    if (done != LOOP_RUNNING && kv > len) kv = len;
    s[LS_STEP] = step + 1;
    s[LS_LEN] = len;
    s[LS_NEW] = nw;
    s[LS_NOUT] = nout;
    s[LS_DONE] = done;
    s[LS_KVPOS] = kv;
    *a.pos = kv;
}

/* the commit by one thread (k_loop_commit_draft, or the greedy walk's thread after the walk),
 * then (LS_NEW, LS_DONE) to the host flags */
__device__ inline void loop_commit_thread(const LoopArgs &a) {
    int *s = a.state;
    const int bs = s[LS_BSTEP];
    s[LS_BSTEP] = bs + 1;
    if (s[LS_DONE] == LOOP_RUNNING) commit_step(a);
    if (a.hflag) {
        a.hflag[2 * (bs & 1)] = s[LS_NEW];
        a.hflag[2 * (bs & 1) + 1] = s[LS_DONE];
    }
}

/* the draft of the next step, by every thread of the workgroup */
__device__ inline void draft_body(const LoopArgs &a) {
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

} // namespace hxd
