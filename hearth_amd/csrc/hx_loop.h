/*
 * hx_loop.h — the device loop's commit of one verify step, shared by k_loop_commit and
 * the greedy acceptance walk that commits in the same thread (k_loop.hip, k_layer.hip).
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

/* the commit by one thread (k_loop_commit, or the greedy walk's thread after the walk),
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

} // namespace hxd
