/*
 * k_loop.hip — the speculative decoding loop on the device: the prompt-lookup
 * drafter (the reference's NgramIndex, python/hearth/generate.py:150-186) and the
 * commit of one verify step's tokens (the verify block, generate.py:365-392, and the
 * token loop of generate(), generate.py:292-400), so that a run of verify steps needs no
 * host round trip.
 *
 * A batch starts with k_loop_draft (the drafts, the forward's token ids and RoPE rows,
 * and for a sampled run the step's uniforms); one step is then the forward of T = k + 1
 * rows, the greedy or sampled acceptance, the commit and the next step's draft (in the
 * greedy walk's launch, accept_greedy_commit, or in k_loop_commit_draft after
 * accept_sample_dev; the draft after a batch's last step is unused and the next batch
 * drafts again). T is the same for every step of a run, so one captured graph serves
 * them all. A step whose
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

__global__ __launch_bounds__(1024) void k_loop_draft(LoopArgs a) { draft_body(a); }

/* a step's commit, then the next step's draft (the state the draft reads is the
 * committed one: the barrier orders thread 0's writes before it) */
__global__ __launch_bounds__(1024) void k_loop_commit_draft(LoopArgs a) {
    if (threadIdx.x == 0) loop_commit_thread(a);
    __syncthreads();
    draft_body(a);
}

} // namespace

namespace hxl {

void loop_draft(const LoopArgs &a, hipStream_t st) { k_loop_draft<<<1, 1024, 0, st>>>(a); }

void loop_commit_draft(const LoopArgs &a, hipStream_t st) { k_loop_commit_draft<<<1, 1024, 0, st>>>(a); }

} // namespace hxl
