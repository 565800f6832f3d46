/*
 * hearth_gpu.h — extension entry points of the MI355X verify engine. None of these
 * has a counterpart in the reference ABI (engine/include/hearth.h); they follow its
 * conventions: 0 or a negative HX error code (-1 argument, -2 token id, -3 KV
 * capacity, -4 device/IO error, -5 memory), caller-owned buffers, and a failed call
 * changes nothing.
 *
 * Speculative verification (reference flow: python/hearth/generate.py:365-392, i.e.
 * hearth_eval([last] + draft, all_logits) -> acceptance -> hearth_rewind):
 *   tokens[0] is the last committed token (the one the reference feeds first),
 *   tokens[1..n) the draft. parent == NULL means a linear chain (parent[i] = i - 1);
 *   otherwise parent[0] = -1 and 0 <= parent[i] < i (a tree in topological order).
 *   Node i is evaluated at position pos + depth(i) and attends to the committed
 *   context followed by its ancestors, so every node's logits equal those of
 *   evaluating the chain root -> node with hearth_eval.
 */
#ifndef HEARTH_GPU_H
#define HEARTH_GPU_H

#include "hearth.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Evaluates a draft tree; node i's K/V go to KV slot pos + i. The position is left
 * unchanged until hearth_commit_path. logits: NULL or [n][vocab]. */
HEARTH_API int hearth_verify_tree(hearth_engine *e, const int32_t *tokens, const int32_t *parent, int n, float *logits);

/* Commits the accepted root path of the last hearth_verify_tree: path[j] is the node
 * at depth j (path[0] = 0). Its K/V move to slots pos .. pos+n-1 and pos += n. */
HEARTH_API int hearth_commit_path(hearth_engine *e, const int32_t *path, int n);

/* Greedy speculative verification in one call, acceptance on the GPU: evaluates the
 * chain or tree, walks from the root taking the child whose token equals the argmax
 * of its parent's logits (first index wins ties, first child wins), commits the
 * accepted path and writes it to path_out (path_out[0] = 0), its length to *n_path
 * and the token that follows it (the argmax at the last accepted node) to *final_tok.
 * After the call pos = old pos + *n_path, exactly as hearth_eval + generate.py's
 * acceptance + hearth_rewind(base + 1 + n_accepted). logits: NULL or [n][vocab]. */
HEARTH_API int hearth_verify_greedy(hearth_engine *e, const int32_t *tokens, const int32_t *parent, int n,
                                    int32_t *path_out, int *n_path, int32_t *final_tok, float *logits);

/* Greedy speculative decoding with the drafting on the device: replaces the loop of
 * the reference's generate() (python/hearth/generate.py:292-400) around its verify
 * block (365-392) with prompt-lookup drafts (NgramIndex, generate.py:150-186), for a
 * greedy sampler without a repetition penalty. Runs up to max_steps verify steps
 * without a host round trip per step: each proposes up to draft_len tokens that follow
 * the latest earlier occurrence of the longest suffix of at most ngram_n tokens
 * (ngram_n or draft_len 0: no drafts; the draft also leaves room in the token budget
 * for the step's own token), verifies [last] + draft, accepts greedily (as
 * hearth_verify_greedy) and handles the step's tokens as generate() does: each, in
 * order, ends the run if it is one of stop_ids (it is not committed), else is
 * committed, and the run ends once new_tokens reaches max_new.
 *
 * The engine must hold seq[0 .. n_seq - 2] (pos == n_seq - 1); new_tokens counts the
 * tokens already yielded (0 <= new_tokens < max_new). Every step evaluates
 * draft_len + 1 rows (rows past a shorter draft are padding), so only
 * (capacity - pos) / (draft_len + 1) steps fit: 0 of them returns -3 and the caller
 * finishes with hearth_verify_greedy and shorter drafts. out receives the tokens each
 * step handled (the accepted drafts, then the final token; a stop token that ended the
 * run included), at least max_steps * (draft_len + 1) entries; records[3 s ..] the
 * draft length, the drafts accepted and the tokens handled of step s (3 * max_steps
 * entries). Afterwards pos is the position generate() leaves: n_seq - 1 plus the
 * committed tokens, or at most the committed sequence's length once the run has ended.
 * Limits: draft_len + 1 <= min(max_batch, 128), n_stop <= 64, max_steps <= 1024.
 * Returns -1 for arguments outside them, and when the engine cannot run the loop
 * (expert streaming, route replay or a routing trace, profiling; see
 * hearth_gpu_spec_loop_ok). No counterpart in the reference's C API. */
#define HEARTH_GPU_SPEC_MAX_STEPS 1024
#define HEARTH_GPU_SPEC_RUNNING 0   /* max_steps ran (or the capacity ended them) */
#define HEARTH_GPU_SPEC_STOP 1      /* a stop token ended the run */
#define HEARTH_GPU_SPEC_LENGTH 2    /* the token budget ended the run */
#define HEARTH_GPU_SPEC_BAD 3       /* the step after the reported ones met a NaN/+inf/all -inf row */
typedef struct hearth_gpu_spec_result {
    int32_t n_out;      /* entries written to out */
    int32_t n_steps;    /* steps reported in records */
    int32_t finish;     /* HEARTH_GPU_SPEC_* */
    int32_t stop_id;    /* the stop token (finish STOP) */
    int32_t pos;        /* the engine position afterwards */
} hearth_gpu_spec_result;
HEARTH_API int hearth_gpu_spec_greedy(hearth_engine *e, const int32_t *seq, int n_seq, int new_tokens, int max_new,
                                      int draft_len, int ngram_n, const int32_t *stop_ids, int n_stop, int max_steps,
                                      int32_t *out, int32_t *records, hearth_gpu_spec_result *res);
/* 1 if the engine can run hearth_gpu_spec_greedy, else 0. */
HEARTH_API int hearth_gpu_spec_loop_ok(hearth_engine *e);

/* The acceptance kernel alone on caller logits (no engine): rows [n][V] f32. Same
 * result as hearth_verify_greedy's walk. Returns -1 for NaN/+inf/all -inf rows
 * (the reference Sampler raises for those, generate.py:69-79). */
HEARTH_API int hearth_gpu_accept_greedy(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                                        int32_t *path_out, int *n_path, int32_t *final_tok);

/* No counterpart in the reference. For callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops that forbid hipMalloc): the acceptance of
 * hearth_gpu_accept_greedy on the caller's DEVICE buffers, enqueued on `stream` (a
 * hipStream_t of the current device; NULL = the null stream) without waiting for it.
 * rows [n][V] f32, tokens [n], parent [n] or NULL for a chain; results land in path_out
 * [n] (accepted nodes from the root) and result [3] = {path length, final token,
 * status: 0, or -1 for NaN/+inf/all -inf rows}. The kernels' scratch is a fixed array
 * of HEARTH_GPU_NOALLOC_MAX_ROWS rows (392 KiB) in the library, one per GPU, held until
 * the process ends: the call allocates nothing, and calls that overlap on one GPU race
 * on it. Returns 0, -1 for bad arguments, -3 when n exceeds the limit, -4 for a
 * device error of this call's launches, or -4 without launching when the calling thread
 * holds a HIP error it has not read yet (that error is left for the caller); parent
 * entries are not checked (any values give a bounded walk). */
#define HEARTH_GPU_NOALLOC_MAX_ROWS 1024
HEARTH_API int hearth_gpu_accept_greedy_noalloc(const float *rows, int n, int V, const int32_t *tokens,
                                                const int32_t *parent, int32_t *path_out, int32_t *result,
                                                void *stream);

/* Sampler settings of sampled acceptance: the fields of the reference's Sampler
 * (python/hearth/generate.py:31-56) with its validation. temperature 0 gives the one-hot
 * argmax distribution; top_k 0, top_p 1, min_p 0 and repetition_penalty 1 are "off".
 * The penalty applies to the distinct ids of context[0..n_context) (normally the
 * committed sequence, ending with tokens[0]) plus, for node v, the draft tokens of the
 * path nodes 1..v (generate.py:380: full[:len(seq) + i]). */
typedef struct hearth_sampler {
    double temperature;
    int32_t top_k;
    double top_p;
    double min_p;
    double repetition_penalty;
    const int32_t *context;
    int32_t n_context;
} hearth_sampler;

/* Sampled speculative verification in one call, acceptance on the GPU in float64 with
 * the reference's operation order (Sampler.probs, accept_point_mass, draw;
 * generate.py:84-147,365-392). Children of a node are tried in index order: child c
 * (token x) is accepted when u[2c] < p_cur[x] / q_v[x], where p_cur is the node's
 * distribution, after each rejected child replaced by max(0, p_cur - q_v) renormalised;
 * if no child is accepted the next token is drawn from p_cur by inverse CDF with
 * u[2v + 1]. q == NULL: every draft is a point mass (q_v = one-hot of the child's token,
 * the reference's case); otherwise q is [n][V] float64 and row v is the distribution
 * v's children were drafted from. u: [2n] uniforms in [0, 1). For a chain, the
 * reference's random stream r0, r1, ... maps to u[2c] = r[c-1] (c = 1..k),
 * u[2v+1] = r[v+1] (v < k) and u[2k+1] = r[k]. Commits the accepted path like
 * hearth_verify_greedy. Returns -1 for bad settings or when a visited row has
 * NaN/+inf/only -inf logits (the reference raises ValueError there). V <= 262144,
 * n <= 4096. logits: NULL or [n][vocab]. */
HEARTH_API int hearth_verify_sample(hearth_engine *e, const int32_t *tokens, const int32_t *parent, int n,
                                    const hearth_sampler *s, const double *q, const double *u, int32_t *path_out,
                                    int *n_path, int32_t *final_tok, float *logits);

/* hearth_verify_sample with the draft distributions q_dev [n][V] float64 already in the
 * engine GPU's memory (hearth_gpu_malloc / hearth_gpu_upload, or a draft model's output
 * on the same device): read in place, so a step moves no q bytes over the host link.
 * -1 also when q_dev is not device memory of the engine's GPU. The reference's
 * hearth_verify_sample (hearth.h) takes q in host memory only. */
HEARTH_API int hearth_gpu_verify_sample_dq(hearth_engine *e, const int32_t *tokens, const int32_t *parent, int n,
                                           const hearth_sampler *s, const double *q_dev, const double *u,
                                           int32_t *path_out, int *n_path, int32_t *final_tok, float *logits);

/* Device memory on the engine's GPU for inputs such as q_dev: NULL on failure; upload
 * copies host bytes into it after the engine's queued work; free releases it (NULL is
 * allowed). No counterpart in the reference (its engine has no device). */
HEARTH_API void *hearth_gpu_malloc(hearth_engine *e, size_t bytes);
HEARTH_API int hearth_gpu_upload(hearth_engine *e, void *dst, const void *src, size_t bytes);
HEARTH_API int hearth_gpu_free(hearth_engine *e, void *p);

/* The sampled acceptance alone on caller logits rows [n][V] (no engine); same result as
 * hearth_verify_sample's walk. */
HEARTH_API int hearth_gpu_accept_sample(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                                        const hearth_sampler *s, const double *q, const double *u,
                                        int32_t *path_out, int *n_path, int32_t *final_tok);

/* Sampler.probs on the GPU for every row of caller logits rows [n][V] (float64 result
 * p_out [n][V], the distributions hearth_gpu_accept_sample works with). The penalty
 * context of row v is s->context plus the tokens of the path nodes 1..v of the tree
 * given by tokens/parent (parent NULL: chain). Returns -1 if a row has NaN/+inf/only
 * -inf logits. */
HEARTH_API int hearth_gpu_probs(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                                const hearth_sampler *s, double *p_out);

/* The loop of hearth_gpu_spec_greedy with sampled acceptance (hearth_verify_sample's
 * walk over each step's chain, the Sampler smp; its penalty context is the committed
 * sequence, so smp->context is not read). A positive temperature draws from the run's
 * random stream uniforms[0 .. n_uniforms), at least max_steps * (draft_len + 1) values,
 * in the reference's order (generate.py:376-392: one per tried draft, then one for the
 * draw where the walk ends; step after step); *n_used reports how many the run consumed,
 * so the caller's generator can be advanced by exactly that many. Temperature 0 (a
 * penalised argmax) reads no uniforms (uniforms may be NULL) and reports 0. Same
 * arguments, results and limits as hearth_gpu_spec_greedy otherwise, plus the sampled
 * acceptance's (draft_len + 1 <= 128, vocabulary within its limit); -1 also for a
 * sampler that hearth_verify_sample would reject. No counterpart in the reference's C
 * API (the reference draws its uniforms on the host, step by step). */
HEARTH_API int hearth_gpu_spec_sample(hearth_engine *e, const int32_t *seq, int n_seq, int new_tokens, int max_new,
                                      int draft_len, int ngram_n, const int32_t *stop_ids, int n_stop, int max_steps,
                                      const hearth_sampler *smp, const double *uniforms, int n_uniforms, int32_t *out,
                                      int32_t *records, hearth_gpu_spec_result *res, int *n_used);

/* Attention order of the engine's GQA layers. No counterpart in the reference, whose
 * ADR-0003-canonical-numerics.md:44-45 lets a GPU backend document its tolerance:
 *   HEARTH_GPU_ATTN_CANONICAL  the reference's order (engine/src/model.c:519-589): dot16
 *                              scores, one softmax over the row list, sequential value
 *                              sums; logits bit-exact to the reference engine.
 *   HEARTH_GPU_ATTN_CHUNKED    the row list in chunks of 64 rows, scores and value sums by
 *                              fused multiply-adds, one partial softmax per chunk, chunks
 *                              folded in order (oracle/hx_oracle.h lists the exact steps).
 *                              Each head's output is within about 1e-6 of the canonical one,
 *                              but models that quantize activations to int8 amplify that:
 *                              it is an opt-in order with a measured, not a guaranteed,
 *                              agreement with the reference.
 * Either order depends on a token's row list only, so batch == sequential and tree ==
 * chain hold bit for bit in both. Default: canonical; HEARTH_GPU_ATTN=chunked at open
 * selects the chunked order where the shape allows it (GQA with head_dim 64 or 128).
 * MLA attention is canonical in both modes. set returns -1 for an unknown mode or a
 * model the chunked order does not cover; call it between calls that use the engine.
 * get returns the order in use. */
#define HEARTH_GPU_ATTN_CANONICAL 0
#define HEARTH_GPU_ATTN_CHUNKED 1
HEARTH_API int hearth_gpu_set_attn_mode(hearth_engine *e, int mode);
HEARTH_API int hearth_gpu_get_attn_mode(hearth_engine *e);

/* GPU time per kernel class, accumulated while profiling is on (HIP event pairs on the
 * engine's stream; see hearth_gpu_set_profiling for the levels). */
typedef struct hearth_gpu_kstats {
    double attn_s;        /* q/k post-processing and RoPE, scores, softmax, value sum (MLA: latent post
                           * step, absorbed queries, RoPE scores) */
    double router_s;      /* router logits + routing + bucketing */
    double expert_s;      /* grouped expert gate/up (one launch per MoE layer and expert dtype) */
    double norm_s;        /* residual, RMSNorm, activation quantization */
    double head_s;        /* lm_head */
    double dense_s;       /* dense FFN layers and shared experts */
    uint64_t expert_launches;   /* MoE layers run (gate/up launch groups) */
    uint64_t expert_bytes;      /* algorithmic weight bytes of the active experts' gate and up matrices */
    uint64_t dense_bytes;       /* algorithmic weight bytes of the attention projections, dense FFN and
                                 * shared-expert matrices and the lm_head read by the profiled forwards */
    uint64_t kv_bytes;          /* KV bytes read by attention (each row once per call and head group) */
    double expert_down_s;       /* SwiGLU activation quantization + grouped expert down projection */
    uint64_t expert_down_bytes; /* algorithmic weight bytes of the active experts' down matrices */
    double accept_s;            /* device acceptance (greedy argmax + walk, or sampled) */
    double proj_s;              /* attention projections: q, k, v, o (MLA: q_a, q_b, kv_a, W_UV per head, o) */
} hearth_gpu_kstats;

/* level 0: off; 1: HIP events around the grouped expert launches only (expert_s,
 * expert_down_s); 2: events around every launch group. Event pairs are recorded on the
 * engine's stream and read when a call completes. */
HEARTH_API int hearth_gpu_set_profiling(hearth_engine *e, int on);
HEARTH_API int hearth_gpu_get_kstats(hearth_engine *e, hearth_gpu_kstats *out);
HEARTH_API void hearth_gpu_reset_kstats(hearth_engine *e);

/* KV-cache snapshot of positions [0, n) (a conversation to resume later, or a context
 * computed elsewhere). Layout, every layer in turn: GQA K [n_kv_heads][n][head_dim] then
 * V [n_kv_heads][n][head_dim]; MLA latent c [n][kv_lora] then rotated k_pe [n][rope_dim]
 * (the reference engine's per-layer cache arrays, engine/src/model.c, cut to n
 * positions). hearth_gpu_kv_row_floats: floats per position and layer, so a snapshot
 * holds n_layers * n * that many floats. Export needs n <= pos; import needs
 * n <= the KV capacity, writes the rows and sets pos = n (the rows past n are left as
 * they were). `count` is the buffer's size in floats. */
HEARTH_API int64_t hearth_gpu_kv_row_floats(hearth_engine *e);
HEARTH_API int hearth_gpu_kv_export(hearth_engine *e, int n, float *dst, int64_t count);
HEARTH_API int hearth_gpu_kv_import(hearth_engine *e, int n, const float *src, int64_t count);

/* The HBM expert cache of an engine. streamed 0: every routed expert is resident in
 * HBM (the other fields are 0). streamed 1: experts are loaded into `slots` HBM slots of
 * `slot_bytes` each when a layer demands them (or ahead of it, prefetch); host_tier 1:
 * a load is one copy of a slot image kept in pinned host memory (host_tier_bytes in all,
 * one image per physical slab of the container), 0: a load stages the container's slab
 * and repacks it on the device. copy_s: time the copy stream spent on load batches since
 * the engine opened (HIP events around the loads of each layer's demand and of each
 * prefetch; bytes_read of hearth_get_stats / copy_s is the host-link rate). No
 * counterpart in the reference (its store, engine/src/store.c, has no device tier). */
typedef struct hearth_gpu_store_info {
    int32_t streamed;
    int32_t host_tier;
    int64_t slots;
    uint64_t slot_bytes;
    uint64_t host_tier_bytes;
    double copy_s;
} hearth_gpu_store_info;

HEARTH_API int hearth_gpu_get_store_info(hearth_engine *e, hearth_gpu_store_info *out);

/* Device the library runs on (HEARTH_DEVICE, default 0) and its name. */
HEARTH_API int hearth_gpu_device(char *name, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* HEARTH_GPU_H */
