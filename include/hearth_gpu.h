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

/* The acceptance kernel alone on caller logits (no engine): rows [n][V] f32. Same
 * result as hearth_verify_greedy's walk. Returns -1 for NaN/+inf/all -inf rows
 * (the reference Sampler raises for those, generate.py:69-79). */
HEARTH_API int hearth_gpu_accept_greedy(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                                        int32_t *path_out, int *n_path, int32_t *final_tok);

/* GPU time per kernel class, accumulated while profiling is on (HIP event pairs on the
 * engine's stream; see hearth_gpu_set_profiling for the levels). */
typedef struct hearth_gpu_kstats {
    double attn_s;        /* QKV projection, post-processing, attention, output projection */
    double router_s;      /* router logits + routing + bucketing */
    double expert_s;      /* grouped expert gate/up (one launch per MoE layer and expert dtype) */
    double norm_s;        /* residual, RMSNorm, activation quantization */
    double head_s;        /* lm_head */
    double dense_s;       /* dense FFN layers and shared experts */
    uint64_t expert_launches;   /* MoE layers run (gate/up launch groups) */
    uint64_t expert_bytes;      /* algorithmic weight bytes of the active experts' gate and up matrices */
    uint64_t dense_bytes;       /* algorithmic weight bytes of attention + lm_head matrices */
    uint64_t kv_bytes;          /* KV bytes read by attention (each row once per call and head group) */
    double expert_down_s;       /* SwiGLU activation quantization + grouped expert down projection */
    uint64_t expert_down_bytes; /* algorithmic weight bytes of the active experts' down matrices */
} hearth_gpu_kstats;

/* level 0: off; 1: HIP events around the grouped expert launches only (expert_s,
 * expert_down_s); 2: events around every launch group. Event pairs are recorded on the
 * engine's stream and read when a call completes. */
HEARTH_API int hearth_gpu_set_profiling(hearth_engine *e, int on);
HEARTH_API int hearth_gpu_get_kstats(hearth_engine *e, hearth_gpu_kstats *out);
HEARTH_API void hearth_gpu_reset_kstats(hearth_engine *e);

/* Device the library runs on (HEARTH_DEVICE, default 0) and its name. */
HEARTH_API int hearth_gpu_device(char *name, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* HEARTH_GPU_H */
