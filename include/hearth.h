/*
 * hearth.h — C ABI of the MI355X verify engine (libhearth.so in hearth_amd/).
 *
 * Layout-compatible replacement for the reference engine's public header
 * (engine/include/hearth.h:1-164): every struct field, its order and type, every
 * enum value and every function signature is the same, so the reference's Python
 * package (python/hearth/engine.py:29-148, _native.py:84-153) drives this library
 * unchanged when HEARTH_LIB points at it. Compute runs on an AMD Instinct MI355X
 * (gfx950) through HIP; the host code only validates, schedules and copies.
 *
 * Differences in meaning (not in layout):
 *   - isa / hearth_cpu_isa: accepted and reported as before; the forward pass runs on
 *     the GPU whatever value is given. The GPU is chosen with HEARTH_DEVICE (default 0).
 *   - cache_gb: budget of the HBM expert cache when the routed experts do not all fit
 *     in HBM (else every expert is resident and cache_gb is ignored).
 *   - n_threads / n_io_threads / direct_io / policy / mirror_paths: accepted and
 *     validated as before; host threads only copy data.
 *
 * Thread-compatible: one engine handle must not be used by two threads at once
 * (reference hearth.h:10-12).
 */
#ifndef HEARTH_H
#define HEARTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HEARTH_API __attribute__((visibility("default")))

#define HEARTH_VERSION_MAJOR 0
#define HEARTH_VERSION_MINOR 1
#define HEARTH_VERSION_PATCH 0

/* dtypes, FORMAT.md §6 (reference hearth.h:40-44) */
enum {
    HEARTH_F32 = 0, HEARTH_F16 = 1, HEARTH_BF16 = 2,
    HEARTH_Q8 = 3, HEARTH_Q4 = 4, HEARTH_I32 = 5, HEARTH_U8 = 6
};

/* expert cache eviction policies (reference hearth.h:46-50) */
enum { HEARTH_POLICY_LRU = 0, HEARTH_POLICY_LFU = 1 };

/* prefetch modes (reference hearth.h:52-57) */
enum { HEARTH_PREFETCH_OFF = 0, HEARTH_PREFETCH_NEXT = 1, HEARTH_PREFETCH_SHARED = 2 };

/* ISA selection (reference hearth.h:59-60) */
enum { HEARTH_ISA_AUTO = 0, HEARTH_ISA_SCALAR = 1, HEARTH_ISA_AVX2 = 2, HEARTH_ISA_AVX512 = 3 };

typedef struct hearth_engine hearth_engine;

/* reference hearth.h:64-83 */
typedef struct hearth_options {
    const char *model_path;
    const char *mirror_paths[8];
    int n_mirrors;
    double cache_gb;
    int n_threads;
    int n_io_threads;
    int direct_io;
    int policy;
    int prefetch;
    int prefetch_extra;
    const char *usage_in;
    const char *usage_out;
    float pin_fraction;
    int warm_start;
    int max_seq;
    int max_batch;
    int isa;
    int verbose;
} hearth_options;

/* reference hearth.h:85-100 */
typedef struct hearth_model_info {
    char arch[32];
    int n_layers, d_model, vocab_size, max_seq;
    int n_heads, n_kv_heads, head_dim, attn_kind;
    int n_experts, top_k, expert_ffn_dim, n_moe_layers;
    int bos_id;
    int n_eos; int eos_ids[8];
    uint64_t dense_bytes;
    uint64_t expert_bytes;
    uint64_t slab_bytes_max;
    double params_total;
    double params_active;
    int cache_slots;
    int isa;
    int n_threads, n_io_threads;
} hearth_model_info;

/* reference hearth.h:102-116. The phase times attn_s / moe_s / dense_s are GPU time
 * measured with HIP events when profiling is on (hearth_gpu_set_profiling), else the
 * host time of the calls; stall_s is time spent waiting for expert copies. */
typedef struct hearth_stats {
    uint64_t tokens;
    uint64_t forward_calls;
    double   wall_s;
    double   attn_s, moe_s, dense_s, stall_s;
    uint64_t expert_uses;
    uint64_t expert_loads_unique;
    uint64_t cache_hits, cache_misses;
    uint64_t prefetch_issued, prefetch_used, prefetch_wasted;
    uint64_t bytes_read;
    double   read_s;
    uint64_t evictions;
    int      cache_slots, cache_resident, cache_pinned;
    uint64_t read_errors;
} hearth_stats;

/* ---- lifecycle (reference hearth.h:118-124) ------------------------------- */
HEARTH_API const char *hearth_version(void);
HEARTH_API void hearth_default_options(hearth_options *opt);
HEARTH_API hearth_engine *hearth_open(const hearth_options *opt, char *err, size_t errlen);
HEARTH_API void hearth_close(hearth_engine *e);
HEARTH_API int hearth_info(hearth_engine *e, hearth_model_info *out);

/* ---- evaluation (reference hearth.h:126-136) ------------------------------
 * tokens[0..n) at positions [pos, pos+n); logits NULL, [vocab] (all_logits 0) or
 * [n][vocab]. 0 on success, < 0 on error; a failed call changes nothing. */
HEARTH_API int hearth_eval(hearth_engine *e, const int32_t *tokens, int n, float *logits, int all_logits);
HEARTH_API int hearth_pos(hearth_engine *e);
HEARTH_API int hearth_reset(hearth_engine *e);
HEARTH_API int hearth_rewind(hearth_engine *e, int pos);

/* ---- telemetry (reference hearth.h:138-147) ------------------------------- */
HEARTH_API int hearth_get_stats(hearth_engine *e, hearth_stats *out);
HEARTH_API void hearth_reset_stats(hearth_engine *e);
HEARTH_API int hearth_trace_start(hearth_engine *e, const char *path);
HEARTH_API int hearth_trace_stop(hearth_engine *e);
HEARTH_API int hearth_route_replay(hearth_engine *e, const char *trace_path);

/* ---- quantization utilities (reference hearth.h:149-159) ------------------
 * hearth_matmul runs NUMERICS §3 on the GPU (the isa argument is validated only). */
HEARTH_API size_t hearth_row_bytes(int dtype, int64_t n_cols);
HEARTH_API int hearth_quantize(int dtype, const float *src, int64_t n_rows, int64_t n_cols, void *dst, int n_threads);
HEARTH_API int hearth_dequantize(int dtype, const void *src, int64_t n_rows, int64_t n_cols, float *dst);
HEARTH_API int hearth_matmul(int dtype, const void *W, int64_t n_rows, int64_t n_cols,
                             const float *X, int T, float *Y, int isa);
HEARTH_API int hearth_cpu_isa(void);

#ifdef __cplusplus
}
#endif
#endif /* HEARTH_H */
