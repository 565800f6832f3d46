/*
 * hx_oracle.h — CPU restatement of the reference engine's numerics, used as the
 * checker for the MI355X build.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load liboracle.so, and only as the checker or the timed
 * CPU baseline; the product library never links, loads or calls it.
 *
 * What each function restates (reference paths relative to the reference tree):
 *   ho_f16_to_f32 / ho_f32_to_f16   engine/src/platform_common.inc:19-65 (IEEE binary16, RNE)
 *   ho_exp_glibc_f                  the platform libm's expf the reference calls (glibc 2.35,
 *                                   sysdeps/ieee754/flt-32/e_expf.c; FMA build)
 *   ho_quantize (Q8, Q4)            engine/src/quant.c:99-228, docs/NUMERICS.md §6
 *   ho_act_quant                    engine/src/quant.c:325-348, docs/NUMERICS.md §2
 *   ho_matmul                       engine/src/quant.c:352-427, docs/NUMERICS.md §3
 *   ho_dot16 / ho_sum16 / rmsnorm / softmax / silu / sigmoid
 *                                   engine/src/quant.c:604-667, docs/NUMERICS.md §1, §4
 *   ho_open / ho_eval               engine/src/model.c:1171-1234 (forward), written as the
 *                                   single-token loop of engine/tests/test_model.c:788-1197
 *   ho_eval_tree / ho_commit_path   new (tree verification): node i runs at position
 *                                   pos0 + depth(i) and attends to the context followed by
 *                                   its ancestors in path order, i.e. exactly the chain
 *                                   root -> i; no reference counterpart
 *   ho_kv_export / ho_kv_import     the reference engine's cache layout (model.c, [Hkv][cap][hd]
 *                                   per K and V) cut to n positions; test plumbing, no arithmetic
 *   ho_probs / ho_accept_*          python/hearth/generate.py:84-147,365-392
 *
 * Exponential mode (ho_set_exp_mode):
 *   HO_EXP_LIBM      expf from the platform libm, as the reference calls it
 *                    (docs/NUMERICS.md "expf ... come from the platform libm");
 *                    with this mode the restatement is bit-exact to the reference
 *                    engine (checked against the reference built from source).
 *   HO_EXP_PORTABLE  ho_exp_port_f: Cody-Waite reduction + degree-13 Taylor in IEEE
 *                    double using only +, -, * and exact conversions (no FMA, no libm),
 *                    so it yields the same bits on any IEEE machine (within 1 ulp of libm).
 *   HO_EXP_GLIBC     ho_exp_glibc_f: glibc's expf (sysdeps/ieee754/flt-32/e_expf.c, the
 *                    x86-64 FMA build) restated with explicit fmas; equal to this image's
 *                    libm expf on all 2^32 inputs. The HIP kernels use the same
 *                    definition; with this mode the GPU must match the restatement bit
 *                    for bit, and so the reference engine.
 * Attention mode (ho_set_attn_mode):
 *   HO_ATTN_CANONICAL  the reference's order (engine/src/model.c:519-589): dot16 scores,
 *                      one softmax over the whole row list, sequential value sums.
 *   HO_ATTN_CHUNKED    the GPU engine's opt-in order for GQA attention (its default is the
 *                      canonical order): the row list in chunks of HO_ATTN_CHUNK rows, one partial softmax and value sum per
 *                      chunk, combined in chunk order (ho_set_attn_mode documents the exact
 *                      steps). Within the north star's tolerance of the reference, not
 *                      bit-exact to it; no reference counterpart (the reference allows a GPU
 *                      backend to document its tolerance, ADR-0003-canonical-numerics.md:44-45).
 *                      MLA attention keeps the canonical order in both modes.
 * Parity status: every function above is pinned (pinned FNV hashes of the reference's
 * test_quant.c, bit-exact comparison with the reference engine built from source on
 * whole forward passes, closed forms for acceptance); see tests/ for each check.
 */
#ifndef HX_ORACLE_H
#define HX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { HO_F32 = 0, HO_F16 = 1, HO_BF16 = 2, HO_Q8 = 3, HO_Q4 = 4, HO_I32 = 5, HO_U8 = 6 };
enum { HO_EXP_LIBM = 0, HO_EXP_PORTABLE = 1, HO_EXP_GLIBC = 2 };
enum { HO_ATTN_CANONICAL = 0, HO_ATTN_CHUNKED = 1, HO_ATTN_CHUNK = 64 };

/* ---- formats and kernels -------------------------------------------------- */
float    ho_f16_to_f32(uint16_t h);
uint16_t ho_f32_to_f16(float f);
uint16_t ho_f32_to_bf16(float f);
size_t   ho_row_bytes(int dtype, int64_t n);
int      ho_quantize(int dtype, const float *src, int64_t rows, int64_t cols, void *dst);
int      ho_dequantize(int dtype, const void *src, int64_t rows, int64_t cols, float *dst);
/* n % 64 == 0; out: n/64 blocks of { float d; int32 sum; int8 q[64] } (72 bytes) */
void     ho_act_quant(const float *x, int64_t n, void *out);
/* Y[t][r] = row r . X[t] per NUMERICS §3 (activation quantization inside). */
int      ho_matmul(int dtype, const void *W, int64_t rows, int64_t cols, const float *X, int T, float *Y);

/* ---- canonical helpers ---------------------------------------------------- */
void  ho_set_exp_mode(int mode);
int   ho_get_exp_mode(void);
float ho_expf(float x);                 /* in the current mode */
float ho_exp_port_f(float x);
float ho_exp_glibc_f(float x);
/* inputs u in [lo, hi) (float bit patterns) where ho_exp_glibc_f and the libm expf differ */
uint64_t ho_exp_glibc_mismatches(uint64_t lo, uint64_t hi, int nthreads);
double ho_exp_port_d(double x);
float ho_dot16(const float *a, const float *b, int64_t n);
/* Attention order of GQA layers (default HO_ATTN_CANONICAL). HO_ATTN_CHUNKED, for one
 * head with query q and the token's row list rows[0..nr) (logical row i reads K/V cache
 * slot rows[i]); chunk c holds logical rows 64c .. min(64c + 64, nr) - 1:
 *   s_i = scale * dotf(q, k_rows[i]), dotf = fmaf(a[d], b[d], acc) for d = 0 .. hd-1
 *         from acc = 0.0f
 *   m_c = max of s_i over the chunk (NaN if one of them is NaN)
 *   e_i = expf(s_i - m_c)                                  (ho_expf, the exp mode)
 *   l_c = pairwise sum of the chunk's 64 positions (e_i, 0.0f past row nr - 1): for
 *         w = 1, 2, 4, 8, 16, 32: a[k] = a[k] + a[k + w] for k = 0, 2w, 4w ..; l_c = a[0]
 *   o_c[d] = fmaf(e_i, v_rows[i][d], o) over the chunk's rows in order, from 0.0f
 *   M = max of m_c over the chunks; w_c = expf(m_c - M)
 *   L = fmaf(l_c, w_c, L) over c in order from 0.0f; O[d] the same with o_c[d]
 *   out[d] = O[d] / L
 * Every step depends on the row list only: batch == sequential and tree == chain hold
 * bit for bit in either mode. */
void  ho_set_attn_mode(int mode);
int   ho_get_attn_mode(void);
/* One head's attention in the current mode: query q [n], K and V rows at K + rows[i] *
 * stride and V + rows[i] * stride (n floats each) for i < nr; out [n]. The GQA layers'
 * per-head step, exposed for tests. Returns 0, -1 for bad arguments. */
int   ho_attn_head(const float *q, const float *K, const float *V, size_t stride, const int32_t *rows, int nr, int n,
                   float scale, float *out);
float ho_sum16(const float *a, int64_t n);

/* ---- model ---------------------------------------------------------------- */
typedef struct ho_model ho_model;
/* cap: KV capacity (0 = min(model max_seq, 4096)). Returns NULL with a message. */
ho_model *ho_open(const char *path, int cap, char *err, size_t errlen);
void      ho_close(ho_model *m);
/* out[0..]: n_layers, d_model, vocab, n_heads, n_kv_heads, head_dim, n_experts, top_k,
 * expert_ffn, n_moe_layers, cap, attn_kind */
void      ho_info(const ho_model *m, int *out);
int       ho_pos(const ho_model *m);
int       ho_rewind(ho_model *m, int pos);
/* Chain evaluation at positions pos..pos+n-1 (pos += n). logits [n][V] or NULL;
 * routes [n][n_moe][K] or NULL. Returns 0, or < 0 like hearth_eval. */
int       ho_eval(ho_model *m, const int32_t *tokens, int n, float *logits, int32_t *routes);
/* The next ho_eval / ho_eval_tree writes, for token i and MoE layer j, the routing margin
 * to buf[i * n_moe + j]: the smallest gap between consecutive selection scores among the
 * top K + 1, relative to the larger score for softmax scoring and absolute for sigmoid
 * scoring (the quantities the reference's synthetic models keep clear, python/hearth/
 * synth.py:171-186). Test instrumentation; buf must hold n * n_moe floats. */
void      ho_set_margins(ho_model *m, float *buf);
/* Tree evaluation: parent[0] = -1, parent[i] < i. Node i runs at pos + depth(i) and its
 * K/V go to slot pos + i. pos is left unchanged (ho_commit_path advances it). */
int       ho_eval_tree(ho_model *m, const int32_t *tokens, const int32_t *parent, int n,
                       float *logits, int32_t *routes);
/* Moves the K/V of nodes path[0..n) (path[j] at depth j) to slots pos..pos+n-1 and
 * sets pos += n. */
int       ho_commit_path(ho_model *m, const int32_t *path, int n);
/* Route replay (model.c:1004-1012): the token at position p takes the experts of trace
 * row p % rows for each MoE layer, weights from the router's scores. ids [rows][n_moe][K]
 * (the caller checks them); NULL turns replay off. Returns 0 or -5. */
int       ho_set_replay(ho_model *m, const uint16_t *ids, int64_t rows);
/* Sets the number of worker threads for the big matrix-vector products (>= 1). */
void      ho_set_threads(ho_model *m, int n);
/* Debug: append per-token intermediates (q, att, h_mid, x_ffn, router, ids, h) to
 * <dir>/l<layer>_<name>.bin ("" turns it off). */
void      ho_set_dump(ho_model *m, const char *dir);

/* KV snapshot of positions [0, n) of every layer, layer by layer: GQA K [Hkv][n][hd]
 * then V [Hkv][n][hd]; MLA latent c [n][C] then rotated k_pe [n][rope_dim] (the reference
 * engine's per-layer cache arrays cut to n positions). ho_kv_row_floats: floats per
 * position and layer. Import sets pos = n. Return 0 or -1. */
int64_t   ho_kv_row_floats(const ho_model *m);
int       ho_kv_export(const ho_model *m, int n, float *dst);
int       ho_kv_import(ho_model *m, int n, const float *src);

/* ---- acceptance ----------------------------------------------------------- */
/* Sampler settings (generate.py:31-56): temperature 0 = one-hot argmax; top_k 0 = off;
 * top_p 1 = off; min_p 0 = off; repetition_penalty 1 = off. context: the tokens the
 * penalty applies to (the committed sequence, normally ending with the verify root's
 * token); each node of a verify tree adds its path's draft tokens (nodes 1..v). */
typedef struct ho_sampler {
    double temperature;
    int top_k;
    double top_p;
    double min_p;
    double repetition_penalty;
    const int32_t *context;
    int n_context;
} ho_sampler;

/* numpy's float64 sum of a contiguous array, as `p.sum()` computes it in generate.py:
 * 0.0, then in order the pairwise sum (8 accumulators over blocks of at most 128) of
 * each 8192-element buffer. */
double ho_np_sum(const double *a, int64_t n);
/* Sampler.probs (generate.py:84-111) on one row of f32 logits: float64 result.
 * temperature 0 = one-hot argmax. Returns 0, or -1 for NaN/+inf/all -inf logits. */
int ho_probs(const float *logits, int V, double temperature, int top_k, double top_p, double min_p,
             double *p_out);
/* The same with the repetition penalty (Sampler._penalised, generate.py:68-79) over
 * s->context plus extra[0..n_extra). */
int ho_probs_s(const float *logits, int V, const ho_sampler *s, const int32_t *extra, int n_extra, double *p_out);
/* Greedy argmax, first index on ties; -1 on NaN/+inf/all -inf. */
int ho_argmax(const float *logits, int V);
/* Inverse-CDF draw (generate.py:113-121) with a given uniform u in [0,1). */
int ho_draw(const double *p, int V, double u);
/* Point-mass acceptance (generate.py:129-147): returns accepted(0/1), *tok. u0 decides,
 * u1 draws the residual. */
int ho_accept_point_mass(const double *p, int V, int d, double u0, double u1, int *tok);
/* Speculative sampling with a general draft distribution q: accept d with probability
 * min(1, p[d]/q[d]) (u0 < p[d]/q[d]); on rejection draw from max(0, p - q) normalised
 * (u1). Reduces to ho_accept_point_mass when q is one-hot on d. */
int ho_accept_general(const double *p, const double *q, int V, int d, double u0, double u1, int *tok);
/* Chain verification (generate.py:365-392): rows [k+1][V], drafts[k] (node i + 1 holds
 * draft i). mode 0 greedy, 1 point-mass sampling, 2 general q (q [k+1][V] float64, row
 * i = the distribution draft i was drawn from). Uniforms as for ho_accept_tree (2k + 2
 * entries). Writes n_acc and the final token; returns 0 or -1 (bad logits). */
int ho_accept_chain(const float *rows, int k, int V, const int32_t *drafts, int mode,
                    double temperature, int top_k, double top_p, double min_p,
                    const double *q, const double *u, int *n_acc, int *final_tok);
/* Tree verification: nodes 0..n-1 (parent[0] = -1, parent[i] < i), rows [n][V] are the
 * target logits at each node, tokens[i] the draft token of node i (node 0 = the last
 * committed token). Children of a node are tried in index order (recursive rejection
 * sampling, SpecInfer-style): accept child c with prob min(1, p[c.tok]/q_c[c.tok]); on
 * rejection p := norm(max(0, p - q_c)) and the next child is tried; if none is accepted
 * the correction is drawn from the current p. Greedy (mode 0): the child whose token is
 * argmax(p) is taken. q: [n][V] float64, row v = the draft distribution of v's children
 * (unused for greedy / point-mass). u: [2n] uniforms in [0, 1): u[2c] decides child c,
 * u[2v + 1] draws the token at node v (the correction, or the bonus at a leaf).
 * path_out gets the accepted node ids from the root (path_out[0] = 0), *n_path their
 * count, *final_tok the token that follows. */
int ho_accept_tree(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                   int mode, double temperature, int top_k, double top_p, double min_p,
                   const double *q, const double *u, int32_t *path_out, int *n_path, int *final_tok);
/* ho_accept_tree with a sampler (penalty included): point-mass mode when q is NULL,
 * general-q mode otherwise; temperature 0 gives the one-hot distribution. */
int ho_accept_tree_s(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                     const ho_sampler *s, const double *q, const double *u, int32_t *path_out, int *n_path,
                     int *final_tok);

#ifdef __cplusplus
}
#endif
#endif /* HX_ORACLE_H */
