/*
 * hx_launch.h — kernel argument blocks and host-side launchers of the verify step.
 * Every launcher only enqueues work on the given stream; shapes are checked by the
 * engine before any launch (engine.cpp).
 */
#pragma once

#include "hx_device.h"

#include <vector>

namespace hxd {

struct GemmSeg {
    QMat m;
    float *Y;          /* Y[t * ldy + row] */
    int ldy;
    int scale_on;      /* 1: y = canon(scale * canon(acc)) (logit_scale) */
    float scale;
    int wg0;           /* first workgroup of the segment (set by the launcher) */
};

struct GemmArgs {
    GemmSeg seg[4];
    int nseg;
    Act a;             /* activations of tokens [0, T) */
    int T, t0;
    /* device [1] or null: tokens t >= *live are padding, whose output rows the split-K
     * product leaves unwritten (nothing reads them) */
    const int *live;
};

struct ExpertW { QMat gate, up, down; };

/* One active expert slot of a routed batch, written by the bucketing step: the expert's
 * matrices, its first pair and its pair count (n = 0: slot unused). */
struct SlotDesc {
    ExpertW w;
    int p0, n, e, pad;
};

struct MoeArgs {
    const ExpertW *table;     /* [n_experts] of this layer */
    const SlotDesc *desc;     /* [n_slots] active expert slots */
    const int *n_active;      /* number of active experts (device scalar) */
    const int *ulist, *u_p0, *u_n;
    const int *pair_tok;      /* pair -> token */
    Act x;                    /* normalized token activations [T] */
    Act mid;                  /* SwiGLU activations per pair [P] */
    float *midf;              /* SwiGLU activations per pair before quantization, f32 [P][F] */
    float *Y;                 /* expert outputs [P][D] */
    int T, F, D;
    int P;                    /* pairs: T * top_k */
    int dtype_mask;           /* bit dt set when some expert of the layer has dtype dt */
    int head_slots;           /* 1: slot u is table[u] for pairs [u * T, u * T + T) (MLA W_UV per head) */
};

/* Routing (NUMERICS §5.3) of T tokens from router logits. */
struct RouteArgs {
    const float *logits;      /* [T][E] */
    const float *bias;        /* [E] or null */
    int T, E, K, score_fn, n_group, topk_group, norm_topk;
    float routed_scale;
    int *ids;                 /* [T][K] */
    float *wts;               /* [T][K] */
    int *n_active, *ulist, *u_p0, *u_n, *pair_tok, *pair_of;
    int *route_out;           /* [T][n_moe][K] or null */
    int moe_ord, n_moe;
    unsigned long long *stats;   /* [0] expert uses, [1] unique expert loads */
    const ExpertW *table;     /* [E] expert matrices of the layer */
    SlotDesc *desc;           /* [n_slots] out: active slots, then n = 0 */
    int n_slots;
    /* route replay (model.c:1004-1012): token t takes the experts of trace row
     * (pos0 + depth[t]) % replay_rows, this MoE layer's K entries; null = routing */
    const int *replay;        /* [replay_rows][n_moe][K] */
    long long replay_rows;
    int pos0;
    const int *depth;         /* [T] */
    /* device [1] or null: tokens t >= *live are padding and take the experts and weights
     * of token 0 (their rows are computed from token 0's router logits) */
    const int *live;
};

/* Per-call token geometry: token t sits at KV slot pos0 + t, has RoPE position
 * pos0 + depth[t] and attends to slots 0..pos0-1 followed by pos0 + anc[t][j] for
 * j = 0..depth[t] (its ancestors from the root, itself last). A chain has depth[t] = t
 * and anc[t][j] = j. pos0 is read from device memory, so that one captured launch
 * sequence serves every position; nr_max bounds every token's row count pos0 +
 * depth[t] + 1 and sizes the grids that cover rows. */
struct TokGeom {
    const int *depth;         /* [T] */
    const int *anc;           /* [T][anc_ld] */
    int anc_ld;
    const int *pos;           /* device [1]: pos0 */
    int nr_max;
    int chain;                /* 1: token t sits at slot pos0 + t with ancestors pos0..pos0 + t */
    /* device [1] or null: tokens t >= *live are padding; the GQA score, softmax and value
     * kernels skip them (their attention output rows are not written) */
    const int *live;
};

constexpr int AF_NR = 10;     /* read-ahead ranges of the value kernel */

struct AttnArgs {
    const float *q;           /* [T][H][hd] after qk-norm and RoPE */
    const float *kc, *vc;     /* layer caches [Hkv][cap][hd] */
    float *S;                 /* scratch [T][H][ldS] */
    int ldS;
    float *out;               /* [T][H*hd] */
    int T, H, Hkv, hd, cap;
    float scale;
    TokGeom g;
    Act qo;                   /* NUMERICS §2 blocks of out (when qo_on; head_dim % 64 == 0) */
    int qo_on;
    int qo_hm;                /* 1: qo rows are (head, token) = h * T + t with hd / 64 blocks each */
    float *po, *pm, *pl;      /* chunked attention partials: [T * H][nc_ld][hd], [T * H][nc_ld] twice */
    int nc_ld;                /* chunks per partial row: at least ceil(nr_max / 64) */
    const uint8_t *pf_p[AF_NR];   /* k_attn_values: byte ranges its pf_wgs extra workgroups read */
    unsigned long long pf_n[AF_NR];
    int pf_wgs;
    /* post = 1: the score kernel does the QKV post-step itself. q is then the raw query
     * projection and rk, rv the raw key and value projections ([T][Hkv*hd]); bias,
     * qk-norm (qk_norm 0 or 1) and RoPE (NEOX halves over the whole head) are applied to
     * q as it is staged and to the step's new K rows as they are loaded, token t's K and
     * V rows of group g go to slot pos0 + t, and the processed q to qout */
    int post, qk_norm;
    const float *rk, *rv, *bq, *bk, *bv, *qn, *kn, *rope;
    float *qout;
    float eps;
};

struct QkvArgs {
    const float *q, *k, *v;   /* GEMM outputs [T][H*hd], [T][Hkv*hd] */
    const float *bq, *bk, *bv, *qn, *kn;
    float *qout;              /* [T][H*hd] */
    float *kc, *vc;           /* layer caches [Hkv][cap][hd] */
    const float *rope;        /* [T][rope_dim]: (cos, sin) pairs, host computed */
    float *rfull;             /* [T][2] scratch for qk_norm = 2 */
    int T, H, Hkv, hd, cap, qk_norm, rope_dim, rope_style;
    float eps;
    const int *pos;           /* device [1]: pos0; token t's K/V go to slot pos0 + t */
    const int *live;          /* device [1] or null: tokens t >= *live are padding (skipped) */
};

/* Residual update + RMSNorm + activation quantization, one workgroup per token:
 *   mode 0: h = es * embed(tok[t])
 *   mode 1: h = h + rs * add[t]
 *   mode 2: h = h + rs * (sum_j w[t][j] * Y[pair_of[t][j]] (+ shared[t]))
 *   mode 3: h unchanged
 *   mode 4: v = h (+ rs * add[t], gated as in mode 2), h unchanged (prediction input)
 * then x = rmsnorm(h or v, w) and its activation blocks. */
struct NormArgs {
    int mode;
    float *h;                 /* [T][D] */
    const float *add;         /* mode 1 / shared expert output (modes 2 and 4, may be null) */
    const float *add_gate;    /* modes 2, 4: per-token shared gate logit (add * sigmoid(gate)), or null */
    const float *Y;           /* mode 2 */
    const float *wts;
    const int *pair_of;
    int K;
    const int *tokens;        /* mode 0 */
    const uint8_t *emb;       /* mode 0: FORMAT rows */
    int emb_dtype;
    size_t emb_rb;
    float es, rs;
    const float *norm_w;      /* [D] */
    float eps;
    float *x;                 /* [T][D] or null */
    Act a;
    int T, D;
    const int *live;          /* device [1] or null: tokens t >= *live are padding (skipped) */
};

constexpr int ACCEPT_PARTS = 32;   /* slices per logits row in the argmax */

struct AcceptArgs {
    const float *rows;        /* [n][V] */
    int n, V;
    const int *tokens, *parent;
    int *amax;                /* [n] argmax or -1 for bad rows */
    float *part_v;            /* [n][ACCEPT_PARTS] per-slice maxima */
    int *part_i, *part_f;     /* [n][ACCEPT_PARTS] their indexes, flags (1 NaN/+inf, 2 not -inf) */
    int *path;                /* [n] */
    int *result;              /* [0] n_path, [1] final token, [2] status (0 ok, -1 bad logits) */
};

/* Multi-head latent attention of one layer (absorbed form, reference model.c:632-787). */
constexpr int MLA_RMAX = 64;          /* qk_rope_dim limit (register tile of the RoPE scores) */
constexpr int MLA_NOPE_MAX = 256;     /* qk_nope_dim limit */
struct MlaArgs {
    int T, H, C, rdim, nope, vd, qh;  /* qh = nope + rdim */
    const float *kva;                 /* [T][C + rdim] kv_a output */
    float *q;                         /* [T][H][qh]; q_pe is rotated in place */
    const float *kv_norm;             /* [C] */
    float *cc, *kp;                   /* layer caches: latent c [cap][C], rotated k_pe [cap][rdim] */
    const float *rope;                /* [T][rope_dim] (cos, sin) pairs */
    int rope_dim, rope_style;
    float eps;
    const int *pos;                   /* device [1]: pos0 */
    const uint8_t *wuk;               /* attn_kv_b as stored (FORMAT rows of C) */
    int wuk_dtype;
    size_t wuk_rb;
    float *qlat;                      /* [T][H][C] absorbed queries */
    float *S;                         /* scores [T][H][ldS] */
    int ldS;
    float scale;
    TokGeom g;
    const float *Yv;                  /* per-head W_UV outputs [H][T][vd] */
    float *att;                       /* [T][H * vd] */
    Act aatt;                         /* NUMERICS §2 blocks of att */
};

/* numpy's pairwise summation tree of the last (partial) 8192-element buffer of a row:
 * leaves in index order, and per level the additions slot[a] = slot[a] + slot[b]
 * (a subtree's value lives in the slot of its leftmost leaf). Built on the host. */
constexpr int PW_MAXLEAF = 72;
struct PwTail {
    int len, nleaf, nlev;
    unsigned short leaf_start[PW_MAXLEAF];
    unsigned char leaf_len[PW_MAXLEAF];
    unsigned char op_a[PW_MAXLEAF], op_b[PW_MAXLEAF];
    unsigned char lev_off[12];       /* ops of level h: [lev_off[h-1], lev_off[h]) */
};

constexpr int SAMPLE_VMAX = 262144;  /* vocabulary limit of sampled acceptance */
constexpr int SAMPLE_NMAX = 4096;    /* verify nodes per call */
constexpr int SAMPLE_WB = SAMPLE_VMAX / 8192;   /* numpy reduction buffers of a row */
constexpr int SAMPLE_HBINS = 2048;   /* top-p histogram bins (exponent and first significand bit of p in (0, 1]) */

/* Sampled acceptance of a verify tree (chain: parent[i] = i - 1). */
struct SampleArgs {
    const float *rows;                /* [n][V] target logits */
    int n, V;
    const int *tokens, *parent;       /* [n] */
    const double *q;                  /* [n][V] draft distributions (row v: v's children) or null */
    const double *u;                  /* [2n] uniforms */
    double temperature, top_p, min_p, rp;
    int top_k;
    const int *ctx;                   /* penalty context ids [n_ctx] */
    int n_ctx;
    double *P;                        /* [n][V] final distributions */
    unsigned long long *skey;         /* [n][sort_n] top-p candidates (tier 0), in index order; then sort scratch */
    int *sidx;                        /* [n][sort_n] */
    unsigned long long *skey2;        /* [n][sort_n] sort scratch of a fine bin too large for LDS */
    int *sidx2;                       /* [n][sort_n] */
    int *seg_begin, *seg_end;         /* [n] row v's candidates: [seg_begin, seg_end) = v * sort_n + [0, m) */
    int *bstar;                       /* [n] first histogram bin of tier 0 (-1: every nonzero entry) */
    int sort_n;                       /* power of two >= V */
    double *cc;                       /* [V / 8] the draw's running sum at the end of each group of 8 entries */
    int *row_rc;                      /* [n] 0 ok, -1 bad logits */
    int *path;                        /* [n] accepted nodes from the root */
    int *result;                      /* [0] path length, [1] final token, [2] status */
    PwTail tail;                      /* pairwise tree of the row's last numpy buffer */
    const int *live;                  /* device [1] or null: rows >= *live are padding (no distribution, never walked) */
    const int *n_ctx_dev;             /* device [1] or null: the penalty context length (else n_ctx) */
    double *wmax, *wsum;              /* [n][SAMPLE_WB] per reduction buffer of a row: max, then pairwise sum */
    int *widx, *wflag;                /* [n][SAMPLE_WB] first argmax, flags */
    unsigned long long *whist;        /* [n][SAMPLE_HBINS] approximate bin masses of a row */
    int *bcnt, *brel;                 /* [n][SAMPLE_HBINS] top-p candidates per fine bin; places taken so far */
    int *tcut;                        /* [n] top-p: every entry of a histogram bin below this one is dropped */
    int tail_wide;                    /* top-p's renormalization runs a workgroup per numpy buffer */
    double *R;                        /* [n][V] residual after node c is rejected (unnormalized) */
    double *rsum;                     /* [n][SAMPLE_WB] its numpy buffers' pairwise sums */
    int *sib_prev, *sib_rank;         /* [n] the sibling before c in index order (-1: none), c's place among them */
};

/* Greedy speculative decoding loop on the device (k_loop.hip): fields of the state block. */
enum LoopField {
    LS_LEN,       /* length of the committed sequence in hist */
    LS_NEW,       /* tokens yielded by the generation so far */
    LS_DONE,      /* LOOP_* */
    LS_STOP,      /* the stop token that ended the run */
    LS_STEP,      /* verify steps committed */
    LS_NOUT,      /* tokens written to out */
    LS_ND,        /* draft length of the current step */
    LS_LIVE,      /* rows of the current step that are not padding (ND + 1) */
    LS_MAXNEW,    /* the generation's token budget */
    LS_NGRAM,     /* longest n-gram the prompt lookup matches (0: no drafts) */
    LS_NSTOP,     /* stop ids */
    LS_KVPOS,     /* the engine position after the last committed step */
    LS_UOFF,      /* sampled runs: uniforms of the run's stream consumed so far */
    LS_BSTEP,     /* commits of the current batch (the host-visible flag slot) */
    LS_FIELDS = 16
};
enum LoopDone { LOOP_RUNNING = 0, LOOP_STOP = 1, LOOP_LENGTH = 2, LOOP_BAD = 3 };
constexpr int LOOP_STOPS_MAX = 64;

struct LoopArgs {
    int *state;                       /* [LS_FIELDS] */
    int *hist;                        /* [hist_cap] committed sequence */
    int hist_cap;
    const int *stops;                 /* [LOOP_STOPS_MAX] */
    int *out;                         /* [out_cap] tokens each step handled, in order */
    int out_cap;
    int *rec;                         /* [rec_cap][3] per step: drafted, accepted, tokens handled */
    int rec_cap;
    int *tokens;                      /* [T] the forward's token ids */
    int *cmp;                         /* [T] the acceptance's draft ids (-1 for padding) */
    float *rope;                      /* [T][rope_dim] the forward's (cos, sin) rows */
    const float *rtab;                /* [cap][rope_dim] (cos, sin) of every position */
    int rope_dim, cap;
    int *pos;                         /* device [1]: the forward's pos0, advanced by the commit */
    const int *result;                /* the acceptance's n_path, final token, status */
    int T;                            /* rows per step: draft length + 1 */
    /* sampled runs (null ustream: no uniforms are used): the run's random stream, the
     * sampled acceptance's uniforms [2T] that the drafter fills from it in the
     * reference's order, and whether the commit advances LS_UOFF */
    const double *ustream;
    int ustream_n;
    double *u;
    int sampled;
    /* host-visible memory [4] or null: every commit of the batch (committing or not)
     * writes (LS_NEW, LS_DONE) after it to [2 (s & 1)], s = LS_BSTEP before it, so the
     * host sees a step's outcome without a copy */
    int *hflag;
};

} // namespace hxd

namespace hxl {
using namespace hxd;
/* rows [r0, r0 + count) of m from FORMAT.md bytes at src_dev (count may run into the pad rows) */
void repack(const uint8_t *src_dev, int r0, int count, const QMat &m, hipStream_t st);
void quant_rows(const float *x, int64_t ldx, int T, int nb, const Act &a, hipStream_t st);
void gemm(const GemmArgs &a, hipStream_t st);
bool expert_gateup(const MoeArgs &a, int n_slots, hipStream_t st, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
void expert_down(const MoeArgs &a, int n_slots, hipStream_t st, bool mid_done = false);
/* the down kernel alone on already quantized pair activations (a.mid) */
void expert_down_q(const MoeArgs &a, int n_slots, hipStream_t st);
/* MLA: latent post step, absorbed queries, RoPE score term, output gather */
void mla_post(const MlaArgs &a, hipStream_t st);
void mla_qlat(const MlaArgs &a, hipStream_t st);
void mla_pe_scores(const MlaArgs &a, hipStream_t st);
void mla_gather(const MlaArgs &a, hipStream_t st);
void fgemv(int dtype, const void *W, int rows, int cols, const float *X, int ldx, int T, float *Y, int ldy, hipStream_t st);
void route(const RouteArgs &a, hipStream_t st);
void norm(const NormArgs &a, hipStream_t st);
void swiglu_quant(float *g, const float *u, int T, int F, const Act &a, hipStream_t st);
void scale_rows(float *y, int ldy, int T, int n, float s, hipStream_t st);
void qkv_post(const QkvArgs &a, hipStream_t st);
void attention(const AttnArgs &a, hipStream_t st);
/* the two halves of attention(): scores; softmax + value sum */
void attention_scores(const AttnArgs &a, hipStream_t st);
void attention_finish(const AttnArgs &a, hipStream_t st);
/* attention in the chunked order (64-row chunks folded in order; see k_attn.hip), for
 * head_dim 64 or 128 and grp * head_dim <= 12288 (attention_chunked_ok) */
bool attention_chunked_ok(int hd, int grp);
void attention_chunked(const AttnArgs &a, hipStream_t st);
void kv_move(float *cache_layer0, size_t layer_stride, int L, int Hkv, int cap, int hd, int pos0, const int *path_dev,
             int n, hipStream_t st);
/* rows pos0 + path[j] -> pos0 + j of a [cap][width] array at offset off of every layer */
void kv_move_rows(float *cache, size_t layer_stride, int L, size_t off, int width, int pos0, const int *path, int n,
                  hipStream_t st);
/* desc[u].w = table[ulist[u]] for u < *n_active (after the expert cache served a layer) */
void desc_refresh(SlotDesc *desc, const ExpertW *table, const int *ulist, const int *n_active, int n_slots,
                  hipStream_t st);
void accept_greedy(const AcceptArgs &a, hipStream_t st);
/* the same, then the device loop's commit of the step and the next step's draft */
void accept_greedy_commit(const AcceptArgs &a, const LoopArgs &la, hipStream_t st);
/* Sampler settings of one sampled acceptance (the reference's Sampler fields). */
struct SamplerSpec {
    double temperature, top_p, min_p, rp;
    int top_k;
    const int *ctx;          /* host penalty context ids */
    int n_ctx;
};

/* Device scratch of sampled acceptance, grown on demand (every call on one stream). */
struct SampleScratch {
    int n_cap = 0, V = 0, ctx_cap = 0, sort_n = 0;
    bool has_q = false;
    double *P = nullptr, *q = nullptr, *u = nullptr, *cc = nullptr;
    unsigned long long *skey = nullptr, *skey2 = nullptr;
    int *sidx = nullptr, *sidx2 = nullptr, *seg_begin = nullptr, *seg_end = nullptr, *bstar = nullptr,
        *row_rc = nullptr, *path = nullptr, *result = nullptr, *ctx = nullptr, *tok = nullptr, *par = nullptr;
    double *wmax = nullptr, *wsum = nullptr;
    int *widx = nullptr, *wflag = nullptr;
    unsigned long long *whist = nullptr;
    int *bcnt = nullptr, *brel = nullptr, *tcut = nullptr;
    double *R = nullptr, *rsum = nullptr;
    int *sib_prev = nullptr, *sib_rank = nullptr;
    hipError_t ensure(int n, int V, bool need_q, int n_ctx);
    void release();
    ~SampleScratch() { release(); }
};

/* Uploads q (host [n][V] float64, or null for point-mass drafts), u (host [2n]) and the
 * penalty context, then runs the distribution and walk kernels on rows (device [n][V])
 * with device tokens/parent. The accepted path is left in m.path, and n_path, final
 * token and status (0, or -1 for bad logits) in m.result[0..2]. */
hipError_t accept_sample(SampleScratch &m, const float *rows, int n, int V, const int *tok, const int *par,
                         const SamplerSpec &s, const double *q, const double *u, hipStream_t st, bool q_dev = false,
                         int max_sib = -1);
/* the most children of one node of a verify tree (host parent[], or null for a chain);
 * the residual steps of accept_sample run that many launches (-1 there: n - 1) */
inline int max_siblings(const int *parent, int n) {
    if (n <= 1) return 0;
    if (!parent) return 1;
    std::vector<int> kids(n, 0);
    int mx = 0;
    for (int c = 1; c < n; c++)
        if (parent[c] >= 0 && parent[c] < n && ++kids[parent[c]] > mx) mx = kids[parent[c]];
    return mx;
}
/* The distribution kernel alone: m.P[v] = the final distribution of row v (the penalty
 * context of row v includes the path tokens of nodes 1..v), m.row_rc[v] its status. */
hipError_t sample_probs(SampleScratch &m, const float *rows, int n, int V, const int *tok, const int *par,
                        const SamplerSpec &s, hipStream_t st);
/* accept_sample with every input already on the device and nothing copied (so it can be
 * captured): the uniforms in m.u, the penalty context ctx_dev[0 .. *n_ctx_dev), rows
 * >= *live treated as padding */
hipError_t accept_sample_dev(SampleScratch &m, const float *rows, int n, int V, const int *tok, const int *par,
                             const SamplerSpec &s, const int *ctx_dev, const int *n_ctx_dev, const int *live,
                             hipStream_t st);
/* One step of the greedy loop: the drafts, token ids and RoPE rows of the next forward
 * (loop_draft), and the commit of the acceptance that followed it (loop_commit). */
void loop_draft(const LoopArgs &a, hipStream_t st);
void loop_commit_draft(const LoopArgs &a, hipStream_t st);
} // namespace hxl
