/*
 * engine.cpp — the hearth.h engine on an MI355X: open (container -> HBM), the
 * verify/eval forward pass as a sequence of HIP kernels on one stream, rewind,
 * telemetry, routing traces, and the tree / on-device acceptance extensions.
 *
 * Reference behaviour followed: engine/src/api.c (argument checks, env overrides,
 * defaults, error codes), engine/src/model.c:1171-1331 (forward, chunking by
 * max_batch, a failed call changes nothing), model.c:1148-1168 and 1885-1959
 * (routing trace / replay), FORMAT.md §9 (trace file).
 *
 * Residency: every weight lives in HBM (288 GB per MI355X) in the GPU layouts of
 * hx_device.h; the reference's NVMe->DRAM expert store is not needed when the routed
 * experts fit, which is every model up to ~280 GB of Q4 experts.
 */
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "hearth.h"
#include "hearth_gpu.h"
#include "hx_host.h"
#include "hx_launch.h"
#include "expert_store.h"

using namespace hx;
using hxd::Act;
using hxd::ExpertW;
using hxd::QMat;

namespace {

constexpr int MAX_BATCH = 4096;

void fail(char *err, size_t n, const char *fmt, ...) {
    if (!err || !n) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, n, fmt, ap);
    va_end(ap);
}

int env_int(const char *k, int def) {
    const char *s = getenv(k);
    if (!s || !*s) return def;
    char *end = nullptr;
    const long v = strtol(s, &end, 10);
    return end && *end == 0 ? (int)v : def;
}

double env_double(const char *k, double def) {
    const char *s = getenv(k);
    if (!s || !*s) return def;
    char *end = nullptr;
    const double v = strtod(s, &end);
    return end && *end == 0 ? v : def;
}

int device_index() { return env_int("HEARTH_DEVICE", 0); }

/* cos/sin as separate non-inlined calls, as the reference does (model.c:201-202), so
 * no compiler fuses them into a sincos routine that can differ by an ulp. */
__attribute__((noinline)) float host_cosf(float x) { return cosf(x); }
__attribute__((noinline)) float host_sinf(float x) { return sinf(x); }

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

/* A matrix on the device: Q8/Q4 in the tiled layout, or F32/F16/BF16 rows as stored. */
struct DMat {
    bool quant = false;
    QMat q{};
    const void *f = nullptr;
    int dtype = 0, rows = 0, cols = 0;
};

struct Layer {
    bool moe = false;
    const float *attn_norm = nullptr, *ffn_norm = nullptr;
    DMat q, k, v, o;
    const float *bq = nullptr, *bk = nullptr, *bv = nullptr, *qn = nullptr, *kn = nullptr;
    DMat gate, up, down;            /* dense FFN */
    DMat sh_gate, sh_up, sh_down;   /* shared expert (MoE layers, shared_ffn_dim > 0) */
    /* MLA: q (q_lora 0) or q_a -> rmsnorm -> q_b; kv_a; W_UK rows as stored; W_UV per head */
    DMat q_a, q_b, kv_a;
    const float *q_a_norm = nullptr, *kv_a_norm = nullptr;
    const uint8_t *kvb_raw = nullptr;
    int kvb_dtype = 0;
    size_t kvb_rb = 0;
    ExpertW *uv = nullptr;          /* device [H]: .down = W_UV of head h */
    const float *sh_gate_inp = nullptr; /* F32 [D]: shared output scaled by sigmoid(dot16(., x)) */
    const float *router = nullptr;  /* F32 [E][D] */
    const float *router_bias = nullptr;
    const float *router_bias_host = nullptr;   /* the same in the mapped container (prediction) */
    ExpertW *experts = nullptr;     /* device table [E] */
    uint64_t proj_bytes = 0;        /* algorithmic bytes of the attention projections (MLA: with W_UV) */
    uint64_t ffn_bytes = 0;         /* of the dense FFN or the shared expert */
    uint64_t expert_bytes_each = 0; /* algorithmic bytes of one expert (gate+up+down) */
    uint64_t expert_gateup_bytes = 0; /* of which gate + up */
    int dtype_mask = 0;             /* bit dt set when some expert has dtype dt */
};


} // namespace

struct hearth_engine {
    hearth_options opt{};
    int verbose = 0;
    ModelFile mf;
    Config c;
    int dev = 0;
    hipStream_t st = nullptr;
    std::vector<void *> allocs;

    int L = 0, D = 0, V = 0, H = 0, Hkv = 0, hd = 0, q_dim = 0, kv_dim = 0, E = 0, K = 0, F = 0, Fd = 0;
    int cap = 0, B = 0, rope_dim = 0, Fs = 0;
    bool mla = false;
    int C = 0, rdim = 0, nope = 0, vd = 0, qlr = 0, qh = 0;   /* MLA shape */
    std::vector<Layer> layers;
    std::vector<int> moe_ord;
    const uint8_t *emb = nullptr;
    int emb_dtype = 0;
    size_t emb_rb = 0;
    DMat lm_head;
    uint64_t head_bytes = 0;
    const float *out_norm = nullptr;
    std::vector<float> inv_freq;

    float *kv = nullptr;
    size_t kv_layer = 0;   /* floats per layer: [K, V][Hkv][cap][hd] */

    /* scratch for B tokens */
    float *h = nullptr, *x = nullptr, *qb = nullptr, *kb = nullptr, *vb = nullptr, *qr = nullptr, *att = nullptr,
          *ao = nullptr, *S = nullptr, *lge = nullptr, *wts = nullptr, *Y = nullptr, *f1 = nullptr, *f2 = nullptr,
          *logits = nullptr, *rope = nullptr, *rfull = nullptr, *midf = nullptr, *sf1 = nullptr, *sf2 = nullptr,
          *shb = nullptr, *shg = nullptr, *qa = nullptr, *kva = nullptr, *olat = nullptr, *yv = nullptr;
    int ldS = 0;
    Act ax{}, aatt{}, amid{}, af{}, asf{}, aqa{}, alat{};
    hxd::SlotDesc *slot_desc = nullptr;
    int *ids = nullptr, *route_meta = nullptr, *pair_tok = nullptr, *pair_of = nullptr, *tokens = nullptr,
        *depth = nullptr, *anc = nullptr, *route_out = nullptr, *acc_i = nullptr, *acc_part = nullptr;
    unsigned long long *dstats = nullptr;
    /* pinned host staging */
    int *h_geom = nullptr;   /* tokens | depth | anc */
    float *h_rope = nullptr;
    int *h_res = nullptr;
    hipEvent_t geom_ev = nullptr;   /* recorded after the last upload from h_geom / h_rope */
    bool geom_pending = false;
    int geom_chain = 1;           /* the uploaded geometry is a chain (no parent table, or parent[i] = i - 1) */

    int pos = 0;
    int *d_pos = nullptr;    /* device [1]: pos of the forward being run (the kernels' pos0) */
    /* Captured forwards: the launch sequence of one forward, replayed as a hipGraph, per
     * (tokens, logits wanted, chain geometry, row bound). pos0 and the geometry live in
     * device memory, so a graph serves every position up to its row bound. */
    struct Captured {
        int T, chain, rows;
        bool logits;
        bool loop;           /* a whole step of the device loop (loop_step), not a forward alone */
        uint64_t skey;       /* loop steps: the sampler they accept with (0: greedy) */
        hipGraph_t graph;
        hipGraphExec_t exec;
    };
    std::vector<Captured> graphs;
    bool graph_on = true;    /* HEARTH_GPU_GRAPH=0 turns capture off */
    bool graph_report = false;   /* HEARTH_GPU_GRAPH_REPORT=1: describe each captured graph on stderr */
    /* attention order of the GQA layers: 0 the reference's canonical order (default), 1
     * chunked (where the shape allows it, attn_chunk_ok); MLA layers are canonical */
    int attn_mode = 0;
    int read_ahead = 0;      /* extra workgroups of the value kernel that read the next weights ahead */
    bool attn_chunk_ok = false;
    float *apo = nullptr, *apm = nullptr, *apl = nullptr;   /* chunked partials (alias S) */
    int anc_ld = 0;                                         /* chunks per partial row */
    void drop_graphs();
    int rows_bound = 0;      /* nonzero while capturing: the graph's bound on pos + T */
    int nr_max(int T) const { return rows_bound ? rows_bound : pos + T; }
    void run_forward(int T, bool want_logits);
    /* telemetry */
    uint64_t tokens_done = 0, forward_calls = 0;
    double wall_s = 0.0;
    int profiling = 0;   /* 0 off, 1 expert launches, 2 every launch group */
    hearth_gpu_kstats ks{};
    struct Ev { hipEvent_t a, b; double *acc; };
    std::vector<Ev> pending_ev;
    std::vector<hipEvent_t> ev_pool;
    size_t ev_next = 0;
    unsigned long long stats_base[2] = {0, 0};
    unsigned long long ks_base = 0;   /* distinct-expert loads counter at hearth_gpu_reset_kstats */
    /* routing trace / replay */
    FILE *trace = nullptr;
    std::vector<int> h_routes;
    int *replay_dev = nullptr;
    int64_t replay_rows = 0;
    /* tree verification: slots of the last uncommitted tree */
    int tree_n = 0;
    /* the greedy speculative loop on the device (hearth_gpu_spec_greedy), allocated on
     * first use: state block, committed sequence, stop ids, handled tokens, per-step
     * records, the acceptance's draft ids and chain parents, its path, and the RoPE
     * table indexed by position (rows [lp_rtab_lo, lp_rtab_hi) filled) */
    int *lp_state = nullptr, *lp_hist = nullptr, *lp_stops = nullptr, *lp_out = nullptr, *lp_rec = nullptr,
        *lp_cmp = nullptr, *lp_par = nullptr, *lp_path = nullptr;
    float *lp_rtab = nullptr;
    int lp_rtab_lo = 0, lp_rtab_hi = 0;
    int *h_lp = nullptr;                 /* pinned: the state block after a batch */
    int *h_lpf = nullptr, *d_lpf = nullptr;   /* pinned, coherent [4]: the commits' (LS_NEW, LS_DONE) flags */
    hipEvent_t lp_ev[2] = {nullptr, nullptr};
    /* sampled runs (hearth_gpu_spec_sample): the acceptance scratch of the loop (its own,
     * so that growing the call-by-call scratch never moves what a captured step reads),
     * the run's uniform stream, the sampler, and its key among the captured steps (0:
     * greedy acceptance) */
    hxl::SampleScratch lp_samp;
    double *lp_ustream = nullptr;
    hxl::SamplerSpec lp_spec{};
    uint64_t lp_skey = 0;
    const int *route_live = nullptr;     /* RouteArgs.live of the forwards being launched */
    void loop_prepare();
    void loop_rope_table(int lo, int hi);
    hxd::LoopArgs loop_args(int T);
    void loop_step(int T);
    void launch_loop_step(int T, int rows);
    bool loop_ok() const { return !store && !replay_dev && !trace && !profiling && dump_dir.empty(); }
    /* sampled acceptance scratch, grown on demand */
    hxl::SampleScratch samp;
    /* HBM expert cache (null: every expert resident) */
    std::unique_ptr<GpuExpertStore> store;
    int *h_meta = nullptr;   /* pinned [1 + E]: n_active, active experts of a layer */
    StoreStats store_base;   /* store counters at hearth_reset_stats */
    /* With the expert cache, a call that fails (a load that could not be enqueued) must
     * leave the statistics as they were: the store's counters and the routing counters
     * dstats[0..1] (copied to dstats[2..3] at the start of the call, in stream order) are
     * put back. Without the cache a failure is a device error and nothing is kept. */
    void call_mark() {
        if (!store) return;
        store->mark();
        (void)hipMemcpyAsync(dstats + 2, dstats, 2 * sizeof(unsigned long long), hipMemcpyDeviceToDevice, st);
    }
    void call_rollback() {
        if (!store) return;
        store->rollback();
        (void)hipMemcpyAsync(dstats, dstats + 2, 2 * sizeof(unsigned long long), hipMemcpyDeviceToDevice, st);
    }
    /* next-layer prediction (model.c:935-984): router of the next MoE layer on the
     * predicted input, top_k + prefetch_extra per token, union over the batch */
    float *pxs = nullptr, *plog = nullptr, *h_plog = nullptr;   /* [B][D], [B][E], pinned [B][E] */
    Act apx{};
    double pf_prec = 1.0;            /* recent precision (EWMA) */
    int pred_layer = -1;
    std::vector<int> pred_list;
    std::vector<uint8_t> pf_mark;
    void predict_select(const float *logits, const float *bias, int kk, int *out) const;
    void prefetch_next(int nl, int T);
    void score_prediction(int l, const int *ulist, int nu);
    /* HEARTH_DEBUG_DUMP=<dir>: every forward writes named intermediate buffers there
     * (T rows each, appended per call) for layer-by-layer comparisons */
    std::string dump_dir;
    void dump(const char *name, int layer, const void *dptr, int T, int width, size_t elem = 4) {
        if (dump_dir.empty()) return;
        std::vector<uint8_t> buf((size_t)T * width * elem);
        ck(hipMemcpyAsync(buf.data(), dptr, buf.size(), hipMemcpyDeviceToHost, st));
        ck(hipStreamSynchronize(st));
        char path[1024];
        std::snprintf(path, sizeof path, "%s/l%d_%s.bin", dump_dir.c_str(), layer, name);
        if (FILE *f = fopen(path, "ab")) { fwrite(buf.data(), 1, buf.size(), f); fclose(f); }
    }

    /* HEARTH_GPU_POISON=1 fills every work buffer with 0xFF bytes (a NaN in every float)
     * when it is allocated: a kernel that reads memory no kernel wrote then shows */
    void *dalloc(size_t n) {
        void *p = nullptr;
        ck(hipMalloc(&p, n ? n : 256));
        allocs.push_back(p);
        static const bool poison = [] {
            const char *s = getenv("HEARTH_GPU_POISON");
            return s && strcmp(s, "0") != 0;
        }();
        if (poison) ck(hipMemset(p, 0xFF, n ? n : 256));
        return p;
    }
    template <class T> T *dnew(size_t count) { return (T *)dalloc(sizeof(T) * count); }
    Act make_act(int rows, int n) {
        Act a{};
        a.nbp = ((n / 64) + 1) & ~1;
        a.q = dnew<int8_t>((size_t)rows * a.nbp * 64);
        a.d = dnew<float>((size_t)rows * a.nbp);
        a.s = dnew<int32_t>((size_t)rows * a.nbp);
        ck(hipMemset(a.q, 0, (size_t)rows * a.nbp * 64));
        ck(hipMemset(a.d, 0, sizeof(float) * (size_t)rows * a.nbp));
        ck(hipMemset(a.s, 0, sizeof(int32_t) * (size_t)rows * a.nbp));
        return a;
    }
    ~hearth_engine() {
        if (dev >= 0) (void)hipSetDevice(dev);
        if (st) (void)hipStreamSynchronize(st);
        for (Captured &g : graphs) {
            (void)hipGraphExecDestroy(g.exec);
            (void)hipGraphDestroy(g.graph);
        }
        for (auto &e : ev_pool) (void)hipEventDestroy(e);
        if (geom_ev) (void)hipEventDestroy(geom_ev);
        for (void *p : allocs) (void)hipFree(p);
        samp.release();
        lp_samp.release();
        if (h_geom) (void)hipHostFree(h_geom);
        if (h_rope) (void)hipHostFree(h_rope);
        if (h_res) (void)hipHostFree(h_res);
        if (h_meta) (void)hipHostFree(h_meta);
        if (h_plog) (void)hipHostFree(h_plog);
        if (h_lp) (void)hipHostFree(h_lp);
        if (h_lpf) (void)hipHostFree(h_lpf);
        for (hipEvent_t &ev : lp_ev)
            if (ev) (void)hipEventDestroy(ev);
        if (replay_dev) (void)hipFree(replay_dev);
        store.reset();
        if (st) (void)hipStreamDestroy(st);
        if (trace) fclose(trace);
    }

    /* ---- profiling: events around launch groups ---- */
    hipEvent_t next_event() {
        if (ev_next == ev_pool.size()) {
            hipEvent_t e;
            ck(hipEventCreate(&e));
            ev_pool.push_back(e);
        }
        return ev_pool[ev_next++];
    }
    template <class Fn> void timed(double *acc, Fn fn, int level = 2) {
        if (profiling < level) { fn(); return; }
        hipEvent_t a = next_event(), b = next_event();
        ck(hipEventRecord(a, st));
        fn();
        ck(hipEventRecord(b, st));
        pending_ev.push_back({a, b, acc});
    }
    /* the same, with the events handed to the launch so that the dispatch records them
     * (kernel start and end, no enqueue gaps) */
    template <class Fn> void timed_dispatch(double *acc, Fn fn, int level) {
        if (profiling < level) { fn(nullptr, nullptr); return; }
        hipEvent_t a = next_event(), b = next_event();
        fn(a, b);
        pending_ev.push_back({a, b, acc});
    }
    void collect_events() {
        for (auto &p : pending_ev) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) *p.acc += ms * 1e-3;
        }
        pending_ev.clear();
        ev_next = 0;
    }

    bool open_model(char *err, size_t errlen);
    bool upload(std::string &msg);
    void forward(int T, bool want_logits, int logit_rows_from);
    void attn_mla(const Layer &w, int l, int T);
    /* KV of slots pos + path[j] -> pos + j (path on the device) */
    void move_kv(const int *path_dev, int n) {
        if (mla) {
            hxl::kv_move_rows(kv, kv_layer, L, 0, C, pos, path_dev, n, st);
            hxl::kv_move_rows(kv, kv_layer, L, (size_t)cap * C, rdim, pos, path_dev, n, st);
        } else {
            hxl::kv_move(kv, kv_layer, L, Hkv, cap, hd, pos, path_dev, n, st);
        }
    }
    int eval_chunked(const int32_t *tokens, int n, float *logits_out, int all_logits);
    int run_geometry(const int32_t *tok, const int32_t *parent, int n, float *logits_out, bool keep_logits_dev);
    void matmul(const DMat &m, const Act &a, const float *xf, int ldx, int T, float *Y, int ldy, bool scale_on, float scale);
    void write_trace(int T);
    void flush_trace();
    std::vector<uint8_t> trace_pend;   /* trace rows of the call in progress */
    std::vector<int> tree_parent;      /* parent table of the last uncommitted tree */
};

/* ---------------------------------------------------------------- upload */

namespace {

struct Uploader {
    hipStream_t st;
    uint8_t *pinned[2] = {nullptr, nullptr};
    uint8_t *dstage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    size_t cap = (size_t)128 << 20;
    int cur = 0;

    explicit Uploader(hipStream_t s) : st(s) {
        for (int i = 0; i < 2; i++) {
            ck(hipHostMalloc((void **)&pinned[i], cap, hipHostMallocDefault));
            ck(hipMalloc((void **)&dstage[i], cap));
            ck(hipEventCreate(&done[i]));
        }
    }
    ~Uploader() {
        for (int i = 0; i < 2; i++) {
            if (done[i]) (void)hipEventSynchronize(done[i]);
            if (pinned[i]) (void)hipHostFree(pinned[i]);
            if (dstage[i]) (void)hipFree(dstage[i]);
            if (done[i]) (void)hipEventDestroy(done[i]);
        }
    }
    /* next staging pair, free once its previous user has finished */
    int take() {
        const int i = cur;
        cur ^= 1;
        if (used[i]) ck(hipEventSynchronize(done[i]));
        used[i] = true;
        return i;
    }
    void raw(void *dst, const uint8_t *src, size_t n) {
        for (size_t off = 0; off < n; off += cap) {
            const size_t len = std::min(cap, n - off);
            const int i = take();
            std::memcpy(pinned[i], src + off, len);
            ck(hipMemcpyAsync((uint8_t *)dst + off, pinned[i], len, hipMemcpyHostToDevice, st));
            ck(hipEventRecord(done[i], st));
        }
    }
    void quant(const QMat &m, const uint8_t *src) {
        const size_t rb = row_bytes(m.dtype, (int64_t)m.nb * 64);
        int chunk = (int)std::min<size_t>((size_t)m.rows_pad, cap / rb) & ~15;
        if (chunk < 16) chunk = 16;
        for (int r0 = 0; r0 < m.rows_pad; r0 += chunk) {
            const int count = std::min(chunk, m.rows_pad - r0);
            const int real = std::max(0, std::min(count, m.rows - r0));
            const int i = take();
            if (real) {
                std::memcpy(pinned[i], src + (size_t)r0 * rb, (size_t)real * rb);
                ck(hipMemcpyAsync(dstage[i], pinned[i], (size_t)real * rb, hipMemcpyHostToDevice, st));
            }
            hxl::repack(dstage[i], r0, count, m, st);
            ck(hipEventRecord(done[i], st));
        }
    }
};

} // namespace

bool hearth_engine::upload(std::string &msg) {
    Uploader up(st);
    auto vec = [&](int layer, const char *name) -> const float * {
        const Tensor *t = layer < 0 ? mf.tensor(name) : mf.layer_tensor(layer, name);
        if (!t) return nullptr;
        float *d = (float *)dalloc(t->nbytes);
        up.raw(d, mf.data(t->offset), t->nbytes);
        return d;
    };
    auto qmat_alloc = [&](int dtype, int rows, int cols) -> QMat {
        QMat m{};
        m.dtype = dtype;
        m.rows = rows;
        m.rows_pad = (rows + 15) & ~15;
        m.nb = cols / 64;
        m.nbp = (m.nb + 1) & ~1;
        m.w = (const uint8_t *)dalloc((size_t)(m.rows_pad / 16) * m.nbp * 1024 / (dtype == HEARTH_Q4 ? 2 : 1));
        m.d = (const uint16_t *)dalloc(sizeof(uint16_t) * (size_t)m.nbp * m.rows_pad);
        return m;
    };
    auto qmat_copy = [&](const QMat &dst, const QMat &src) {   /* same dtype and shape */
        const size_t wb = (size_t)(src.rows_pad / 16) * src.nbp * 1024 / (src.dtype == HEARTH_Q4 ? 2 : 1);
        ck(hipMemcpyAsync((void *)dst.w, src.w, wb, hipMemcpyDeviceToDevice, st));
        ck(hipMemcpyAsync((void *)dst.d, src.d, sizeof(uint16_t) * (size_t)src.nbp * src.rows_pad,
                          hipMemcpyDeviceToDevice, st));
    };
    std::unordered_map<uint64_t, ExpertW> first_copy;   /* slab offset -> the matrices of its first entry */
    auto mat = [&](int layer, const char *name, DMat &out) -> bool {
        const Tensor *t = layer < 0 ? mf.tensor(name) : mf.layer_tensor(layer, name);
        if (!t) { msg = std::string("tensor '") + name + "' is missing"; return false; }
        out.dtype = t->dtype;
        out.rows = (int)t->shape[0];
        out.cols = (int)t->shape[1];
        if (dtype_is_quant(t->dtype)) {
            out.quant = true;
            out.q = qmat_alloc(t->dtype, out.rows, out.cols);
            up.quant(out.q, mf.data(t->offset));
        } else {
            out.quant = false;
            void *d = dalloc(t->nbytes);
            up.raw(d, mf.data(t->offset), t->nbytes);
            out.f = d;
        }
        return true;
    };

    /* embedding rows as stored (a gather of T rows per call) */
    {
        const Tensor *t = mf.tensor("tok_embd");
        emb_dtype = t->dtype;
        emb_rb = row_bytes(t->dtype, D);
        uint8_t *d = (uint8_t *)dalloc(t->nbytes);
        up.raw(d, mf.data(t->offset), t->nbytes);
        emb = d;
    }
    if (!mat(-1, c.tie ? "tok_embd" : "lm_head", lm_head)) return false;
    out_norm = vec(-1, "out_norm");
    layers.resize(L);
    for (int l = 0; l < L; l++) {
        Layer &w = layers[l];
        w.moe = c.layer_kind[l] != 0;
        w.attn_norm = vec(l, "attn_norm");
        w.ffn_norm = vec(l, "ffn_norm");
        if (mla) {
            if (qlr) {
                if (!mat(l, "attn_q_a", w.q_a) || !mat(l, "attn_q_b", w.q_b)) return false;
                w.q_a_norm = vec(l, "attn_q_a_norm");
            } else if (!mat(l, "attn_q", w.q)) {
                return false;
            }
            if (!mat(l, "attn_kv_a", w.kv_a) || !mat(l, "attn_o", w.o)) return false;
            w.kv_a_norm = vec(l, "attn_kv_a_norm");
            const Tensor *t = mf.layer_tensor(l, "attn_kv_b");
            if (!t) { msg = "tensor 'attn_kv_b' is missing"; return false; }
            if (!dtype_is_quant(t->dtype) && t->dtype > HEARTH_BF16) { msg = "attn_kv_b has an unsupported dtype"; return false; }
            w.kvb_dtype = t->dtype;
            w.kvb_rb = row_bytes(t->dtype, C);
            uint8_t *raw = (uint8_t *)dalloc(t->nbytes);
            up.raw(raw, mf.data(t->offset), t->nbytes);
            w.kvb_raw = raw;
            if (!dtype_is_quant(t->dtype)) { msg = "attn_kv_b must be Q8 or Q4 for the per-head W_UV kernel"; return false; }
            std::vector<ExpertW> uvt(H);
            for (int h = 0; h < H; h++) {
                uvt[h] = ExpertW{};
                uvt[h].down = qmat_alloc(t->dtype, vd, C);
                up.quant(uvt[h].down, mf.data(t->offset) + ((size_t)h * (nope + vd) + nope) * w.kvb_rb);
            }
            w.uv = (ExpertW *)dalloc(sizeof(ExpertW) * (size_t)H);
            ck(hipMemcpyAsync(w.uv, uvt.data(), sizeof(ExpertW) * (size_t)H, hipMemcpyHostToDevice, st));
            ck(hipStreamSynchronize(st));   /* the host table goes out of scope */
        } else if (!mat(l, "attn_q", w.q) || !mat(l, "attn_k", w.k) || !mat(l, "attn_v", w.v) || !mat(l, "attn_o", w.o)) {
            return false;
        }
        if (c.qkv_bias) {
            w.bq = vec(l, "attn_q_bias");
            w.bk = vec(l, "attn_k_bias");
            w.bv = vec(l, "attn_v_bias");
        }
        if (c.qk_norm) {
            w.qn = vec(l, "attn_q_norm");
            w.kn = vec(l, "attn_k_norm");
        }
        if (!w.moe) {
            if (!mat(l, "ffn_gate", w.gate) || !mat(l, "ffn_up", w.up) || !mat(l, "ffn_down", w.down)) return false;
            continue;
        }
        w.router = vec(l, "moe_router");
        if (c.score_bias) {
            w.router_bias = vec(l, "moe_router_bias");
            if (const Tensor *tb = mf.layer_tensor(l, "moe_router_bias")) w.router_bias_host = (const float *)mf.data(tb->offset);
        }
        if (c.shared_ffn > 0) {
            if (!mat(l, "shexp_gate", w.sh_gate) || !mat(l, "shexp_up", w.sh_up) || !mat(l, "shexp_down", w.sh_down))
                return false;
            if (c.shared_gate) w.sh_gate_inp = vec(l, "shexp_gate_inp");
        }
        if (store) {   /* experts stream through the HBM cache */
            for (int e = 0; e < E; e++) {
                const int dt = (int)mf.expert(l, e)->dtype;
                w.expert_bytes_each = 2 * (uint64_t)F * row_bytes(dt, D) + (uint64_t)D * row_bytes(dt, F);
                w.expert_gateup_bytes = 2 * (uint64_t)F * row_bytes(dt, D);
                w.dtype_mask |= 1 << dt;
            }
            w.experts = (ExpertW *)dalloc(sizeof(ExpertW) * (size_t)E);
            ck(hipMemset(w.experts, 0, sizeof(ExpertW) * (size_t)E));
            continue;
        }
        std::vector<ExpertW> table(E);
        for (int e = 0; e < E; e++) {
            const ExpertEntry *ent = mf.expert(l, e);
            const int dt = (int)ent->dtype;
            uint64_t og, ou, od;
            slab_layout(dt, D, F, &og, &ou, &od);
            const uint8_t *slab = mf.data(ent->offset);
            table[e].gate = qmat_alloc(dt, F, D);
            table[e].up = qmat_alloc(dt, F, D);
            table[e].down = qmat_alloc(dt, D, F);
            auto seen = first_copy.find(ent->offset);
            if (seen != first_copy.end()) {   /* an aliased slab: its own copy, made on the device */
                qmat_copy(table[e].gate, seen->second.gate);
                qmat_copy(table[e].up, seen->second.up);
                qmat_copy(table[e].down, seen->second.down);
            } else {
                up.quant(table[e].gate, slab + og);
                up.quant(table[e].up, slab + ou);
                up.quant(table[e].down, slab + od);
                first_copy.emplace(ent->offset, table[e]);
            }
            w.expert_bytes_each = 2 * (uint64_t)F * row_bytes(dt, D) + (uint64_t)D * row_bytes(dt, F);
            w.expert_gateup_bytes = 2 * (uint64_t)F * row_bytes(dt, D);
            w.dtype_mask |= 1 << dt;
        }
        w.experts = (ExpertW *)dalloc(sizeof(ExpertW) * (size_t)E);
        ck(hipMemcpyAsync(w.experts, table.data(), sizeof(ExpertW) * (size_t)E, hipMemcpyHostToDevice, st));
        ck(hipStreamSynchronize(st));   /* the host table goes out of scope */
    }
    ck(hipStreamSynchronize(st));
    /* algorithmic weight bytes per forward, for the profiling counters */
    auto mb = [](const DMat &m) -> uint64_t { return m.rows ? (uint64_t)m.rows * row_bytes(m.dtype, m.cols) : 0; };
    for (Layer &w : layers) {
        w.proj_bytes = mb(w.q) + mb(w.k) + mb(w.v) + mb(w.o) + mb(w.q_a) + mb(w.q_b) + mb(w.kv_a);
        if (mla) w.proj_bytes += (uint64_t)H * vd * row_bytes(w.kvb_dtype, C);
        w.ffn_bytes = mb(w.gate) + mb(w.up) + mb(w.down) + mb(w.sh_gate) + mb(w.sh_up) + mb(w.sh_down);
    }
    head_bytes = mb(lm_head);
    return true;
}

bool hearth_engine::open_model(char *err, size_t errlen) {
    std::string msg;
    if (!mf.open(opt.model_path, msg)) { fail(err, errlen, "%s: %s", opt.model_path, msg.c_str()); return false; }
    c = mf.cfg;
    mla = c.attn_kind == ATTN_MLA;
    L = c.n_layers; D = c.d_model; V = c.vocab; H = c.n_heads; Hkv = c.n_kv_heads; hd = c.head_dim;
    q_dim = H * hd; kv_dim = Hkv * hd; E = c.n_experts; K = c.top_k; F = c.expert_ffn; Fd = c.dense_ffn;
    Fs = c.n_moe ? c.shared_ffn : 0;
    if (mla) {
        C = c.kv_lora; rdim = c.rope_qk; nope = c.nope; vd = c.v_head; qlr = c.q_lora; qh = nope + rdim;
        if (C < 128 || C > 512 || C % 128 || rdim > hxd::MLA_RMAX || rdim % 2 || nope < 1 || nope > hxd::MLA_NOPE_MAX ||
            vd < 64 || vd % 64 || (qlr && qlr % 64) || c.rope_dim > rdim) {
            fail(err, errlen, "%s: MLA shape (kv_lora %d, rope %d, nope %d, v %d, q_lora %d) is outside this build's kernels",
                 opt.model_path, C, rdim, nope, vd, qlr);
            return false;
        }
        Hkv = 1; hd = C; q_dim = H * qh; kv_dim = 0;
    }
    rope_dim = c.rope_dim;
    if (!mla && (hd > 512 || hd % 16)) { fail(err, errlen, "%s: head_dim %d unsupported (needs a multiple of 16 <= 512)", opt.model_path, hd); return false; }
    if (E > 1024) { fail(err, errlen, "%s: %d experts exceed this build's limit of 1024", opt.model_path, E); return false; }
    if (c.n_moe && K > 64) { fail(err, errlen, "%s: top_k %d exceeds this build's limit of 64", opt.model_path, K); return false; }
    if (c.n_group > 64) { fail(err, errlen, "%s: n_group %d exceeds this build's limit of 64", opt.model_path, c.n_group); return false; }
    if (c.n_moe && (K < 1 || K > E || c.n_group < 1 || E % c.n_group ||
                    (c.n_group > 1 && (c.topk_group < 1 || c.topk_group > c.n_group)))) {
        fail(err, errlen, "%s: routing shape (experts %d, top_k %d, groups %d keep %d) is inconsistent", opt.model_path,
             E, K, c.n_group, c.topk_group);
        return false;
    }
    if (c.n_moe && F % 64) { fail(err, errlen, "%s: expert_ffn_dim %d is not a multiple of 64", opt.model_path, F); return false; }
    if (c.n_moe && (D > 16384 || F > 16384)) {
        fail(err, errlen, "%s: expert matrices of %d x %d exceed this build's limit of 16384", opt.model_path, F, D);
        return false;
    }
    for (int l = 0; l < L && c.n_moe; l++)
        for (int e = 0; e < E && c.layer_kind[l]; e++)
            if (!dtype_is_quant((int)mf.expert(l, e)->dtype)) {
                fail(err, errlen, "%s: expert (%d, %d) is %s; this build runs Q8/Q4 experts", opt.model_path, l, e,
                     dtype_name((int)mf.expert(l, e)->dtype));
                return false;
            }
    moe_ord.assign(L, -1);
    for (int l = 0, k = 0; l < L; l++) moe_ord[l] = c.layer_kind[l] ? k++ : -1;
    cap = opt.max_seq > 0 ? std::min(opt.max_seq, c.max_seq) : std::min(c.max_seq, 4096);
    if (cap < 1) cap = 1;
    B = opt.max_batch;
    if (rope_dim) {
        const Tensor *t = mf.tensor("rope_inv_freq");
        inv_freq.resize(rope_dim / 2);
        std::memcpy(inv_freq.data(), mf.data(t->offset), sizeof(float) * inv_freq.size());
    }

    dev = device_index();
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) { fail(err, errlen, "no HIP device is available"); return false; }
    if (dev < 0 || dev >= ndev) { fail(err, errlen, "HEARTH_DEVICE=%d but %d device(s) exist", dev, ndev); return false; }
    try {
        ck(hipSetDevice(dev));
        ck(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
        if (c.n_moe) {
            /* HBM expert cache when HEARTH_GPU_EXPERT_CACHE_GB is below the expert set, or
             * when the experts do not fit next to the dense weights, KV cache and scratch */
            const uint64_t slot_b = GpuExpertStore::slot_bytes_for(D, F, GpuExpertStore::room_dtype(mf, L, E));
            const uint64_t all = slot_b * (uint64_t)c.n_moe * E;
            const uint64_t kvb = (uint64_t)L * cap * 4 * (mla ? (uint64_t)(C + rdim) : 2ull * Hkv * hd);
            uint64_t budget = UINT64_MAX;
            size_t freeb = 0, totb = 0;
            ck(hipMemGetInfo(&freeb, &totb));
            const uint64_t other = mf.dense_bytes + kvb + (4ull << 30);
            budget = freeb > other ? freeb - other : 0;
            if (const char *g = getenv("HEARTH_GPU_EXPERT_CACHE_GB"))
                if (*g) budget = std::min<uint64_t>(budget, (uint64_t)(std::max(0.0, atof(g)) * 1073741824.0));
            if (all > budget) {
                const int n_slots = (int)std::max<uint64_t>((uint64_t)E, budget / slot_b);
                store = std::make_unique<GpuExpertStore>();
                const char *ht = getenv("HEARTH_GPU_HOST_TIER");
                if (!store->open(mf, L, E, D, F, n_slots, opt.policy, !(ht && !strcmp(ht, "0")), msg)) {
                    fail(err, errlen, "%s: %s", opt.model_path, msg.c_str());
                    return false;
                }
                ck(hipHostMalloc((void **)&h_meta, sizeof(int) * (size_t)(1 + E), hipHostMallocDefault));
                log_msg(LOG_INFO, "expert cache: %d HBM slots of %.1f MiB for %d experts; %s", n_slots,
                        slot_b / 1048576.0, c.n_moe * E,
                        store->host_tier() ? "loads from pinned slot images" : "staged loads from the container");
            }
        }
        if (!upload(msg)) { fail(err, errlen, "%s: %s", opt.model_path, msg.c_str()); return false; }
        /* KV cache and scratch */
        kv_layer = mla ? (size_t)cap * (C + rdim) : (size_t)2 * Hkv * cap * hd;
        kv = dnew<float>(kv_layer * L);
        ck(hipMemset(kv, 0, sizeof(float) * kv_layer * L));
        const size_t Bs = (size_t)B, P = Bs * (size_t)std::max(K, 1);
        h = dnew<float>(Bs * D);
        x = dnew<float>(Bs * D);
        qb = dnew<float>(Bs * q_dim);
        if (mla) {
            qr = dnew<float>(Bs * H * C);                 /* absorbed queries [T][H][C] */
            olat = dnew<float>(Bs * H * C);               /* latent attention outputs [T][H][C] */
            alat = make_act(H * B, C);                    /* their blocks, rows (head, token) */
            yv = dnew<float>(Bs * H * vd);                /* W_UV outputs [H][T][vd] */
            att = dnew<float>(Bs * H * vd);
            kva = dnew<float>(Bs * (C + rdim));
            if (qlr) {
                qa = dnew<float>(Bs * qlr);
                aqa = make_act(B, qlr);
            }
        } else {
            kb = dnew<float>(Bs * kv_dim);
            vb = dnew<float>(Bs * kv_dim);
            qr = dnew<float>(Bs * q_dim);
            att = dnew<float>(Bs * q_dim);
        }
        ao = dnew<float>(Bs * D);
        ldS = (cap + 63) & ~63;
        attn_chunk_ok = !mla && hxl::attention_chunked_ok(hd, H / Hkv);
        if (attn_chunk_ok) {
            /* one buffer serves either order: the canonical scores S or the chunked
             * partials (a call uses one of them) */
            anc_ld = (cap + 63) / 64;
            const size_t part = Bs * H * (size_t)anc_ld;
            S = dnew<float>(std::max(Bs * H * (size_t)ldS, part * (size_t)(hd + 2)));
            apo = S;
            apm = apo + part * (size_t)hd;
            apl = apm + part;
        } else {
            S = dnew<float>(Bs * H * (size_t)ldS);
        }
        ax = make_act(B, D);
        aatt = make_act(B, mla ? H * vd : q_dim);
        logits = dnew<float>(Bs * V);
        rope = dnew<float>(Bs * (size_t)std::max(rope_dim, 2));
        rfull = dnew<float>(Bs * 2);
        tokens = dnew<int>(Bs);
        depth = dnew<int>(Bs);
        anc = dnew<int>(Bs * Bs);
        acc_i = dnew<int>(Bs * 2 + 8);
        acc_part = dnew<int>(Bs * hxd::ACCEPT_PARTS * 3);
        dstats = dnew<unsigned long long>(4);
        ck(hipMemset(dstats, 0, sizeof(unsigned long long) * 4));
        if (c.n_moe) {
            lge = dnew<float>(Bs * E);
            ids = dnew<int>(P);
            wts = dnew<float>(P);
            route_meta = dnew<int>(1 + 3 * (size_t)E);
            slot_desc = (hxd::SlotDesc *)dalloc(sizeof(hxd::SlotDesc) * (size_t)E);
            pair_tok = dnew<int>(P);
            pair_of = dnew<int>(P);
            amid = make_act((int)P, F);
            midf = dnew<float>(P * F);
            Y = dnew<float>(P * D);
            route_out = dnew<int>(Bs * c.n_moe * K);
        }
        if (Fd) {
            f1 = dnew<float>(Bs * Fd);
            f2 = dnew<float>(Bs * Fd);
            af = make_act(B, Fd);
        }
        if (Fs) {
            sf1 = dnew<float>(Bs * Fs);
            sf2 = dnew<float>(Bs * Fs);
            asf = make_act(B, Fs);
            shb = dnew<float>(Bs * D);
            shg = dnew<float>(Bs);
        }
        if (store && opt.prefetch != HEARTH_PREFETCH_OFF) {
            pxs = dnew<float>(Bs * D);
            plog = dnew<float>(Bs * E);
            apx = make_act(B, D);
            ck(hipHostMalloc((void **)&h_plog, sizeof(float) * Bs * E, hipHostMallocDefault));
            pf_mark.assign(E, 0);
        }
        ck(hipHostMalloc((void **)&h_geom, sizeof(int) * (2 * Bs + Bs * Bs + 1), hipHostMallocDefault));
        d_pos = dnew<int>(1);
        ck(hipHostMalloc((void **)&h_rope, sizeof(float) * Bs * std::max(rope_dim, 2), hipHostMallocDefault));
        ck(hipHostMalloc((void **)&h_res, sizeof(int) * (2 * Bs + 8), hipHostMallocDefault));
        ck(hipEventCreateWithFlags(&geom_ev, hipEventDisableTiming));
        ck(hipDeviceSynchronize());
    } catch (const DeviceError &e) {
        fail(err, errlen, "%s: HIP error during open: %s", opt.model_path, hipGetErrorString(e.e));
        return false;
    }
    return true;
}

/* ---------------------------------------------------------------- forward */

void hearth_engine::matmul(const DMat &m, const Act &a, const float *xf, int ldx, int T, float *Yp, int ldy,
                           bool scale_on, float scale) {
    if (m.quant) {
        hxd::GemmArgs g{};
        g.nseg = 1;
        g.seg[0].m = m.q;
        g.seg[0].Y = Yp;
        g.seg[0].ldy = ldy;
        g.seg[0].scale_on = scale_on;
        g.seg[0].scale = scale;
        g.a = a;
        g.T = T;
        g.live = route_live;
        hxl::gemm(g, st);
    } else {
        hxl::fgemv(m.dtype, m.f, m.rows, m.cols, xf, ldx, T, Yp, ldy, st);
        if (scale_on) hxl::scale_rows(Yp, ldy, T, m.rows, scale, st);
    }
}

/* Multi-head latent attention of layer l for T tokens (reference attn_mla,
 * model.c:739-787): projections, latent post step, absorbed queries, latent scores +
 * RoPE term, softmax and latent value sum (GQA kernels, one shared group of width C),
 * W_UV per head (grouped projection, one slot per head), output projection. */
void hearth_engine::attn_mla(const Layer &w, int l, int T) {
    const int kvd = C + rdim;
    const DMat &qin = qlr ? w.q_a : w.q;
    float *qdst = qlr ? qa : qb;
    const int qld = qlr ? qlr : q_dim;
    timed(&ks.proj_s, [&] {
    if (qin.quant && w.kv_a.quant) {
        hxd::GemmArgs g{};
        g.nseg = 2;
        g.seg[0].m = qin.q; g.seg[0].Y = qdst; g.seg[0].ldy = qld;
        g.seg[1].m = w.kv_a.q; g.seg[1].Y = kva; g.seg[1].ldy = kvd;
        g.a = ax;
        g.T = T;
        g.live = route_live;
        hxl::gemm(g, st);
    } else {
        matmul(qin, ax, x, D, T, qdst, qld, false, 1.0f);
        matmul(w.kv_a, ax, x, D, T, kva, kvd, false, 1.0f);
    }
    if (qlr) {
        hxd::NormArgs n{};
        n.mode = 3; n.h = qa; n.norm_w = w.q_a_norm; n.eps = c.eps; n.x = qa; n.a = aqa; n.T = T; n.D = qlr;
        hxl::norm(n, st);
        matmul(w.q_b, aqa, qa, qlr, T, qb, q_dim, false, 1.0f);
    }
    });
    float *cc = kv + (size_t)l * kv_layer;
    hxd::MlaArgs ma{};
    ma.T = T; ma.H = H; ma.C = C; ma.rdim = rdim; ma.nope = nope; ma.vd = vd; ma.qh = qh;
    ma.kva = kva; ma.q = qb; ma.kv_norm = w.kv_a_norm; ma.cc = cc; ma.kp = cc + (size_t)cap * C;
    ma.rope = rope; ma.rope_dim = rope_dim; ma.rope_style = c.rope_style; ma.eps = c.eps; ma.pos = d_pos;
    ma.wuk = w.kvb_raw; ma.wuk_dtype = w.kvb_dtype; ma.wuk_rb = w.kvb_rb; ma.qlat = qr;
    ma.S = S; ma.ldS = ldS; ma.scale = c.attn_scale;
    ma.g.depth = depth; ma.g.anc = anc; ma.g.anc_ld = B; ma.g.pos = d_pos; ma.g.nr_max = nr_max(T); ma.g.chain = geom_chain;
    ma.Yv = yv; ma.att = att; ma.aatt = aatt;
    hxd::AttnArgs at{};
    timed(&ks.attn_s, [&] {
    hxl::mla_post(ma, st);
    hxl::mla_qlat(ma, st);
    at.q = qr; at.kc = cc; at.vc = cc; at.S = S; at.ldS = ldS; at.out = olat; at.T = T; at.H = H; at.Hkv = 1;
    at.hd = C; at.cap = cap; at.scale = 1.0f;
    at.g = ma.g;
    at.qo = alat; at.qo_on = 1; at.qo_hm = 1;
    hxl::attention_scores(at, st);
    hxl::mla_pe_scores(ma, st);
    hxl::attention_finish(at, st);
    });
    dump("att", l, olat, T, H * C);
    timed(&ks.proj_s, [&] {
        hxd::MoeArgs m{};
        m.table = w.uv; m.head_slots = 1; m.mid = alat; m.T = T; m.D = vd; m.F = C; m.Y = yv; m.P = H * T;
        m.dtype_mask = 1 << w.kvb_dtype;
        hxl::expert_down_q(m, H, st);
        hxl::mla_gather(ma, st);
        matmul(w.o, aatt, att, H * vd, T, ao, D, false, 1.0f);
    });
}

/* One forward of T tokens whose geometry (tokens, depth, anc, rope) is already on the
 * device; logits of all T rows into this->logits when want_logits. */
void hearth_engine::forward(int T, bool want_logits, int /*logit_rows_from*/) {
    const float rs = c.resid_scale;
    timed(&ks.norm_s, [&] {
        hxd::NormArgs n{};
        n.mode = 0; n.h = h; n.tokens = tokens; n.emb = emb; n.emb_dtype = emb_dtype; n.emb_rb = emb_rb;
        n.es = c.emb_scale; n.norm_w = layers[0].attn_norm; n.eps = c.eps; n.x = x; n.a = ax; n.T = T; n.D = D;
        n.live = route_live;
        hxl::norm(n, st);
    });
    for (int l = 0; l < L; l++) {
        const Layer &w = layers[l];
        if (profiling) ks.dense_bytes += w.proj_bytes + w.ffn_bytes;
        if (mla) attn_mla(w, l, T);
        else {
        timed(&ks.proj_s, [&] {
            if (w.q.quant && w.k.quant && w.v.quant) {
                hxd::GemmArgs g{};
                g.nseg = 3;
                const DMat *ms[3] = {&w.q, &w.k, &w.v};
                float *ys[3] = {qb, kb, vb};
                const int ld[3] = {q_dim, kv_dim, kv_dim};
                for (int s = 0; s < 3; s++) { g.seg[s].m = ms[s]->q; g.seg[s].Y = ys[s]; g.seg[s].ldy = ld[s]; }
                g.a = ax;
                g.T = T;
                g.live = route_live;
                hxl::gemm(g, st);
            } else {
                matmul(w.q, ax, x, D, T, qb, q_dim, false, 1.0f);
                matmul(w.k, ax, x, D, T, kb, kv_dim, false, 1.0f);
                matmul(w.v, ax, x, D, T, vb, kv_dim, false, 1.0f);
            }
        });
        timed(&ks.attn_s, [&] {
            hxd::QkvArgs qa{};
            qa.q = qb; qa.k = kb; qa.v = vb; qa.bq = w.bq; qa.bk = w.bk; qa.bv = w.bv; qa.qn = w.qn; qa.kn = w.kn;
            qa.qout = qr; qa.kc = kv + (size_t)l * kv_layer; qa.vc = qa.kc + (size_t)Hkv * cap * hd;
            qa.rope = rope; qa.rfull = rfull; qa.T = T; qa.H = H; qa.Hkv = Hkv; qa.hd = hd; qa.cap = cap;
            qa.qk_norm = c.qk_norm; qa.rope_dim = rope_dim; qa.rope_style = c.rope_style; qa.eps = c.eps; qa.pos = d_pos;
            qa.live = route_live;
            /* the canonical score kernel does the post-step itself (one launch fewer) for
             * per-head or no qk-norm and NEOX RoPE over the whole head, at most 16 tokens
             * (every score workgroup redoes its token's q: with a tree's 85 tokens that cost
             * more than the launch it saves, 17.01 -> 17.41 ms per step; the chain of 9
             * gained 6.545 -> 6.507 ms) */
            const bool fuse_post = T <= 16 && attn_mode != 1 && dump_dir.empty() && hd % 64 == 0 && hd <= 256 &&
                                   (c.qk_norm == 0 || c.qk_norm == 1) && c.rope_style == 0 && rope_dim == hd;
            if (!fuse_post) {
                hxl::qkv_post(qa, st);
                dump("q", l, qr, T, q_dim);
            }
            hxd::AttnArgs at{};
            at.q = fuse_post ? qb : qr;
            if (fuse_post) {
                at.post = 1; at.qk_norm = c.qk_norm; at.rk = kb; at.rv = vb; at.bq = w.bq; at.bk = w.bk; at.bv = w.bv;
                at.qn = w.qn; at.kn = w.kn; at.rope = rope; at.qout = qr; at.eps = c.eps;
            }
            at.kc = qa.kc; at.vc = qa.vc; at.S = S; at.ldS = ldS; at.out = att; at.T = T; at.H = H;
            at.Hkv = Hkv; at.hd = hd; at.cap = cap; at.scale = c.attn_scale;
            at.g.depth = depth; at.g.anc = anc; at.g.anc_ld = B; at.g.pos = d_pos; at.g.nr_max = nr_max(T); at.g.chain = geom_chain;
            at.g.live = route_live;
            at.qo = aatt; at.qo_on = w.o.quant && hd % 64 == 0;
            if (read_ahead > 0) {
                /* the value kernel reads ahead this layer's output projection and router and
                 * the next layer's QKV weights */
                int r = 0;
                auto add = [&](const DMat &m) {
                    if (!m.quant || r + 2 > hxd::AF_NR) return;
                    at.pf_p[r] = m.q.w;
                    at.pf_n[r++] = hxd::qmat_w_bytes(m.q);
                    at.pf_p[r] = (const uint8_t *)m.q.d;
                    at.pf_n[r++] = hxd::qmat_d_bytes(m.q);
                };
                add(w.o);
                if (w.moe && w.router) {
                    at.pf_p[r] = (const uint8_t *)w.router;
                    at.pf_n[r++] = sizeof(float) * (size_t)E * D;
                }
                if (l + 1 < L) { add(layers[l + 1].q); add(layers[l + 1].k); add(layers[l + 1].v); }
                at.pf_wgs = read_ahead;
            }
            if (attn_mode == 1) {
                at.po = apo; at.pm = apm; at.pl = apl; at.nc_ld = anc_ld;
                hxl::attention_chunked(at, st);
            } else {
                hxl::attention(at, st);
            }
            dump("att", l, att, T, q_dim);
            if (w.o.quant && !at.qo_on) hxl::quant_rows(att, q_dim, T, q_dim / 64, aatt, st);
        });
        timed(&ks.proj_s, [&] { matmul(w.o, aatt, att, q_dim, T, ao, D, false, 1.0f); });
        }
        timed(&ks.norm_s, [&] {
            hxd::NormArgs n{};
            n.mode = 1; n.h = h; n.add = ao; n.rs = rs; n.norm_w = w.ffn_norm; n.eps = c.eps; n.x = x; n.a = ax;
            n.T = T; n.D = D; n.live = route_live;
            hxl::norm(n, st);
        });
        dump("h_mid", l, h, T, D);
        dump("x_ffn", l, x, T, D);
        const float *next_norm = l + 1 < L ? layers[l + 1].attn_norm : out_norm;
        if (w.moe) {
            int *n_active = route_meta, *ulist = route_meta + 1, *u_p0 = ulist + E, *u_n = u_p0 + E;
            /* next-layer prediction (model.c:989-991, 1049-1063): 1 = on h, 2 = on h plus
             * the shared expert's output (shared mode with a shared expert) */
            const int nl = l + 1 < L && layers[l + 1].moe ? l + 1 : -1;
            const int pf = !pxs || nl < 0 ? 0 : opt.prefetch == HEARTH_PREFETCH_SHARED && Fs ? 2 : 1;
            auto shared_expert = [&] {   /* reference model.c:925-934: SwiGLU FFN of x, optional sigmoid gate */
                timed(&ks.dense_s, [&] {
                    matmul(w.sh_gate, ax, x, D, T, sf1, Fs, false, 1.0f);
                    matmul(w.sh_up, ax, x, D, T, sf2, Fs, false, 1.0f);
                    hxl::swiglu_quant(sf1, sf2, T, Fs, asf, st);
                    matmul(w.sh_down, asf, sf1, Fs, T, shb, D, false, 1.0f);
                    if (w.sh_gate_inp) hxl::fgemv(0, w.sh_gate_inp, 1, D, x, D, T, shg, 1, st);
                });
            };
            if (pf == 2) shared_expert();
            if (pf) {   /* predicted input rmsnorm(h (+ rs * shared), ffn_norm of nl); h unchanged */
                hxd::NormArgs n{};
                n.mode = 4; n.h = h; n.rs = rs; n.add = pf == 2 ? shb : nullptr;
                n.add_gate = pf == 2 && w.sh_gate_inp ? shg : nullptr;
                n.norm_w = layers[nl].ffn_norm; n.eps = c.eps; n.x = pxs; n.a = apx; n.T = T; n.D = D;
                hxl::norm(n, st);
                hxl::fgemv(0, layers[nl].router, E, D, pxs, D, T, plog, E, st);
                ck(hipMemcpyAsync(h_plog, plog, sizeof(float) * (size_t)T * E, hipMemcpyDeviceToHost, st));
            }
            timed(&ks.router_s, [&] {
                hxl::fgemv(0, w.router, E, D, x, D, T, lge, E, st);
                hxd::RouteArgs r{};
                r.logits = lge; r.bias = w.router_bias; r.T = T; r.E = E; r.K = K; r.score_fn = c.score_fn;
                r.n_group = c.n_group; r.topk_group = c.topk_group; r.norm_topk = c.norm_topk;
                r.routed_scale = c.routed_scale; r.ids = ids; r.wts = wts; r.n_active = n_active; r.ulist = ulist;
                r.u_p0 = u_p0; r.u_n = u_n; r.pair_tok = pair_tok; r.pair_of = pair_of;
                r.route_out = route_out; r.moe_ord = moe_ord[l]; r.n_moe = c.n_moe; r.stats = dstats;
                r.table = w.experts; r.desc = slot_desc; r.n_slots = std::min(E, T * K);
                r.replay = replay_dev; r.replay_rows = replay_rows; r.pos0 = pos; r.depth = depth;
                r.live = route_live;
                hxl::route(r, st);
            });
            if (store) {
                ck(hipMemcpyAsync(h_meta, route_meta, sizeof(int) * (size_t)(1 + E), hipMemcpyDeviceToHost, st));
                ck(hipStreamSynchronize(st));
                score_prediction(l, h_meta + 1, h_meta[0]);
                store->ensure(l, h_meta + 1, h_meta[0], w.experts, st);
                hxl::desc_refresh(slot_desc, w.experts, route_meta + 1, route_meta, std::min(E, T * K), st);
            }
            dump("router", l, lge, T, E);
            dump("ids", l, ids, T, K);
            {
                hxd::MoeArgs m{};
                m.table = w.experts; m.desc = slot_desc; m.n_active = n_active; m.ulist = ulist; m.u_p0 = u_p0; m.u_n = u_n;
                m.pair_tok = pair_tok; m.x = ax; m.mid = amid; m.midf = midf; m.Y = Y; m.T = T; m.F = F; m.D = D;
                m.P = T * K; m.dtype_mask = w.dtype_mask;
                const int slots = std::min(E, T * K);
                bool mid_done = false;
                timed_dispatch(&ks.expert_s, [&](hipEvent_t e0, hipEvent_t e1) { mid_done = hxl::expert_gateup(m, slots, st, e0, e1); }, 1);
                timed(&ks.expert_down_s, [&] { hxl::expert_down(m, slots, st, mid_done); }, 1);
            }
            if (profiling) ks.expert_launches++;
            if (Fs && pf != 2) shared_expert();
            timed(&ks.norm_s, [&] {
                hxd::NormArgs n{};
                n.mode = 2; n.h = h; n.Y = Y; n.wts = wts; n.pair_of = pair_of; n.K = K; n.rs = rs;
                n.add = Fs ? shb : nullptr; n.add_gate = w.sh_gate_inp ? shg : nullptr;
                n.norm_w = next_norm; n.eps = c.eps; n.x = x; n.a = ax; n.T = T; n.D = D; n.live = route_live;
                hxl::norm(n, st);
            });
            /* the layer's work is queued: the prediction's loads overlap it */
            if (pf) prefetch_next(nl, T);
            dump("h", l, h, T, D);
        } else {
            timed(&ks.dense_s, [&] {
                matmul(w.gate, ax, x, D, T, f1, Fd, false, 1.0f);
                matmul(w.up, ax, x, D, T, f2, Fd, false, 1.0f);
                hxl::swiglu_quant(f1, f2, T, Fd, af, st);
                matmul(w.down, af, f1, Fd, T, ao, D, false, 1.0f);
            });
            timed(&ks.norm_s, [&] {
                hxd::NormArgs n{};
                n.mode = 1; n.h = h; n.add = ao; n.rs = rs; n.norm_w = next_norm; n.eps = c.eps; n.x = x; n.a = ax;
                n.T = T; n.D = D; n.live = route_live;
                hxl::norm(n, st);
            });
        }
    }
    if (want_logits) {
        timed(&ks.head_s, [&] { matmul(lm_head, ax, x, D, T, logits, V, true, c.logit_scale); });
        if (profiling) ks.dense_bytes += head_bytes;
    }
    if (store) store->tick();
}

/* route_select (model.c:793-830) for the prediction: score = softmax or sigmoid of the
 * logits, sel = score (+ bias), group limit, then the kk best by sel (larger first, NaN
 * last, ties to the lower index). Host arithmetic: it only picks experts to load. */
void hearth_engine::predict_select(const float *lg, const float *bias, int kk, int *out) const {
    std::vector<float> score(lg, lg + E), sel(E);
    if (c.score_fn == 0) {
        float m = score[0];
        for (int e = 1; e < E; e++) m = score[e] > m ? score[e] : m;
        float sum = 0.0f;
        for (int e = 0; e < E; e++) sum += (score[e] = std::exp(score[e] - m));
        for (int e = 0; e < E; e++) score[e] /= sum;
    } else {
        for (int e = 0; e < E; e++) score[e] = 1.0f / (1.0f + std::exp(-score[e]));
    }
    for (int e = 0; e < E; e++) sel[e] = bias ? score[e] + bias[e] : score[e];
    auto before = [](float va, int ia, float vb, int ib) {
        const bool na = va != va, nb = vb != vb;
        if (na || nb) return na == nb ? ia < ib : nb;
        if (va != vb) return va > vb;
        return ia < ib;
    };
    if (c.n_group > 1) {
        const int ng = c.n_group, gs = E / ng;
        std::vector<float> gsc(ng);
        std::vector<uint8_t> keep(ng, 0);
        for (int g = 0; g < ng; g++) {
            const float *v = sel.data() + (size_t)g * gs;
            int i1 = 0, i2 = -1;
            for (int i = 1; i < gs; i++) {
                if (before(v[i], i, v[i1], i1)) { i2 = i1; i1 = i; }
                else if (i2 < 0 || before(v[i], i, v[i2], i2)) i2 = i;
            }
            gsc[g] = i2 >= 0 ? v[i1] + v[i2] : v[i1];
        }
        for (int r = 0; r < c.topk_group; r++) {
            int best = -1;
            for (int g = 0; g < ng; g++)
                if (!keep[g] && (best < 0 || before(gsc[g], g, gsc[best], best))) best = g;
            keep[best] = 1;
        }
        for (int g = 0; g < ng; g++)
            if (!keep[g]) std::fill(sel.begin() + (size_t)g * gs, sel.begin() + (size_t)(g + 1) * gs, 0.0f);
    }
    std::vector<uint8_t> taken(E, 0);
    for (int j = 0; j < kk; j++) {
        int best = -1;
        for (int e = 0; e < E; e++)
            if (!taken[e] && (best < 0 || before(sel[e], e, sel[best], best))) best = e;
        out[j] = best;
        taken[best] = 1;
    }
}

/* prefetch_next (model.c:944-973): the prediction for layer nl is always made and
 * scored when nl routes; it goes to the store only while the recent precision is at
 * least 0.5 * top_k / (top_k + prefetch_extra). */
void hearth_engine::prefetch_next(int nl, int T) {
    const int kk = std::min(K + opt.prefetch_extra, E);
    for (int e : pred_list) pf_mark[e] = 0;
    pred_list.clear();
    std::vector<int> sel(kk);
    for (int t = 0; t < T; t++) {
        predict_select(h_plog + (size_t)t * E, layers[nl].router_bias_host, kk, sel.data());
        for (int j = 0; j < kk; j++)
            if (!pf_mark[sel[j]]) {
                pf_mark[sel[j]] = 1;
                pred_list.push_back(sel[j]);
            }
    }
    pred_layer = nl;
    if (pf_prec >= 0.5 * (double)K / (double)kk) store->prefetch(nl, pred_list.data(), (int)pred_list.size());
}

/* score_prediction (model.c:976-984): precision = predicted experts used / predicted */
void hearth_engine::score_prediction(int l, const int *ulist, int nu) {
    if (pred_layer != l || pred_list.empty()) return;
    int hit = 0;
    for (int u = 0; u < nu; u++) hit += pf_mark[ulist[u]];
    pf_prec += 0.05 * ((double)hit / (double)pred_list.size() - pf_prec);
    for (int e : pred_list) pf_mark[e] = 0;
    pred_list.clear();
    pred_layer = -1;
}

/* Uploads tokens and geometry for n tokens at pos (parent NULL: chain) and runs the
 * forward; returns 0 or a negative code (nothing changed on failure). */
int hearth_engine::run_geometry(const int32_t *tok, const int32_t *parent, int n, float *logits_out, bool) {
    /* the staging buffers may still feed the previous call's uploads */
    if (geom_pending) ck(hipEventSynchronize(geom_ev));
    int *ht = h_geom, *hdp = h_geom + B, *hanc = h_geom + 2 * B;
    geom_chain = 1;
    for (int i = 0; parent && i < n; i++) geom_chain &= parent[i] == i - 1;
    for (int i = 0; i < n; i++) {
        ht[i] = tok[i];
        hdp[i] = parent ? (i == 0 ? 0 : hdp[parent[i]] + 1) : i;
        for (int v = i, j = hdp[i]; v >= 0 && j >= 0; v = parent ? parent[v] : v - 1, j--) hanc[(size_t)i * B + j] = v;
    }
    for (int i = 0; i < n; i++) {
        const float p = (float)(pos + hdp[i]);
        for (int j = 0; j < rope_dim / 2; j++) {
            const float th = p * inv_freq[j];
            h_rope[(size_t)i * rope_dim + 2 * j] = host_cosf(th) * c.rope_factor;
            h_rope[(size_t)i * rope_dim + 2 * j + 1] = host_sinf(th) * c.rope_factor;
        }
    }
    int *hpos = h_geom + 2 * B + (size_t)B * B;
    *hpos = pos;
    ck(hipMemcpyAsync(tokens, ht, sizeof(int) * n, hipMemcpyHostToDevice, st));
    ck(hipMemcpyAsync(depth, hdp, sizeof(int) * n, hipMemcpyHostToDevice, st));
    ck(hipMemcpyAsync(anc, hanc, sizeof(int) * (size_t)n * B, hipMemcpyHostToDevice, st));
    if (rope_dim) ck(hipMemcpyAsync(rope, h_rope, sizeof(float) * (size_t)n * rope_dim, hipMemcpyHostToDevice, st));
    ck(hipMemcpyAsync(d_pos, hpos, sizeof(int), hipMemcpyHostToDevice, st));
    ck(hipEventRecord(geom_ev, st));
    geom_pending = true;
    run_forward(n, logits_out != nullptr);
    if (logits_out) ck(hipMemcpyAsync(logits_out, logits, sizeof(float) * (size_t)n * V, hipMemcpyDeviceToHost, st));
    return OK;
}

/* HEARTH_GPU_GRAPH_REPORT: the node census of a captured graph (node types, kernel
 * nodes' distinct functions, the largest grid, block and LDS request, dependency edges),
 * for comparing what a tool that walks the graph at launch has to handle. */
static void report_graph(hipGraph_t g, const char *what, int T) {
    size_t n = 0;
    if (hipGraphGetNodes(g, nullptr, &n) != hipSuccess) return;
    std::vector<hipGraphNode_t> nodes(n);
    if (n && hipGraphGetNodes(g, nodes.data(), &n) != hipSuccess) return;
    size_t edges = 0;
    (void)hipGraphGetEdges(g, nullptr, nullptr, &edges);
    int counts[16] = {};
    std::vector<const void *> funcs;
    unsigned max_grid = 0, max_block = 0, max_lds = 0, null_params = 0;
    for (hipGraphNode_t nd : nodes) {
        hipGraphNodeType t{};
        if (hipGraphNodeGetType(nd, &t) != hipSuccess) continue;
        counts[(int)t & 15]++;
        if (t != hipGraphNodeTypeKernel) continue;
        hipKernelNodeParams kp{};
        if (hipGraphKernelNodeGetParams(nd, &kp) != hipSuccess) continue;
        if (std::find(funcs.begin(), funcs.end(), kp.func) == funcs.end()) funcs.push_back(kp.func);
        max_grid = std::max(max_grid, kp.gridDim.x * kp.gridDim.y * kp.gridDim.z);
        max_block = std::max(max_block, kp.blockDim.x * kp.blockDim.y * kp.blockDim.z);
        max_lds = std::max(max_lds, kp.sharedMemBytes);
        if (!kp.kernelParams && !kp.extra) null_params++;
    }
    (void)hipGetLastError();
    log_msg(LOG_ERROR,
            "graph report (%s, T=%d): %zu nodes (kernel %d, memcpy %d, memset %d, host %d, graph %d, empty %d, "
            "wait event %d, record event %d), %zu edges, %zu distinct kernels, largest grid %u workgroups, block %u, "
            "dynamic LDS %u B, %u kernel nodes without arguments",
            what, T, n, counts[hipGraphNodeTypeKernel], counts[hipGraphNodeTypeMemcpy], counts[hipGraphNodeTypeMemset],
            counts[hipGraphNodeTypeHost], counts[hipGraphNodeTypeGraph], counts[hipGraphNodeTypeEmpty],
            counts[hipGraphNodeTypeWaitEvent], counts[hipGraphNodeTypeEventRecord], edges, funcs.size(), max_grid,
            max_block, max_lds, null_params);
}

/* The forward of T tokens whose geometry is uploaded: replayed from a captured graph
 * when the call is one a graph can serve (experts resident, no route replay, no
 * per-launch timing or debug dumps, at most 128 tokens), else launched directly. The
 * graph's grids cover rows up to the next multiple of 1024 (at most the capacity), and
 * the kernels read pos0 from d_pos, so the replay computes what the direct launches
 * would. At most 32 graphs are kept (the oldest is dropped). */
/* Captured forwards hold the launches of the attention order they were captured with;
 * a change of order drops them (after the stream has finished with them). */
void hearth_engine::drop_graphs() {
    if (graphs.empty()) return;
    (void)hipSetDevice(dev);
    (void)hipStreamSynchronize(st);
    for (Captured &g : graphs) {
        (void)hipGraphExecDestroy(g.exec);
        (void)hipGraphDestroy(g.graph);
    }
    graphs.clear();
}

void hearth_engine::run_forward(int T, bool want_logits) {
    if (!graph_on || store || replay_dev || profiling || !dump_dir.empty() || T > 128) {
        forward(T, want_logits, 0);
        return;
    }
    const int rows = std::min(cap, (pos + T + 1023) / 1024 * 1024);
    Captured *cg = nullptr;
    for (Captured &g : graphs)
        if (!g.loop && g.T == T && g.chain == geom_chain && g.rows == rows && g.logits == want_logits) cg = &g;
    if (!cg) {
        if (graphs.size() >= 32) {
            (void)hipGraphExecDestroy(graphs.front().exec);
            (void)hipGraphDestroy(graphs.front().graph);
            graphs.erase(graphs.begin());
        }
        Captured g{T, geom_chain, rows, want_logits, false, 0, nullptr, nullptr};
        ck(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        rows_bound = rows;
        try {
            forward(T, want_logits, 0);
        } catch (const DeviceError &) {
            rows_bound = 0;
            hipGraph_t dead = nullptr;
            if (hipStreamEndCapture(st, &dead) == hipSuccess && dead) (void)hipGraphDestroy(dead);
            throw;
        }
        rows_bound = 0;
        ck(hipStreamEndCapture(st, &g.graph));
        if (graph_report) report_graph(g.graph, "forward", T);
        const hipError_t e = hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(g.graph);
            throw DeviceError{e};
        }
        graphs.push_back(g);
        cg = &graphs.back();
    }
    ck(hipGraphLaunch(cg->exec, st));
}

/* ---------------------------------------------------------------- greedy loop on the device */

void hearth_engine::loop_prepare() {
    if (lp_state) return;
    lp_hist = dnew<int>((size_t)cap + B + 2);
    lp_stops = dnew<int>(hxd::LOOP_STOPS_MAX);
    lp_out = dnew<int>((size_t)HEARTH_GPU_SPEC_MAX_STEPS * B);
    lp_rec = dnew<int>((size_t)HEARTH_GPU_SPEC_MAX_STEPS * 3);
    lp_cmp = dnew<int>(B);
    lp_par = dnew<int>(B);
    lp_path = dnew<int>(B);
    if (rope_dim) lp_rtab = dnew<float>((size_t)cap * rope_dim);
    lp_ustream = dnew<double>((size_t)HEARTH_GPU_SPEC_MAX_STEPS * 128);
    if (!h_lp) ck(hipHostMalloc((void **)&h_lp, sizeof(int) * hxd::LS_FIELDS, hipHostMallocDefault));
    if (!h_lpf) {
        /* fine-grained host memory the commit kernel writes directly */
        ck(hipHostMalloc((void **)&h_lpf, 4 * sizeof(int), hipHostMallocCoherent | hipHostMallocMapped));
        ck(hipHostGetDevicePointer((void **)&d_lpf, h_lpf, 0));
    }
    for (hipEvent_t &ev : lp_ev)
        if (!ev) ck(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    lp_state = dnew<int>(hxd::LS_FIELDS);   /* last: a failure above retries everything */
}

/* RoPE rows of positions [lo, hi) in the table: the same host cosf/sinf values that
 * run_geometry uploads per call (rope_tables, model.c:386-397). Only rows not filled
 * yet are computed: a run's batches extend the filled range, and a batch that starts
 * outside it (after a rewind) starts a new range, so a run after a long prompt pays for
 * its own positions, not every position before them. */
void hearth_engine::loop_rope_table(int lo, int hi) {
    if (!rope_dim) return;
    if (lo < lp_rtab_lo || lo > lp_rtab_hi) lp_rtab_lo = lp_rtab_hi = lo;
    if (hi <= lp_rtab_hi) return;
    const int half = rope_dim / 2, r0 = lp_rtab_hi;
    std::vector<float> tab((size_t)(hi - r0) * rope_dim);
    for (int p = r0; p < hi; p++) {
        float *r = tab.data() + (size_t)(p - r0) * rope_dim;
        for (int j = 0; j < half; j++) {
            const float th = (float)p * inv_freq[j];
            r[2 * j] = host_cosf(th) * c.rope_factor;
            r[2 * j + 1] = host_sinf(th) * c.rope_factor;
        }
    }
    ck(hipMemcpy(lp_rtab + (size_t)r0 * rope_dim, tab.data(), sizeof(float) * tab.size(), hipMemcpyHostToDevice));
    lp_rtab_hi = hi;
}

hxd::LoopArgs hearth_engine::loop_args(int T) {
    hxd::LoopArgs a{};
    a.state = lp_state; a.hist = lp_hist; a.hist_cap = cap + B + 2; a.stops = lp_stops;
    a.out = lp_out; a.out_cap = HEARTH_GPU_SPEC_MAX_STEPS * B; a.rec = lp_rec; a.rec_cap = HEARTH_GPU_SPEC_MAX_STEPS;
    a.tokens = tokens; a.cmp = lp_cmp; a.rope = rope; a.rtab = lp_rtab; a.rope_dim = rope_dim; a.cap = cap;
    a.pos = d_pos; a.result = lp_skey ? lp_samp.result : acc_i + 2 * B; a.T = T; a.hflag = d_lpf;
    if (lp_skey) {
        /* temperature 0 (a penalised argmax) draws nothing: zero uniforms, as the host
         * steps pass */
        a.sampled = lp_spec.temperature > 0.0;
        a.ustream = a.sampled ? lp_ustream : nullptr;
        a.ustream_n = HEARTH_GPU_SPEC_MAX_STEPS * 128;
        a.u = lp_samp.u;
    }
    return a;
}

/* One step (its draft already made): the forward of T rows with the head, the greedy or
 * sampled acceptance of the live rows, the commit and the next step's draft. */
void hearth_engine::loop_step(int T) {
    const hxd::LoopArgs la = loop_args(T);
    forward(T, true, 0);
    if (lp_skey) {
        /* the sampled walk over the live rows (the chain parents of lp_par), penalty context
         * = the committed sequence (it ends with the step's first token) */
        ck(hxl::accept_sample_dev(lp_samp, logits, T, V, tokens, lp_par, lp_spec, lp_hist, lp_state + hxd::LS_LEN,
                                  lp_state + hxd::LS_LIVE, st));
        hxl::loop_commit_draft(la, st);
        return;
    }
    hxd::AcceptArgs a{};
    a.rows = logits; a.n = T; a.V = V; a.tokens = lp_cmp; a.parent = lp_par; a.amax = acc_i + B;
    a.part_v = (float *)acc_part; a.part_i = acc_part + (size_t)T * hxd::ACCEPT_PARTS;
    a.part_f = acc_part + 2 * (size_t)T * hxd::ACCEPT_PARTS;
    a.path = lp_path; a.result = acc_i + 2 * B;
    hxl::accept_greedy_commit(a, la, st);
}

/* A step of T rows whose positions stay below rows: replayed from a captured graph
 * (graphs on), else launched directly with the same row bound. */
void hearth_engine::launch_loop_step(int T, int rows) {
    struct Bound {   /* the launch bounds of a loop step, reset on every exit */
        hearth_engine *e;
        Bound(hearth_engine *x, int rows) : e(x) { e->rows_bound = rows; e->route_live = e->lp_state + hxd::LS_LIVE; }
        ~Bound() { e->rows_bound = 0; e->route_live = nullptr; }
    };
    if (!graph_on) {
        Bound b(this, rows);
        loop_step(T);
        return;
    }
    Captured *cg = nullptr;
    for (Captured &g : graphs)
        if (g.loop && g.T == T && g.rows == rows && g.skey == lp_skey) cg = &g;
    if (!cg) {
        if (graphs.size() >= 32) {
            (void)hipGraphExecDestroy(graphs.front().exec);
            (void)hipGraphDestroy(graphs.front().graph);
            graphs.erase(graphs.begin());
        }
        Captured g{T, 1, rows, true, true, lp_skey, nullptr, nullptr};
        ck(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        try {
            Bound b(this, rows);
            loop_step(T);
        } catch (const DeviceError &) {
            hipGraph_t dead = nullptr;
            if (hipStreamEndCapture(st, &dead) == hipSuccess && dead) (void)hipGraphDestroy(dead);
            throw;
        }
        ck(hipStreamEndCapture(st, &g.graph));
        if (graph_report) report_graph(g.graph, "loop step", T);
        const hipError_t e = hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(g.graph);
            throw DeviceError{e};
        }
        graphs.push_back(g);
        cg = &graphs.back();
    }
    ck(hipGraphLaunch(cg->exec, st));
}

/* Routing-trace rows of the T tokens just evaluated: appended to trace_pend, which the
 * call writes out only once it has succeeded (a failed call leaves the trace as it was,
 * as the reference's tpend does, model.c:1287-1323). */
void hearth_engine::write_trace(int T) {
    if (!trace || !c.n_moe) return;
    const size_t n = (size_t)T * c.n_moe * K;
    h_routes.resize(n);
    ck(hipMemcpyAsync(h_routes.data(), route_out, sizeof(int) * n, hipMemcpyDeviceToHost, st));
    ck(hipStreamSynchronize(st));
    const size_t o = trace_pend.size();
    trace_pend.resize(o + 2 * n);
    for (size_t i = 0; i < n; i++) {
        trace_pend[o + 2 * i] = (uint8_t)(h_routes[i] & 0xff);
        trace_pend[o + 2 * i + 1] = (uint8_t)((h_routes[i] >> 8) & 0xff);
    }
}

void hearth_engine::flush_trace() {
    if (trace && !trace_pend.empty() && fwrite(trace_pend.data(), 1, trace_pend.size(), trace) != trace_pend.size()) {
        log_msg(LOG_ERROR, "routing trace: write failed; tracing stopped");
        fclose(trace);
        trace = nullptr;
    }
    trace_pend.clear();
}

int hearth_engine::eval_chunked(const int32_t *tok, int n, float *logits_out, int all_logits) {
    const double t0 = now_s();
    const int start = pos;
    const uint64_t tokens0 = tokens_done, calls0 = forward_calls;
    trace_pend.clear();
    call_mark();
    try {
        for (int off = 0; off < n; off += B) {
            const int T = std::min(B, n - off);
            float *lg = nullptr;
            bool copy_last = false;
            if (logits_out && all_logits) lg = logits_out + (size_t)off * V;
            else if (logits_out && off + T == n) copy_last = true;
            /* all_logits 0: compute the chunk's logits only for its last row */
            run_geometry(tok + off, nullptr, T, lg, false);
            if (copy_last) {
                if (!lg) {
                    /* run_geometry skipped the head: run it for the last row only */
                    timed(&ks.head_s, [&] {
                        hxd::Act last = ax;
                        last.q += (size_t)(T - 1) * ax.nbp * 64;
                        last.d += (size_t)(T - 1) * ax.nbp;
                        last.s += (size_t)(T - 1) * ax.nbp;
                        matmul(lm_head, last, x + (size_t)(T - 1) * D, D, 1, logits, V, true, c.logit_scale);
                    });
                    ck(hipMemcpyAsync(logits_out, logits, sizeof(float) * V, hipMemcpyDeviceToHost, st));
                }
            }
            write_trace(T);
            pos += T;
            tokens_done += T;
            forward_calls++;
        }
        ck(hipStreamSynchronize(st));
        if (profiling) collect_events();
    } catch (const DeviceError &e) {
        log_msg(LOG_ERROR, "HIP error in hearth_eval: %s", hipGetErrorString(e.e));
        call_rollback();
        pos = start;
        tokens_done = tokens0;
        forward_calls = calls0;
        trace_pend.clear();
        return E_IO;
    }
    flush_trace();
    wall_s += now_s() - t0;
    return OK;
}

/* ---------------------------------------------------------------- C ABI */

namespace {
std::atomic<int> g_log_init{0};
void init_log_level(int verbose) {
    const char *s = getenv("HEARTH_LOG");
    if (s && *s) set_log_level(env_int("HEARTH_LOG", LOG_WARN));
    else if (verbose > 0 && get_log_level() < (verbose == 1 ? LOG_INFO : LOG_DEBUG))
        set_log_level(verbose == 1 ? LOG_INFO : LOG_DEBUG);
    g_log_init = 1;
}

bool parse_isa(const char *s, int *out) {
    static const char *names[] = {"auto", "scalar", "avx2", "avx512"};
    while (*s == ' ') s++;
    for (int i = 0; i < 4; i++) {
        const char *a = s, *b = names[i];
        while (*a && *b && ((*a >= 'A' && *a <= 'Z') ? *a - 'A' + 'a' : *a) == *b) { a++; b++; }
        if (!*a && !*b) { *out = i; return true; }
    }
    if (s[0] >= '0' && s[0] <= '3' && s[1] == 0) { *out = s[0] - '0'; return true; }
    return false;
}

int cpu_isa() {
#if defined(__x86_64__) && !defined(__HIP_DEVICE_COMPILE__)
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl") &&
        __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("avx2"))
        return HEARTH_ISA_AVX512;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return HEARTH_ISA_AVX2;
#endif
    return HEARTH_ISA_SCALAR;
}
} // namespace

extern "C" {

HEARTH_API const char *hearth_version(void) { return "0.1.0"; }

HEARTH_API int hearth_cpu_isa(void) { return cpu_isa(); }

HEARTH_API void hearth_default_options(hearth_options *o) {
    if (!o) return;
    std::memset(o, 0, sizeof *o);
    o->cache_gb = 8.0;
    o->direct_io = 1;
    o->policy = HEARTH_POLICY_LFU;
    o->prefetch = HEARTH_PREFETCH_SHARED;
    o->isa = HEARTH_ISA_AUTO;
}

/* reference api.c:108-196: env overrides, validation, defaults; then the model */
HEARTH_API hearth_engine *hearth_open(const hearth_options *in, char *err, size_t errlen) {
    if (err && errlen) err[0] = 0;
    if (!in) { fail(err, errlen, "hearth_open: options are NULL"); return nullptr; }
    hearth_options o = *in;
    init_log_level(o.verbose);
    const char *s = getenv("HEARTH_ISA");
    if (s && *s && !parse_isa(s, &o.isa)) {
        fail(err, errlen, "HEARTH_ISA=%s is not one of auto, scalar, avx2, avx512", s);
        return nullptr;
    }
    o.n_threads = env_int("HEARTH_THREADS", o.n_threads);
    o.n_io_threads = env_int("HEARTH_IO_THREADS", o.n_io_threads);
    o.cache_gb = env_double("HEARTH_CACHE_GB", o.cache_gb);
    if (!o.model_path || !*o.model_path) { fail(err, errlen, "hearth_open: no model path"); return nullptr; }
    if (o.n_mirrors < 0 || o.n_mirrors > 8) { fail(err, errlen, "hearth_open: n_mirrors %d outside 0..8", o.n_mirrors); return nullptr; }
    for (int i = 0; i < o.n_mirrors; i++)
        if (!o.mirror_paths[i] || !*o.mirror_paths[i]) { fail(err, errlen, "hearth_open: mirror %d has no path", i); return nullptr; }
    if (!(o.cache_gb >= 0.0) || std::isinf(o.cache_gb)) { fail(err, errlen, "hearth_open: cache_gb must be a finite number >= 0"); return nullptr; }
    if (!(o.pin_fraction >= 0.0f) || o.pin_fraction > 1.0f) { fail(err, errlen, "hearth_open: pin_fraction must be in [0, 1]"); return nullptr; }
    if (o.n_threads < 0 || o.n_io_threads < 0 || o.max_seq < 0 || o.max_batch < 0 || o.prefetch_extra < 0) {
        fail(err, errlen, "hearth_open: n_threads, n_io_threads, max_seq, max_batch and prefetch_extra must be >= 0");
        return nullptr;
    }
    if (o.policy != HEARTH_POLICY_LRU && o.policy != HEARTH_POLICY_LFU) { fail(err, errlen, "hearth_open: unknown cache policy %d", o.policy); return nullptr; }
    if (o.prefetch < HEARTH_PREFETCH_OFF || o.prefetch > HEARTH_PREFETCH_SHARED) { fail(err, errlen, "hearth_open: unknown prefetch mode %d", o.prefetch); return nullptr; }
    if (o.isa < HEARTH_ISA_AUTO || o.isa > HEARTH_ISA_AVX512) { fail(err, errlen, "hearth_open: unknown ISA %d", o.isa); return nullptr; }
    if (o.isa == HEARTH_ISA_AUTO) o.isa = cpu_isa();
    else if (o.isa > cpu_isa()) { fail(err, errlen, "hearth_open: ISA %d is not supported by this CPU", o.isa); return nullptr; }
    if (o.n_threads == 0) o.n_threads = std::max(1, (int)std::thread::hardware_concurrency());
    if (o.n_io_threads == 0) o.n_io_threads = 8;
    if (o.max_batch == 0) o.max_batch = 512;
    if (o.max_batch > MAX_BATCH) o.max_batch = MAX_BATCH;
    o.direct_io = o.direct_io ? 1 : 0;
    o.warm_start = o.warm_start ? 1 : 0;

    std::unique_ptr<hearth_engine> e(new (std::nothrow) hearth_engine());
    if (!e) { fail(err, errlen, "out of memory"); return nullptr; }
    e->opt = o;
    e->verbose = o.verbose;
    if (const char *dd = getenv("HEARTH_DEBUG_DUMP")) e->dump_dir = dd;
    if (const char *gg = getenv("HEARTH_GPU_GRAPH")) e->graph_on = strcmp(gg, "0") != 0;
    if (const char *gr = getenv("HEARTH_GPU_GRAPH_REPORT")) e->graph_report = strcmp(gr, "0") != 0;
    if (!e->open_model(err, errlen)) return nullptr;
    const char *am = getenv("HEARTH_GPU_ATTN");
    e->attn_mode = e->attn_chunk_ok && am && strcmp(am, "chunked") == 0 ? 1 : 0;
    e->read_ahead = std::max(0, std::min(256, env_int("HEARTH_GPU_READ_AHEAD", 64)));
    log_msg(LOG_INFO, "%s: %s, %d layers (%d MoE), d_model %d, vocab %d, KV %d positions, device %d", o.model_path,
            e->c.arch.c_str(), e->L, e->c.n_moe, e->D, e->V, e->cap, e->dev);
    return e.release();
}

HEARTH_API void hearth_close(hearth_engine *e) { delete e; }

HEARTH_API int hearth_info(hearth_engine *e, hearth_model_info *out) {
    if (!e || !out) return E_ARG;
    std::memset(out, 0, sizeof *out);
    std::snprintf(out->arch, sizeof out->arch, "%s", e->c.arch.c_str());
    out->n_layers = e->L;
    out->d_model = e->D;
    out->vocab_size = e->V;
    out->max_seq = e->c.max_seq;
    out->n_heads = e->H;
    out->n_kv_heads = e->Hkv;
    out->head_dim = e->hd;
    out->attn_kind = e->c.attn_kind;
    out->n_experts = e->E;
    out->top_k = e->K;
    out->expert_ffn_dim = e->c.expert_ffn;
    out->n_moe_layers = e->c.n_moe;
    out->bos_id = e->c.bos_id;
    out->n_eos = (int)std::min<size_t>(8, e->c.eos_ids.size());
    for (int i = 0; i < out->n_eos; i++) out->eos_ids[i] = e->c.eos_ids[i];

    out->expert_bytes = e->mf.expert_region_bytes;
    out->slab_bytes_max = e->mf.slab_bytes_max;
    out->params_total = e->mf.params_total;
    out->params_active = e->mf.params_active;
    out->cache_slots = e->store ? e->store->slots() : e->c.n_moe * e->E;
    out->isa = e->opt.isa;
    out->n_threads = e->opt.n_threads;
    out->n_io_threads = e->opt.n_io_threads;
    return OK;
}

HEARTH_API int hearth_eval(hearth_engine *e, const int32_t *tokens, int n, float *logits, int all_logits) {
    if (!e || n < 0) return E_ARG;
    if (n == 0) return OK;
    if (!tokens) return E_ARG;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= e->V) return E_TOKEN;
    if ((int64_t)e->pos + n > (int64_t)e->cap) return E_CAPACITY;
    if (hipSetDevice(e->dev) != hipSuccess) return E_IO;
    e->tree_n = 0;
    return e->eval_chunked(tokens, n, logits, all_logits ? 1 : 0);
}

HEARTH_API int hearth_pos(hearth_engine *e) { return e ? e->pos : E_ARG; }

HEARTH_API int hearth_reset(hearth_engine *e) {
    if (!e) return E_ARG;
    e->pos = 0;
    e->tree_n = 0;
    return OK;
}

HEARTH_API int hearth_rewind(hearth_engine *e, int pos) {
    if (!e || pos < 0) return E_ARG;
    if (pos > e->pos) return E_CAPACITY;
    e->pos = pos;
    e->tree_n = 0;
    return OK;
}

HEARTH_API int hearth_get_stats(hearth_engine *e, hearth_stats *out) {
    if (!e || !out) return E_ARG;
    std::memset(out, 0, sizeof *out);
    unsigned long long d[2] = {0, 0};
    if (hipSetDevice(e->dev) == hipSuccess && hipStreamSynchronize(e->st) == hipSuccess)
        (void)hipMemcpy(d, e->dstats, sizeof d, hipMemcpyDeviceToHost);
    out->tokens = e->tokens_done;
    out->forward_calls = e->forward_calls;
    out->wall_s = e->wall_s;
    out->attn_s = e->ks.attn_s + e->ks.proj_s;
    out->moe_s = e->ks.router_s + e->ks.expert_s + e->ks.expert_down_s;
    out->dense_s = e->ks.dense_s + e->ks.head_s + e->ks.norm_s;
    out->expert_uses = d[0] - e->stats_base[0];
    out->expert_loads_unique = d[1] - e->stats_base[1];
    if (e->store) {
        const StoreStats &ss = e->store->stats;
        out->prefetch_issued = ss.prefetch_issued - e->store_base.prefetch_issued;
        out->prefetch_used = ss.prefetch_used - e->store_base.prefetch_used;
        out->prefetch_wasted = ss.prefetch_wasted - e->store_base.prefetch_wasted;
        out->cache_hits = ss.hits - e->store_base.hits;
        out->cache_misses = ss.misses - e->store_base.misses;
        out->evictions = ss.evictions - e->store_base.evictions;
        out->bytes_read = ss.bytes_read - e->store_base.bytes_read;
        out->read_s = ss.load_s - e->store_base.load_s;
        out->cache_slots = e->store->slots();
        out->cache_resident = e->store->resident();
    } else {
        out->cache_hits = out->expert_uses;   /* every expert is resident in HBM */
        out->cache_slots = e->c.n_moe * e->E;
        out->cache_resident = out->cache_slots;
    }
    return OK;
}

HEARTH_API void hearth_reset_stats(hearth_engine *e) {
    if (!e) return;
    unsigned long long d[2] = {0, 0};
    if (hipSetDevice(e->dev) == hipSuccess && hipStreamSynchronize(e->st) == hipSuccess)
        (void)hipMemcpy(d, e->dstats, sizeof d, hipMemcpyDeviceToHost);
    e->stats_base[0] = d[0];
    e->stats_base[1] = d[1];
    if (e->store) e->store_base = e->store->stats;
    e->tokens_done = e->forward_calls = 0;
    e->wall_s = 0.0;
    e->ks = hearth_gpu_kstats{};
}

/* FORMAT.md §9; refuses to overwrite an existing non-empty file that is not a trace
 * (reference model.c:1148-1168 rule). */
HEARTH_API int hearth_trace_start(hearth_engine *e, const char *path) {
    if (!e || !path || !*path) return E_ARG;
    FILE *f = fopen(path, "rb");
    if (f) {
        unsigned char m[4];
        fseek(f, 0, SEEK_END);
        const long size = ftell(f);
        fseek(f, 0, SEEK_SET);
        const bool ok = size == 0 || (size >= 4 && fread(m, 1, 4, f) == 4 && m[0] == 'H' && m[1] == 'R' && m[2] == 'T' && m[3] == 'R');
        fclose(f);
        if (!ok) return E_ARG;
    }
    f = fopen(path, "wb");
    if (!f) return E_IO;
    uint32_t hdr[6] = {0x52545248u, 1u, (uint32_t)e->L, (uint32_t)e->E, (uint32_t)e->K, (uint32_t)e->c.n_moe};
    if (fwrite(hdr, 4, 6, f) != 6) { fclose(f); return E_IO; }
    if (e->trace) fclose(e->trace);
    e->trace = f;
    return OK;
}

HEARTH_API int hearth_trace_stop(hearth_engine *e) {
    if (!e) return E_ARG;
    if (e->trace) { fclose(e->trace); e->trace = nullptr; }
    return OK;
}

/* hx_model_route_replay (model.c:1885-1960): "" or NULL turns replay off; else the
 * trace must match the model (E, K, n_moe; n_layers >= n_moe), hold whole rows of
 * n_moe * K little-endian uint16 ids (at most 4 GiB), and every row must name K
 * distinct experts below E. A failed call keeps the previous replay. */
HEARTH_API int hearth_route_replay(hearth_engine *e, const char *path) {
    if (!e) return E_ARG;
    if (!path || !*path) {
        if (e->replay_dev) (void)hipSetDevice(e->dev), (void)hipFree(e->replay_dev);
        e->replay_dev = nullptr;
        e->replay_rows = 0;
        return OK;
    }
    if (!e->c.n_moe) { log_msg(LOG_ERROR, "route replay: the model has no MoE layers"); return E_FORMAT; }
    FILE *f = fopen(path, "rb");
    if (!f) { log_msg(LOG_ERROR, "route replay: cannot open %s", path); return E_IO; }
    std::vector<uint8_t> buf;
    {
        uint8_t chunk[1 << 16];
        size_t got;
        while ((got = fread(chunk, 1, sizeof chunk, f)) > 0) {
            buf.insert(buf.end(), chunk, chunk + got);
            if (buf.size() > (4ull << 30) + 24) break;
        }
        const bool err = ferror(f);
        fclose(f);
        if (err) { log_msg(LOG_ERROR, "route replay: cannot read %s", path); return E_IO; }
    }
    auto rd32 = [&](size_t o) { return (uint32_t)buf[o] | ((uint32_t)buf[o + 1] << 8) | ((uint32_t)buf[o + 2] << 16) | ((uint32_t)buf[o + 3] << 24); };
    const int E = e->E, K = e->K, nm = e->c.n_moe;
    if (buf.size() < 24) { log_msg(LOG_ERROR, "route replay: %s is not a routing trace", path); return E_FORMAT; }
    if (rd32(0) != 0x52545248u || rd32(4) != 1u || rd32(8) < (uint32_t)nm || rd32(12) != (uint32_t)E ||
        rd32(16) != (uint32_t)K || rd32(20) != (uint32_t)nm) {
        log_msg(LOG_ERROR, "route replay: %s does not match this model (needs %d experts, top-%d, %d MoE layers)", path, E,
                K, nm);
        return E_FORMAT;
    }
    const uint64_t row = (uint64_t)nm * K, body = buf.size() - 24;
    if (body == 0 || body % (2 * row) != 0 || body > (1ull << 32)) {
        log_msg(LOG_ERROR, "route replay: %s has a body of %llu bytes (rows of %llu bytes)", path,
                (unsigned long long)body, (unsigned long long)(2 * row));
        return E_FORMAT;
    }
    const uint64_t rows = body / (2 * row);
    std::vector<int> ids(body / 2);
    for (size_t i = 0; i < ids.size(); i++) ids[i] = buf[24 + 2 * i] | (buf[24 + 2 * i + 1] << 8);
    for (uint64_t r = 0; r < rows * nm; r++) {
        const int *v = ids.data() + r * K;
        for (int j = 0; j < K; j++) {
            bool bad = v[j] >= E;
            for (int i = 0; i < j && !bad; i++) bad = v[i] == v[j];
            if (bad) {
                log_msg(LOG_ERROR, "route replay: %s token %llu has an invalid or repeated expert id", path,
                        (unsigned long long)(r / nm));
                return E_FORMAT;
            }
        }
    }
    int *d = nullptr;
    if (hipSetDevice(e->dev) != hipSuccess || hipMalloc((void **)&d, sizeof(int) * ids.size()) != hipSuccess) return E_NOMEM;
    if (hipMemcpy(d, ids.data(), sizeof(int) * ids.size(), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return E_NOMEM;
    }
    if (e->replay_dev) (void)hipFree(e->replay_dev);   /* kernels that read it have finished: eval is synchronous */
    e->replay_dev = d;
    e->replay_rows = (int64_t)rows;
    return OK;
}

/* ---- extensions (hearth_gpu.h) ---- */

HEARTH_API int hearth_verify_tree(hearth_engine *e, const int32_t *tokens, const int32_t *parent, int n, float *logits) {
    if (!e || n < 1 || !tokens) return E_ARG;
    if (n > e->B) return E_ARG;
    for (int i = 0; i < n; i++) {
        if (tokens[i] < 0 || tokens[i] >= e->V) return E_TOKEN;
        if (parent && ((i == 0 && parent[i] != -1) || (i > 0 && (parent[i] < 0 || parent[i] >= i)))) return E_ARG;
    }
    if ((int64_t)e->pos + n > (int64_t)e->cap) return E_CAPACITY;
    if (hipSetDevice(e->dev) != hipSuccess) return E_IO;
    const double t0 = now_s();
    e->trace_pend.clear();
    e->call_mark();
    try {
        e->run_geometry(tokens, parent, n, logits, false);
        e->write_trace(n);
        ck(hipStreamSynchronize(e->st));
        if (e->profiling) e->collect_events();
    } catch (const DeviceError &err) {
        log_msg(LOG_ERROR, "HIP error in hearth_verify_tree: %s", hipGetErrorString(err.e));
        e->call_rollback();
        e->trace_pend.clear();
        return E_IO;
    }
    e->flush_trace();
    e->tree_parent.resize(n);
    for (int i = 0; i < n; i++) e->tree_parent[i] = parent ? parent[i] : i - 1;
    e->tree_n = n;
    e->tokens_done += n;
    e->forward_calls++;
    e->wall_s += now_s() - t0;
    return OK;
}

HEARTH_API int hearth_commit_path(hearth_engine *e, const int32_t *path, int n) {
    if (!e || n < 0 || (n && !path)) return E_ARG;
    if (n > e->tree_n) return E_ARG;
    /* a root path of the last tree: path[0] = 0 and each node the child of the previous */
    for (int j = 0; j < n; j++) {
        if (path[j] < j || path[j] >= e->tree_n || (j && path[j] <= path[j - 1])) return E_ARG;
        if (j == 0 ? path[0] != 0 : e->tree_parent[path[j]] != path[j - 1]) return E_ARG;
    }
    if (hipSetDevice(e->dev) != hipSuccess) return E_IO;
    try {
        bool moves = false;
        for (int j = 0; j < n; j++) moves = moves || path[j] != j;
        if (moves) {
            std::memcpy(e->h_res, path, sizeof(int) * n);
            ck(hipMemcpyAsync(e->acc_i, e->h_res, sizeof(int) * n, hipMemcpyHostToDevice, e->st));
            e->move_kv(e->acc_i, n);
            ck(hipStreamSynchronize(e->st));
        }
    } catch (const DeviceError &err) {
        log_msg(LOG_ERROR, "HIP error in hearth_commit_path: %s", hipGetErrorString(err.e));
        return E_IO;
    }
    e->pos += n;
    e->tree_n = 0;
    return OK;
}

} // extern "C"

namespace {

/* The verify-and-accept calls: forward + head for the tree, the acceptance enqueued by
 * accept(d_parent) (which returns the device path and the device result triple
 * {n_path, final token, status}), then the commit of the accepted path. */
template <class Accept>
int verify_and_commit(hearth_engine *e, const int32_t *tokens, const int32_t *parent, int n, float *logits,
                      int32_t *path_out, int *n_path, int32_t *final_tok, const char *what, Accept accept) {
    if (!e || n < 1 || !tokens || !path_out || !n_path || !final_tok) return E_ARG;
    if (n > e->B) return E_ARG;
    for (int i = 0; i < n; i++) {
        if (tokens[i] < 0 || tokens[i] >= e->V) return E_TOKEN;
        if (parent && ((i == 0 && parent[i] != -1) || (i > 0 && (parent[i] < 0 || parent[i] >= i)))) return E_ARG;
    }
    if ((int64_t)e->pos + n > (int64_t)e->cap) return E_CAPACITY;
    if (hipSetDevice(e->dev) != hipSuccess) return E_IO;
    const double t0 = now_s();
    int np = 0, fin = -1, status = 0;
    e->trace_pend.clear();
    e->call_mark();
    try {
        e->run_geometry(tokens, parent, n, nullptr, false);
        /* logits stay in HBM; the head ran only if requested -> force it here */
        e->timed(&e->ks.head_s, [&] { e->matmul(e->lm_head, e->ax, e->x, e->D, n, e->logits, e->V, true, e->c.logit_scale); });
        if (logits) ck(hipMemcpyAsync(logits, e->logits, sizeof(float) * (size_t)n * e->V, hipMemcpyDeviceToHost, e->st));
        int *d_par = e->acc_i;
        int *h_par = e->h_res;
        for (int i = 0; i < n; i++) h_par[i] = parent ? parent[i] : i - 1;
        ck(hipMemcpyAsync(d_par, h_par, sizeof(int) * n, hipMemcpyHostToDevice, e->st));
        const int *d_path = nullptr, *d_res = nullptr;
        e->timed(&e->ks.accept_s, [&] { accept(d_par, d_path, d_res); });
        ck(hipMemcpyAsync(e->h_res + e->B, d_path, sizeof(int) * n, hipMemcpyDeviceToHost, e->st));
        ck(hipMemcpyAsync(e->h_res + 2 * e->B, d_res, sizeof(int) * 3, hipMemcpyDeviceToHost, e->st));
        ck(hipStreamSynchronize(e->st));
        np = e->h_res[2 * e->B];
        fin = e->h_res[2 * e->B + 1];
        status = e->h_res[2 * e->B + 2];
        if (status == 0) {
            for (int j = 0; j < np; j++) path_out[j] = e->h_res[e->B + j];
            bool moves = false;
            for (int j = 0; j < np; j++) moves = moves || path_out[j] != j;
            if (moves) {
                ck(hipMemcpyAsync(e->acc_i, path_out, sizeof(int) * np, hipMemcpyHostToDevice, e->st));
                e->move_kv(e->acc_i, np);
                ck(hipStreamSynchronize(e->st));
            }
        }
        e->write_trace(n);
        if (e->profiling) e->collect_events();
    } catch (const DeviceError &err) {
        log_msg(LOG_ERROR, "HIP error in %s: %s", what, hipGetErrorString(err.e));
        e->call_rollback();
        e->trace_pend.clear();
        return E_IO;
    }
    if (status != 0) {
        e->trace_pend.clear();
        return E_ARG;
    }
    e->flush_trace();
    *n_path = np;
    *final_tok = fin;
    e->pos += np;
    e->tree_n = 0;
    e->tokens_done += n;
    e->forward_calls++;
    e->wall_s += now_s() - t0;
    return OK;
}

/* rows [0, n) of every layer's cache <-> the snapshot layout of hearth_gpu_kv_export */
int kv_snapshot(hearth_engine *e, int n, float *host, int64_t count, bool to_host) {
    const int64_t W = hearth_gpu_kv_row_floats(e);
    if (count < (int64_t)e->L * n * W) return E_ARG;
    if (hipSetDevice(e->dev) != hipSuccess) return E_IO;
    try {
        const hipMemcpyKind kind = to_host ? hipMemcpyDeviceToHost : hipMemcpyHostToDevice;
        for (int l = 0; l < e->L; l++) {
            float *dev = e->kv + (size_t)l * e->kv_layer, *h = host + (size_t)l * n * W;
            /* (device offset, host offset, floats) of each contiguous piece */
            auto piece = [&](size_t doff, size_t hoff, size_t nf) {
                if (to_host) ck(hipMemcpyAsync(h + hoff, dev + doff, sizeof(float) * nf, kind, e->st));
                else ck(hipMemcpyAsync(dev + doff, h + hoff, sizeof(float) * nf, kind, e->st));
            };
            if (e->mla) {
                piece(0, 0, (size_t)n * e->C);
                piece((size_t)e->cap * e->C, (size_t)n * e->C, (size_t)n * e->rdim);
            } else {
                for (int b = 0; b < 2 * e->Hkv; b++)   /* K groups, then V groups: [cap][hd] each */
                    piece((size_t)b * e->cap * e->hd, (size_t)b * n * e->hd, (size_t)n * e->hd);
            }
        }
        ck(hipStreamSynchronize(e->st));
    } catch (const DeviceError &err) {
        log_msg(LOG_ERROR, "HIP error in the KV snapshot: %s", hipGetErrorString(err.e));
        return E_IO;
    }
    return OK;
}

} // namespace

extern "C" {

HEARTH_API int hearth_verify_greedy(hearth_engine *e, const int32_t *tokens, const int32_t *parent, int n,
                                    int32_t *path_out, int *n_path, int32_t *final_tok, float *logits) {
    return verify_and_commit(e, tokens, parent, n, logits, path_out, n_path, final_tok, "hearth_verify_greedy",
                             [&](int *d_par, const int *&d_path, const int *&d_res) {
        hxd::AcceptArgs a{};
        a.rows = e->logits; a.n = n; a.V = e->V; a.tokens = e->tokens; a.parent = d_par; a.amax = e->acc_i + e->B;
        a.part_v = (float *)e->acc_part; a.part_i = e->acc_part + (size_t)n * hxd::ACCEPT_PARTS;
        a.part_f = e->acc_part + 2 * (size_t)n * hxd::ACCEPT_PARTS;
        a.path = e->depth; /* reuse: depth is not needed after the forward */
        a.result = e->acc_i + 2 * e->B;
        hxl::accept_greedy(a, e->st);
        d_path = a.path;
        d_res = a.result;
    });
}

HEARTH_API int hearth_gpu_spec_loop_ok(hearth_engine *e) { return e && e->loop_ok() ? 1 : 0; }

/* The speculative loop on the device (greedy: smp null; sampled: smp and, at a positive
 * temperature, uni[0 .. n_uni) the run's uniform stream, of which *n_used were consumed). */
static int spec_run(hearth_engine *e, const int32_t *seq, int n_seq, int new_tokens, int max_new, int draft_len,
                    int ngram_n, const int32_t *stop_ids, int n_stop, int max_steps, const hearth_sampler *smp,
                    const double *uni, int n_uni, int32_t *out, int32_t *records, hearth_gpu_spec_result *res,
                    int *n_used) {
    const char *what = smp ? "hearth_gpu_spec_sample" : "hearth_gpu_spec_greedy";
    if (!e || !seq || n_seq < 1 || !out || !records || !res) return E_ARG;
    if (new_tokens < 0 || max_new <= new_tokens || draft_len < 0 || ngram_n < 0) return E_ARG;
    if (n_stop < 0 || n_stop > hxd::LOOP_STOPS_MAX || (n_stop && !stop_ids)) return E_ARG;
    if (max_steps < 1 || max_steps > HEARTH_GPU_SPEC_MAX_STEPS) return E_ARG;
    const int T = draft_len + 1;
    if (T > e->B || T > 128) return E_ARG;
    if (smp) {
        if (!n_used || check_sampler(smp) != OK || T > hxd::SAMPLE_NMAX || e->V > hxd::SAMPLE_VMAX) return E_ARG;
        /* a step uses at most T uniforms */
        if (smp->temperature > 0.0 && (!uni || n_uni < max_steps * T)) return E_ARG;
    }
    if (!e->loop_ok()) {
        log_msg(LOG_ERROR, "%s: not available with expert streaming, route replay, a routing trace or profiling", what);
        return E_ARG;
    }
    if (e->pos != n_seq - 1) return E_ARG;
    for (int i = 0; i < n_seq; i++)
        if (seq[i] < 0 || seq[i] >= e->V) return E_TOKEN;
    /* step s runs at a position <= pos + s T and writes rows below pos + (s + 1) T */
    const int S = std::min(max_steps, (e->cap - e->pos) / T);
    if (S < 1) return E_CAPACITY;
    if (hipSetDevice(e->dev) != hipSuccess) return E_IO;
    const double t0 = now_s();
    const int pos0 = e->pos, rows = std::min(e->cap, (pos0 + S * T + 1023) / 1024 * 1024);
    int launched = 0;
    int state[hxd::LS_FIELDS] = {};
    try {
        ck(hipStreamSynchronize(e->st));
        e->loop_prepare();
        e->loop_rope_table(pos0, std::min(e->cap, pos0 + S * T));
        e->lp_skey = 0;
        if (smp) {
            /* a captured step bakes the sampler settings into its kernel arguments: they
             * key the step (never 0); a larger scratch drops the captured steps */
            const double f[5] = {smp->temperature, (double)smp->top_k, smp->top_p, smp->min_p, smp->repetition_penalty};
            uint64_t k = 1469598103934665603ull;
            for (double x : f) {
                uint64_t bits;
                std::memcpy(&bits, &x, 8);
                k = (k ^ bits) * 1099511628211ull;
            }
            e->lp_skey = k ? k : 1;
            e->lp_spec = hxl::SamplerSpec{smp->temperature, smp->top_p, smp->min_p, smp->repetition_penalty, smp->top_k,
                                          nullptr, 0};
            const int cap0 = e->lp_samp.n_cap;
            ck(e->lp_samp.ensure(T, e->V, false, 0));
            if (e->lp_samp.n_cap != cap0) e->drop_graphs();
            if (smp->temperature > 0.0)
                ck(hipMemcpy(e->lp_ustream, uni, sizeof(double) * (size_t)S * T, hipMemcpyHostToDevice));
        }
        state[hxd::LS_LEN] = n_seq;
        state[hxd::LS_NEW] = new_tokens;
        state[hxd::LS_MAXNEW] = max_new;
        state[hxd::LS_NGRAM] = draft_len ? ngram_n : 0;
        state[hxd::LS_NSTOP] = n_stop;
        state[hxd::LS_KVPOS] = pos0;
        state[hxd::LS_LIVE] = 1;
        /* chain geometry of T rows: depth i, ancestors 0..i; parents i - 1 */
        std::vector<int> depth_h(T), anc_h((size_t)T * e->B, 0), par_h(T);
        for (int i = 0; i < T; i++) {
            depth_h[i] = i;
            par_h[i] = i - 1;
            for (int j = 0; j <= i; j++) anc_h[(size_t)i * e->B + j] = j;
        }
        ck(hipMemcpy(e->lp_state, state, sizeof state, hipMemcpyHostToDevice));
        ck(hipMemcpy(e->lp_hist, seq, sizeof(int) * n_seq, hipMemcpyHostToDevice));
        if (n_stop) ck(hipMemcpy(e->lp_stops, stop_ids, sizeof(int) * n_stop, hipMemcpyHostToDevice));
        ck(hipMemcpy(e->depth, depth_h.data(), sizeof(int) * T, hipMemcpyHostToDevice));
        ck(hipMemcpy(e->anc, anc_h.data(), sizeof(int) * anc_h.size(), hipMemcpyHostToDevice));
        ck(hipMemcpy(e->lp_par, par_h.data(), sizeof(int) * T, hipMemcpyHostToDevice));
        ck(hipMemcpy(e->d_pos, &pos0, sizeof(int), hipMemcpyHostToDevice));
        e->geom_chain = 1;
        e->tree_n = 0;
        /* two steps in flight: before step i is queued, step i - 2 has finished, and step
         * i - 1 too when it could spend the token budget (a step yields at most T tokens),
         * so a run that ends on its budget queues no step after the last; a stop token or
         * bad logits can leave two more, which commit nothing. Step i's commit writes its
         * (LS_NEW, LS_DONE) pair to h_lpf + 2 (i & 1) (LS_BSTEP counts the batch's
         * commits from 0); step i + 2, which reuses the pair, is queued only after it is
         * read. */
        /* the first step's draft; every step then drafts the next after its commit */
        hxl::loop_draft(e->loop_args(T), e->st);
        int seen = new_tokens;   /* tokens yielded as of the last step read */
        auto finished = [&](int j) {
            ck(hipEventSynchronize(e->lp_ev[j & 1]));
            const volatile int *f = e->h_lpf + 2 * (j & 1);
            seen = f[0];
            return f[1] != hxd::LOOP_RUNNING;
        };
        for (int i = 0; i < S; i++) {
            if (i >= 2 && finished(i - 2)) break;
            if (i >= 1 && seen + T >= max_new && finished(i - 1)) break;
            e->launch_loop_step(T, rows);
            launched++;
            ck(hipEventRecord(e->lp_ev[i & 1], e->st));
        }
        ck(hipMemcpyAsync(e->h_lp, e->lp_state, sizeof(int) * hxd::LS_FIELDS, hipMemcpyDeviceToHost, e->st));
        ck(hipStreamSynchronize(e->st));
        std::memcpy(state, e->h_lp, sizeof state);
        const int nout = std::min(state[hxd::LS_NOUT], S * T), nst = std::min(state[hxd::LS_STEP], S);
        if (nout) ck(hipMemcpy(out, e->lp_out, sizeof(int) * nout, hipMemcpyDeviceToHost));
        if (nst) ck(hipMemcpy(records, e->lp_rec, sizeof(int) * 3 * nst, hipMemcpyDeviceToHost));
        res->n_out = nout;
        res->n_steps = nst;
    } catch (const DeviceError &err) {
        log_msg(LOG_ERROR, "HIP error in %s: %s", what, hipGetErrorString(err.e));
        e->lp_skey = 0;
        return E_IO;
    }
    e->lp_skey = 0;
    res->finish = state[hxd::LS_DONE];
    res->stop_id = state[hxd::LS_STOP];
    res->pos = state[hxd::LS_KVPOS];
    if (n_used) *n_used = state[hxd::LS_UOFF];
    e->pos = state[hxd::LS_KVPOS];
    e->tokens_done += (uint64_t)launched * T;
    e->forward_calls += launched;
    e->wall_s += now_s() - t0;
    return OK;
}

HEARTH_API int hearth_gpu_spec_greedy(hearth_engine *e, const int32_t *seq, int n_seq, int new_tokens, int max_new,
                                      int draft_len, int ngram_n, const int32_t *stop_ids, int n_stop, int max_steps,
                                      int32_t *out, int32_t *records, hearth_gpu_spec_result *res) {
    return spec_run(e, seq, n_seq, new_tokens, max_new, draft_len, ngram_n, stop_ids, n_stop, max_steps, nullptr,
                    nullptr, 0, out, records, res, nullptr);
}

HEARTH_API int hearth_gpu_spec_sample(hearth_engine *e, const int32_t *seq, int n_seq, int new_tokens, int max_new,
                                      int draft_len, int ngram_n, const int32_t *stop_ids, int n_stop, int max_steps,
                                      const hearth_sampler *smp, const double *uniforms, int n_uniforms, int32_t *out,
                                      int32_t *records, hearth_gpu_spec_result *res, int *n_used) {
    if (!smp) return E_ARG;
    return spec_run(e, seq, n_seq, new_tokens, max_new, draft_len, ngram_n, stop_ids, n_stop, max_steps, smp,
                    uniforms, n_uniforms, out, records, res, n_used);
}

HEARTH_API int hearth_verify_sample(hearth_engine *e, const int32_t *tokens, const int32_t *parent, int n,
                                    const hearth_sampler *s, const double *q, const double *u, int32_t *path_out,
                                    int *n_path, int32_t *final_tok, float *logits) {
    if (!e || !u || check_sampler(s) != OK) return E_ARG;
    if (n > hxd::SAMPLE_NMAX || e->V > hxd::SAMPLE_VMAX) return E_ARG;
    return verify_and_commit(e, tokens, parent, n, logits, path_out, n_path, final_tok, "hearth_verify_sample",
                             [&](int *d_par, const int *&d_path, const int *&d_res) {
        const int n_ctx = s->repetition_penalty != 1.0 ? s->n_context : 0;
        ck(e->samp.ensure(n, e->V, q != nullptr, n_ctx));
        hxl::SamplerSpec sp{s->temperature, s->top_p, s->min_p, s->repetition_penalty, s->top_k, s->context, n_ctx};
        ck(hxl::accept_sample(e->samp, e->logits, n, e->V, e->tokens, d_par, sp, q, u, e->st, false,
                              hxl::max_siblings(parent, n)));
        d_path = e->samp.path;
        d_res = e->samp.result;
    });
}

HEARTH_API int hearth_gpu_verify_sample_dq(hearth_engine *e, const int32_t *tokens, const int32_t *parent, int n,
                                           const hearth_sampler *s, const double *q_dev, const double *u,
                                           int32_t *path_out, int *n_path, int32_t *final_tok, float *logits) {
    if (!e || !u || !q_dev || check_sampler(s) != OK) return E_ARG;
    if (n > hxd::SAMPLE_NMAX || e->V > hxd::SAMPLE_VMAX) return E_ARG;
    hipPointerAttribute_t pa{};
    if (hipPointerGetAttributes(&pa, q_dev) != hipSuccess || pa.type != hipMemoryTypeDevice || pa.device != e->dev) {
        (void)hipGetLastError();
        log_msg(LOG_ERROR, "hearth_gpu_verify_sample_dq: q is not device memory of the engine's GPU");
        return E_ARG;
    }
    return verify_and_commit(e, tokens, parent, n, logits, path_out, n_path, final_tok, "hearth_gpu_verify_sample_dq",
                             [&](int *d_par, const int *&d_path, const int *&d_res) {
        const int n_ctx = s->repetition_penalty != 1.0 ? s->n_context : 0;
        ck(e->samp.ensure(n, e->V, false, n_ctx));
        hxl::SamplerSpec sp{s->temperature, s->top_p, s->min_p, s->repetition_penalty, s->top_k, s->context, n_ctx};
        ck(hxl::accept_sample(e->samp, e->logits, n, e->V, e->tokens, d_par, sp, q_dev, u, e->st, true,
                              hxl::max_siblings(parent, n)));
        d_path = e->samp.path;
        d_res = e->samp.result;
    });
}

HEARTH_API void *hearth_gpu_malloc(hearth_engine *e, size_t bytes) {
    if (!e || !bytes || hipSetDevice(e->dev) != hipSuccess) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

HEARTH_API int hearth_gpu_upload(hearth_engine *e, void *dst, const void *src, size_t bytes) {
    if (!e || !dst || (!src && bytes)) return E_ARG;
    if (hipSetDevice(e->dev) != hipSuccess || hipStreamSynchronize(e->st) != hipSuccess ||
        hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        return E_IO;
    }
    return OK;
}

HEARTH_API int hearth_gpu_free(hearth_engine *e, void *p) {
    if (!e) return E_ARG;
    if (!p) return OK;
    if (hipSetDevice(e->dev) != hipSuccess || hipStreamSynchronize(e->st) != hipSuccess || hipFree(p) != hipSuccess) {
        (void)hipGetLastError();
        return E_IO;
    }
    return OK;
}

HEARTH_API int hearth_gpu_set_attn_mode(hearth_engine *e, int mode) {
    if (!e || (mode != HEARTH_GPU_ATTN_CANONICAL && mode != HEARTH_GPU_ATTN_CHUNKED)) return E_ARG;
    if (mode == HEARTH_GPU_ATTN_CHUNKED && !e->attn_chunk_ok) return E_ARG;
    if (mode != e->attn_mode) {
        e->drop_graphs();
        e->attn_mode = mode;
    }
    return OK;
}

HEARTH_API int hearth_gpu_get_attn_mode(hearth_engine *e) { return e ? e->attn_mode : E_ARG; }

HEARTH_API int hearth_gpu_set_profiling(hearth_engine *e, int on) {
    if (!e) return E_ARG;
    e->profiling = on < 0 ? 0 : (on > 2 ? 2 : on);
    return OK;
}

HEARTH_API int hearth_gpu_get_kstats(hearth_engine *e, hearth_gpu_kstats *out) {
    if (!e || !out) return E_ARG;
    *out = e->ks;
    unsigned long long d[2] = {0, 0};
    if (hipSetDevice(e->dev) == hipSuccess && hipStreamSynchronize(e->st) == hipSuccess)
        (void)hipMemcpy(d, e->dstats, sizeof d, hipMemcpyDeviceToHost);
    uint64_t per_gu = 0, per_dn = 0;
    for (const Layer &l : e->layers)
        if (l.moe) { per_gu = l.expert_gateup_bytes; per_dn = l.expert_bytes_each - l.expert_gateup_bytes; break; }
    out->expert_bytes = (d[1] - e->ks_base) * per_gu;
    out->expert_down_bytes = (d[1] - e->ks_base) * per_dn;
    return OK;
}

HEARTH_API void hearth_gpu_reset_kstats(hearth_engine *e) {
    if (!e) return;
    e->ks = hearth_gpu_kstats{};
    unsigned long long d[2] = {0, 0};
    if (hipSetDevice(e->dev) == hipSuccess && hipStreamSynchronize(e->st) == hipSuccess)
        (void)hipMemcpy(d, e->dstats, sizeof d, hipMemcpyDeviceToHost);
    e->ks_base = d[1];
}

HEARTH_API int hearth_gpu_get_store_info(hearth_engine *e, hearth_gpu_store_info *out) {
    if (!e || !out) return E_ARG;
    *out = hearth_gpu_store_info{};
    if (!e->store) return OK;
    try {
        ck(hipSetDevice(e->dev));
        e->store->harvest(true);
    } catch (const DeviceError &) {
        return E_IO;
    }
    out->streamed = 1;
    out->host_tier = e->store->host_tier();
    out->slots = e->store->slots();
    out->slot_bytes = e->store->slot_bytes();
    out->host_tier_bytes = e->store->host_tier_bytes();
    out->copy_s = e->store->stats.copy_s;
    return OK;
}

HEARTH_API int64_t hearth_gpu_kv_row_floats(hearth_engine *e) {
    if (!e) return E_ARG;
    return e->mla ? (int64_t)e->C + e->rdim : 2 * (int64_t)e->Hkv * e->hd;
}


HEARTH_API int hearth_gpu_kv_export(hearth_engine *e, int n, float *dst, int64_t count) {
    if (!e || n < 0 || n > e->pos || (n && !dst)) return E_ARG;
    return n ? kv_snapshot(e, n, dst, count, true) : OK;
}

HEARTH_API int hearth_gpu_kv_import(hearth_engine *e, int n, const float *src, int64_t count) {
    if (!e || n < 0 || (n && !src)) return E_ARG;
    if (n > e->cap) return E_CAPACITY;
    const int rc = n ? kv_snapshot(e, n, const_cast<float *>(src), count, false) : OK;
    if (rc == OK) {
        e->pos = n;
        e->tree_n = 0;
    }
    return rc;
}

HEARTH_API int hearth_gpu_device(char *name, size_t n) {
    const int d = device_index();
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, d) != hipSuccess) return E_IO;
    if (name && n) std::snprintf(name, n, "%s (%s)", p.name, p.gcnArchName);
    return d;
}

} // extern "C"
